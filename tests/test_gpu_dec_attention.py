"""llhip_dec_attention (one decode row's attention + the output projection's partial sums) with its
state (long contexts as ONE launch of H x S workgroups exchanging tagged partials) against the same
call without state (the split-context launches) and against the C oracle's attention with a numpy
output projection, bit-exact, over consecutive launches that share one state."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from llaccel_amd import _lib
from oracle import golden_np as O
from tests.gpu_helpers import ptr, stream, torch, up, workspace

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(4242)


def _launch(q, kc, vc, posd, H, Hkv, D, max_seq, prm, wo, N, state):
    t = torch()
    out = t.full((H * D,), 77, dtype=t.int8, device="cuda")
    acc = t.zeros(N, dtype=t.int32, device="cuda")
    zero = t.full((8 * N,), 5, dtype=t.int32, device="cuda")
    d = _lib.DecAttnDesc()
    d.q, d.kc, d.vc, d.out, d.pos_dev, d.pos = ptr(q), ptr(kc), ptr(vc), ptr(out), ptr(posd), 0
    d.H, d.Hkv, d.D, d.max_seq = H, Hkv, D, max_seq
    d.Ms, d.Ss, d.Mo, d.So, d.prob_bits = prm
    d.wo_panel, d.N, d.acc, d.zero, d.zero_n = ptr(wo), N, ptr(acc), ptr(zero), 8 * N
    d.state, d.state_bytes = (ptr(state), state.numel()) if state is not None else (None, 0)
    _lib.call("llhip_dec_attention", ctypes.byref(d), ptr(workspace()), stream())
    assert int(zero.abs().sum().item()) == 0  # the down projection's accumulators cleared
    return out.cpu().numpy().astype(np.int64), acc.cpu().numpy().astype(np.int64)


@pytest.mark.parametrize("H,Hkv,D,N", [(16, 8, 128, 1024), (14, 2, 64, 896), (9, 3, 64, 576)])
def test_one_launch_attention_equals_split_and_oracle(H, Hkv, D, N):
    t = torch()
    max_seq = 4096
    kc = RNG.integers(-128, 128, (Hkv, max_seq, D)).astype(np.int8)  # the C oracle reads int8 caches
    vc = RNG.integers(-128, 128, (Hkv, max_seq, D)).astype(np.int8)
    wo = RNG.integers(-128, 128, (H, N, D))  # panel [h][n][d] = W[n][h D + d]
    W = wo.transpose(1, 0, 2).reshape(N, H * D)
    kcd, vcd, wod = up(kc, np.int8), up(vc, np.int8), up(wo, np.int8)
    nb = int(_lib.lib().llhip_dec_attn_state_bytes(H, D))
    state = t.zeros(nb, dtype=t.uint8, device="cuda")
    posd = t.zeros(1, dtype=t.int32, device="cuda")
    launches = 0
    for i, (pos, pb) in enumerate(((4095, 15), (4095, 8), (2047, 15), (3000, 8), (36, 15), (0, 15), (4000, 15))):
        print(f"dec_attention H={H} D={D} pos={pos} pb={pb}", flush=True)
        q = RNG.integers(-128, 128, H * D)
        Ms = int(RNG.integers(1 << 30, 1 << 31))
        Ss = 31 + int(round(np.log2(5372 * np.sqrt(D) / 768)))
        Mo, So = int(RNG.integers(1 << 30, 1 << 31)), 38
        qd = up(q, np.int8)
        posd.fill_(pos)
        prm = (Ms, Ss, Mo, So, pb)
        got_o, got_a = _launch(qd, kcd, vcd, posd, H, Hkv, D, max_seq, prm, wod, N, state)
        launches += 1
        want_o, want_a = _launch(qd, kcd, vcd, posd, H, Hkv, D, max_seq, prm, wod, N, None)
        assert np.array_equal(got_o, want_o), (pos, pb)
        assert np.array_equal(got_a, want_a), (pos, pb)
        ref = O.attention_c(q[None, :], kc, vc, pos, H, Hkv, D, Ms, Ss, Mo, So, pb)[0]
        assert np.array_equal(got_o, ref), (pos, pb)
        assert np.array_equal(got_a, W.astype(np.int64) @ ref), (pos, pb)
    n, err = ctypes.c_int64(), ctypes.c_int64()
    _lib.call("llhip_dec_attn_status", ptr(state), ctypes.byref(n), ctypes.byref(err))
    assert err.value == 0 and n.value == launches  # every launch took the one-launch form
