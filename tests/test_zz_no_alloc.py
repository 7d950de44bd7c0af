"""GPU parity of llhip_attention_noalloc (the allocation-free attention entry point, its split-context
partials in a static device array) with llhip_attention (partials in the caller's workspace) and
with the C oracle: bit-exact on every one of consecutive calls, each later call smaller than a call
before it (the reduced-split plan of call 2 included), through the C ABI."""
from __future__ import annotations

import numpy as np
import pytest

from llaccel_amd import _lib
from oracle import golden_np as O
from tests.gpu_helpers import down, ptr, stream, up, workspace

pytestmark = pytest.mark.gpu

# M, H, Hkv, D, pos, max_seq: the first four take the split-context path (the third needs fewer
# splits than llhip_attention takes: its natural plan's partials exceed the static array), the last
# two the single-launch kernels (no scratch)
CALLS = [
    (1, 16, 8, 128, 4095, 4096),
    (1, 16, 8, 128, 2100, 4096),
    (1, 64, 8, 256, 2047, 2048),
    (16, 8, 2, 256, 2020, 2048),
    (1, 14, 2, 64, 700, 1024),
    (40, 14, 2, 64, 0, 64),
]


def _run(entry, q, kd, vd, M, H, Hkv, D, pos, max_seq, Ms, Ss, Mo, So, pb):
    t = __import__("torch")
    out = t.full((M, H * D), 77, dtype=t.int8, device="cuda")
    args = [ptr(q), M, H, Hkv, D, H * D, pos, None, None, 0, ptr(kd), ptr(vd), max_seq, Ms, Ss, Mo, So, pb, ptr(out),
            H * D]
    if entry == "llhip_attention":
        args.append(ptr(workspace()))
    _lib.call(entry, *args, stream())
    return down(out)


def test_noalloc_attention_equals_workspace_attention():
    scratch = int(_lib.lib().llhip_workspace_bytes())  # the allocating entry point's workspace
    assert scratch > 4 << 20
    for i, (M, H, Hkv, D, pos, max_seq) in enumerate(CALLS):
        print(f"noalloc call {i}: M={M} H={H} Hkv={Hkv} D={D} pos={pos}", flush=True)
        rng = np.random.default_rng(100 + i)
        kc = rng.integers(-128, 128, (Hkv, max_seq, D)).astype(np.int8)
        vc = rng.integers(-128, 128, (Hkv, max_seq, D)).astype(np.int8)
        q = rng.integers(-128, 128, (M, H * D))
        Ms, Ss = int(rng.integers(1 << 30, 1 << 31)), 31 + int(round(np.log2(5372 * np.sqrt(D) / 768)))
        Mo, So = int(rng.integers(1 << 30, 1 << 31)), 38
        qd, kd, vd = up(q, np.int8), up(kc, np.int8), up(vc, np.int8)
        for pb in (15, 8):
            want = _run("llhip_attention", qd, kd, vd, M, H, Hkv, D, pos, max_seq, Ms, Ss, Mo, So, pb)
            got = _run("llhip_attention_noalloc", qd, kd, vd, M, H, Hkv, D, pos, max_seq, Ms, Ss, Mo, So, pb)
            assert np.array_equal(got, want), (i, pb)
            assert np.array_equal(got, O.attention_c(q, kc, vc, pos, H, Hkv, D, Ms, Ss, Mo, So, pb)), (i, pb)
        assert np.abs(got).max() > 0


def test_noalloc_attention_errors_match():
    t = __import__("torch")
    q = t.zeros((1, 64), dtype=t.int8, device="cuda")
    kc = t.zeros((1, 64, 64), dtype=t.int8, device="cuda")
    with pytest.raises(ValueError, match="prob_bits"):
        _lib.call("llhip_attention_noalloc", ptr(q), 1, 1, 1, 64, 64, 0, None, None, 0, ptr(kc), ptr(kc), 64, 1, 0, 1,
                  0, 9, ptr(q), 64, stream())
    with pytest.raises(ValueError, match="max_seq"):
        _lib.call("llhip_attention_noalloc", ptr(q), 1, 1, 1, 64, 64, 64, None, None, 0, ptr(kc), ptr(kc), 64, 1, 0, 1,
                  0, 15, ptr(q), 64, stream())
