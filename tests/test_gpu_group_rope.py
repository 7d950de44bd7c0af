"""llhip_linear_group_rope (the q, k, v projections of a prompt chunk with the rope -> quant of the q
and k rows and the layer's K/V cache write as the GEMM's epilogue, one launch) against
llhip_linear_group followed by llhip_rope_quant2, bit-exact in every output: the three linear outputs,
the rotated and quantised q and k rows and both caches -- 64x64 tiles (512 and 40 rows) and 64x128
tiles (2100 and 4608 rows, the latter more A than an L2 holds), positions from the
argument, from a device word, per row (own cache slots) and per sequence of a batched prefill -- and
the oracle's rope and quant on one case."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from llaccel_amd import _lib
from oracle import golden_np as O
from tests.gpu_helpers import down, ptr, stream, torch, up, workspace

pytestmark = pytest.mark.gpu

H, HKV, D = 14, 2, 64


def _tables(rows):
    inv = 1e6 ** (-np.arange(0, D, 2) / D)
    ang = np.outer(np.arange(rows), inv)
    return np.round(np.cos(ang) * 16384).astype(np.int64), np.round(np.sin(ang) * 16384).astype(np.int64)


def _rq(rng, N, out8):
    return np.stack([rng.integers(1 << 29, 1 << 31, N), rng.integers(36 if out8 else 30, 40 if out8 else 34, N)], 1)


class _Run:
    """Output buffers of one run (the fused launch or the two launches) and their descriptors."""

    def __init__(self, t, M, slots, max_seq, kc0, vc0):
        z = lambda shape, dt: t.full(shape, 11, dtype=dt, device="cuda")  # noqa: E731
        self.lin = [z((M, H * D), t.int16), z((M, HKV * D), t.int16), z((M, HKV * D), t.int8)]
        self.y = [z((M, H * D), t.int16), z((M, HKV * D), t.int16)]
        self.yq = [z((M, H * D), t.int8), z((M, HKV * D), t.int8)]
        self.kc, self.vc = up(kc0, np.int8), up(vc0, np.int8)

    def outputs(self):
        return [down(x) for x in self.lin + self.y + self.yq + [self.kc, self.vc]]


@pytest.mark.parametrize("M,K,mode", [(512, 896, "pos"), (40, 896, "pos"), (2100, 1024, "pos"), (100, 896, "pos_dev"),
                                      (64, 896, "row_pos"), (128, 896, "seq_rows"), (4608, 1024, "seq_rows")])
def test_group_rope_equals_group_then_rope_quant2(M, K, mode):
    t = torch()
    rng = np.random.default_rng(M + K)
    max_seq = 256 if M <= 128 else 4096  # the positions pos .. pos + M - 1 fit the table and the caches
    slots = M if mode == "row_pos" else (M // 64 if mode == "seq_rows" else 1)
    slot_stride = HKV * max_seq * D if slots > 1 else 0
    pos = 0 if mode == "row_pos" else (10 if mode == "seq_rows" else 37)
    a = rng.integers(-127, 128, (M, K))
    Ns = (H * D, HKV * D, HKV * D)
    W = [rng.integers(-127, 128, (N, K)) for N in Ns]
    rq = [_rq(rng, N, q == 2) for q, N in enumerate(Ns)]
    bias = [rng.integers(-(1 << 18), 1 << 18, Ns[0]), rng.integers(-(1 << 18), 1 << 18, Ns[1]), None]
    c, s = _tables(max_seq)
    kc0 = rng.integers(-128, 128, (slots, HKV, max_seq, D))
    vc0 = rng.integers(-128, 128, (slots, HKV, max_seq, D))
    ad = up(a, np.int8)
    wd = [up(w, np.int8) for w in W]
    rqd = [up(r, np.int32) for r in rq]
    bd = [None if b is None else up(b, np.int32) for b in bias]
    cd, sd = up(c, np.int16), up(s, np.int16)
    posd = t.full((1,), pos, dtype=t.int32, device="cuda")
    rowp = rng.permutation(max_seq)[:M] if mode == "row_pos" else None
    rowpd = up(rowp, np.int32) if rowp is not None else None
    qq, qk = (1234567891, 40), (987654321, 39)

    def descs(run):
        probs = (_lib.LinearProblem * 3)()
        for q, pr in enumerate(probs):
            pr.W, pr.N, pr.rq, pr.bias = ptr(wd[q]), Ns[q], ptr(rqd[q]), ptr(bd[q])
            pr.out, pr.ldo, pr.out_i8 = ptr(run.lin[q]), Ns[q], int(q == 2)
        rd = []
        for q, (n, qp) in enumerate(((H, qq), (HKV, qk))):
            d = _lib.RopeQuantDesc()
            d.x, d.M, d.H, d.D, d.ldx = ptr(run.lin[q]), M, n, D, n * D
            d.cos_tab, d.sin_tab, d.table_rows, d.pos = ptr(cd), ptr(sd), max_seq, pos
            d.pos_dev = ptr(posd) if mode == "pos_dev" else None
            d.row_pos = ptr(rowpd) if mode == "row_pos" else None
            d.seq_rows = 64 if mode == "seq_rows" else 0
            d.y, d.yq, d.qM, d.qS = ptr(run.y[q]), ptr(run.yq[q]), qp[0], qp[1]
            if q == 1:
                d.kc, d.v, d.ldv, d.vc = ptr(run.kc), ptr(run.lin[2]), HKV * D, ptr(run.vc)
                d.max_seq, d.slot_stride = max_seq, slot_stride
            rd.append(d)
        return probs, rd

    print(f"group_rope M={M} K={K} mode={mode}", flush=True)
    fused, split = _Run(t, M, slots, max_seq, kc0, vc0), _Run(t, M, slots, max_seq, kc0, vc0)
    probs, rd = descs(fused)
    _lib.call("llhip_linear_group_rope", ptr(ad), M, K, K, probs, ctypes.byref(rd[0]), ctypes.byref(rd[1]),
              ptr(workspace()), stream())
    probs2, rd2 = descs(split)
    _lib.call("llhip_linear_group", ptr(ad), M, K, K, 3, probs2, ptr(workspace()), stream())
    _lib.call("llhip_rope_quant2", ctypes.byref(rd2[0]), ctypes.byref(rd2[1]), stream())
    names = ["q", "k", "v", "q rope", "k rope", "q quant", "k quant", "K cache", "V cache"]
    for name, x, y in zip(names, fused.outputs(), split.outputs()):
        assert np.array_equal(x, y), name
    if mode == "pos" and M == 40:  # the oracle's linear, rope and quant of the query rows
        lin_q = O.linear_c(a, W[0], rq[0], bias[0], False, "none", None, 0, None)
        assert np.array_equal(down(fused.lin[0]), lin_q)
        yq = O.rope(lin_q, H, D, c, s, pos)
        assert np.array_equal(down(fused.y[0]), yq) and np.array_equal(down(fused.yq[0]), O.vquant(yq, *qq))


def test_group_rope_refuses_what_it_does_not_cover():
    t = torch()
    M, K = 64, 896
    ad = t.zeros((M, K), dtype=t.int8, device="cuda")
    w = t.zeros((H * D, K), dtype=t.int8, device="cuda")
    rqd = t.zeros((H * D, 2), dtype=t.int32, device="cuda")
    outs = [t.zeros((M, H * D), dtype=t.int16, device="cuda") for _ in range(6)]
    vq = t.zeros((M, HKV * D), dtype=t.int8, device="cuda")
    cd = t.zeros((256, D // 2), dtype=t.int16, device="cuda")
    probs = (_lib.LinearProblem * 3)()
    for q, pr in enumerate(probs):
        n = H * D if q == 0 else HKV * D
        pr.W, pr.N, pr.rq, pr.bias = ptr(w), n, ptr(rqd), None
        pr.out, pr.ldo, pr.out_i8 = (ptr(vq) if q == 2 else ptr(outs[q])), n, int(q == 2)

    def desc(q, hd=D):
        d = _lib.RopeQuantDesc()
        n = H if q == 0 else HKV
        d.x, d.M, d.H, d.D, d.ldx = ptr(outs[q]), M, n * D // hd, hd, n * D
        d.cos_tab, d.sin_tab, d.table_rows, d.pos = ptr(cd), ptr(cd), 256, 0
        d.y, d.yq, d.qM, d.qS = ptr(outs[2 + q]), ptr(outs[4 + q]), 1 << 30, 38
        return d

    def call(k, a=None, b=None):
        _lib.call("llhip_linear_group_rope", ptr(ad), M, k, k, probs, ctypes.byref(a or desc(0)),
                  ctypes.byref(b or desc(1)), ptr(workspace()), stream())

    with pytest.raises(ValueError):
        call(K, a=desc(0, hd=128))  # head_dim 128: a 64-column tile is half a head
    with pytest.raises(ValueError):
        call(832)  # K not a multiple of 128
    call(K)  # the same operands otherwise taken
    t.cuda.synchronize()
