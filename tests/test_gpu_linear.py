"""GPU parity of the gemm engine (llhip_linear) against the CPU oracle, bit-exact.

Covers BASELINE config 2 (M in {1,16,128,2048} x (K,N) in {(896,896),(896,4864),(4864,896),
(896,151936)}) plus every epilogue, bias, i8/i16 output, ragged K/N/M, split-K on and off, and both
K-tile sizes of the MFMA kernels (128 bytes when K % 128 == 0, else 64: K = 192, 576).
At M=2048 x N=151936 the oracle checks 8 sampled rows over all columns and 96 sampled
columns over all rows (an output element depends only on its A row and W row)."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from oracle import golden_np as O
from tests.gpu_helpers import gpu_linear, random_rq

pytestmark = pytest.mark.gpu
SHAPES_KN = [(896, 896), (896, 4864), (4864, 896), (896, 151936)]


def _operands(rng, M, K, N, out_i8=True):
    a = rng.integers(-127, 128, (M, K)).astype(np.int8)
    w = rng.integers(-127, 128, (N, K)).astype(np.int8)
    return a, w, random_rq(rng, N, K, out_i8)


@pytest.mark.parametrize("K,N", SHAPES_KN)
@pytest.mark.parametrize("M", [1, 16, 128, 2048])
def test_config2_sweep(M, K, N):
    rng = np.random.default_rng(M * 7 + K + N)
    a, w, rq = _operands(rng, M, K, N)
    got = gpu_linear(a, w, rq, out_i8=True)
    if M * N * K <= 20e9:
        want = O.linear_c(a, w, rq, None, True, "none", None, 0, None)
        assert np.array_equal(got, want)
    else:
        rows = np.sort(rng.choice(M, 8, replace=False))
        cols = np.sort(rng.choice(N, 96, replace=False))
        want_r = O.linear_c(a[rows], w, rq, None, True, "none", None, 0, None)
        want_c = O.linear_c(a, w[cols], rq[cols], None, True, "none", None, 0, None)
        assert np.array_equal(got[rows], want_r)
        assert np.array_equal(got[:, cols], want_c)
    # outputs are not degenerate (the requant spans the i8 range)
    assert got.min() < -60 and got.max() > 60 and np.mean(np.abs(got) == 127) < 0.2


@pytest.mark.parametrize("epilogue", ["none", "resadd", "silu", "mul"])
@pytest.mark.parametrize("M", [1, 3, 16, 40, 200])
def test_epilogues_and_bias(M, epilogue):
    rng = np.random.default_rng(M + len(epilogue))
    K, N = 896, 1152
    a, w, rq = _operands(rng, M, K, N, out_i8=False)
    bias = rng.integers(-(2**31), 2**31 - 1, N) if M != 3 else rng.integers(-3000, 3000, N)
    aux = rng.integers(-32768, 32768, (M, N))
    silu = {"Mi": 1 << 30, "Si": 30, "sh_out": 16}
    kw = dict(bias=bias, out_i8=False, epilogue=epilogue, aux=aux if epilogue in ("resadd", "mul") else None,
              aux_shift=11 if epilogue == "mul" else 0, silu=silu if epilogue == "silu" else None)
    got = gpu_linear(a, w, rq, **kw)
    want = O.linear_c(a, w, rq, bias, False, epilogue, kw["aux"], kw["aux_shift"], kw["silu"])
    assert np.array_equal(got, want)


@pytest.mark.parametrize("M,K,N", [(1, 64, 64), (16, 64, 172), (16, 172, 64), (5, 16, 3), (1, 4864, 896),
                                   (17, 172, 33), (33, 96, 130), (2, 1, 5), (16, 65, 17), (300, 64, 1000),
                                   (300, 576, 1000)])
def test_ragged_shapes(M, K, N):
    rng = np.random.default_rng(M * 131 + K * 7 + N)
    a, w, rq = _operands(rng, M, K, N, out_i8=False)
    bias = rng.integers(-5000, 5000, N)
    got = gpu_linear(a, w, rq, bias=bias)
    assert np.array_equal(got, O.linear_c(a, w, rq, bias, False, "none", None, 0, None))


def test_split_k_matches_unsplit_and_self_cleans():
    """The split-K path (workspace) and the one-wave-per-tile path give identical results, and
    repeated calls stay exact (the workspace is left zeroed)."""
    rng = np.random.default_rng(5)
    a, w, rq = _operands(rng, 1, 4864, 896)
    r1 = gpu_linear(a, w, rq, out_i8=True, ws=True)
    r2 = gpu_linear(a, w, rq, out_i8=True, ws=False)
    r3 = gpu_linear(a, w, rq, out_i8=True, ws=True)
    want = O.linear_c(a, w, rq, None, True, "none", None, 0, None)
    assert np.array_equal(r1, want) and np.array_equal(r2, want) and np.array_equal(r3, want)


def test_extreme_operands():
    """All -128 operands: |acc| = K * 2^14 at K=4864, full-range bias, M = 2^31 - 1."""
    K, N = 4864, 64
    a = np.full((16, K), -128, np.int8)
    w = np.full((N, K), -128, np.int8)
    w[1::2] = 127
    rq = np.stack([np.full(N, 2**31 - 1), np.arange(N) % 64], 1).astype(np.int32)
    bias = np.where(np.arange(N) % 3 == 0, 2**31 - 1, -(2**31))
    for out_i8 in (True, False):
        got = gpu_linear(a, w, rq, bias=bias, out_i8=out_i8)
        assert np.array_equal(got, O.linear_c(a, w, rq, bias, out_i8, "none", None, 0, None))


def test_error_paths():
    rng = np.random.default_rng(1)
    a, w, rq = _operands(rng, 2, 64, 16)
    with pytest.raises(ValueError, match="i8 output"):
        gpu_linear(a, w, rq, out_i8=True, epilogue="resadd", aux=np.zeros((2, 16)))
    with pytest.raises(ValueError):
        gpu_linear(a, w, rq, out_i8=False, epilogue="mul", aux=np.zeros((2, 16)), aux_shift=64)


@pytest.mark.parametrize("epilogue,out_i8", [("none", True), ("none", False), ("resadd", False), ("silu", False),
                                             ("mul", False)])
def test_large_gemm_path_ragged_with_epilogues(epilogue, out_i8):
    """Shapes large enough for the 256x256 LDS-ring MFMA kernel, with M and N not multiples of
    the block tile, a full-range bias and every epilogue; sampled rows x all columns and all
    rows x sampled columns against the oracle."""
    rng = np.random.default_rng(len(epilogue) + out_i8)
    M, K, N = 300, 896, 76000
    a, w, rq = _operands(rng, M, K, N, out_i8=out_i8)
    bias = rng.integers(-(2**31), 2**31 - 1, N)
    aux = rng.integers(-32768, 32768, (M, N)) if epilogue in ("resadd", "mul") else None
    silu = {"Mi": 1 << 30, "Si": 30, "sh_out": 16} if epilogue == "silu" else None
    sh = 11 if epilogue == "mul" else 0
    got = gpu_linear(a, w, rq, bias=bias, out_i8=out_i8, epilogue=epilogue, aux=aux, aux_shift=sh, silu=silu)
    rows = np.array([0, 1, 127, 128, 255, 256, 298, 299])
    cols = np.concatenate([np.arange(0, 40), np.arange(75900, 76000), rng.choice(N, 60, replace=False)])
    want_r = O.linear_c(a[rows], w, rq, bias, out_i8, epilogue, None if aux is None else aux[rows], sh, silu)
    want_c = O.linear_c(a, w[cols], rq[cols], bias[cols], out_i8, epilogue, None if aux is None else aux[:, cols], sh,
                        silu)
    assert np.array_equal(got[rows], want_r)
    assert np.array_equal(got[:, cols], want_c)


@pytest.mark.parametrize("epilogue,out_i8", [("none", True), ("none", False), ("resadd", False), ("silu", False),
                                             ("mul", False)])
@pytest.mark.parametrize("M,K,N", [(512, 4864, 896), (300, 2048, 900), (2048, 4864, 896), (130, 4864, 130),
                                   (512, 896, 896), (33, 256, 130), (2048, 256, 1152)])
def test_split_k_gemm(M, K, N, epilogue, out_i8):
    """Prompt-sized GEMMs with too few output tiles for the GPU take the split-K path (int32
    partial planes in the workspace, summed by a second kernel): equal to the oracle and to the
    unsplit kernel (no workspace), with a full-range bias and every epilogue; ragged M and N.  The
    2048-row shapes: K = 4864 on 64x128 tiles split along K, K = 256 on 64x128 tiles unsplit."""
    rng = np.random.default_rng(M + K + N + len(epilogue) + out_i8)
    a, w, rq = _operands(rng, M, K, N, out_i8=out_i8)
    bias = rng.integers(-(2**31), 2**31 - 1, N)
    aux = rng.integers(-32768, 32768, (M, N)) if epilogue in ("resadd", "mul") else None
    silu = {"Mi": 1 << 30, "Si": 30, "sh_out": 16} if epilogue == "silu" else None
    sh = 11 if epilogue == "mul" else 0
    kw = dict(bias=bias, out_i8=out_i8, epilogue=epilogue, aux=aux, aux_shift=sh, silu=silu)
    got = gpu_linear(a, w, rq, **kw)
    assert np.array_equal(got, gpu_linear(a, w, rq, ws=False, **kw))
    rows = np.unique(np.concatenate([np.arange(4), np.arange(M - 4, M), rng.choice(M, 12, replace=False)]))
    want = O.linear_c(a[rows], w, rq, bias, out_i8, epilogue, None if aux is None else aux[rows], sh, silu)
    assert np.array_equal(got[rows], want)


@pytest.mark.parametrize("epilogue,out_i8", [("none", True), ("resadd", False)])
@pytest.mark.parametrize("M,K,N", [(4100, 256, 1000), (8192, 896, 896), (2100, 4864, 300), (16384, 128, 4096),
                                   (3000, 2048, 1000), (4608, 1024, 32768)])
def test_gemm_tile_orders(M, K, N, epilogue, out_i8):
    """The MFMA GEMM's tile orders.  At least four times as many rows as columns: N-block fastest (an
    XCD's run of tiles shares A rows) -- ragged M and N on 128x128 tiles, 448 tiles of 128x128, a split
    along K on 64x64 tiles, persistent workgroups (4096 tiles).  More A than an L2 holds otherwise:
    M-block fastest within groups of M-blocks -- a partial last group (3000 rows) and persistent
    workgroups (4608 x 1024 x 32768: groups of 8 256-row or 16 128-row blocks).  Sampled rows against the
    oracle, all columns."""
    rng = np.random.default_rng(M + K + N + out_i8)
    a, w, rq = _operands(rng, M, K, N, out_i8=out_i8)
    bias = rng.integers(-(2**31), 2**31 - 1, N)
    aux = rng.integers(-32768, 32768, (M, N)) if epilogue == "resadd" else None
    got = gpu_linear(a, w, rq, bias=bias, out_i8=out_i8, epilogue=epilogue, aux=aux)
    rows = np.unique(np.concatenate([np.arange(4), np.arange(M - 70, M), rng.choice(M, 24, replace=False)]))
    want = O.linear_c(a[rows], w, rq, bias, out_i8, epilogue, None if aux is None else aux[rows], 0, None)
    assert np.array_equal(got[rows], want)


@pytest.mark.parametrize("M,K", [(2048, 896), (512, 896), (300, 896), (300, 576), (37, 128), (64, 100), (5000, 1024)])
def test_linear_group_equals_separate_launches(M, K):
    """llhip_linear_group (q, k, v of a prompt chunk in one launch: i16, i16 and i8 outputs, bias
    on two of them) equals one llhip_linear launch per problem: 64x64 tiles (512 and 300 rows,
    K = 896), 64x128 tiles (2048 rows; K = 576 with 64-byte K tiles); K = 100 runs the
    per-problem fallback."""
    import ctypes

    from llaccel_amd import _lib
    from tests.gpu_helpers import ptr, stream, torch, up, workspace

    t = torch()
    rng = np.random.default_rng(M + K)
    a = rng.integers(-127, 128, (M, K)).astype(np.int8)
    shapes = [(896, False, True), (128, False, True), (130, True, False)]
    probs = (_lib.LinearProblem * 3)()
    outs, want = [], []
    ad = up(a, np.int8)
    for pr, (N, out8, has_bias) in zip(probs, shapes):
        w = rng.integers(-127, 128, (N, K)).astype(np.int8)
        rq = random_rq(rng, N, K, out8)
        bias = rng.integers(-(2**20), 2**20, N) if has_bias else None
        wd, rqd = up(w, np.int8), up(rq, np.int32)
        bd = up(bias, np.int32) if has_bias else None
        od = t.zeros((M, N + 3), dtype=t.int8 if out8 else t.int16, device="cuda")
        pr.W, pr.N, pr.rq, pr.bias = ptr(wd), N, ptr(rqd), ptr(bd)
        pr.out, pr.ldo, pr.out_i8 = ptr(od), N + 3, int(out8)
        outs.append((od, wd, rqd, bd))
        want.append(gpu_linear(a, w, rq, bias=bias, out_i8=out8))
    _lib.call("llhip_linear_group", ptr(ad), M, K, K, 3, probs, ptr(workspace()), stream())
    for (od, *_keep), (N, _, _), wnt in zip(outs, shapes, want):
        assert np.array_equal(od.cpu().numpy()[:, :N], wnt) and not od.cpu().numpy()[:, N:].any()
    with pytest.raises(ValueError):
        _lib.call("llhip_linear_group", ptr(ad), M, K, K, 5, probs, ptr(workspace()), stream())


# (silu Mi, Si, sh_out, mul_sh, fq_M, fq_S): the model's kind of parameters, then the extremes of the
# shifts the exact double-precision and 32-bit epilogue arithmetic must hold for (0, 31, 32, 52, 53, 63)
PARAMS = [(1 << 30, 30, 16, 11, 1518500250, 38), ((1 << 32) - 1, 0, 31, 31, (1 << 32) - 1, 52),
          ((1 << 32) - 1, 53, 0, 32, 3, 0), (12345, 63, 63, 0, (1 << 31) + 7, 63), (987654321, 52, 32, 30, 1, 53)]


@pytest.mark.parametrize("M,K,N,pad,par", [(512, 896, 4864, 0, 0), (512, 896, 4864, 5, 0), (1024, 256, 4864, 0, 0),
                                           (300, 128, 200, 4, 0),
                                           (200, 192, 256, 0, 0),
                                           (40, 100, 64, 5, 0), (5000, 1024, 1000, 4, 0)]
                         + [(70, 128, 256, 0, i) for i in range(1, 5)])
def test_gate_up_equals_the_three_ops(M, K, N, pad, par):
    """llhip_gate_up (gate linear with the silu epilogue, up linear with the mul epilogue on the
    gate's output, quant of the product, in one launch) equals the three ops run one by one; output
    rows of N + pad elements (pad 0 and 4: the word stores, 5: element stores); 64x64 tiles up to
    three workgroups per CU, 64x128 beyond (1024 rows) and for 64-byte K tiles, their M-blocks in groups
    when A exceeds an L2 (5000 x 1024: groups of 32, 32 and 15 64-row blocks); K = 100 runs the
    op-by-op fallback inside the entry point; PARAMS[1:] put every shift at its extremes."""
    from llaccel_amd import _lib
    from oracle import golden_np as OO
    from tests.gpu_helpers import ptr, stream, torch, up

    t = torch()
    rng = np.random.default_rng(M + K + N)
    a = rng.integers(-127, 128, (M, K)).astype(np.int8)
    wg, wu = (rng.integers(-127, 128, (N, K)).astype(np.int8) for _ in range(2))
    rqg, rqu = random_rq(rng, N, K, False), random_rq(rng, N, K, False)
    bg, bu = rng.integers(-(2**20), 2**20, N), None
    Mi, Si, sh_out, mul_sh, fqM, fqS = PARAMS[par]
    silu = {"Mi": Mi, "Si": Si, "sh_out": sh_out}
    # the three ops in the oracle
    sg = O.linear_c(a, wg, rqg, bg, False, "silu", None, 0, silu)
    f = O.linear_c(a, wu, rqu, None, False, "mul", sg, mul_sh, None)
    fq = OO.vquant(f, fqM, fqS)
    d = _lib.GateUpDesc()
    keep = [up(a, np.int8), up(wg, np.int8), up(rqg, np.int32), up(bg, np.int32), up(wu, np.int8), up(rqu, np.int32)]
    ld = N + pad
    outs = [t.zeros((M, ld), dtype=t.int16, device="cuda"), t.zeros((M, ld), dtype=t.int16, device="cuda"),
            t.zeros((M, ld), dtype=t.int8, device="cuda")]
    d.A, d.M, d.K, d.lda = ptr(keep[0]), M, K, K
    d.Wg, d.rqg, d.bg, d.Wu, d.rqu, d.bu = ptr(keep[1]), ptr(keep[2]), ptr(keep[3]), ptr(keep[4]), ptr(keep[5]), None
    d.N, d.ld = N, ld
    d.silu_Mi, d.silu_Si, d.silu_sh, d.mul_sh, d.fq_M, d.fq_S = silu["Mi"], silu["Si"], silu["sh_out"], mul_sh, fqM, fqS
    d.sg_out, d.f_out, d.fq_out = (ptr(o) for o in outs)
    _lib.call("llhip_gate_up", ctypes.byref(d), stream())
    got = [o.cpu().numpy() for o in outs]
    for g_, w_ in zip(got, (sg, f, fq)):
        assert np.array_equal(g_[:, :N], w_) and not g_[:, N:].any()
    if par == 0:
        assert np.count_nonzero(f) > f.size // 2  # the products are not degenerate
    # NULL gate and up outputs: only the quantised product is written, the same one; the
    # op-by-op fallback (K % 64 != 0) needs them and refuses NULL
    fq2 = t.zeros((M, ld), dtype=t.int8, device="cuda")
    d.sg_out, d.f_out, d.fq_out = None, None, ptr(fq2)
    if K % 64:
        with pytest.raises(ValueError, match="may be NULL only"):
            _lib.call("llhip_gate_up", ctypes.byref(d), stream())
    else:
        _lib.call("llhip_gate_up", ctypes.byref(d), stream())
        assert np.array_equal(fq2.cpu().numpy(), got[2])


@pytest.mark.parametrize("M,K,N", [(512, 4864, 896), (300, 2048, 576), (300, 896, 896), (40, 896, 896), (16, 896, 896),
                                   (16, 4864, 896), (5, 2048, 576), (2, 896, 1024), (512, 896, 896), (256, 1024, 576),
                                   (128, 896, 1024)])
def test_linear_norm_equals_linear_then_rmsnorm_quant(M, K, N):
    """llhip_linear_norm (a resadd linear, then rmsnorm + quant of its output rows) equals the resadd
    linear checked against the oracle followed by the oracle's rmsnorm and quant: with the split-K
    finishing kernel (512 x 4864 x 896, 300 x 2048 x 576) and with the separate launches (unsplit
    300 x 896 x 896, the 40-row tiled path, the GEMV rows of a batch decode launch, M <= 16, and the
    prompt's o_proj shapes 512 x 896 x 896, 256 x 1024 x 576, 128 x 896 x 1024), each twice in a row,
    the first call with another residual."""
    import math

    from llaccel_amd import _lib
    from tests.gpu_helpers import down, ptr, stream, torch, up, workspace

    t = torch()
    rng = np.random.default_rng(M + K + N)
    a, w, rq = _operands(rng, M, K, N, out_i8=False)
    bias = rng.integers(-(1 << 20), 1 << 20, N)
    aux = rng.integers(-20000, 20000, (M, N))
    g = rng.integers(-32768, 32768, N)
    eps_t, C, sh, qM, qS = 12345, int(2**24 * math.sqrt(N)), 24, 1234567891, 38
    ad, wd, rqd, bd, auxd, gd = up(a, np.int8), up(w, np.int8), up(rq, np.int32), up(bias, np.int32), up(aux, np.int16), \
        up(g, np.int16)
    xd = t.zeros((M, N), dtype=t.int16, device="cuda")
    hd = t.zeros((M, N), dtype=t.int16, device="cuda")
    hqd = t.zeros((M, N), dtype=t.int8, device="cuda")
    d = _lib.NormQuantDesc()
    d.x, d.gamma, d.h_out, d.hq_out, d.ldx, d.K = ptr(xd), ptr(gd), ptr(hd), ptr(hqd), N, N
    d.eps_t, d.C, d.sh_post, d.Mq, d.Sq, d.prequant = eps_t, C, sh, qM, qS, 0
    aux_other = up(rng.integers(-20000, 20000, (M, N)), np.int16)
    for ax in (aux_other, auxd):
        _lib.call("llhip_linear_norm", ptr(ad), M, K, K, ptr(wd), N, ptr(rqd), ptr(bd), ptr(ax), N, ptr(xd), N,
                  ctypes.byref(d), ptr(workspace()), stream())
    x_want = O.linear_c(a, w, rq, bias, False, "resadd", aux, 0, None)
    assert np.array_equal(down(xd), x_want)
    h_want = O.rmsnorm(x_want, g, eps_t, C, sh)
    assert np.array_equal(down(hd), h_want) and np.array_equal(down(hqd), O.vquant(h_want, qM, qS))
    d.x = ptr(hd)  # the norm must read the linear's output
    with pytest.raises(ValueError):
        _lib.call("llhip_linear_norm", ptr(ad), M, K, K, ptr(wd), N, ptr(rqd), ptr(bd), ptr(auxd), N, ptr(xd), N,
                  ctypes.byref(d), ptr(workspace()), stream())
