"""GPU parity of the elementwise primitives and vec-engine kernels against the CPU oracle
(bit-exact).  Calls go through llaccel_amd.golden, i.e. through the libllhip C ABI."""
from __future__ import annotations

import ctypes
import math

import numpy as np
import pytest

from llaccel_amd import golden as G
from oracle import golden_np as O

pytestmark = pytest.mark.gpu
RNG = np.random.default_rng(7)


def test_rshr_full_domain():
    vals = np.concatenate([np.array([-(1 << 63), (1 << 63) - 1, -1, 0, 1], np.int64),
                           RNG.integers(-(1 << 63), (1 << 63) - 1, 500, dtype=np.int64)])
    for s in (0, 1, 2, 7, 14, 31, 32, 62, 63):
        assert np.array_equal(G.rshr(vals, s), O.rshr(vals, s))
    shifts = RNG.integers(0, 64, vals.shape[0])
    assert np.array_equal(G.rshr(vals, shifts), O.rshr(vals, shifts))
    assert G.rshr(np.array([5]), 1)[0] == 3 and G.rshr(np.array([-5]), 1)[0] == -2
    with pytest.raises(ValueError):
        G.rshr(np.array([1]), 64)


def test_saturation_and_mulshift():
    v = np.array([-10**9, -32769, -32768, -129, -128, 0, 127, 128, 255, 256, 32767, 32768, 65535, 65536, 10**9])
    for f in ("sat8", "satu8", "sat16", "satu16"):
        assert np.array_equal(getattr(G, f)(v), getattr(O, f)(v)), f
    x = RNG.integers(-(1 << 40), 1 << 40, 4000)
    M = RNG.integers(0, 1 << 32, 4000)
    S = RNG.integers(0, 64, 4000)
    assert np.array_equal(G.mulshift(x, M, S), O.mulshift(x, M, S))
    assert np.array_equal(G.requant16(x >> 10, M, S), O.requant16(x >> 10, M, S))
    assert np.array_equal(G.requant8(x >> 10, M, S), O.requant8(x >> 10, M, S))
    # broadcasting of per-channel parameters like golden.py:329
    acc = RNG.integers(-(1 << 30), 1 << 30, (5, 7))
    Mn, Sn = RNG.integers(1 << 30, 1 << 31, 7)[None, :], RNG.integers(20, 50, 7)[None, :]
    assert np.array_equal(G.requant16(acc, Mn, Sn), O.requant16(acc, Mn, Sn))


def test_isqrt_udiv():
    for t in [0, 1, 2, 3, (1 << 48) - 1, 1 << 47, 65535**2] + RNG.integers(0, 1 << 48, 20).tolist():
        assert G.isqrt48(t) == math.isqrt(t)
    # perfect squares and their neighbours, where a rounded floating-point root can land on
    # either side of the integer root
    n = np.concatenate([np.arange(1, 3000), (1 << 24) - np.arange(1, 3000), RNG.integers(1, 1 << 24, 6000)])
    t = np.concatenate([n * n - 1, n * n, n * n + 1, n * n + 2 * n])
    t = t[(t >= 0) & (t < (1 << 48))]
    want = np.array([math.isqrt(int(v)) for v in t])
    assert np.array_equal(G._elementwise("llhip_isqrt48", [t.astype(np.int64)]), want)
    with pytest.raises(ValueError):
        G.isqrt48(1 << 48)
    assert G.udiv(10, 3) == 3 and G.udiv(10, 0) == 10 and G.udiv(2**31, 65534) == 32769
    assert G.udiv(2**40, 1) == (2**40) & 0xFFFFFFFF
    with pytest.raises(ValueError):
        G.udiv(-1, 2)


def test_silu_vmul_vadd_vquant():
    x = np.arange(-32768, 32768, 3)
    for Mi, Si, sh in ((2**30, 30, 16), (1518500250, 31, 15), (2**31 - 1, 33, 14)):
        assert np.array_equal(G.silu16(x, Mi, Si, sh), O.silu16(x, Mi, Si, sh))
    a = RNG.integers(-32768, 32768, 5000)
    b = RNG.integers(-32768, 32768, 5000)
    for sh in (0, 1, 10, 15, 31):
        assert np.array_equal(G.vmul(a, b, sh), O.vmul(a, b, sh))
        assert np.array_equal(G.vadd(a, b, sh), O.vadd(a, b, sh))
    assert np.array_equal(G.vquant(a, 2**30, 38), O.vquant(a, 2**30, 38))
    assert G.vmul(np.array([1000, -1000, 32767]), np.array([1000, 1000, 32767]), 10).tolist() == [977, -977, 32767]


@pytest.mark.parametrize("K", [16, 64, 128, 172, 576, 896, 1024, 4864])
def test_rmsnorm(K):
    x = RNG.integers(-32768, 32768, (9, K)) >> RNG.integers(0, 12, (9, 1))
    x[0] = 0
    g = RNG.integers(-32768, 32768, K)
    for eps_t, C, sh in ((0, 2**32 - 1, 40), (12345, int(2**24 * math.sqrt(K)), 24), (2**32 - 1, 1, 0)):
        assert np.array_equal(G.rmsnorm(x, g, eps_t, C, sh), O.rmsnorm(x, g, eps_t, C, sh))


@pytest.mark.parametrize("H,D", [(4, 16), (2, 64), (14, 64), (16, 128), (8, 256)])
def test_rope(H, D):
    inv = 1e6 ** (-np.arange(0, D, 2) / D)
    ang = np.outer(np.arange(300), inv)
    c = np.round(np.cos(ang) * 16384).astype(np.int64)
    s = np.round(np.sin(ang) * 16384).astype(np.int64)
    x = RNG.integers(-32768, 32768, (16, H * D))
    for pos in (0, 17, 284):
        assert np.array_equal(G.rope(x, H, D, c, s, pos), O.rope(x, H, D, c, s, pos))


def test_attention_head_known_answers():
    """test_golden_primitives.py:141-155, 197-231 and test_rounding_boundaries.py:19-29 on the GPU."""
    D = 16
    v = RNG.integers(-127, 128, (1, D))
    out = G.attention_head(RNG.integers(-127, 128, D), RNG.integers(-127, 128, (1, D)), v, 2**30, 40, 2155905153, 39)
    assert np.array_equal(out, v[0])
    for pb in (8, 15):
        for dim in (16, 32, 64):
            q = np.zeros(dim, np.int64)
            q[0] = 127
            vals = np.zeros((2, dim), np.int64)
            vals[:, 0] = [-127, 127]
            outs = []
            for off in (0, 126, -128):
                keys = np.zeros((2, dim), np.int64)
                keys[:, 0] = [off, off + 1]
                outs.append(G.attention_head(q, keys, vals, 1 << 30, 24, 1 << 30, 38, pb))
            assert all(np.array_equal(o, outs[0]) for o in outs) and outs[0][0] == 127
            q.fill(127)
            keys = np.array([[-128] * dim, [127] * dim], np.int64)
            assert G.attention_head(q, keys, vals, 2**32 - 1, 0, 1 << 30, 38, pb)[0] == 127
    for T in (1, 2, 100, 171, 255, 256):
        for val in (-128, -1, 0, 127):
            got = G.attention_head(np.zeros(16), np.zeros((T, 16)), np.full((T, 16), val), 1, 0, 1 << 30, 38, 15)
            assert np.max(np.abs(got - val)) <= 1
    assert int(G.attention_head(np.zeros(16), np.zeros((171, 16)), np.full((171, 16), 127), 1, 0, 1 << 30, 38)[0]) == 85


@pytest.mark.parametrize("D", [16, 32, 64, 128, 256])
def test_attention_head_random(D):
    for T in (1, 3, 255, 256, 257, 1000):
        q = RNG.integers(-128, 128, D)
        k = RNG.integers(-128, 128, (T, D))
        v = RNG.integers(-128, 128, (T, D))
        Ms, Ss = int(RNG.integers(1 << 30, 1 << 31)), int(RNG.integers(30, 40))
        Mo, So = int(RNG.integers(1 << 30, 1 << 31)), int(RNG.integers(36, 42))
        for pb in (8, 15):
            assert np.array_equal(G.attention_head(q, k, v, Ms, Ss, Mo, So, pb),
                                  O.attention_head(q, k, v, Ms, Ss, Mo, So, pb)), (T, pb)


def test_exact_blas_matmul():
    """test_exact_blas.py:6-19 on the GPU."""
    for m, n, k in ((1, 17, 16), (4, 33, 4096), (16, 257, 512), (3, 1025, 32)):
        a = RNG.integers(-32768, 32768, (m, k), dtype=np.int64)
        w = RNG.integers(-128, 128, (n, k), dtype=np.int8)
        a[0, :] = -32768
        w[0, :] = -128
        assert np.array_equal(G.exact_blas_matmul(a, w, 17), a @ w.astype(np.int64).T)
    # any integer weight dtype, as the reference accepts (golden.py:226): int8-valued int32 weights, and
    # int16 weights beyond int8 (the FP64 path, exact under the 2^53 bound)
    a = RNG.integers(-1000, 1000, (5, 300), dtype=np.int64)
    for w in (RNG.integers(-128, 128, (70, 300)).astype(np.int32),
              RNG.integers(-32768, 32768, (70, 300)).astype(np.int16)):
        w[0, 0] = np.iinfo(w.dtype).min if w.dtype == np.int16 else -128
        assert np.array_equal(G.exact_blas_matmul(a, w, 3), a @ w.astype(np.int64).T), w.dtype
    with pytest.raises(ValueError, match="bound"):
        G.exact_blas_matmul(np.array([[2**53]], np.int64), np.array([[127]], np.int8))
    with pytest.raises(ValueError, match="integer"):
        G.exact_blas_matmul(np.ones((1, 1)), np.ones((1, 1), np.int8))


@pytest.mark.parametrize("vocab", [1, 7, 8, 9, 2047, 2048, 16385, 151936])
def test_argmax_row_lengths_and_tails(vocab):
    """llhip_argmax_i16 over rows of every tail length (16-byte chunks of 8 values, eight chunks
    per thread in flight), maxima in the last partial chunk and ties across chunks and threads;
    rows at a 16-byte-aligned and at an odd row stride (the one-value-at-a-time form)."""
    from llaccel_amd import _lib
    from tests.gpu_helpers import ptr, stream, torch, up

    t = torch()
    rows = RNG.integers(-32768, 32767, (4, vocab))
    rows[1, -1] = 32767  # the last value
    rows[2, :] = -5
    rows[2, [vocab // 3, vocab - 1]] = 9  # a tie: the lower index wins
    rows[3, :] = 32767  # all equal: index 0
    for ld in (vocab + (-vocab) % 8, vocab + 1):
        buf = np.zeros((4, ld), np.int64)
        buf[:, :vocab] = rows
        buf[:, vocab:] = 32767  # past vocab: never chosen
        d = up(buf, np.int16)
        idx = t.empty(4, dtype=t.int32, device="cuda")
        _lib.call("llhip_argmax_i16", ptr(d), 4, ld, vocab, ptr(idx), stream())
        assert idx.cpu().numpy().tolist() == [int(np.argmax(r)) for r in rows], ld


@pytest.mark.parametrize("vocab", [1, 7, 8, 9, 2047, 65537, 151936])
def test_greedy_rows_argmax_record_and_positions(vocab):
    """llhip_greedy_rows (the batch decode's greedy step) against numpy's argmax per row (the first
    index of the maximum, golden.py's greedy choice): every tail length of the 16-byte chunks, ties
    across chunks and threads, values past vocab never chosen; row r recorded at ring slot
    s = positions[r] - base[r] only when 0 <= s < ring_cap (rows and tokens elsewhere untouched),
    at a record stride that is a multiple of 8 (16-byte stores) and at an odd one; positions + 1."""
    from llaccel_amd import _lib
    from tests.gpu_helpers import ptr, stream, torch, up

    t = torch()
    R, cap = 5, 3
    rows = RNG.integers(-32768, 32767, (R, vocab))
    rows[1, -1] = 32767  # the last value
    rows[2, :] = -5
    rows[2, [vocab // 3, vocab - 1]] = 9  # a tie: the lower index wins
    rows[3, :] = 32767  # all equal: index 0
    want = [int(np.argmax(r)) for r in rows]
    base = np.array([100, 7, 0, 50, 3], np.int32)
    pos = base + np.array([0, 2, cap, -1, 1], np.int32)  # slots 0, 2, none (= cap), none (< 0), 1
    ld = vocab + (vocab & 1)
    for ring_ld in (vocab + (-vocab) % 8, vocab + 1 + vocab % 2):  # a multiple of 8, odd
        buf = np.full((R, ld), 32767, np.int64)
        buf[:, :vocab] = rows  # past vocab: never chosen
        d = up(buf, np.int16)
        tok = t.full((R,), -1, dtype=t.int32, device="cuda")
        posd = t.tensor(pos, dtype=t.int32, device="cuda")
        based = t.tensor(base, dtype=t.int32, device="cuda")
        ring = t.full((cap * R * ring_ld,), -7, dtype=t.int16, device="cuda")
        ring_tok = t.full((cap * R,), -3, dtype=t.int32, device="cuda")
        _lib.call("llhip_greedy_rows", ptr(d), R, ld, vocab, ptr(tok), ptr(posd), ptr(based), ptr(ring), ring_ld,
                  ptr(ring_tok), cap, stream())
        t.cuda.synchronize()
        assert tok.cpu().numpy().tolist() == want, ring_ld
        assert np.array_equal(posd.cpu().numpy(), pos + 1)
        got_ring = ring.cpu().numpy().reshape(cap, R, ring_ld)
        got_tok = ring_tok.cpu().numpy().reshape(cap, R)
        exp_ring = np.full((cap, R, ring_ld), -7, np.int64)
        exp_tok = np.full((cap, R), -3, np.int64)
        for r in range(R):
            s = int(pos[r] - base[r])
            if 0 <= s < cap:
                exp_ring[s, r, :vocab] = rows[r]
                exp_tok[s, r] = want[r]
        assert np.array_equal(got_ring, exp_ring), ring_ld
        assert np.array_equal(got_tok, exp_tok), ring_ld


def test_argmax_lowest_index_on_ties():
    row = np.zeros(151936, np.int64)
    row[[5, 100, 151935]] = 7
    assert G.GoldenModel.argmax(row, 151936) == 5
    row = RNG.integers(-32768, 32768, 49152)
    assert G.GoldenModel.argmax(row, 49152) == int(np.argmax(row))
    assert G.GoldenModel.argmax(row, 1000) == int(np.argmax(row[:1000]))


@pytest.mark.parametrize("H,D,rows", [(2, 64, False), (8, 128, False), (4, 16, True)])
def test_rope_quant_with_cache_writes(H, D, rows):
    """llhip_rope_quant (the prompt-chunk launch of rope -> quant [-> kv_write]) equals the oracle's
    rope, vquant and cache write; with per-row positions each row writes its own cache slot."""
    from llaccel_amd import _lib
    from tests.gpu_helpers import ptr, stream, torch, up

    t = torch()
    M, max_seq, pos, qM, qS = 40, 96, 50, 1234567891, 40
    inv = 1e6 ** (-np.arange(0, D, 2) / D)
    ang = np.outer(np.arange(max_seq), inv)
    c = np.round(np.cos(ang) * 16384).astype(np.int64)
    s = np.round(np.sin(ang) * 16384).astype(np.int64)
    x = RNG.integers(-32768, 32768, (M, H * D))
    v = RNG.integers(-128, 128, (M, H * D + 8))
    slots = M if rows else 1
    kc0 = RNG.integers(-128, 128, (slots, H, max_seq, D))
    vc0 = RNG.integers(-128, 128, (slots, H, max_seq, D))
    rp = RNG.integers(0, max_seq, M) if rows else None
    xd, cd, sd, vd = up(x, np.int16), up(c, np.int16), up(s, np.int16), up(v, np.int8)
    kcd, vcd = up(kc0, np.int8), up(vc0, np.int8)
    rpd = up(rp, np.int32) if rows else None
    yd = t.zeros((M, H * D), dtype=t.int16, device="cuda")
    yqd = t.zeros((M, H * D), dtype=t.int8, device="cuda")
    stride = H * max_seq * D
    _lib.call("llhip_rope_quant", ptr(xd), M, H, D, H * D, ptr(cd), ptr(sd), max_seq, pos, None, ptr(rpd), ptr(yd),
              ptr(yqd), qM, qS, ptr(kcd), ptr(vd), H * D + 8, ptr(vcd), max_seq, stride if rows else 0, stream())
    if rows:
        want_y = np.stack([O.rope(x[m:m + 1], H, D, c, s, int(rp[m]))[0] for m in range(M)])
    else:
        want_y = O.rope(x, H, D, c, s, pos)
    want_q = O.vquant(want_y, qM, qS)
    assert np.array_equal(yd.cpu().numpy(), want_y) and np.array_equal(yqd.cpu().numpy(), want_q)
    kc, vc = kc0.copy(), vc0.copy()
    for m in range(M):
        slot, pm = (m, int(rp[m])) if rows else (0, pos + m)
        kc[slot, :, pm] = want_q[m].reshape(H, D)
        vc[slot, :, pm] = v[m, :H * D].reshape(H, D)
    assert np.array_equal(kcd.cpu().numpy(), kc) and np.array_equal(vcd.cpu().numpy(), vc)
    # without caches: the query rows (y and yq only)
    yqd.zero_()
    _lib.call("llhip_rope_quant", ptr(xd), M, H, D, H * D, ptr(cd), ptr(sd), max_seq, 7, None, None, ptr(yd), ptr(yqd),
              qM, qS, None, None, 0, None, max_seq, 0, stream())
    assert np.array_equal(yqd.cpu().numpy(), O.vquant(O.rope(x, H, D, c, s, 7), qM, qS))
    with pytest.raises(ValueError):
        _lib.call("llhip_rope_quant", ptr(xd), M, H, D, H * D, ptr(cd), ptr(sd), max_seq, 60, None, None, ptr(yd),
                  ptr(yqd), qM, qS, ptr(kcd), ptr(vd), H * D, ptr(vcd), max_seq, 0, stream())


def test_rope_quant_extreme_table_entries():
    """Table entries and inputs of -32768 (x2 c + x1 s = 2^31, past int32): llhip_rope and
    llhip_rope_quant equal the oracle's int64 rotation (saturated to 32767)."""
    from llaccel_amd import _lib
    from tests.gpu_helpers import ptr, stream, torch, up

    t = torch()
    M, H, D, max_seq, qM, qS = 8, 2, 16, 4, 1234567891, 40
    c = RNG.choice([-32768, 32767, 16384, -1], (max_seq, D // 2))
    s = RNG.choice([-32768, 32767, -16384, 1], (max_seq, D // 2))
    c[0], s[0] = -32768, -32768
    x = RNG.choice([-32768, 32767, 5, -7], (M, H * D))
    x[0] = -32768
    want = O.rope(x[:1], H, D, c, s, 0)
    assert want[0, D // 2] == 32767
    assert np.array_equal(G.rope(x[:1], H, D, c, s, 0), want)
    xd, cd, sd = up(x, np.int16), up(c, np.int16), up(s, np.int16)
    yd = t.zeros((M, H * D), dtype=t.int16, device="cuda")
    yqd = t.zeros((M, H * D), dtype=t.int8, device="cuda")
    rp = up(np.arange(M) % max_seq, np.int32)
    _lib.call("llhip_rope_quant", ptr(xd), M, H, D, H * D, ptr(cd), ptr(sd), max_seq, 0, None, ptr(rp), ptr(yd),
              ptr(yqd), qM, qS, None, None, 0, None, max_seq, 0, stream())
    want_y = np.stack([O.rope(x[m:m + 1], H, D, c, s, m % max_seq)[0] for m in range(M)])
    assert np.array_equal(yd.cpu().numpy(), want_y)
    assert np.array_equal(yqd.cpu().numpy(), O.vquant(want_y, qM, qS))


def test_rope_quant2_equals_two_calls():
    """llhip_rope_quant2 (the query rows, then the key rows with the layer's kv_write, in one launch)
    equals the oracle's rope, vquant and cache write of each part, and refuses a bad part as the
    single call would."""
    from llaccel_amd import _lib
    from tests.gpu_helpers import ptr, stream, torch, up

    t = torch()
    M, H, Hkv, D, max_seq, pos = 37, 14, 2, 64, 96, 41
    qq, qk = (1234567891, 40), (987654321, 39)
    inv = 1e6 ** (-np.arange(0, D, 2) / D)
    ang = np.outer(np.arange(max_seq), inv)
    c = np.round(np.cos(ang) * 16384).astype(np.int64)
    s = np.round(np.sin(ang) * 16384).astype(np.int64)
    xq = RNG.integers(-32768, 32768, (M, H * D))
    xk = RNG.integers(-32768, 32768, (M, Hkv * D))
    v = RNG.integers(-128, 128, (M, Hkv * D))
    kc0 = RNG.integers(-128, 128, (Hkv, max_seq, D))
    vc0 = RNG.integers(-128, 128, (Hkv, max_seq, D))
    xqd, xkd, cd, sd, vd = up(xq, np.int16), up(xk, np.int16), up(c, np.int16), up(s, np.int16), up(v, np.int8)
    kcd, vcd = up(kc0, np.int8), up(vc0, np.int8)
    outs = [t.zeros((M, n * D), dtype=dt, device="cuda") for n in (H, Hkv) for dt in (t.int16, t.int8)]

    def desc(x, n, y, yq, q, kc=None, vv=None, vc=None, p=pos):
        d = _lib.RopeQuantDesc()
        d.x, d.M, d.H, d.D, d.ldx = ptr(x), M, n, D, n * D
        d.cos_tab, d.sin_tab, d.table_rows, d.pos = ptr(cd), ptr(sd), max_seq, p
        d.y, d.yq, d.qM, d.qS = ptr(y), ptr(yq), q[0], q[1]
        d.kc, d.v, d.ldv, d.vc, d.max_seq = ptr(kc), ptr(vv), n * D if vv is not None else 0, ptr(vc), max_seq
        return d

    a = desc(xqd, H, outs[0], outs[1], qq)
    b = desc(xkd, Hkv, outs[2], outs[3], qk, kcd, vd, vcd)
    _lib.call("llhip_rope_quant2", ctypes.byref(a), ctypes.byref(b), stream())
    yq_want, yk_want = O.rope(xq, H, D, c, s, pos), O.rope(xk, Hkv, D, c, s, pos)
    kq_want = O.vquant(yk_want, *qk)
    assert np.array_equal(outs[0].cpu().numpy(), yq_want)
    assert np.array_equal(outs[1].cpu().numpy(), O.vquant(yq_want, *qq))
    assert np.array_equal(outs[2].cpu().numpy(), yk_want) and np.array_equal(outs[3].cpu().numpy(), kq_want)
    kc, vc = kc0.copy(), vc0.copy()
    for m in range(M):
        kc[:, pos + m] = kq_want[m].reshape(Hkv, D)
        vc[:, pos + m] = v[m].reshape(Hkv, D)
    assert np.array_equal(kcd.cpu().numpy(), kc) and np.array_equal(vcd.cpu().numpy(), vc)
    with pytest.raises(ValueError):  # the key part's positions run past the cache
        _lib.call("llhip_rope_quant2", ctypes.byref(a), ctypes.byref(desc(xkd, Hkv, outs[2], outs[3], qk, kcd, vd, vcd,
                                                                          p=max_seq - 10)), stream())
