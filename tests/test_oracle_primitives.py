"""Pins the CPU oracle's primitives (oracle/golden_np.py, oracle/numerics.c) against
things other than themselves: Python big-integer closed forms, math.isqrt, the known
answers of the reference's tests (tests/python/test_golden_primitives.py,
test_rounding_boundaries.py, test_luts.py), the LUT constants the reference commits
(include/llaccel/luts.h -> tests/golden/luts_ref.json) and the reference's numerics.h
compiled into oracle/_ref."""
from __future__ import annotations

import ctypes
import json
import math

import numpy as np
import pytest

from oracle import golden_np as O

RNG = np.random.default_rng(20261201)


def big_rshr(v: int, s: int) -> int:
    """floor((v + 2^(s-1)) / 2^s) over the integers (NUMERICS.md:15-18)."""
    return v if s == 0 else (v + (1 << (s - 1))) >> s


def wrap64(x: int) -> int:
    x &= (1 << 64) - 1
    return x - (1 << 64) if x >= 1 << 63 else x


# ---- LUTs ----------------------------------------------------------------------------------
def test_luts_equal_reference_committed_constants(golden_dir):
    ref = json.loads((golden_dir / "luts_ref.json").read_text())
    assert O.sigmoid_table().tolist() == ref["kSigmoidLut"]
    assert O.exp_int_table().tolist() == ref["kExpIntLut"]
    assert O.exp_frac_table().tolist() == ref["kExpFracLut"]


def test_lut_anchors():
    sig = O.sigmoid_table().astype(np.int64)
    assert sig.shape == (257,) and sig[128] == 32768 and sig[256] == 65514
    assert np.all(np.diff(sig) >= 0)
    assert O.exp_int_table()[0] == 65535 and O.exp_frac_table()[0] == 65535


def test_luts_equal_oracle_ref(ref_lib):
    sig, ei, ef = np.zeros(257, np.uint16), np.zeros(16, np.uint16), np.zeros(256, np.uint16)
    ref_lib.ref_luts(sig.ctypes.data, ei.ctypes.data, ef.ctypes.data)
    assert np.array_equal(sig, O.sigmoid_table())
    assert np.array_equal(ei, O.exp_int_table()) and np.array_equal(ef, O.exp_frac_table())


# ---- rshr / sat / mulshift -------------------------------------------------------------------
def test_rshr_known_answers():
    # test_golden_primitives.py:16-22
    assert O.rshr(5, 1) == 3 and O.rshr(-5, 1) == -2 and O.rshr(-6, 1) == -3
    assert O.rshr(7, 2) == 2 and O.rshr(6, 2) == 2 and O.rshr(-7, 0) == -7


def test_rshr_full_i64_domain_against_big_integers():
    vals = np.concatenate([np.array([-(1 << 63), (1 << 63) - 1, -1, 0, 1], np.int64),
                           RNG.integers(-(1 << 63), (1 << 63) - 1, 300, dtype=np.int64)])
    for s in range(64):
        exp = [big_rshr(int(v), s) for v in vals]
        assert O.rshr(vals, s).tolist() == exp
    shifts = np.arange(64, dtype=np.int64)
    top = (1 << 63) - 1
    assert O.rshr(np.int64(top), shifts).tolist() == [big_rshr(top, int(s)) for s in shifts]


def test_rshr_c_twin_and_reference(ref_lib):
    lib = O.c_oracle()
    vals = [-(1 << 63), (1 << 63) - 1, -1, 0, 1] + RNG.integers(-(1 << 63), (1 << 63) - 1, 64, dtype=np.int64).tolist()
    for s in range(64):
        for v in vals:
            e = big_rshr(v, s)
            assert lib.orc_rshr(v, s) == e
            assert ref_lib.ref_rshr(v, s) == e


def test_saturation_known_answers():
    # test_golden_primitives.py:31-36
    v = np.array([-10**9, -32769, -32768, -129, -128, 0, 127, 128, 255, 256, 32767, 32768, 65535, 65536, 10**9])
    assert O.sat8(v).tolist() == [-128] * 5 + [0] + [127] * 9
    assert O.satu8(v).tolist() == [0] * 6 + [127, 128, 255] + [255] * 6
    assert O.sat16(v).tolist() == [-32768] * 3 + [-129, -128, 0, 127, 128, 255, 256] + [32767] * 5
    assert O.satu16(v).tolist() == [0] * 6 + [127, 128, 255, 256, 32767, 32768, 65535, 65535, 65535]


def test_mulshift_wraps_like_int64_and_matches_reference(ref_lib):
    lib = O.c_oracle()
    v = RNG.integers(-(1 << 40), 1 << 40, 2000)
    M = RNG.integers(0, 1 << 32, 2000)
    S = RNG.integers(0, 64, 2000)
    got = O.mulshift(v, M, S)
    for i in range(0, 2000, 7):
        e = big_rshr(wrap64(int(v[i]) * int(M[i])), int(S[i]))
        assert got[i] == e
        assert lib.orc_mulshift(int(v[i]), int(M[i]), int(S[i])) == e
        assert ref_lib.ref_mulshift(int(v[i]), int(M[i]), int(S[i])) == e


def test_requant_matches_reference(ref_lib):
    acc = RNG.integers(-(1 << 30), 1 << 30, 3000)
    M = RNG.integers(1 << 30, 1 << 31, 3000)
    S = RNG.integers(20, 50, 3000)
    r16, r8 = O.requant16(acc, M, S), O.requant8(acc, M, S)
    for i in range(0, 3000, 5):
        assert r16[i] == ref_lib.ref_requant16(int(acc[i]), int(M[i]), int(S[i]))
        assert r8[i] == ref_lib.ref_requant8(int(acc[i]), int(M[i]), int(S[i]))


# ---- isqrt48 / udiv ----------------------------------------------------------------------------
def test_isqrt48_equals_math_isqrt(ref_lib):
    lib = O.c_oracle()
    vals = RNG.integers(0, 1 << 48, 3000).tolist() + [0, 1, 2, 3, 4, (1 << 48) - 1, 1 << 47, (1 << 46) - 1,
                                                      65535**2, 65536**2, 65536**2 - 1]
    for t in vals:
        r = math.isqrt(t)
        assert O.isqrt48(t) == r
        assert lib.orc_isqrt48(t) == r
        assert ref_lib.ref_isqrt48(t) == r


def test_isqrt48_domain():
    with pytest.raises(ValueError):
        O.isqrt48(1 << 48)
    with pytest.raises(ValueError):
        O.isqrt48(-1)


def test_udiv_known_answers():
    # test_golden_primitives.py:45-49
    assert O.udiv(10, 3) == 3 and O.udiv(10, 0) == 10
    assert O.udiv(2**31, 65534) == 32769
    assert O.udiv(2**40, 1) == (2**40) & 0xFFFFFFFF
    with pytest.raises(ValueError):
        O.udiv(-1, 3)


# ---- elementwise ---------------------------------------------------------------------------
def test_vmul_vadd_vquant_known_answers(ref_lib):
    # test_golden_primitives.py:158-163
    a, b = np.array([1000, -1000, 32767]), np.array([1000, 1000, 32767])
    assert O.vmul(a, b, 10).tolist() == [977, -977, 32767]
    assert O.vadd(a, b, 1).tolist() == [1500, -500, 32767]
    assert O.vquant(np.array([32767, -32768, 100]), 2**30, 38).tolist() == [127, -128, 0]
    x = RNG.integers(-32768, 32768, 500)
    y = RNG.integers(-32768, 32768, 500)
    sh = RNG.integers(0, 40, 500)
    for i in range(500):
        assert O.vmul(x[i], y[i], sh[i]) == ref_lib.ref_vmul(int(x[i]), int(y[i]), int(sh[i]))
        assert O.vadd(x[i], y[i], sh[i]) == ref_lib.ref_vadd(int(x[i]), int(y[i]), int(sh[i]))
        assert O.vquant(x[i], 1 << 30, sh[i] + 20) == ref_lib.ref_vquant(int(x[i]), 1 << 30, int(sh[i]) + 20)


def test_silu16_lut_points_and_reference(ref_lib):
    # test_golden_primitives.py:166-176: at f = 0 the interpolation returns the table entry
    sig = O.SIG
    for x in (-32768, -4096, -256, 0, 256, 4096, 32512):
        j = (x >> 8) + 128
        assert O.silu16(np.array([x]), 2**30, 30, 16)[0] == O.sat16(O.rshr(np.array([x * int(sig[j])]), 16))[0]
    assert O.silu16(np.array([0]), 2**30, 30, 16)[0] == 0
    for x in (32000, -32000, 25600):
        assert abs(int(O.silu16(np.array([x]), 2**30, 30, 16)[0]) - x / (1 + math.exp(-x / 4096))) <= 1.0
    lib = O.c_oracle()
    xs = RNG.integers(-32768, 32768, 3000)
    for Mi, Si, sh in ((2**30, 30, 16), (1518500250, 31, 15), (2**30, 28, 17), (2**31 - 1, 33, 14)):
        got = O.silu16(xs, Mi, Si, sh)
        for i in range(0, 3000, 3):
            e = ref_lib.ref_silu16(int(xs[i]), Mi, Si, sh)
            assert got[i] == e and lib.orc_silu16(int(xs[i]), Mi, Si, sh) == e


def test_silu16_tolerance_vs_float():
    # test_golden_primitives.py:71-80 (e_x = e_y = -12)
    x = RNG.integers(-32768, 32768, 4096)
    y = O.silu16(x, 2**30, 30, 16)
    xr = x * 2.0**-12
    err = np.abs(y * 2.0**-12 - xr / (1 + np.exp(-xr)))
    assert err.max() < 0.16 and err.mean() < 0.004


# ---- rmsnorm / rope ---------------------------------------------------------------------------
def test_rmsnorm_zero_row_and_clamp():
    # test_golden_primitives.py:179-186
    K = 32
    g = np.full(K, 16384)
    C = int(round(2.0**24 * math.sqrt(K)))
    assert np.all(O.rmsnorm(np.zeros((1, K), np.int64), g, 3, C, 20) == 0)
    y = O.rmsnorm(np.ones((1, K), np.int64), g, 0, C, 20)[0]
    assert np.all(y == O.sat16(O.rshr(np.array([16384 * 65535]), 20))[0])


def test_rmsnorm_quiet_row():
    """Quiet-row known answer (reference tests/cpp/numerics_selftest.cpp:27-47): x = 102 at
    e_x = -10 normalises to ~1 at e_y = -10 with C/eps from the compiler rule."""
    K, e_x = 896, -10
    eps_t = int(round(1e-6 * K * 2.0 ** (-2 * e_x)))
    # the compiler rule with measured rms 102: largest R with floor(C / 3053) < 65535/4 is 20
    R = 20
    C = int(round(2.0**R * math.sqrt(K)))
    assert math.floor(C / math.isqrt(K * 102 * 102 + eps_t)) < 65535 / 4 <= math.floor(2 * C / 3053)
    y = O.rmsnorm(np.full((1, K), 102), np.full(K, 16384), eps_t, C, R + 14 - 10)[0]
    val = 102 / 1024
    assert abs(y[0] / 1024.0 - val / math.sqrt(val * val + 1e-6)) < 0.002


def test_rmsnorm_matches_reference(ref_lib):
    lib = O.c_oracle()
    for K in (16, 64, 128, 896, 1024):
        for trial in range(6):
            x = RNG.integers(-32768, 32768, K) // (1 << int(RNG.integers(0, 12)))
            g = RNG.integers(-32768, 32768, K)
            eps_t = int(RNG.integers(0, 1 << 32))
            C = int(RNG.integers(0, 1 << 32))
            sh = int(RNG.integers(10, 50))
            got = O.rmsnorm(x[None, :], g, eps_t, C, sh)[0]
            x16, g16, y16 = x.astype(np.int16), g.astype(np.int16), np.zeros(K, np.int16)
            ref_lib.ref_rmsnorm(x16.ctypes.data, g16.ctypes.data, y16.ctypes.data, K, eps_t, C, sh)
            assert got.tolist() == y16.tolist()
            yc = np.zeros(K, np.int64)
            xs, gs = x.astype(np.int64), g.astype(np.int64)
            assert lib.orc_rmsnorm_row(xs.ctypes.data, gs.ctypes.data, K, eps_t, C, sh, yc.ctypes.data) == 0
            assert yc.tolist() == y16.tolist()


def test_rmsnorm_tolerance_vs_float():
    # test_golden_primitives.py:82-99
    K, e_x, e_y, e_g = 128, -10, -12, -14
    g = RNG.uniform(0.5, 2.0, K)
    gq = np.round(g / 2.0**-14).astype(np.int64)
    gq = np.minimum(gq, 32767)
    R = 24
    C = int(round(2.0**R * math.sqrt(K)))
    eps_t = int(round(1e-5 * K * 2.0 ** (-2 * e_x)))
    for _ in range(10):
        x = np.clip(np.round(RNG.normal(0, RNG.uniform(0.3, 3.0), K) / 2.0**e_x), -32768, 32767).astype(np.int64)
        y = O.rmsnorm(x[None, :], gq, eps_t, C, R - e_g + e_y)[0]
        xq = x * 2.0**e_x
        ref = xq / np.sqrt(np.mean(xq**2) + 1e-5) * (gq * 2.0**e_g)
        assert (np.abs(y * 2.0**e_y - ref) / np.abs(ref).max()).max() < 2e-3


def test_rope_identity_at_position_zero():
    # test_golden_primitives.py:189-194
    D, H = 16, 2
    x = RNG.integers(-32768, 32768, (2, H * D))
    assert np.array_equal(O.rope(x, H, D, np.full((4, D // 2), 16384), np.zeros((4, D // 2), np.int64), 0), x)


def test_rope_matches_reference_and_float(ref_lib):
    for H, D in ((4, 32), (2, 64), (1, 128), (2, 256)):
        inv_freq = 10000.0 ** (-np.arange(0, D, 2) / D)
        ang = np.outer(np.arange(64), inv_freq)
        cos_t = np.round(np.cos(ang) * 16384).astype(np.int64)
        sin_t = np.round(np.sin(ang) * 16384).astype(np.int64)
        x = RNG.integers(-32768, 32768, (3, H * D))
        y = O.rope(x, H, D, cos_t, sin_t, 17)
        for m in range(3):
            out = np.zeros(H * D, np.int16)
            xm = x[m].astype(np.int16)
            c, s = cos_t[17 + m].astype(np.int16), sin_t[17 + m].astype(np.int16)
            ref_lib.ref_rope(xm.ctypes.data, out.ctypes.data, H, D, c.ctypes.data, s.ctypes.data)
            assert y[m].tolist() == out.tolist()
        # rotation agrees with float within the two Q1.14 roundings (test_golden_primitives.py:102-116)
        xr = x.reshape(3, H, D).astype(np.float64)
        c = np.concatenate([np.cos(ang), np.cos(ang)], -1)[17:20][:, None, :]
        s = np.concatenate([np.sin(ang), np.sin(ang)], -1)[17:20][:, None, :]
        rot = np.concatenate([-xr[..., D // 2:], xr[..., :D // 2]], -1)
        ref = np.clip(xr * c + rot * s, -32768, 32767).reshape(3, H * D)
        assert np.abs(y - ref).max() < 3 + 1e-9


def test_rope_extreme_table_entries(ref_lib):
    """Table entries and inputs of -32768: x2 c + x1 s = 2^31, past int32 (golden.py:141-158 sums in
    int64), so the rotated value saturates to 32767; the compiled numerics.h agrees."""
    H, D = 1, 16
    cos_t = np.full((2, D // 2), -32768, np.int64)
    sin_t = np.full((2, D // 2), -32768, np.int64)
    cos_t[1, ::2], sin_t[1, 1::2] = 32767, 32767
    x = np.full((2, H * D), -32768, np.int64)
    x[1, 3] = 32767
    y = O.rope(x, H, D, cos_t, sin_t, 0)
    assert y[0, D // 2] == 32767  # b c + a s = 2^31 -> rshr 2^17 -> sat16 32767
    assert y[0, 0] == 0  # a c - b s = 0
    for m in range(2):
        out = np.zeros(H * D, np.int16)
        xm = x[m].astype(np.int16)
        c, s = cos_t[m].astype(np.int16), sin_t[m].astype(np.int16)
        ref_lib.ref_rope(xm.ctypes.data, out.ctypes.data, H, D, c.ctypes.data, s.ctypes.data)
        assert y[m].tolist() == out.tolist()


# ---- attention -------------------------------------------------------------------------------
def _ref_attn(ref_lib, q, k, v, Ms, Ss, Mo, So, wide):
    D, T = q.shape[0], k.shape[0]
    q8, k8, v8 = (np.ascontiguousarray(a, dtype=np.int8) for a in (q, k, v))
    out = np.zeros(D, np.int8)
    ref_lib.ref_attention_head(q8.ctypes.data, D, T, k8.ctypes.data, v8.ctypes.data, Ms, Ss, Mo, So,
                               out.ctypes.data, int(wide))
    return out.astype(np.int64)


def test_attention_max_key_probability():
    # test_golden_primitives.py:151-155
    z = np.array([0])
    assert ((O.EXPI[z >> 8] * O.EXPF[z & 255] + (1 << 15)) >> 16)[0] == 65534


def test_attention_single_key_identity():
    # test_golden_primitives.py:141-148: T=1 -> pn = 255, Mo/So undo it
    D = 16
    v = RNG.integers(-127, 128, (1, D))
    Mo, So = 2155905153, 39   # (M, S) of 1/255 normalised to [2^30, 2^31)
    assert abs(Mo * 2.0**-So - 1 / 255) < 1e-12
    out = O.attention_head(RNG.integers(-127, 128, D), RNG.integers(-127, 128, (1, D)), v, 2**30, 40, Mo, So)
    assert np.array_equal(out, v[0])


def test_attention_offset_invariance_and_extremes():
    # test_golden_primitives.py:197-215
    for pb in (8, 15):
        for D in (16, 32, 64):
            q = np.zeros(D, np.int64)
            q[0] = 127
            vals = np.zeros((2, D), np.int64)
            vals[:, 0] = [-127, 127]
            outs = []
            for off in (0, 126, -128):
                keys = np.zeros((2, D), np.int64)
                keys[:, 0] = [off, off + 1]
                outs.append(O.attention_head(q, keys, vals, 1 << 30, 24, 1 << 30, 38, pb))
            assert all(np.array_equal(o, outs[0]) for o in outs) and outs[0][0] == 127
            q.fill(127)
            keys = np.array([[-128] * D, [127] * D], np.int64)
            assert O.attention_head(q, keys, vals, 2**32 - 1, 0, 1 << 30, 38, pb)[0] == 127


def test_attention_common_offset_nontrivial():
    # test_golden_primitives.py:218-231
    q = np.zeros(16, np.int64)
    q[0], q[1] = 1, 127
    keys = np.zeros((2, 16), np.int64)
    keys[:, 0] = [0, 1]
    vals = np.zeros((2, 16), np.int64)
    vals[:, 0] = [-127, 127]
    for pb in (8, 15):
        base = O.attention_head(q, keys, vals, 1 << 30, 24, 1 << 30, 38, pb)
        sh = keys.copy()
        sh[:, 1] = 126
        out = O.attention_head(q, sh, vals, 1 << 30, 24, 1 << 30, 38, pb)
        assert np.array_equal(out, base) and abs(int(out[0]) - 127 * math.tanh(0.125)) <= 1


def test_wide_attention_constant_values_and_legacy_bias():
    # test_rounding_boundaries.py:19-29
    for T in list(range(1, 40)) + [100, 171, 255, 256]:
        q = np.zeros(16, np.int64)
        keys = np.zeros((T, 16), np.int64)
        for val in (-128, -1, 0, 1, 127):
            got = O.attention_head(q, keys, np.full((T, 16), val), 1, 0, 1 << 30, 38, prob_bits=15)
            assert np.max(np.abs(got - val)) <= 1
    legacy = O.attention_head(np.zeros(16), np.zeros((171, 16)), np.full((171, 16), 127), 1, 0, 1 << 30, 38)
    assert int(legacy[0]) == 85


def test_attention_prob_bits_validated():
    with pytest.raises(ValueError):
        O.attention_head(np.zeros(16), np.zeros((2, 16)), np.zeros((2, 16)), 1, 0, 1, 0, prob_bits=9)


@pytest.mark.parametrize("D", [16, 64, 128, 256])
def test_attention_matches_reference_and_c(ref_lib, D):
    lib = O.c_oracle()
    for T in (1, 2, 7, 255, 256, 257, 600):
        q = RNG.integers(-128, 128, D)
        k = RNG.integers(-128, 128, (T, D))
        v = RNG.integers(-128, 128, (T, D))
        Ms = int(RNG.integers(1 << 30, 1 << 31))
        Ss = int(RNG.integers(30, 40))
        Mo, So = int(RNG.integers(1 << 30, 1 << 31)), int(RNG.integers(36, 42))
        for pb in (8, 15):
            got = O.attention_head(q, k, v, Ms, Ss, Mo, So, pb)
            assert got.tolist() == _ref_attn(ref_lib, q, k, v, Ms, Ss, Mo, So, pb == 15).tolist()
            out = np.zeros(D, np.int64)
            q8, k8, v8 = (np.ascontiguousarray(a, dtype=np.int8) for a in (q, k, v))
            assert lib.orc_attention_head(q8.ctypes.data, k8.ctypes.data, v8.ctypes.data, T, D, Ms, Ss, Mo, So, pb,
                                          out.ctypes.data) == 0
            assert out.tolist() == got.tolist()


def test_attention_tolerance_vs_float_softmax():
    # test_golden_primitives.py:119-138 (legacy prob_bits 8)
    D = 32
    s_q = s_k = 0.02
    s_v = s_out = 0.03
    from llaccel_amd.synth import scalar_pair
    Ms, Ss = scalar_pair(256 * s_q * s_k / math.sqrt(D))
    Mo, So = scalar_pair(s_v / (256 * s_out))
    for T in (1, 5, 40, 200):
        q = RNG.integers(-127, 128, D)
        k = RNG.integers(-127, 128, (T, D))
        v = RNG.integers(-127, 128, (T, D))
        out = O.attention_head(q, k, v, Ms, Ss, Mo, So)
        sc = (k * s_k) @ (q * s_q) / math.sqrt(D)
        p = np.exp(sc - sc.max())
        p /= p.sum()
        ref = p @ (v * s_v)
        assert np.abs(out * s_out - ref).max() < 0.15


# ---- planted mistakes are caught (the checks above are not tautological) -----------------------
def test_planted_rshr_mistake_is_caught():
    def bad_rshr(v, s):  # round half to -inf instead of half up
        return (np.asarray(v, np.int64) + (1 << (s - 1)) - 1) >> s if s else np.asarray(v)
    assert bad_rshr(5, 1) != big_rshr(5, 1)


def test_planted_lut_mistake_is_caught(golden_dir):
    ref = json.loads((golden_dir / "luts_ref.json").read_text())
    half_up = [min(65535, math.floor(65536 / (1 + math.exp(8 - j / 16)) + 0.5)) for j in range(257)]
    # Python round (half-even) and half-up differ nowhere here, but a truncating table would:
    trunc = [min(65535, int(65536 / (1 + math.exp(8 - j / 16)))) for j in range(257)]
    assert half_up == ref["kSigmoidLut"] and trunc != ref["kSigmoidLut"]
