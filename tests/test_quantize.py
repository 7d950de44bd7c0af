"""CPU checks of the qgraph producer (llaccel_amd.quantize) and of its oracle (oracle/quant_np.py).

The host formulas are held to the known answers of the reference quantizer's own tests
(test_refquant.py: llround ties :18-27, (M, S) normalisation :36-56, exponents and scales :59-62,
row scales and biases :65-70, the R rule :90-110, shifts :115-136, attention and RoPE parameters
:139-148) and to what those formulas are meant to realise through the oracle's integer primitives.
The device conversions are checked against the oracle in tests/test_gpu_quantize.py."""
from __future__ import annotations

import dataclasses
import json
import math
from fractions import Fraction

import numpy as np
import pytest

from llaccel_amd import quantize as Q
from llaccel_amd import synth
from oracle import golden_np as O
from oracle import quant_np as QN

RNG = np.random.default_rng(7)


# ---- rounding -------------------------------------------------------------------------------
LLROUND_KATS = {2.5: 3, -2.5: -3, 0.5: 1, -0.5: -1, 1.4999: 1, -1.4999: -1, 3.0: 3, 0.0: 0,
                0.49999999999999994: 0, -0.49999999999999994: 0, 1e15 + 0.5: 1000000000000001}


def test_llround_known_answers():
    for x, want in LLROUND_KATS.items():
        assert Q.llround(x) == want, x
    xs = np.array(list(LLROUND_KATS))
    assert Q.llround_vec(xs).tolist() == list(LLROUND_KATS.values())
    assert QN.llround(xs).tolist() == list(LLROUND_KATS.values())
    assert round(2.5) == 2  # Python's round is half-even; llround is not
    with pytest.raises(ValueError):
        Q.llround(float("nan"))
    with pytest.raises(ValueError):
        Q.llround_vec([1.0, float("inf")])


def _exact_round_away(x: float) -> int:
    """Rounding of the exact binary value of x, halves away from zero, in rational arithmetic."""
    f = Fraction(x)
    n = math.floor(abs(f) + Fraction(1, 2))
    return n if f >= 0 else -n


def test_llround_against_exact_rational_rounding():
    xs = np.concatenate([RNG.uniform(-300, 300, 2000), RNG.integers(-1000, 1000, 500) + 0.5,
                         np.ldexp(RNG.integers(-2**20, 2**20, 500).astype(np.float64), -8)])
    want = [_exact_round_away(float(x)) for x in xs]
    assert Q.llround_vec(xs).tolist() == want
    assert QN.llround(xs).tolist() == want
    assert [Q.llround(float(x)) for x in xs[:300]] == want[:300]


# ---- (M, S) pairs ------------------------------------------------------------------------------
def test_mulshift_pairs_match_the_frexp_definition():
    rs = [1e-9, 1e-6, 0.001, 0.37, 0.5, 1.0, 1.0 - 2.0**-40, 3.5, 1000.0, 2.0**30, 2.0**30.999]
    M, S = Q.mulshift_pairs(rs)
    for r, m, s in zip(rs, M.tolist(), S.tolist()):
        assert (m, s) == Q.mulshift_pair(r)
        assert 0 <= s <= 63
        if s < 63:
            assert 2**30 <= m < 2**31 and abs(m * 2.0**-s / r - 1) <= 2.0**-30
    assert Q.mulshift_pair(1.0 - 2.0**-40) == (2**30, 30)  # mantissa rounds up to 1.0
    assert Q.mulshift_pair(2.0**-70) == (0, 63)
    assert Q.mulshift_pair(2.0**-40) == (2**23, 63)
    for bad in (2.0**31, 0.0, -1.0, float("nan")):
        with pytest.raises(ValueError):
            Q.mulshift_pair(bad)


def test_exponents_scales_and_biases():
    assert Q.i16_exponent(32767.0) == 0 and Q.i16_exponent(32767.5) == 1 and Q.i16_exponent(1.0) == -14
    assert Q.i16_exponent(0.5) == -15 and Q.i16_exponent(1e-9) == -15 and Q.i16_exponent(0.0) == -15
    assert Q.i8_scale(127.0) == 1.0 and Q.i8_scale(0.0) == 1.0 and Q.i8_scale(2.54) == 2.54 / 127.0
    assert Q.gemm_bias_rows([1.0, 1e30, -1e30], 0.5, [0.5, 2.0, 2.0]).tolist() == [4, 2**31 - 1, -(2**31)]
    with pytest.raises(ValueError):
        Q.gemm_bias_rows([1.0], 0.0, [1.0])


def test_oracle_row_scales_and_weights():
    w = np.array([[1.0, -2.0, 0.5], [0.0, 0.0, 0.0], [-127.0, 3.0, 3.0]])
    q, s = QN.quant_rows_i8(w)
    assert s.tolist() == [2.0 / 127.0, 1.0, 1.0]
    assert q.tolist() == [[64, -127, 32], [0, 0, 0], [-127, 3, 3]]  # 63.5 -> 64, 31.75 -> 32
    assert QN.quant_i8(np.array([2.5, -2.5, 300.0, -300.0, 0.4]), 1.0).tolist() == [3, -3, 127, -128, 0]
    assert QN.quant_i16(np.array([1.5, -1.5, 1e9]), -1).tolist() == [3, -3, 32767]
    assert QN.quant_i16(np.array([2.5]), 0).tolist() == [3]


# ---- parameter formulas through the integer primitives -------------------------------------
def test_gemm_rq_realises_the_scale():
    s_a, s_w, e_out, s_out = 0.031, 0.0047, -9, 0.02
    acc = RNG.integers(-2**20, 2**20, 1000)
    (M, S), = Q.gemm_rq_rows(s_a, np.array([s_w]), False, e_out, 0.0).tolist()
    y = O.sat16(O.mulshift(acc, M, S))
    ref = acc * s_a * s_w / 2.0**e_out
    ok = np.abs(ref) < 32767
    assert np.all(np.abs(y[ok] - ref[ok]) <= 0.5 + 1e-6 * np.abs(ref[ok]))
    (M, S), = Q.gemm_rq_rows(s_a, np.array([s_w]), True, 0, s_out).tolist()
    a8 = acc[:50] // 4096
    y = O.sat8(O.mulshift(a8, M, S))
    assert np.all(np.abs(y - np.clip(a8 * s_a * s_w / s_out, -128, 127)) <= 0.5 + 1e-6)


def test_quant_params_realise_the_scale():
    e_x, s_y = -11, 0.013
    M, S = Q.quant_params(e_x, s_y)
    x = RNG.integers(-32768, 32768, 2000)
    y = O.sat8(O.mulshift(x, M, S))
    ref = np.clip(x * 2.0**e_x / s_y, -128, 127)
    assert np.all(np.abs(y - ref) <= 0.5 + 1e-6 * np.abs(ref))


def test_rmsnorm_r_rule_is_the_largest_feasible_shift():
    K, eps, e_x, e_g, e_y, absmax = 128, 1e-5, -13, -14, -12, 3.9
    p = Q.rmsnorm_params(K, eps, e_x, e_g, e_y, absmax, "t")
    assert p["eps_t"] == Q.llround(eps * K * 2.0 ** (-2 * e_x)) and p["sh_post"] == p["R"] - e_g + e_y

    def feasible(R):
        C = Q.llround(math.ldexp(math.sqrt(K), R))
        rms_q = (absmax / 4.0) / 2.0**e_x
        r_typ = max(1.0, math.floor(math.sqrt(K * rms_q * rms_q + p["eps_t"])))
        return C < 2**32 and math.floor(C / r_typ) < 65535 / 4

    assert feasible(p["R"]) and not any(feasible(R) for R in range(p["R"] + 1, 32))
    # a row at rms = absmax/4 through the integer RMSNorm matches the float formula
    g = RNG.uniform(0.5, 1.5, K)
    gq = QN.quant_i16(g, e_g).astype(np.int64)
    xr = RNG.normal(0, absmax / 4, K)
    xr *= (absmax / 4) / np.sqrt(np.mean(xr**2))
    x = QN.quant_i16(xr, e_x).astype(np.int64)
    y = O.rmsnorm(x[None], gq, p["eps_t"], p["C"], p["sh_post"])[0]
    xq = x * 2.0**e_x
    ref = xq / np.sqrt(np.mean(xq**2) + eps) * (gq * 2.0**e_g)
    assert np.abs(y * 2.0**e_y - ref).max() / np.abs(ref).max() < 2e-3
    with pytest.raises(ValueError, match="sh_post"):
        Q.rmsnorm_params(K, eps, e_x, 20, -15, absmax, "t")


def test_rmsnorm_minimum_row_statistic():
    args = (896, 1e-6, -10, -14, -10, 100.0, "quiet")
    old, new = Q.rmsnorm_params(*args), Q.rmsnorm_params(*args, rms_min=0.1)
    assert new["C"] < old["C"]
    y = O.rmsnorm(np.full((1, 896), 102, np.int64), np.full(896, 16384, np.int64), new["eps_t"], new["C"],
                  new["sh_post"])
    v = 102 / 1024
    assert np.max(np.abs(y / 1024 - v / math.sqrt(v * v + 1e-6))) < 0.002
    for bad in (-1.0, 101.0, float("inf"), float("nan")):
        with pytest.raises(ValueError, match="rms_min"):
            Q.rmsnorm_params(*args, rms_min=bad)
    assert Q.rmsnorm_params(*args, rms_min=0.0)["C"] > 0


def test_silu_mul_add_shifts():
    e_g, e_sg, e_u, e_f = -12, -13, -12, -14
    sp = Q.silu_params(e_g, e_sg, "t")
    assert sp == {"Mi": 2**30, "Si": 30 - (e_g + 12), "sh_out": 16 + e_sg - e_g}
    x = RNG.integers(-20000, 16000, 500)
    y = O.silu16(x, sp["Mi"], sp["Si"], sp["sh_out"])
    xr = x * 2.0**e_g
    assert np.abs(y * 2.0**e_sg - xr / (1 + np.exp(-xr))).max() < 0.01
    assert Q.mul_shift(e_sg, e_u, e_f, "t") == 11
    assert Q.add_shift(-8, -8, "t") == 0 and Q.add_shift(-8, -10, "t") == 2
    for fn, args in ((Q.add_shift, (-10, -8, "t")), (Q.mul_shift, (-2, -2, -14, "t")), (Q.silu_params, (20, 20, "t"))):
        with pytest.raises(ValueError):
            fn(*args)


def test_attention_parameters_and_rope_tables():
    p = Q.attn_params(0.04, 0.05, 0.01, 0.008, 32)
    assert p["Ms"] * 2.0 ** -p["Ss"] == pytest.approx(256 * 0.04 * 0.05 / math.sqrt(32), rel=2**-30)
    assert p["Mo"] * 2.0 ** -p["So"] == pytest.approx(0.01 / (256 * 0.008), rel=2**-30)
    cos_t, sin_t = Q.rope_tables(40, 16, 10000.0)
    assert cos_t.shape == sin_t.shape == (40, 8) and cos_t.dtype == np.int16
    ang = np.outer(np.arange(40), 10000.0 ** (-np.arange(0, 16, 2) / 16))
    assert np.abs(cos_t - 16384 * np.cos(ang)).max() <= 0.5 + 1e-9
    assert np.abs(sin_t - 16384 * np.sin(ang)).max() <= 0.5 + 1e-9
    assert cos_t[0].tolist() == [16384] * 8 and sin_t[0].tolist() == [0] * 8


# ---- export directory and blob ---------------------------------------------------------------
def test_export_directory_round_trip(tmp_path):
    cfg = dataclasses.replace(synth.CONFIGS["tiny"], name="x", ffn=128, qkv_bias=True)
    d = synth.write_export(tmp_path / "ex", cfg, seed=4)
    attrs, W, calib = Q.load_export(d)
    assert attrs == {"dim": 64, "n_layers": 2, "n_heads": 4, "n_kv_heads": 2, "head_dim": 16, "ffn": 128,
                     "vocab": 256, "max_seq": 64, "rope_base": 10000.0, "rms_eps": 1e-5}
    ref = synth.float_weights(cfg, 4)
    assert set(W) == set(ref) and all(np.array_equal(W[k], ref[k]) for k in ref)
    assert {"input", "logits", "hn", "l0.h", "l1.x2", "l0.sg", "l0.qr", "l0.a"} <= set(calib)
    with pytest.raises(ValueError, match="llaccel.model"):
        Q.parse_model_attrs("module {}")


def test_blob_layout():
    b = Q.Pack(OracleDevice())
    b.put("a", np.arange(3, dtype=np.int64), "i8")
    b.put("r", np.array([[1, 2], [3, 4]], dtype=np.int64), "rq", None)
    b.put("g", np.ones(5, dtype=np.int64), "i16", -3)
    assert b.tensors == {"a": {"dtype": "i8", "shape": [3], "offset": 0},
                         "r": {"dtype": "rq", "shape": [2], "offset": 64},
                         "g": {"dtype": "i16", "shape": [5], "offset": 128, "exp": -3}}
    data = b.bytes()
    assert len(data) == 192 and data[:3] == b"\x00\x01\x02" and data[64:80] == np.array([1, 2, 3, 4], "<i4").tobytes()
    with pytest.raises(ValueError, match="duplicate"):
        b.put("a", np.zeros(1), "i8")


# ---- the whole producer against graphs written by the reference quantizer --------------------
class OracleDevice:
    """The producer's device conversions restated on the CPU by oracle/quant_np.py (refquant.py:119-141),
    so the host side of the producer -- formats, parameters, op list, blob layout -- is checked
    without a GPU.  The GPU conversions themselves are compared with the same fixtures in
    tests/test_gpu_quantize.py."""

    def rows_i8(self, w, n_rows=None):
        w = np.asarray(w, np.float32)
        full = np.zeros((w.shape[0] if n_rows is None else int(n_rows), w.shape[1]), np.float32)
        full[: w.shape[0]] = w
        return QN.quant_rows_i8(full)

    def i16(self, x, e):
        return QN.quant_i16(np.asarray(x, np.float32), e)


REFQUANT = {"llama_v2": ("llama", True), "qwen_v1": ("qwen", False), "qwen_v2": ("qwen", True)}


@pytest.mark.parametrize("name", sorted(REFQUANT))
def test_producer_equals_reference_quantizer(golden_dir, tmp_path, name):
    """tests/golden/refquant/q_*: qgraph.json + qweights.bin written by the reference's
    refquant.quantize_export (refquant.py:493-506) on the committed export directories; the producer
    writes the same graph and byte-identical weights."""
    model, fusion = REFQUANT[name]
    ref = golden_dir / "refquant"
    got = Q.quantize_export(ref / f"export_{model}", tmp_path / "q", fusion=fusion, device=OracleDevice())
    want = json.loads((ref / f"q_{name}" / "qgraph.json").read_text())
    assert json.loads(json.dumps(got)) == want
    assert (tmp_path / "q" / "qweights.bin").read_bytes() == (ref / f"q_{name}" / "qweights.bin").read_bytes()
    assert json.loads((tmp_path / "q" / "qgraph.json").read_text()) == want


def test_producer_fixture_catches_a_planted_formula_change(golden_dir, tmp_path, monkeypatch):
    """A one-step change of the RMSNorm R rule (the largest feasible shift minus one) changes the
    written graph: the fixture comparison is sensitive to the formulas it pins."""
    real = Q._rms_shift

    def off_by_one(K, r_typ):
        R, _ = real(K, r_typ)
        return R - 1, Q.llround(math.ldexp(math.sqrt(float(K)), R - 1))

    monkeypatch.setattr(Q, "_rms_shift", off_by_one)
    ref = golden_dir / "refquant"
    got = Q.quantize_export(ref / "export_llama", tmp_path / "q", fusion=True, device=OracleDevice())
    assert json.loads(json.dumps(got)) != json.loads((ref / "q_llama_v2" / "qgraph.json").read_text())
