"""The float side's CPU restatement (oracle/float_np.py) pinned against the reference's own TinyLlama
and smooth_model outputs (tests/golden/float/, written by tests/golden/make_float_fixtures.py) and
against what the reparameterisation fixes: the smoothed model computes the same logits, and with
alpha = 1/2 each group's largest scaled activation equals its largest scaled weight column."""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

from llaccel_amd.floatside import FloatConfig, export_name
from oracle import float_np as FO

GOLD = Path(__file__).parent / "golden" / "float"
CASES = ["bias", "tied", "gqa_qknorm"]


def load(case):
    meta = json.loads((GOLD / f"{case}.json").read_text())
    z = np.load(GOLD / f"{case}.npz")
    cfg = FloatConfig.from_dict(meta["cfg"])

    def params(prefix):
        p = {export_name(k[len(prefix) + 1:]): z[k].astype(np.float64) for k in z.files if k.startswith(prefix + ".")
             and not k.startswith(prefix + ".logits")}
        return p

    return cfg, meta, z, params


@pytest.mark.parametrize("case", CASES)
def test_oracle_forward_equals_reference_logits(case):
    cfg, meta, z, params = load(case)
    p = params("sd")
    if meta["tied"]:
        p.pop("lm_head")
    for i, ids in enumerate(meta["seqs"]):
        got = FO.forward(cfg, p, ids)
        want = z[f"logits.{i}"]
        np.testing.assert_allclose(got, want, rtol=1e-4, atol=2e-6)


@pytest.mark.parametrize("case", CASES)
def test_oracle_calibration_equals_reference_records(case):
    cfg, meta, z, params = load(case)
    p = params("sd")
    got = FO.calibrate_tokens(cfg, p, meta["seqs"])
    want = meta["amax"] | {f"{k}.rms_min": v for k, v in meta["rms_min"].items()}
    assert set(got) == set(want)
    for k, v in want.items():
        assert got[k] == pytest.approx(v, rel=2e-5, abs=1e-9), k


@pytest.mark.parametrize("case", CASES)
def test_oracle_smoothing_equals_reference(case):
    cfg, meta, z, params = load(case)
    for k, sm in enumerate(meta["smooth"]):
        opts = {o: v for o, v in sm["options"].items() if o != "row_chunk"}
        p = params("sd")
        if meta["tied"]:
            p.pop("lm_head")
        res = FO.smooth_model(cfg, p, meta["seqs"], **opts)
        want = params(f"sm{k}")
        for name, w in want.items():
            got = p[name] if name in p else p["embed"]  # a head left tied is the embedding
            np.testing.assert_allclose(got, w, rtol=3e-5, atol=3e-5 * np.abs(w).max(), err_msg=f"{case} {k} {name}")
        for g in sm["metadata"]["groups"]:
            np.testing.assert_allclose(res["scales"][g["group"]], g["scales"], rtol=3e-5)
            assert res["alpha"][g["group"]] == g["selected_alpha"], (case, k, g["group"])
            if opts.get("auto_alpha"):
                ref_obj = {x["alpha"]: x["weighted_error"] for x in g["alpha_objective"]}
                for a, e in res["objective"][g["group"]].items():
                    assert e == pytest.approx(ref_obj[a], rel=1e-3), (g["group"], a)


@pytest.mark.parametrize("case", CASES)
def test_smoothed_oracle_model_computes_the_same_logits(case):
    """The reparameterisation is exact in real arithmetic: in float64 the logits agree to ~1e-12."""
    cfg, meta, z, params = load(case)
    base = params("sd")
    if meta["tied"]:
        base.pop("lm_head")
    for opts in ({"alpha": 0.5}, {"alpha": 0.9, "auto_alpha": True, "sample_rows": 3}):
        p = {k: v.copy() for k, v in base.items()}
        FO.smooth_model(cfg, p, meta["seqs"], **opts)
        for ids in meta["seqs"][:2]:
            a, b = FO.forward(cfg, base, ids), FO.forward(cfg, p, ids)
            np.testing.assert_allclose(b, a, rtol=1e-9, atol=1e-12)


def test_half_alpha_balances_activation_and_weight_ranges():
    """alpha = 1/2: s = sqrt(max|x| / max|W|) per channel, so max|x| / s = max|W| * s for every
    channel of every RMSNorm group (where neither maximum is clamped)."""
    cfg, meta, z, params = load("bias")
    p = params("sd")
    res = FO.smooth_model(cfg, {k: v.copy() for k, v in p.items()}, meta["seqs"], 0.5)
    members = {"norm": ["lm_head"]}
    for i in range(cfg.n_layers):
        members[f"layers.{i}.input_layernorm"] = [f"l{i}_wq", f"l{i}_wk", f"l{i}_wv"]
        members[f"layers.{i}.post_attention_layernorm"] = [f"l{i}_wg", f"l{i}_wu"]
    for name, wn in members.items():
        s = res["scales"][name]
        colmax = np.max([np.abs(p[w]).max(0) for w in wn], axis=0)
        act = res["maxima"][name]
        ok = (act > 1e-5) & (colmax > 1e-5)
        assert ok.all()
        np.testing.assert_allclose(act / s, colmax * s, rtol=1e-12)


def test_a_planted_transposed_rescale_breaks_equivalence():
    """A mistake in the restatement -- the value/output scales applied to the output projection's
    rows instead of its columns -- changes the logits, so the equivalence test would catch it."""
    cfg, meta, z, params = load("bias")
    assert cfg.dim == cfg.n_heads * cfg.head_dim  # o_proj is square here
    base = params("sd")
    p = {k: v.copy() for k, v in base.items()}
    res = FO.smooth_model(cfg, p, meta["seqs"], 0.5, smooth_ffn=False)
    s = res["scales"]["layers.0.value_output"]
    ds = np.repeat(s.reshape(cfg.n_kv_heads, 1, cfg.head_dim), cfg.n_heads // cfg.n_kv_heads, axis=1).reshape(-1)
    p["l0_wo"] = p["l0_wo"] / ds[None, :] * ds[:, None]
    a, b = FO.forward(cfg, base, meta["seqs"][0]), FO.forward(cfg, p, meta["seqs"][0])
    assert np.abs(a - b).max() > 1e-4


def test_names_map_both_ways_and_shapes_cover_every_parameter():
    from llaccel_amd.floatside import _expected_shapes, state_dict_name

    for case in CASES:
        cfg, meta, z, params = load(case)
        sd_names = {k[3:] for k in z.files if k.startswith("sd.")}
        assert {export_name(n) for n in sd_names} == set(_expected_shapes(cfg))
        assert {state_dict_name(export_name(n)) for n in sd_names} == sd_names


def test_rope_tables_are_the_reference_float32_tables():
    """llaccel_amd.floatside.rope_tables (torch fp32 ops of rope.py:64-99) against the oracle's numpy
    float32 restatement, default and linear kinds"""
    from llaccel_amd.floatside import rope_tables

    for scaling in (None, {"rope_type": "linear", "rope_theta": 5e5, "factor": 4.0}):
        cfg = FloatConfig(head_dim=64, max_seq=200, rope_base=1e6, rope_scaling=scaling)
        c, s = (t.numpy() for t in rope_tables(cfg))
        oc, os_ = FO.rope_tables(cfg)
        # torch's and numpy's float32 power may differ by an ulp of inv_freq, which position 199 turns
        # into ~2e-6 of angle
        np.testing.assert_allclose(c, oc, rtol=0, atol=1e-5)
        np.testing.assert_allclose(s, os_, rtol=0, atol=1e-5)
        assert np.abs(c - oc)[:8].max() < 3e-7  # early positions: the fp32 rounding of cos only


def _rope_fixture():
    meta = json.loads((GOLD / "rope.json").read_text())
    z = np.load(GOLD / "rope.npz")
    return {k: (FloatConfig.from_dict(c), z[f"{k}.cos"], z[f"{k}.sin"]) for k, c in meta.items()}


def _ratios(cfg, cos, sin):
    """default inv_freq / the table's inv_freq per frequency, read off position 1's angle"""
    d = cfg.head_dim
    theta = (cfg.rope_scaling or {}).get("rope_theta", cfg.rope_base)
    ang = np.arctan2(sin[1, :d // 2].astype(np.float64), cos[1, :d // 2].astype(np.float64))
    return theta ** (-np.arange(0, d, 2) / d) / ang


def test_reference_rope_fixture_follows_each_scaling_rule():
    """The reference's tables (tests/golden/float/rope.npz, from rope.py:64-99) against what each scaling
    fixes: cos^2 + sin^2 = amplitude^2 (attention_factor for yarn, 1 otherwise); default keeps the
    frequencies, linear divides all by `factor`; llama3 divides those with wavelength above
    original_max/low_freq_factor by `factor` and blends the band below it monotonically; yarn keeps the
    dimensions below the floor of the beta_fast correction, divides those from the ceiling of the
    beta_slow correction on by `factor`, and ramps 1/ratio linearly in between (here dims 0..6)."""
    tabs = _rope_fixture()
    for kind, (cfg, cos, sin) in tabs.items():
        amp = (cfg.rope_scaling or {}).get("attention_factor", 1.0)
        np.testing.assert_allclose(np.hypot(cos, sin), amp, rtol=3e-7, err_msg=kind)
        np.testing.assert_array_equal(cos[0], np.float32(amp))
        np.testing.assert_array_equal(cos[:, :cfg.head_dim // 2], cos[:, cfg.head_dim // 2:])
    np.testing.assert_allclose(_ratios(*tabs["default"]), 1.0, rtol=1e-5)
    np.testing.assert_allclose(_ratios(*tabs["linear"]), 4.0, rtol=1e-5)
    cfg, cos, sin = tabs["llama3"]
    r = _ratios(cfg, cos, sin)
    p = cfg.rope_scaling
    wave = 2 * np.pi * (p["rope_theta"] ** (np.arange(0, cfg.head_dim, 2) / cfg.head_dim))
    far = wave > p["original_max_position_embeddings"] / p["low_freq_factor"]
    assert far.sum() == 29 and (~far).sum() == 3  # the fixture covers both regions
    np.testing.assert_allclose(r[far], p["factor"], rtol=1e-5)
    assert np.all(np.diff(r[~far]) > 0) and np.all((r[~far] > 1) & (r[~far] < p["factor"]))
    cfg, cos, sin = tabs["yarn"]
    r = _ratios(cfg, cos, sin)
    np.testing.assert_allclose(r[0], 1.0, rtol=1e-5)
    np.testing.assert_allclose(r[6:], 4.0, rtol=1e-5)
    ramp = (1 - 1 / r[:7]) / (1 - 1 / 4.0)
    np.testing.assert_allclose(ramp, np.arange(7) / 6, atol=1e-5)


def test_rope_tables_equal_the_reference_tables_for_every_scaling():
    """llaccel_amd.floatside.rope_tables against the reference's own default, linear, llama3 and yarn tables
    (the same float32 operations in the same order: equal up to the platform's float32 cos/sin)"""
    from llaccel_amd.floatside import rope_tables

    for kind, (cfg, cos, sin) in _rope_fixture().items():
        c, s = (t.numpy() for t in rope_tables(cfg))
        np.testing.assert_allclose(c, cos, rtol=0, atol=2.4e-7, err_msg=kind)
        np.testing.assert_allclose(s, sin, rtol=0, atol=2.4e-7, err_msg=kind)
        if kind in ("default", "linear"):
            oc, os_ = FO.rope_tables(cfg)
            np.testing.assert_allclose(oc, cos, rtol=0, atol=1e-5, err_msg=kind)
            np.testing.assert_allclose(os_, sin, rtol=0, atol=1e-5, err_msg=kind)


def test_float_model_needs_the_library_and_a_gpu():
    """The product path refuses to run without the HIP library and a GPU (no CPU fallback)."""
    import torch

    from llaccel_amd.floatside import FloatModel

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    cfg, meta, z, params = load("bias")
    with pytest.raises((RuntimeError, OSError)):
        FloatModel(cfg, {k: v.astype(np.float32) for k, v in params("sd").items()})
