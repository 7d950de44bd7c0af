"""The float side on the GPU (llaccel_amd.floatside): its kernels against exact host arithmetic, and
calibration and SmoothQuant against the reference's own outputs (tests/golden/float/, written by the
reference's TinyLlama and smooth_model) and the float64 restatement (oracle/float_np.py).

Tolerances: the kernels' maxima and fp32 rescalings are exact (bit-equal); the row-RMS minima and the
objective sums are double sums in another order (rtol 1e-12 / 1e-9); the forward runs fp32 GEMMs and
attention in another order than the reference's CPU torch, so records, scales and smoothed weights
agree to rtol 3e-5 and logits to the reference test's atol 3e-5 / rtol 3e-4."""
from __future__ import annotations

import ctypes
import json
from pathlib import Path

import numpy as np
import pytest

from oracle import float_np as FO

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).parent / "golden" / "float"
CASES = ["bias", "tied", "gqa_qknorm"]


def _t():
    import torch

    return torch


def _p(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _s():
    return ctypes.c_void_p(_t().cuda.current_stream().cuda_stream)


def load(case):
    from llaccel_amd.floatside import FloatConfig

    meta = json.loads((GOLD / f"{case}.json").read_text())
    z = np.load(GOLD / f"{case}.npz")
    return FloatConfig.from_dict(meta["cfg"]), meta, z


def state(z, prefix):
    return {k[len(prefix) + 1:]: z[k] for k in z.files if k.startswith(prefix + ".") and ".logits" not in k[len(prefix):]}


def model_of(case, prefix="sd"):
    from llaccel_amd.floatside import FloatModel

    cfg, meta, z = load(case)
    torch = _t()
    sd = {k: torch.from_numpy(v.copy()) for k, v in state(z, prefix).items()}
    if meta["tied"]:
        sd["lm_head.weight"] = sd["embed_tokens.weight"]  # one tensor, as the tied TinyLlama
    return FloatModel.from_state_dict(cfg, sd), cfg, meta, z


# ---- kernels ---------------------------------------------------------------------------------
def test_absmax_kernel_is_exact_and_counts_nonfinite():
    from llaccel_amd import _lib

    torch = _t()
    rng = np.random.default_rng(5)
    rows, cols, ld = 1000, 777, 800
    x = (rng.standard_normal((rows, ld)) * np.exp(rng.uniform(-20, 20, (rows, ld)))).astype(np.float32)
    x[3, 5], x[900, 776], x[17, 0] = np.nan, np.inf, -np.inf
    xd = torch.from_numpy(x).cuda()
    col = torch.zeros(cols, dtype=torch.float32, device="cuda")
    col[10] = 1e30  # running maxima start at the caller's values
    amax = torch.zeros(1, dtype=torch.float32, device="cuda")
    bad = torch.zeros(1, dtype=torch.int32, device="cuda")
    _lib.call("llhip_f32_absmax", _p(xd), rows, cols, ld, _p(col), _p(amax), _p(bad), _s())
    a = np.abs(x[:, :cols])
    a[~np.isfinite(a)] = 0
    want = a.max(0)
    want[10] = 1e30
    assert np.array_equal(col.cpu().numpy(), want)
    assert amax.cpu().numpy()[0] == a.max()
    assert int(bad.cpu()[0]) == 3


def test_rms_min_kernel_equals_float64():
    from llaccel_amd import _lib

    torch = _t()
    rng = np.random.default_rng(6)
    x = (rng.standard_normal((333, 48)) * rng.uniform(0.01, 5, (333, 1))).astype(np.float32)
    out = torch.full((1,), np.inf, dtype=torch.float64, device="cuda")
    _lib.call("llhip_f32_rms_min", _p(torch.from_numpy(x).cuda()), 333 * 3, 16, _p(out), _s())
    want = np.sqrt((x.astype(np.float64).reshape(-1, 16) ** 2).mean(1)).min()
    assert float(out.cpu()[0]) == pytest.approx(want, rel=1e-14)


def test_rescale_kernel_is_the_fp32_operations_in_order():
    from llaccel_amd import _lib

    torch = _t()
    rng = np.random.default_rng(7)
    rows, cols, ld = 70, 130, 131
    x = rng.standard_normal((rows, ld)).astype(np.float32)
    cm, cd, rd = (np.exp(rng.uniform(-8, 8, n)).astype(np.float32) for n in (cols, cols, rows))
    xd = torch.from_numpy(x.copy()).cuda()
    dev = [torch.from_numpy(v).cuda() for v in (cm, cd, rd)]
    _lib.call("llhip_f32_rescale", _p(xd), rows, cols, ld, *[_p(v) for v in dev], _s())
    want = x.copy()
    want[:, :cols] = ((x[:, :cols] * cm[None, :]) / cd[None, :]) / rd[:, None]
    assert np.array_equal(xd.cpu().numpy(), want)
    _lib.call("llhip_f32_rescale", _p(xd), rows, cols, ld, None, None, _p(dev[2]), _s())
    want[:, :cols] = want[:, :cols] / rd[:, None]
    assert np.array_equal(xd.cpu().numpy(), want)


def test_smooth_objective_kernel_equals_host_terms():
    from llaccel_amd import _lib

    torch = _t()
    rng = np.random.default_rng(8)
    rows, cols = 300, 96
    W = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    W[7] = 0  # an all-zero row takes the 1e-30 step
    s, ae, en = (np.exp(rng.uniform(-3, 3, cols)).astype(np.float32) for _ in range(3))
    out = torch.zeros(2, dtype=torch.float64, device="cuda")
    dv = [torch.from_numpy(v).cuda() for v in (W, s, ae, en)]
    _lib.call("llhip_f32_smooth_objective", _p(dv[0]), rows, cols, _p(dv[1]), _p(dv[2]), _p(dv[3]), _p(out), _s())
    w = W * s[None, :]
    step = np.maximum(np.abs(w).max(1, keepdims=True), np.float32(1e-30)) / np.float32(127)
    q = np.clip(np.rint(w / step), -128, 127).astype(np.float32) * step
    e1 = ((w * w) * ae[None, :]).astype(np.float64).sum()
    e2 = (((q - w) * (q - w)) * en[None, :]).astype(np.float64).sum()
    got = out.cpu().numpy()
    assert got[0] == pytest.approx(e1, rel=1e-9) and got[1] == pytest.approx(e2, rel=1e-9)


# ---- calibration -----------------------------------------------------------------------------
@pytest.mark.parametrize("case", CASES)
def test_gpu_forward_and_calibration_equal_reference(case):
    from llaccel_amd.floatside import calibrate_tokens

    model, cfg, meta, z = model_of(case)
    print("case", case, flush=True)
    for i, ids in enumerate(meta["seqs"]):
        got = model.forward(ids).cpu().numpy()
        np.testing.assert_allclose(got, z[f"logits.{i}"], rtol=3e-4, atol=3e-5)
    rec = calibrate_tokens(model, meta["seqs"])
    want = meta["amax"] | {f"{k}.rms_min": v for k, v in meta["rms_min"].items()}
    assert set(rec) == set(want)
    for k, v in want.items():
        assert rec[k] == pytest.approx(v, rel=3e-5, abs=1e-9), k


def test_gpu_clipping_bounds_equal_reference():
    from llaccel_amd.floatside import calibrate_tokens

    model, cfg, meta, z = model_of("bias")
    rec = calibrate_tokens(model, meta["seqs"], optimize_quantization=True, sample_budget=meta["bounds_budget"])
    # the selected bound is a fraction of the abs-max (rtol 3e-5, as the records); its squared error
    # depends on which sampled values fall on either side of a rounding boundary of the grid, which
    # activations that differ in their last fp32 bits move: rtol 5e-2
    for k, v in meta["bounds"].items():
        assert rec[k] == pytest.approx(v, rel=3e-5 if k.endswith("_absmax") else 5e-2, abs=1e-12), k


def test_gpu_calibration_of_a_larger_model_equals_the_oracle():
    """A synthetic 4-layer GQA model with Q/K norm and biases, 3 sequences up to 96 tokens."""
    from llaccel_amd.floatside import FloatConfig, FloatModel, _expected_shapes, calibrate_tokens

    cfg = FloatConfig(dim=256, n_layers=4, n_heads=8, n_kv_heads=2, head_dim=32, ffn=640, vocab=1000, max_seq=128,
                      qkv_bias=True, qk_norm=True, rope_base=1e6, rms_eps=1e-6)
    rng = np.random.default_rng(9)
    params = {n: (rng.standard_normal(s) * (0.05 if len(s) == 2 else 0.3) + (1.0 if "norm" in n else 0.0))
              .astype(np.float32) for n, s in _expected_shapes(cfg).items()}
    seqs = [rng.integers(0, cfg.vocab, n).tolist() for n in (96, 40, 2)]
    rec = calibrate_tokens(FloatModel(cfg, params), seqs)
    want = FO.calibrate_tokens(cfg, {k: v.astype(np.float64) for k, v in params.items()}, seqs)
    assert set(rec) == set(want)
    for k, v in want.items():
        assert rec[k] == pytest.approx(v, rel=1e-4), k


def test_gpu_calibration_of_an_export_reproduces_its_record():
    """FloatModel.from_export on a committed export directory, over the token sequence its calib.json
    was recorded on (llaccel_amd.synth.write_export: default_rng(seed + 1000), 24 tokens)."""
    from llaccel_amd.floatside import FloatModel, calibrate_tokens

    d = Path(__file__).parent / "golden" / "refquant" / "export_qwen"
    model = FloatModel.from_export(d)
    ids = np.random.default_rng(12 + 1000).integers(0, model.cfg.vocab, 24).tolist()
    rec = calibrate_tokens(model, [ids])
    want = json.loads((d / "calib.json").read_text())
    for k, v in want.items():
        assert rec[k] == pytest.approx(v, rel=1e-4), k


# ---- SmoothQuant -----------------------------------------------------------------------------
@pytest.mark.parametrize("case", CASES)
def test_gpu_smoothing_equals_reference(case):
    from llaccel_amd.floatside import smooth_model

    cfg, meta, z = load(case)
    for k, sm in enumerate(meta["smooth"]):
        print("case", case, sm["options"], flush=True)
        model, *_ = model_of(case)
        md = smooth_model(model, meta["seqs"], **sm["options"])
        ref = sm["metadata"]
        assert set(md) == set(ref) and md["untied_lm_head"] == ref["untied_lm_head"]
        assert [g["group"] for g in md["groups"]] == [g["group"] for g in ref["groups"]]
        for g, r in zip(md["groups"], ref["groups"]):
            assert g["selected_alpha"] == r["selected_alpha"], g["group"]
            np.testing.assert_allclose(g["scales"], r["scales"], rtol=3e-5)
            for key in ("activation_max_before", "activation_max_after", "weight_max_before", "weight_max_after"):
                assert g[key] == pytest.approx(r[key], rel=3e-5), (g["group"], key)
        got = model.state_dict()
        for name, w in state(z, f"sm{k}").items():
            np.testing.assert_allclose(got[name], w, rtol=3e-5, atol=3e-5 * np.abs(w).max(), err_msg=name)
        logits = model.forward(meta["seqs"][0]).cpu().numpy()
        np.testing.assert_allclose(logits, z[f"sm{k}.logits.0"], rtol=3e-4, atol=3e-5)


def test_gpu_smoothing_keeps_the_model_and_balances_outliers():
    """test_smoothquant.py:27-64: the smoothed model's logits equal the original's; a planted
    activation outlier (gamma[0] = 1000) moves into the weights, the two ranges equal at alpha 1/2."""
    from llaccel_amd.floatside import smooth_model

    model, cfg, meta, z = model_of("bias")
    model.p["l0_attn_norm"][0] = 1000.0
    tokens = meta["seqs"][0]
    before = model.forward(tokens).cpu().numpy()
    md = smooth_model(model, meta["seqs"], 0.5)
    g = md["groups"][0]
    assert g["activation_max_after"] < g["activation_max_before"] / 50
    assert g["weight_max_after"] > g["weight_max_before"]
    assert g["activation_max_after"] == pytest.approx(g["weight_max_after"], rel=1e-5)
    np.testing.assert_allclose(model.forward(tokens).cpu().numpy(), before, rtol=3e-4, atol=3e-5)


def test_gpu_smoothing_rejects_what_the_reference_rejects():
    from llaccel_amd.floatside import smooth_model

    model, cfg, meta, z = model_of("bias")
    for alpha in (-1, 1.1, float("nan"), float("inf"), True):
        with pytest.raises(ValueError, match="alpha"):
            smooth_model(model, [[1, 2]], alpha)
    for seqs in ([], [[]], [[1] * 33], [[-1]], [[80]], [[True]], [[1.5]]):
        with pytest.raises(ValueError):
            smooth_model(model, seqs)
    gamma = model.p["l0_attn_norm"].clone()
    model.p["lm_head"][0, 0] = float("nan")
    with pytest.raises(ValueError, match="nonfinite weight"):
        smooth_model(model, [[1, 2, 3]])
    assert _t().equal(gamma, model.p["l0_attn_norm"])  # nothing changed before the error
