"""GPU parity of the qgraph producer (llaccel_amd.quantize): the weight conversions
(llhip_quant_rows_i8, llhip_quant_i16) against the float64 oracle bit for bit, and the produced
graphs against the reference quantizer's contract (test_refquant.py:158-292 restated: tensor
index and alignment, exponent policies, op sequence, fused forms, the late-outlier known answers),
then run through the datapath and equal to the CPU oracle on the same graph."""
from __future__ import annotations

import ctypes
import dataclasses
import json

import numpy as np
import pytest

from llaccel_amd import _lib
from llaccel_amd import golden as G
from llaccel_amd import quantize as Q
from llaccel_amd import synth
from oracle import golden_np as O
from oracle import quant_np as QN
from tests.gpu_helpers import down, ptr, stream, torch, up

pytestmark = pytest.mark.gpu

# dims a multiple of 16 (refquant.py:407-409), two layers, QKV bias
CFG = dataclasses.replace(synth.CONFIGS["tiny"], name="rq", dim=64, ffn=128, vocab=200, qkv_bias=True)
# head_dim 128 with Q/K RMSNorm (beyond the reference quantizer's head_dim limit)
CFG128 = dataclasses.replace(synth.CONFIGS["tiny"], name="rq128", dim=128, n_heads=2, n_kv_heads=1, head_dim=128,
                             ffn=256, vocab=96, max_seq=64, qk_norm=True, rope_base=1e6, rms_eps=1e-6)


def _rows_i8(w, n_rows=None):
    t = torch()
    w = np.ascontiguousarray(w, dtype=np.float32)
    N, K = (w.shape[0] if n_rows is None else n_rows), w.shape[1]
    src = t.zeros((N, K), dtype=t.float32, device="cuda")
    src[: w.shape[0]].copy_(t.from_numpy(w))
    q = t.empty((N, K), dtype=t.int8, device="cuda")
    s = t.empty(N, dtype=t.float64, device="cuda")
    st = t.zeros(1, dtype=t.int32, device="cuda")
    _lib.call("llhip_quant_rows_i8", ptr(src), N, K, K, ptr(q), K, ptr(s), ptr(st), stream())
    return q.cpu().numpy(), s.cpu().numpy(), int(down(st)[0])


def _i16(x, e):
    t = torch()
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    src = t.from_numpy(x).cuda()
    y = t.empty(x.size, dtype=t.int16, device="cuda")
    st = t.zeros(1, dtype=t.int32, device="cuda")
    _lib.call("llhip_quant_i16", ptr(src), x.size, e, ptr(y), ptr(st), stream())
    return y.cpu().numpy(), int(down(st)[0])


@pytest.mark.parametrize("N,K", [(64, 896), (37, 100), (5, 4864), (300, 3)])
def test_quant_rows_i8_equals_oracle(N, K):
    rng = np.random.default_rng(N * 31 + K)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    w[0] = 0.0                                   # all-zero row: scale 1, zeros
    if N > 2:                                    # exact halves: w / s lands on k + 0.5
        w[1, : min(K, 6)] = np.array([127.0, 63.5, -63.5, 0.5, -0.5, 2.5], np.float32)[: min(K, 6)]
        w[2] = np.float32(3.0e38) * np.sign(rng.standard_normal(K)).astype(np.float32)  # near f32 max
    q, s, st = _rows_i8(w)
    wq, ws = QN.quant_rows_i8(w.astype(np.float64))
    assert st == 0
    assert np.array_equal(s, ws) and np.array_equal(q, wq)
    if N > 2 and K >= 6:
        assert q[1, :6].tolist() == [127, 64, -64, 1, -1, 3]
    # rows past the tensor (the padded lm_head) are zero rows
    q2, s2, _ = _rows_i8(w, N + 3)
    assert np.array_equal(q2[:N], q) and not q2[N:].any() and s2[N:].tolist() == [1.0] * 3


@pytest.mark.parametrize("K", [64, 896])
def test_quant_rows_i8_ties_near_ties_and_tiny_rows(K):
    """The wave kernel rounds from a float32 quotient and settles near-halves in float64: exact
    halves (row max 127 * 2^-3, entries (k + 1/2) * 2^-3), entries one ulp either side of them,
    rows whose abs-max is subnormal or just above 2^-100, and rows at the float32 maximum."""
    rng = np.random.default_rng(K)
    rows = []
    k = rng.integers(-127, 127, K)
    half = ((k + 0.5) * 0.125).astype(np.float32)
    half[0] = 127 * 0.125
    rows.append(half)
    rows.append(np.nextafter(half, np.float32(np.inf)))
    rows.append(np.nextafter(half, np.float32(-np.inf)))
    for scale in (1e-39, 3e-45, 2.0**-99, 2.0**-101, 3.0e38, 1.7):
        r = (np.clip(rng.standard_normal(K), -1.1, 1.1) * scale).astype(np.float32)  # finite at 3e38
        r[1] = np.float32(scale)
        rows.append(r)
    w = np.stack(rows)
    q, s, st = _rows_i8(w)
    wq, ws = QN.quant_rows_i8(w.astype(np.float64))
    assert st == 0 and np.array_equal(s, ws) and np.array_equal(q, wq)
    assert np.array_equal(q[0, 1:], np.clip(np.where(k[1:] >= 0, k[1:] + 1, k[1:]), -128, 127))


def test_quant_rows_i8_strided_and_non_finite():
    t = torch()
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((10, 20)) * 3).astype(np.float32)
    src = up(np.pad(w, ((0, 0), (0, 7))), np.float32)  # row stride 27
    q = t.zeros((10, 24), dtype=t.int8, device="cuda")
    s = t.empty(10, dtype=t.float64, device="cuda")
    st = t.zeros(1, dtype=t.int32, device="cuda")
    _lib.call("llhip_quant_rows_i8", ptr(src), 10, 20, 27, ptr(q), 24, ptr(s), ptr(st), stream())
    wq, ws = QN.quant_rows_i8(w.astype(np.float64))
    qh = q.cpu().numpy()
    assert np.array_equal(qh[:, :20], wq) and np.array_equal(s.cpu().numpy(), ws) and not qh[:, 20:].any()
    for bad in (np.inf, -np.inf, np.nan):
        w2 = w.copy()
        w2[4, 7] = bad
        assert _rows_i8(w2)[2] == 1
    with pytest.raises(ValueError):
        _lib.call("llhip_quant_rows_i8", ptr(src), 10, 20, 19, ptr(q), 24, ptr(s), ptr(st), stream())


def test_quant_i16_equals_oracle():
    rng = np.random.default_rng(11)
    x = np.concatenate([rng.standard_normal(5000) * 0.3, np.array([1.5, -1.5, 2.5, -2.5, 1e9, -1e9, 0.0])])
    x = x.astype(np.float32)
    for e in (-15, -12, -1, 0, 3):
        y, st = _i16(x, e)
        assert st == 0 and np.array_equal(y, QN.quant_i16(x.astype(np.float64), e)), e
    y, _ = _i16(np.array([1.5, -1.5, 2.5], np.float32), -1)
    assert y.tolist() == [3, -3, 5]
    assert _i16(np.array([1.0, np.nan], np.float32), 0)[1] == 1


# ---- the produced graphs ------------------------------------------------------------------
@pytest.fixture(scope="module")
def produced(tmp_path_factory):
    base = tmp_path_factory.mktemp("quantize")
    ex = synth.write_export(base / "export", CFG, seed=5)
    g1 = Q.quantize_export(ex, base / "v1", fusion=False)
    g2 = Q.quantize_export(ex, base / "v2", fusion=True)
    return ex, base, g1, g2


def test_graph_contract(produced):
    ex, base, q1, q2 = produced
    calib = json.loads((ex / "calib.json").read_text())
    m = q1["model"]
    assert m["vocab"] == 200 and m["vocab_padded"] == 208 and m["dim"] == 64
    assert q1["input"] == "input" and q1["output"] == "logits"
    assert (base / "v1" / "qweights.bin").read_bytes() == (base / "v2" / "qweights.bin").read_bytes()
    t = q1["tensors"]
    assert t["embed"] == {"dtype": "i16", "shape": [208, 64], "offset": 0, "exp": m["E_RES"]}
    assert t["rope_cos"]["shape"] == [64, 8] and t["l0_wk"]["shape"] == [32, 64] and t["lm_head"]["shape"] == [208, 64]
    assert t["l0_wk.rq"]["dtype"] == "rq" and t["l0_wk.rq"]["shape"] == [32]
    assert t["l0_bq"]["dtype"] == "i32" and t["l0_attn_norm"]["dtype"] == "i16" and "exp" in t["l0_attn_norm"]
    assert all(v["offset"] % 64 == 0 for v in t.values())
    assert m["E_RES"] == Q.i16_exponent(calib["input"]) == q1["exps"]["input"]
    previous = "input"
    for i in range(2):
        for branch, out in ((f"l{i}.o", f"l{i}.x1"), (f"l{i}.d", f"l{i}.x2")):
            want = max(Q.i16_exponent(calib[branch]), Q.i16_exponent(calib[out]), Q.i16_exponent(calib[previous]),
                       q1["exps"][previous])
            assert q1["exps"][branch] == q1["exps"][out] == want
            previous = out
    assert m["E_LOGIT"] == Q.i16_exponent(calib["logits"]) == q1["exps"]["logits"]
    for i in range(2):
        assert q1["exps"][f"l{i}.q"] == q1["exps"][f"l{i}.qr"] >= Q.i16_exponent(calib[f"l{i}.qr"])
        assert q1["exps"][f"l{i}.k"] == q1["exps"][f"l{i}.kr"]
        assert q1["scales"][f"l{i}.h.q"] == calib[f"l{i}.h"] / 127 and q1["scales"][f"l{i}.v"] == calib[f"l{i}.v"] / 127
    layer = ["rmsnorm", "quant", "linear", "linear", "linear", "rope", "rope", "quant", "quant", "kv_write", "attention",
             "linear", "add", "rmsnorm", "quant", "linear", "linear", "silu", "mul", "quant", "linear", "add"]
    kinds = [o["op"] for o in q1["ops"]]
    assert kinds == layer * 2 + ["rmsnorm", "quant", "linear"]
    for o in q1["ops"]:
        if o["op"] == "linear":
            assert o["epilogue"] == "none" and o["out_dtype"] == ("i8" if o["out"].endswith(".v") else "i16")
            assert (o["bias"] is not None) == (o["out"].split(".")[-1] in ("q", "k", "v"))
        elif o["op"] == "quant":
            assert o["out"] == o["in"] + ".q" and 2**30 <= o["M"] < 2**31
        elif o["op"] == "attention":
            assert o["prob_bits"] == 15 and o["q"].endswith(".qr.q")
        elif o["op"] == "add":
            assert o["sh_b"] == q1["exps"][o["a"]] - q1["exps"][o["b"]] >= 0
    k2 = [o["op"] for o in q2["ops"]]
    assert "silu" not in k2 and "mul" not in k2 and k2.count("linear") == kinds.count("linear")
    fused = {o["out"]: o for o in q2["ops"] if o["op"] == "linear" and o["epilogue"] != "none"}
    eligible = {o["out"] for o in q1["ops"] if o["op"] == "add" and o["sh_b"] == 0}
    assert set(fused) == eligible | {f"l{i}.{n}" for i in range(2) for n in ("sg", "f")}
    assert fused["l0.f"]["aux"] == "l0.sg" and fused["l0.f"]["rq"] == "l0_wu.rq"


def test_weights_and_parameters_follow_the_oracle(produced):
    """Every weight tensor of the blob is the oracle's conversion of the export's float weights,
    and every rq pair is the (M, S) of s_a * s_w[n] / 2^e_out."""
    ex, base, q1, _ = produced
    _, W, _ = Q.load_export(ex)
    blob = (base / "v1" / "qweights.bin").read_bytes()
    t = q1["tensors"]

    def read(name, dt):
        spec = t[name]
        n = int(np.prod(spec["shape"])) * (2 if spec["dtype"] == "rq" else 1)
        return np.frombuffer(blob, dtype=dt, count=n, offset=spec["offset"])

    for o in q1["ops"]:
        if o["op"] != "linear":
            continue
        w = np.zeros((o["N"], o["K"]))
        w[: W[o["w"]].shape[0]] = W[o["w"]]
        wq, s_w = QN.quant_rows_i8(w)
        assert np.array_equal(read(o["w"], "<i1").reshape(wq.shape), wq), o["w"]
        s_a = q1["scales"][o["in"]]
        den = q1["scales"][o["out"]] if o["out_dtype"] == "i8" else 2.0 ** q1["exps"][o["out"]]
        rq = read(o["rq"], "<i4").reshape(-1, 2)
        for n in (0, o["N"] // 2, o["N"] - 1):
            assert tuple(rq[n]) == Q.mulshift_pair(s_a * s_w[n] / den)
    e = q1["model"]["E_RES"]
    emb = np.zeros((208, 64))
    emb[:200] = W["embed"]
    assert np.array_equal(read("embed", "<i2").reshape(208, 64), QN.quant_i16(emb, e))


@pytest.mark.parametrize("which", ["v1", "v2"])
def test_produced_graph_runs_exact(produced, which):
    _, base, _, _ = produced
    qdir = base / which
    g, o = G.GoldenModel(qdir), O.OracleModel(qdir, backend="c")
    prompt = list(range(3, 22))
    assert g.generate(prompt, 6) == o.generate(prompt, 6)


def test_late_residual_outlier_known_answers(produced):
    """test_refquant.py:252-276: a late residual outlier does not coarsen the embedding's
    exponent, and its shifted ADD stays unfused (embedding rows 0.01 -> 328 at 2^-15)."""
    ex = produced[0]
    cfg, weights, calib = Q.load_export(ex)
    calib = dict(calib)
    calib["input"] = 0.01
    for layer in range(cfg["n_layers"]):
        for n in ("o", "d", "x1", "x2"):
            calib[f"l{layer}.{n}"] = 0.02
    calib["l1.d"] = calib["l1.x2"] = 1024.0
    weights = dict(weights)
    weights["embed"] = np.full_like(weights["embed"], 0.01)
    qs = [Q.Graph(cfg, weights, calib, fusion) for fusion in (False, True)]
    graphs = [q.build() for q in qs]
    assert qs[0].pack.bytes() == qs[1].pack.bytes()
    for q, gph in zip(qs, graphs):
        assert gph["model"]["E_RES"] == gph["exps"]["input"] == -15
        assert gph["exps"]["l0.x1"] == gph["exps"]["l0.x2"] == -15 and gph["exps"]["l1.x2"] == -4
        off = gph["tensors"]["embed"]["offset"]
        assert np.all(np.frombuffer(q.pack.bytes(), "<i2", count=weights["embed"].size, offset=off) == 328)
        late = next(op for op in gph["ops"] if op["op"] == "add" and op["out"] == "l1.x2")
        assert (late["a"], late["b"], late["sh_b"]) == ("l1.d", "l1.x1", 11)
        assert not any(op.get("epilogue") == "resadd" and op["out"] == "l1.x2" for op in gph["ops"])


def test_head_dim_128_with_qk_norm(tmp_path):
    ex = synth.write_export(tmp_path / "ex", CFG128, seed=9)
    graph = Q.quantize_export(ex, tmp_path / "q", fusion=True)
    assert sum(op["op"] == "rmsnorm" and op.get("heads") == 2 for op in graph["ops"]) == 2
    g, o = G.GoldenModel(tmp_path / "q"), O.OracleModel(tmp_path / "q", backend="c")
    prompt = list(range(5, 25))
    assert g.generate(prompt, 4) == o.generate(prompt, 4)
    with pytest.raises(ValueError, match="head_dim"):
        Q.Graph({**Q.load_export(ex)[0], "head_dim": 8}, {}, {}, False).build()


@pytest.mark.parametrize("name,model,fusion", [("llama_v2", "llama", True), ("qwen_v1", "qwen", False),
                                               ("qwen_v2", "qwen", True)])
def test_gpu_producer_equals_reference_quantizer(golden_dir, tmp_path, name, model, fusion):
    """The producer with its GPU conversions writes the graph and the byte-identical qweights.bin
    that the reference's refquant.quantize_export wrote (tests/golden/refquant/)."""
    ref = golden_dir / "refquant"
    got = Q.quantize_export(ref / f"export_{model}", tmp_path / "q", fusion=fusion)
    assert json.loads(json.dumps(got)) == json.loads((ref / f"q_{name}" / "qgraph.json").read_text())
    assert (tmp_path / "q" / "qweights.bin").read_bytes() == (ref / f"q_{name}" / "qweights.bin").read_bytes()
