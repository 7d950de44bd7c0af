"""Pins the oracle's composition (OracleModel = GoldenModel restatement) against the
outputs of the reference's own golden.py (fixtures in tests/golden/ref_tiny_*) and the
invariants of the reference's tests/python/test_golden_e2e.py."""
from __future__ import annotations

import json
import math

import numpy as np
import pytest

from oracle import golden_np as O

CASES = ["ref_tiny_v2", "ref_tiny_v1", "ref_tiny_v2_pad", "ref_tiny_v2_m4",
         "ref_qwen2_bias", "ref_qwen3_qknorm_d128", "ref_d256"]  # Qwen2 bias, Qwen3 Q/K norm at D = 128, D = 256


def _load(golden_dir, name):
    d = golden_dir / name
    meta = json.loads((d / "meta.json").read_text())
    rec = json.loads((d / "record.json").read_text())
    kv = np.load(d / "kv_final.npz")
    acts = np.load(d / "acts.npz")
    return d / "qgraph", meta, rec, kv, acts


@pytest.mark.parametrize("backend", ["np", "c"])
@pytest.mark.parametrize("name", CASES)
def test_oracle_reproduces_reference_golden_run(golden_dir, name, backend):
    qdir, meta, rec, kv, acts = _load(golden_dir, name)
    m = O.OracleModel(qdir, backend=backend)
    got_acts: list = []
    got = m.generate(meta["prompt"], meta["n_tokens"], got_acts)
    assert got == rec
    for layer, (k, v) in m.kv.items():
        assert np.array_equal(k, kv[f"k{layer}"]) and np.array_equal(v, kv[f"v{layer}"])
    for i in meta["acts_steps"]:
        names = {key.split("/", 1)[1] for key in acts.files if key.startswith(f"step{i}/")}
        assert names == set(got_acts[i]["acts"])
        for n in names:
            assert np.array_equal(got_acts[i]["acts"][n], acts[f"step{i}/{n}"]), (i, n)


def test_launch_record_structure(golden_dir):
    """test_golden_e2e.py:112-141 -- launch sequence and record layout."""
    qdir, meta, rec, _, _ = _load(golden_dir, "ref_tiny_v2_pad")
    assert rec["steps"][0] == {"kind": "prefill", "pos": 0, "rows": 16, "valid_rows": 16}
    assert rec["steps"][1] == {"kind": "prefill", "pos": 16, "rows": 16, "valid_rows": 4}
    assert rec["steps"][2] == {"kind": "decode", "pos": 20, "rows": 1, "valid_rows": 1}
    assert len(rec["generated"]) == 12 and len(rec["steps"]) == 14
    assert rec["generated"] == rec["argmax_per_step"][1:13]
    for row, am in zip(rec["logits_last_rows"], rec["argmax_per_step"]):
        assert am == row.index(max(row))


def test_chunked_prefill_equals_sequential_decode(golden_dir):
    """test_golden_e2e.py:144-155."""
    qdir = golden_dir / "ref_tiny_v2" / "qgraph"
    toks = np.random.default_rng(3).integers(0, 256, 21).tolist()
    a = O.OracleModel(qdir, "c").prefill(toks)
    m2 = O.OracleModel(qdir, "c")
    b = [m2.decode(t, i) for i, t in enumerate(toks)]
    assert all(np.array_equal(x, y) for x, y in zip(a, b))


def test_fused_equals_unfused(golden_dir):
    """test_golden_e2e.py:158-162."""
    r1 = O.OracleModel(golden_dir / "ref_tiny_v1" / "qgraph", "c").generate(list(range(10)), 16)
    r2 = O.OracleModel(golden_dir / "ref_tiny_v2" / "qgraph", "c").generate(list(range(10)), 16)
    assert r1 == r2


def test_max_seq_errors(golden_dir):
    """test_golden_e2e.py:192-204."""
    qdir = golden_dir / "ref_tiny_v2" / "qgraph"
    with pytest.raises(ValueError, match="max_seq"):
        O.OracleModel(qdir).generate(list(range(10)), 64)
    r = O.OracleModel(qdir, "c").generate(list(range(10)), 54)
    assert len(r["generated"]) == 54 and r["steps"][-1]["pos"] == 62 and len(r["steps"]) == 54


def test_pad_rows_do_not_leak(golden_dir):
    """test_golden_e2e.py:207-215."""
    qdir = golden_dir / "ref_tiny_v2" / "qgraph"
    toks = [(3 + i) % 256 for i in range(20)]
    a = O.OracleModel(qdir, "c").prefill(toks)
    b = O.OracleModel(qdir, "c").prefill(toks[:12])
    assert all(np.array_equal(x, y) for x, y in zip(a[:12], b))


def test_planted_composition_mistake_is_caught(golden_dir):
    """A restatement recording the wrong logits row (row 0 of each chunk) fails the fixture."""
    qdir, meta, rec, _, _ = _load(golden_dir, "ref_tiny_v2_pad")
    m = O.OracleModel(qdir, "c")
    rows = m.prefill(meta["prompt"])
    bad_first = [int(v) for v in rows[16][:256]]
    assert bad_first != rec["logits_last_rows"][1]
    assert [int(v) for v in rows[19][:256]] == rec["logits_last_rows"][1]


# ---- the oracle's FP64-BLAS backend (the reference's fast_matmul path) --------------------------
@pytest.mark.parametrize("m,n,k", [(1, 17, 16), (4, 33, 4096), (16, 257, 512), (3, 1025, 32)])
def test_exact_blas_matmul_against_integer(m, n, k):
    """test_exact_blas.py:5-11: exact against int64 matmul at the extreme operands."""
    rng = np.random.default_rng(m + n + k)
    a = rng.integers(-32768, 32768, (m, k), dtype=np.int64)
    w = rng.integers(-128, 128, (n, k), dtype=np.int8)
    a[0, :] = -32768
    w[0, :] = -128
    assert np.array_equal(O.exact_blas_matmul(a, w, 17), a @ w.astype(np.int64).T)


def test_exact_blas_matmul_errors():
    """test_exact_blas.py:13-19: the 2^53 bound and integer-only inputs."""
    with pytest.raises(ValueError, match="bound"):
        O.exact_blas_matmul(np.array([[2**53]], dtype=np.int64), np.array([[127]], dtype=np.int8))
    with pytest.raises(ValueError, match="integer"):
        O.exact_blas_matmul(np.ones((1, 1)), np.ones((1, 1), dtype=np.int8))


def test_blas_backend_equals_the_reference_fixture(golden_dir):
    """The fast_matmul oracle reproduces the reference golden.py's own record and KV."""
    qdir, meta, rec, kv, _ = _load(golden_dir, "ref_tiny_v2")
    o = O.OracleModel(qdir, "blas")
    assert o.generate(meta["prompt"], meta["n_tokens"]) == rec
    for layer, (k, v) in o.kv.items():
        assert np.array_equal(k, kv[f"k{layer}"]) and np.array_equal(v, kv[f"v{layer}"])
