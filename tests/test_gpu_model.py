"""GPU GoldenModel (llaccel_amd.golden) against the outputs of the reference's own
golden.py (tests/golden/ref_tiny_*), the CPU oracle, and the invariants of the reference's
tests/python/test_golden_e2e.py."""
from __future__ import annotations

import json

import numpy as np
import pytest

from llaccel_amd import golden as G
from llaccel_amd import synth
from oracle import golden_np as O

pytestmark = pytest.mark.gpu
CASES = ["ref_tiny_v2", "ref_tiny_v1", "ref_tiny_v2_pad", "ref_tiny_v2_m4",
         "ref_qwen2_bias", "ref_qwen3_qknorm_d128", "ref_d256"]  # Qwen2 bias, Qwen3 Q/K norm at D = 128, D = 256


def _load(golden_dir, name):
    d = golden_dir / name
    return (d / "qgraph", json.loads((d / "meta.json").read_text()), json.loads((d / "record.json").read_text()),
            np.load(d / "kv_final.npz"), np.load(d / "acts.npz"))


@pytest.mark.parametrize("name", CASES)
def test_reproduces_reference_golden_run(golden_dir, name):
    qdir, meta, rec, kv, acts = _load(golden_dir, name)
    g = G.GoldenModel(qdir)
    got_acts: list = []
    got = g.generate(meta["prompt"], meta["n_tokens"], got_acts)
    assert got == rec
    for layer, (k, v) in g.kv.items():
        assert np.array_equal(k, kv[f"k{layer}"]) and np.array_equal(v, kv[f"v{layer}"]), layer
    assert [{k: a[k] for k in ("kind", "pos", "rows", "valid_rows")} for a in got_acts] == meta["steps"]
    for i in meta["acts_steps"]:
        names = {key.split("/", 1)[1] for key in acts.files if key.startswith(f"step{i}/")}
        assert names == set(got_acts[i]["acts"])
        for n in names:
            assert np.array_equal(got_acts[i]["acts"][n], acts[f"step{i}/{n}"]), (i, n)


def test_run_chunk_acts_and_determinism(golden_dir):
    qdir = golden_dir / "ref_tiny_v2" / "qgraph"
    g = G.GoldenModel(qdir)
    o = O.OracleModel(qdir)
    rows = g.embed_rows([1, 2, 3], 16)
    assert np.array_equal(rows, o.embed_rows([1, 2, 3], 16))
    a1, a2 = {}, {}
    l1 = g.run_chunk(rows, 0, a1)
    l2 = o.run_chunk(rows, 0, a2)
    assert np.array_equal(l1, l2) and set(a1) == set(a2)
    for n in a1:
        assert np.array_equal(a1[n], a2[n]), n
    g.reset()
    assert np.array_equal(g.run_chunk(rows, 0), l1)


def test_chunked_prefill_equals_sequential_decode(golden_dir):
    qdir = golden_dir / "ref_tiny_v2" / "qgraph"
    toks = np.random.default_rng(3).integers(0, 256, 21).tolist()
    a = G.GoldenModel(qdir).prefill(toks)
    g2 = G.GoldenModel(qdir)
    b = [g2.decode(t, i) for i, t in enumerate(toks)]
    assert all(np.array_equal(x, y) for x, y in zip(a, b))


def test_errors(golden_dir, tmp_path):
    qdir = golden_dir / "ref_tiny_v2" / "qgraph"
    with pytest.raises(ValueError, match="max_seq"):
        G.GoldenModel(qdir).generate(list(range(10)), 64)
    r = G.GoldenModel(qdir).generate(list(range(10)), 54)
    assert len(r["generated"]) == 54 and r["steps"][-1]["pos"] == 62
    with pytest.raises(ValueError, match="max_seq"):
        G.GoldenModel(qdir).run_chunk(np.zeros((16, 64)), 60)
    for pm in (0, 3, 17):
        d = tmp_path / f"q{pm}"
        d.mkdir()
        g = json.loads((qdir / "qgraph.json").read_text())
        g["model"]["prefill_m"] = pm
        (d / "qgraph.json").write_text(json.dumps(g))
        (d / "qweights.bin").write_bytes((qdir / "qweights.bin").read_bytes())
        with pytest.raises(ValueError, match="max_seq must be divisible by prefill_m"):
            G.GoldenModel(d)


def test_kv_snapshot_and_preinitialised_state(golden_dir):
    """Preinitialised-KV boundary launch (regress_pretrained_boundaries.py:55-69 pattern)."""
    qdir = golden_dir / "ref_tiny_v2" / "qgraph"
    rng = np.random.default_rng(9)
    g, o = G.GoldenModel(qdir), O.OracleModel(qdir)
    for layer in g.kv:
        k = rng.integers(-128, 128, o.kv[layer][0].shape).astype(np.int8)
        v = rng.integers(-128, 128, o.kv[layer][1].shape).astype(np.int8)
        g.set_kv(layer, k, v)
        o.kv[layer][0][...] = k
        o.kv[layer][1][...] = v
    assert np.array_equal(g.decode(17, 50), o.decode(17, 50))
    for layer in g.kv:
        assert np.array_equal(g.kv[layer][0], o.kv[layer][0]) and np.array_equal(g.kv[layer][1], o.kv[layer][1])


@pytest.mark.parametrize("fusion", [True, False])
def test_smol_shape_prefill_decode(tmp_path, fusion):
    """SmolLM2-135M shape (config 3, 30 layers, 9/3 heads): 20-token prompt + 4 decode
    launches, GPU == C oracle on the record and the whole KV state."""
    qdir = synth.build_qgraph(tmp_path / "smol", "smol", seed=3, fusion=fusion)
    prompt = synth.seeded_prompt("smol", 20, 1)
    g = G.GoldenModel(qdir)
    o = O.OracleModel(qdir, backend="c")
    # resadd o_proj and down (the fused graph's; the unfused graph adds separately) each pair with
    # the rmsnorm + quant that opens the next fused run, which the prompt launch takes on its wide
    # path (one llhip_linear_norm call per pair)
    from llaccel_amd import fusion as F

    assert sum(isinstance(s, F._DeferredLinear) for s in g._plan) == (2 * 30 if fusion else 0)
    assert g.generate(prompt, 4) == o.generate(prompt, 4)
    for layer in (0, 17, 29):
        assert np.array_equal(g.kv[layer][0], o.kv[layer][0]) and np.array_equal(g.kv[layer][1], o.kv[layer][1])


def test_graph_decode_equals_eager_and_reference(golden_dir):
    """The captured-graph decode loop (default generate path) reproduces the reference record;
    replays are interleaved with eager launches and checked every time."""
    qdir, meta, rec, kv, _ = _load(golden_dir, "ref_tiny_v2")
    g = G.GoldenModel(qdir)
    assert g.generate(meta["prompt"], meta["n_tokens"]) == rec
    for layer, (k, v) in g.kv.items():
        assert np.array_equal(k, kv[f"k{layer}"]) and np.array_equal(v, kv[f"v{layer}"]), layer
    g.use_graph = False
    assert g.generate(meta["prompt"], meta["n_tokens"]) == rec
    g.use_graph = True
    o = O.OracleModel(qdir, backend="c")
    for seed in range(3):
        prompt = synth.seeded_prompt("tiny", 5 + 7 * seed, 100 + seed)
        assert g.generate(prompt, 20) == o.generate(prompt, 20), seed
        rows = g.embed_rows([seed], 16)
        g.reset()
        o.reset()
        assert np.array_equal(g.run_chunk(rows, 0), o.run_chunk(rows, 0))


def test_decode_loop_matches_sequential_decode(golden_dir):
    qdir = golden_dir / "ref_tiny_v2_pad" / "qgraph"
    prompt = list(range(20))
    g1, g2 = G.GoldenModel(qdir), G.GoldenModel(qdir)
    r1, r2 = g1.prefill(prompt), g2.prefill(prompt)
    nxt = G.GoldenModel.argmax(r1[-1], g1.vocab)
    toks, rows = g1.decode_loop(nxt, 20, 12)
    t = nxt
    for i in range(12):
        row = g2.decode(t, 20 + i)
        assert np.array_equal(rows[i], row[:g2.vocab]), i
        t = G.GoldenModel.argmax(row, g2.vocab)
        assert t == toks[i]


@pytest.mark.parametrize("name,plen", [("ref_tiny_v2", 16), ("ref_tiny_v2", 41), ("ref_tiny_v2_m4", 9),
                                       ("ref_tiny_v1", 33)])
def test_whole_prompt_prefill_equals_chunked(golden_dir, name, plen):
    """One launch of the padded prompt == the chunked launches: logits rows, records, and the
    whole KV state including the pad rows' entries."""
    qdir = golden_dir / name / "qgraph"
    prompt = synth.seeded_prompt("tiny", plen, 77)
    g1, g2 = G.GoldenModel(qdir), G.GoldenModel(qdir)
    g2.whole_prompt_prefill = False
    r1, r2 = g1.prefill(prompt), g2.prefill(prompt)
    assert len(r1) == len(r2) == plen and all(np.array_equal(a, b) for a, b in zip(r1, r2))
    for layer in g1.kv:
        assert np.array_equal(g1.kv[layer][0], g2.kv[layer][0]) and np.array_equal(g1.kv[layer][1], g2.kv[layer][1])
    g1.reset(), g2.reset()
    assert g1.generate(prompt, 5) == g2.generate(prompt, 5) == O.OracleModel(qdir, "c").generate(prompt, 5)


@pytest.mark.parametrize("name,B,L,n", [("ref_tiny_v2", 4, 10, 30), ("ref_tiny_v2_pad", 16, 17, 12),
                                        ("ref_tiny_v1", 3, 5, 58)])
def test_generate_batch_equals_single_sequences(golden_dir, name, B, L, n):
    """Batch decode (config 4's batch-16 form): B sequences with their own prompts, KV slots and
    positions run as the B rows of one launch; every record equals the sequence's own generate()
    run alone and the oracle's.  n reaches max_seq in the last case (the record stops there)."""
    qdir = golden_dir / name / "qgraph"
    prompts = [synth.seeded_prompt("tiny", L, 40 + b) for b in range(B)]
    g = G.GoldenModel(qdir)
    recs = g.generate_batch(prompts, n)
    single = G.GoldenModel(qdir)
    o = O.OracleModel(qdir, backend="c")
    for b in range(B):
        want = single.generate(prompts[b], n)
        assert recs[b] == want, b
        if b in (0, B - 1):
            assert want == o.generate(prompts[b], n), b
    # the KV slot of the last sequence equals its single-sequence caches
    g._slot = B - 1
    for layer, (k, v) in g.kv.items():
        assert np.array_equal(k, single.kv[layer][0]) and np.array_equal(v, single.kv[layer][1]), layer
    g._slot = 0
    # eager batch launches (no graph) give the same records
    g.use_graph = False
    assert g.generate_batch(prompts[:2], 6) == [single.generate(p, 6) for p in prompts[:2]]


def test_generate_batch_qwen_shape(tmp_path):
    """Qwen2.5 GQA shape with QKV bias (reduced to 2 layers, vocab 4096): batch of 4 sequences of
    24 tokens + 6 decode launches, each equal to its single-sequence run."""
    import dataclasses

    cfg = dataclasses.replace(synth.CONFIGS["qwen25"], n_layers=2, vocab=4096, max_seq=64, name="q25s")
    qdir = synth.build_qgraph(tmp_path / "q25s", cfg, seed=5)
    prompts = [synth.seeded_prompt(cfg, 24, 7 + b) for b in range(4)]
    g, single = G.GoldenModel(qdir), G.GoldenModel(qdir)
    recs = g.generate_batch(prompts, 6)
    for b in range(4):
        assert recs[b] == single.generate(prompts[b], 6), b


def test_generate_batch_errors(golden_dir):
    g = G.GoldenModel(golden_dir / "ref_tiny_v2" / "qgraph")
    with pytest.raises(ValueError, match="one length"):
        g.generate_batch([[1, 2], [3]], 2)
    with pytest.raises(ValueError, match="max_seq"):
        g.generate_batch([[1, 2]], 63)


def test_golden_cli_and_dump_acts(golden_dir, tmp_path):
    """The golden CLI and dump_acts (golden.py:443-477), as the reference's
    tests/python/test_golden_e2e.py:165-189 checks them: the record of a 5-token run from a char
    prompt, one int32 .npy per activation per launch named step{i:03d}_{kind}_pos{P}_{name}.npy with
    the launch's shapes, the recorded logits rows equal to the dumped logits activation's rows, and
    the record verifying against itself (MATCH) but not against a perturbed copy ("step 2")."""
    import json as _json

    from llaccel_amd import verify

    qdir = golden_dir / "ref_tiny_v1" / "qgraph"
    graph = _json.loads((qdir / "qgraph.json").read_text())
    m = graph["model"]
    itos = [chr(ord("a") + i) for i in range(26)] + [chr(0x4E00 + i) for i in range(m["vocab"] - 26)]
    (tmp_path / "tok.json").write_text(_json.dumps({"itos": itos}))
    out, acts = tmp_path / "golden.json", tmp_path / "acts"
    G.main(["--qgraph", str(qdir), "--prompt", "abcde", "--tokenizer", str(tmp_path / "tok.json"), "--tokens", "5",
            "-o", str(out), "--dump-acts", str(acts)])
    rec = _json.loads(out.read_text())
    assert rec["prompt_tokens"] == [0, 1, 2, 3, 4] and len(rec["generated"]) == 5 and len(rec["argmax_per_step"]) == 6
    assert rec["argmax_per_step"][:5] == rec["generated"]  # the last decode launch's argmax is not generated
    per_launch = 1 + sum(1 for op in graph["ops"] if "out" in op)  # the input rows and every op output
    files = sorted(acts.glob("*.npy"))
    assert len(files) == 6 * per_launch
    assert all(np.load(f).dtype == np.int32 for f in files)
    H, Hkv, D = m["n_heads"], m["n_kv_heads"], m["head_dim"]
    assert np.load(acts / "step000_prefill_pos0_logits.npy").shape == (16, m["vocab_padded"])
    assert np.load(acts / "step001_decode_pos5_l0.a.npy").shape == (1, H * D)
    assert np.load(acts / "step005_decode_pos9_l0.kr.q.npy").shape == (1, Hkv * D)
    # the golden.json logits row is the recorded row of the dumped logits activation
    assert np.load(acts / "step000_prefill_pos0_logits.npy")[4, :m["vocab"]].tolist() == rec["logits_last_rows"][0]
    assert np.load(acts / "step003_decode_pos7_logits.npy")[0, :m["vocab"]].tolist() == rec["logits_last_rows"][3]
    ok, msg = verify.compare_sim(out, out)
    assert ok and msg.startswith("MATCH")
    bad = dict(rec, generated=list(rec["generated"]))
    bad["generated"][2] = (bad["generated"][2] + 1) % m["vocab"]
    (tmp_path / "sim.json").write_text(_json.dumps(bad))
    ok, msg = verify.compare_sim(tmp_path / "sim.json", out)
    assert not ok and "step 2" in msg
