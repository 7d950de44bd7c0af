"""Fused decoder-block launches (llaccel_amd.fusion -> llhip_attn_in / llhip_mlp_in /
llhip_norm_linear) against the per-op path and the CPU oracle, bit-exact, on every
configuration shape: tiny Llama (fused and unfused graphs), SmolLM2-135M, Qwen2.5-0.5B
(QKV bias) and Qwen3-0.6B (head_dim 128, Q/K RMSNorm)."""
from __future__ import annotations

import numpy as np
import pytest

from llaccel_amd import golden as G
from llaccel_amd import synth
from oracle import golden_np as O

pytestmark = pytest.mark.gpu

_CACHE = {}


def _qgraph(tmp_path_factory, cfg, fusion=True, seed=1):
    key = (cfg, fusion, seed)
    if key not in _CACHE:
        d = tmp_path_factory.mktemp(f"{cfg}_{int(fusion)}")
        _CACHE[key] = synth.build_qgraph(d, cfg, seed=seed, fusion=fusion)
    return _CACHE[key]


def _kinds(g):
    return [getattr(s, "kind", "?") for s in g._plan]


@pytest.mark.parametrize("name", ["ref_tiny_v2", "ref_tiny_v1"])
def test_tiny_plan_is_fused_and_exact(golden_dir, name):
    qdir = golden_dir / name / "qgraph"
    g = G.GoldenModel(qdir)
    k = _kinds(g)
    assert k.count("attn_in") == 2 and k.count("mlp_in") == 2 and k.count("norm_linear") == 1
    u = G.GoldenModel(qdir, fuse=False)
    prompt = list(range(3, 23))
    a1, a2 = [], []
    assert g.generate(prompt, 6, a1) == u.generate(prompt, 6, a2)
    for s1, s2 in zip(a1, a2):
        assert set(s1["acts"]) == set(s2["acts"])
        for n in s1["acts"]:
            assert np.array_equal(s1["acts"][n], s2["acts"][n]), (s1["kind"], s1["pos"], n)


@pytest.mark.parametrize("cfg,fusion", [("smol", True), ("smol", False), ("qwen25", True), ("qwen3", True)])
def test_model_shapes_fused_vs_oracle(tmp_path_factory, cfg, fusion):
    qdir = _qgraph(tmp_path_factory, cfg, fusion)
    g = G.GoldenModel(qdir)
    k = _kinds(g)
    L = g.n_layers
    assert k.count("attn_in") == L and k.count("mlp_in") == L and k.count("norm_linear") == 1, k[:20]
    o = O.OracleModel(qdir, backend="c")
    prompt = synth.seeded_prompt(cfg, 19, 5)
    acts_g, acts_o = [], []
    rg = g.generate(prompt, 3, acts_g)      # eager launches (activations collected)
    ro = o.generate(prompt, 3, acts_o)
    assert rg == ro
    for sg, so in zip(acts_g, acts_o):
        for n in so["acts"]:
            assert np.array_equal(sg["acts"][n], so["acts"][n]), (sg["kind"], sg["pos"], n)
    for layer in (0, L - 1):
        assert np.array_equal(g.kv[layer][0], o.kv[layer][0]) and np.array_equal(g.kv[layer][1], o.kv[layer][1])
    # graph decode path (no activations requested) gives the same record
    assert g.generate(prompt, 3) == ro


def test_qwen3_preinitialised_long_context(tmp_path_factory):
    """Config 5: KV of every layer filled with seeded int8 at positions 0..4094, one decode
    launch at position 4095 (T = 4096 = 16 tiles of 256 keys)."""
    qdir = _qgraph(tmp_path_factory, "qwen3", True)
    g = G.GoldenModel(qdir)
    o = O.OracleModel(qdir, backend="c")
    rng = np.random.default_rng(4095)
    for layer in g.kv:
        shape = o.kv[layer][0].shape
        k = np.zeros(shape, np.int8)
        v = np.zeros(shape, np.int8)
        k[:, :4095] = rng.integers(-128, 128, (shape[0], 4095, shape[2]))
        v[:, :4095] = rng.integers(-128, 128, (shape[0], 4095, shape[2]))
        g.set_kv(layer, k, v)
        o.kv[layer][0][...] = k
        o.kv[layer][1][...] = v
    tok = 12345
    want = o.decode(tok, 4095)
    assert np.array_equal(g.decode(tok, 4095), want)
    kv = g.kv  # every layer's K and V region after the launch (one host snapshot)
    assert sorted(kv) == sorted(o.kv) and len(kv) == 28
    for layer in kv:
        assert np.array_equal(kv[layer][0], o.kv[layer][0]), f"K cache, layer {layer}"
        assert np.array_equal(kv[layer][1], o.kv[layer][1]), f"V cache, layer {layer}"
    # the graph decode launch at the same position rewrites the same KV row and gives the same logits
    toks, rows = g.decode_loop(tok, 4095, 1)
    assert np.array_equal(rows[0], want[:g.vocab]) and toks[0] == int(np.argmax(want[:g.vocab]))


@pytest.mark.parametrize("cfg", ["smol", "qwen25", "qwen3"])
def test_whole_prompt_prefill_large_models(tmp_path_factory, cfg):
    """Config 3-5 shapes: one M = 64 prefill launch (tiled MFMA GEMM, M-row attention; at head_dim 64
    the q/k/v GEMM with the rope/quant/kv_write epilogue) == the chunked M = 16 launches (fused
    kernels), logits and KV."""
    qdir = _qgraph(tmp_path_factory, cfg, True)
    prompt = synth.seeded_prompt(cfg, 61, 3)
    g1, g2 = G.GoldenModel(qdir), G.GoldenModel(qdir)
    g2.whole_prompt_prefill = False
    r1, r2 = g1.prefill(prompt), g2.prefill(prompt)
    assert all(np.array_equal(a, b) for a, b in zip(r1, r2))
    for layer in (0, g1.n_layers // 2, g1.n_layers - 1):
        assert np.array_equal(g1.kv[layer][0], g2.kv[layer][0]) and np.array_equal(g1.kv[layer][1], g2.kv[layer][1])
    from llaccel_amd.fusion import _GroupRopeStep

    gr = [w for st in g1._plan for w in getattr(st, "wide", None) or [] if isinstance(w, _GroupRopeStep)]
    if cfg == "qwen25":  # head_dim 64, K % 128 == 0: q, k, v with their rope, quant and kv_write in one launch
        assert gr and all(w.fused and w.launched > 0 for w in gr)
    if cfg == "smol":  # K = 576: the fused launch refuses and the two launches run
        assert gr and not any(w.fused for w in gr)


def test_prefill_graph_replays_equal_eager_launches(tmp_path_factory):
    """The second whole-prompt prefill of a shape is captured as a HIP graph and later ones replay
    it: four prefills (eager, capture + replay, replay, replay of another prompt of the same
    length), with eager decode launches between them, each equal to the eager model's logits and
    KV; a prompt of another length runs eagerly again."""
    qdir = _qgraph(tmp_path_factory, "qwen25", True)
    g, e = G.GoldenModel(qdir), G.GoldenModel(qdir)
    e.use_graph = False
    prompts = [synth.seeded_prompt("qwen25", 40, 1)] * 3 + [synth.seeded_prompt("qwen25", 40, 2),
                                                           synth.seeded_prompt("qwen25", 37, 3)]
    for i, p in enumerate(prompts):
        g.reset()
        e.reset()
        r1, r2 = g.prefill(p), e.prefill(p)
        assert all(np.array_equal(a, b) for a, b in zip(r1, r2)), i
        for layer in (0, g.n_layers - 1):
            assert np.array_equal(g.kv[layer][0], e.kv[layer][0]) and np.array_equal(g.kv[layer][1], e.kv[layer][1])
        assert np.array_equal(g.decode(5, len(p)), e.decode(5, len(p)))
    assert len(g._pf_graphs) == 1


def test_fused_and_unfused_graph_decode_agree(tmp_path_factory):
    qdir = _qgraph(tmp_path_factory, "smol", True)
    prompt = synth.seeded_prompt("smol", 33, 9)
    g, u = G.GoldenModel(qdir), G.GoldenModel(qdir, fuse=False)
    assert g.generate(prompt, 24) == u.generate(prompt, 24)


@pytest.mark.parametrize("cfg", ["smol", "qwen25", "qwen3"])
def test_prefill_batch_one_launch_equals_separate_prefills(tmp_path_factory, cfg):
    """prefill_batch of prompts of one length runs ONE launch of B x padded rows (sequence-major
    positions, slot per sequence); its logits rows and every slot's KV equal separate prefill()
    calls (each the whole-prompt launch into slot 0 of its own model)."""
    qdir = _qgraph(tmp_path_factory, cfg, True)
    B, L = 3, 61
    prompts = [synth.seeded_prompt(cfg, L, 10 + b) for b in range(B)]
    g = G.GoldenModel(qdir)
    calls = []
    one = g._prefill_seqs
    g._prefill_seqs = lambda *a: calls.append(1) or one(*a)
    rows = g.prefill_batch(prompts)
    assert calls == [1] and len(rows) == B
    for b, p in enumerate(prompts):
        s = G.GoldenModel(qdir)
        want = s.prefill(p)
        assert len(rows[b]) == L == len(want)
        assert np.array_equal(rows[b].numpy(), want.numpy()), b
        got_kv, want_kv = g.kv_of(b), s.kv
        for layer in want_kv:
            assert np.array_equal(got_kv[layer][0], want_kv[layer][0]), (b, layer)
            assert np.array_equal(got_kv[layer][1], want_kv[layer][1]), (b, layer)


def test_prefill_batch_other_lengths_run_separately(tmp_path_factory):
    """Prompts of different lengths (or one chunk long) take one prefill() per prompt."""
    qdir = _qgraph(tmp_path_factory, "qwen25", True)
    g = G.GoldenModel(qdir)
    calls = []
    one = g._prefill_seqs
    g._prefill_seqs = lambda *a: calls.append(1) or one(*a)
    prompts = [synth.seeded_prompt("qwen25", 40, 1), synth.seeded_prompt("qwen25", 33, 2)]
    rows = g.prefill_batch(prompts)
    assert calls == [] and [len(r) for r in rows] == [40, 33]
    s = G.GoldenModel(qdir)
    assert np.array_equal(np.asarray(rows[1][32]), np.asarray(s.prefill(prompts[1])[32]))
