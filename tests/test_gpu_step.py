"""The one-launch decode step (llhip_dec_step: every layer of a decode row in one persistent launch,
stages handed between workgroups through device-scope flags) against the three-launch decode chain
and the C oracle, bit-exact: decode records (tokens and logits rows) and every layer's KV cache."""
from __future__ import annotations

import numpy as np
import pytest

from llaccel_amd import golden as G
from llaccel_amd import synth
from oracle import golden_np as O

pytestmark = pytest.mark.gpu

_CACHE = {}


def _qgraph(tmp_path_factory, cfg, seed=3):
    if (cfg, seed) not in _CACHE:
        _CACHE[(cfg, seed)] = synth.build_qgraph(tmp_path_factory.mktemp(f"step_{cfg}"), cfg, seed=seed)
    return _CACHE[(cfg, seed)]


def _kv_equal(a, b):
    for layer in a.kv:
        ka, va = a.kv[layer]
        kb, vb = b.kv[layer]
        assert np.array_equal(ka, kb), f"K layer {layer}"
        assert np.array_equal(va, vb), f"V layer {layer}"


@pytest.mark.parametrize("cfg", ["smol", "qwen25"])
def test_step_equals_chain_and_oracle(tmp_path_factory, cfg):
    qdir = _qgraph(tmp_path_factory, cfg)
    prompt = synth.seeded_prompt(cfg, 37, 5)
    g = G.GoldenModel(qdir)
    rec = g.generate(prompt, 12)
    assert g._chain._step is not None, g._chain.step_unsupported  # the decode loop ran the one-launch step
    c = G.GoldenModel(qdir)
    c._chain.use_step = False
    c._chain.use_logits = False  # and the head as finish + lm_head + greedy launches
    assert c.generate(prompt, 12) == rec
    assert c._chain._step is None
    _kv_equal(g, c)
    o = O.OracleModel(qdir, backend="c")
    assert o.generate(prompt, 12) == rec
    for layer in g.kv:
        assert np.array_equal(g.kv[layer][0], o.kv[layer][0]) and np.array_equal(g.kv[layer][1], o.kv[layer][1])


def test_step_long_context_and_two_loops(tmp_path_factory):
    """Contexts past the keys and values the step keeps in LDS (768 at head_dim 64): seeded caches
    for every layer, then two decode loops (positions 900.. and 1010..1023, the cache's last row),
    step == chain on tokens, logits rows and caches."""
    qdir = _qgraph(tmp_path_factory, "qwen25")
    rng = np.random.default_rng(17)
    runs = []
    for use_step in (True, False):
        g = G.GoldenModel(qdir)
        g._chain.use_step = use_step
        rng = np.random.default_rng(17)
        for layer in range(g.n_layers):
            k = rng.integers(-128, 128, size=(2, g.max_seq, 64), dtype=np.int8)
            v = rng.integers(-128, 128, size=(2, g.max_seq, 64), dtype=np.int8)
            g.set_kv(layer, k, v)
        t1, r1 = g.decode_loop(123, 900, 9)
        t2, r2 = g.decode_loop(4567, 1010, 14)
        assert (g._chain._step is not None) == use_step
        runs.append((g, t1, r1, t2, r2))
    (gs, *a), (gc, *b) = runs
    for x, y in zip(a, b):
        assert np.array_equal(x, y)
    _kv_equal(gs, gc)


def test_step_graph_equals_eager(tmp_path_factory):
    """The captured decode graph (one step launch + head + greedy per replay) equals eager launches."""
    qdir = _qgraph(tmp_path_factory, "smol")
    prompt = synth.seeded_prompt("smol", 30, 9)
    runs = []
    for use_graph in (True, False):
        g = G.GoldenModel(qdir)
        g.use_graph = use_graph
        rows = g.prefill(prompt)
        first = g.argmax(rows[-1], g.vocab)
        t1, r1 = g.decode_loop(first, 30, 10)
        t2, r2 = g.decode_loop(11, 40, 5)
        assert g._chain._step is not None
        runs.append((t1, r1, t2, r2, g))
    for x, y in zip(runs[0][:4], runs[1][:4]):
        assert np.array_equal(x, y)
    _kv_equal(runs[0][4], runs[1][4])


def test_step_not_used_for_qk_norm(tmp_path_factory):
    """Qwen3 (Q/K norm) keeps the three-launch chain; its decode loop still equals the oracle."""
    qdir = _qgraph(tmp_path_factory, "qwen3")
    g = G.GoldenModel(qdir)
    prompt = synth.seeded_prompt("qwen3", 9, 2)
    rec = g.generate(prompt, 4)
    assert g._chain._step is None and g._chain.step_unsupported
    assert O.OracleModel(qdir, backend="c").generate(prompt, 4) == rec
