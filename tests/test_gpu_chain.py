"""The decode chain (llaccel_amd.chain: three launches per layer, the output and down projections as
int32 partial sums finished by the next launch) against the fused per-block plan and the C oracle,
bit-exact: records, every activation of the decode launches, and the KV caches."""
from __future__ import annotations

import numpy as np
import pytest

from llaccel_amd import golden as G
from llaccel_amd import synth
from oracle import golden_np as O

pytestmark = pytest.mark.gpu

_CACHE = {}


def _qgraph(tmp_path_factory, cfg, seed=2):
    if (cfg, seed) not in _CACHE:
        _CACHE[(cfg, seed)] = synth.build_qgraph(tmp_path_factory.mktemp(f"chain_{cfg}"), cfg, seed=seed)
    return _CACHE[(cfg, seed)]


def _decode_acts(g, prompt, n):
    acts: list = []
    rec = g.generate(prompt, n, acts)
    return rec, [a for a in acts if a["kind"] == "decode"]


@pytest.mark.parametrize("cfg", ["tiny", "smol", "qwen25", "qwen3"])
def test_chain_equals_fused_plan_and_oracle(tmp_path_factory, golden_dir, cfg):
    qdir = golden_dir / "ref_tiny_v2" / "qgraph" if cfg == "tiny" else _qgraph(tmp_path_factory, cfg)
    g = G.GoldenModel(qdir)
    assert g._chain is not None and g.use_chain
    assert len(g._chain.layers) == g.n_layers
    f = G.GoldenModel(qdir)
    f.use_chain = False
    prompt = list(range(5, 26)) if cfg == "tiny" else synth.seeded_prompt(cfg, 21, 7)
    rc, ac = _decode_acts(g, prompt, 5)
    rf, af = _decode_acts(f, prompt, 5)
    assert rc == rf
    for sc, sf in zip(ac, af):
        assert set(sc["acts"]) == set(sf["acts"])
        for name in sf["acts"]:
            assert np.array_equal(sc["acts"][name], sf["acts"][name]), (sc["pos"], name)
    o = O.OracleModel(qdir, backend="c")
    assert g.generate(prompt, 9) == o.generate(prompt, 9)  # the captured chain decode loop
    for layer in g.kv:
        assert np.array_equal(g.kv[layer][0], o.kv[layer][0]) and np.array_equal(g.kv[layer][1], o.kv[layer][1])


def test_chain_decode_loop_graph_equals_eager(tmp_path_factory):
    """Graph replays of the chain (the greedy step gathers the next input row) equal eager chain
    launches and the fused plan's loop, over two decode_loop calls from different tokens."""
    qdir = _qgraph(tmp_path_factory, "qwen25")
    prompt = synth.seeded_prompt("qwen25", 40, 11)
    runs = []
    for use_graph, use_chain in ((True, True), (False, True), (True, False)):
        g = G.GoldenModel(qdir)
        g.use_graph, g.use_chain = use_graph, use_chain
        rows = g.prefill(prompt)
        first = g.argmax(rows[-1], g.vocab)
        t1, r1 = g.decode_loop(first, 40, 12)
        t2, r2 = g.decode_loop(7, 52, 6)
        runs.append((t1, r1, t2, r2, g.kv[0], g.kv[g.n_layers - 1]))
    base = runs[0]
    for other in runs[1:]:
        for a, b in zip(base[:4], other[:4]):
            assert np.array_equal(a, b)
        for kv_a, kv_b in zip(base[4:], other[4:]):
            assert np.array_equal(kv_a[0], kv_b[0]) and np.array_equal(kv_a[1], kv_b[1])


@pytest.mark.parametrize("ffn", [4112, 6000, 7008])
def test_chain_ffn_tail_groups(tmp_path, ffn):
    """FFN widths whose 16-column tiles outnumber the CUs (on a 256-CU device): the MLP launch runs one
    workgroup per CU, each with one tile and at most one group of columns of the tiles past the CU
    count -- 4112: one such tile in groups of 4; 6000: 119 tiles in groups of 8; 7008: 182 tiles in
    groups of 16.  Chain == fused plan == oracle on a 2-layer Qwen2.5-shaped model."""
    import dataclasses

    cfg = dataclasses.replace(synth.CONFIGS["qwen25"], n_layers=2, vocab=4096, ffn=ffn, max_seq=64,
                              name=f"q25f{ffn}")
    qdir = synth.build_qgraph(tmp_path / cfg.name, cfg, seed=4)
    g = G.GoldenModel(qdir)
    assert g._chain is not None and g.use_chain
    f = G.GoldenModel(qdir)
    f.use_chain = False
    prompt = synth.seeded_prompt(cfg, 13, 5)
    rc, ac = _decode_acts(g, prompt, 4)
    rf, af = _decode_acts(f, prompt, 4)
    assert rc == rf
    for sc, sf in zip(ac, af):
        for name in sf["acts"]:
            assert np.array_equal(sc["acts"][name], sf["acts"][name]), (sc["pos"], name)
    assert g.generate(prompt, 6) == O.OracleModel(qdir, backend="c").generate(prompt, 6)
