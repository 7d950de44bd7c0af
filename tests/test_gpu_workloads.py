"""Configs 3 and 4 at the workloads BASELINE.json states, on the GPU against the C oracle, bit-exact:

* config 3 (SmolLM2-135M shape): 128-token prefill + 64-token greedy decode at batch 1;
* config 4 (Qwen2.5-0.5B shape): 512-token prefill through the default whole-prompt launch + 256-token
  greedy decode at batch 1, and the same at batch 16 (prompts with seeds s + b, one KV slot per
  sequence) with every sequence b = 0..15 checked against its own oracle run.

Each check compares the whole golden.json record (every recorded logits row and argmax, the launch
list) and the K and V caches of every layer.  The reference runs the same launches in
golden.py:399-440; the oracle restates it (oracle/golden_np.py, heavy ops in oracle/numerics.c)."""
from __future__ import annotations

import numpy as np
import pytest

from llaccel_amd import golden as G
from llaccel_amd import synth
from oracle import golden_np as O

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(600)]

SEED = 0
B16_SEQS = tuple(range(16))


def _note(msg: str) -> None:
    print(msg, flush=True)


@pytest.fixture(scope="module")
def smol_q(tmp_path_factory):
    return synth.build_qgraph(tmp_path_factory.mktemp("smol"), "smol", seed=SEED)


@pytest.fixture(scope="module")
def qwen_q(tmp_path_factory):
    return synth.build_qgraph(tmp_path_factory.mktemp("qwen25"), "qwen25", seed=SEED)


def _assert_kv_equal(got: dict, want: dict) -> None:
    assert set(got) == set(want)
    for layer in sorted(want):
        assert np.array_equal(got[layer][0], want[layer][0]), f"K cache, layer {layer}"
        assert np.array_equal(got[layer][1], want[layer][1]), f"V cache, layer {layer}"


def _assert_record_equal(got: dict, want: dict) -> None:
    assert got["steps"] == want["steps"]
    assert got["argmax_per_step"] == want["argmax_per_step"]
    assert got["generated"] == want["generated"]
    assert got["model"] == want["model"] and got["prompt_tokens"] == want["prompt_tokens"]
    assert len(got["logits_last_rows"]) == len(want["logits_last_rows"])
    for i, (a, b) in enumerate(zip(got["logits_last_rows"], want["logits_last_rows"])):
        assert a == b, f"logits row of launch {i}"


def test_config3_smol_prefill128_decode64(smol_q):
    prompt = synth.seeded_prompt("smol", 128, seed=SEED)
    _note("config 3: GPU 128 + 64")
    g = G.GoldenModel(smol_q)
    got = g.generate(prompt, 64)
    _note("config 3: oracle 128 + 64")
    o = O.OracleModel(smol_q, backend="c")
    want = o.generate(prompt, 64)
    assert len(got["steps"]) == 128 // 16 + 64
    _assert_record_equal(got, want)
    _assert_kv_equal(g.kv, {L: o.kv[L] for L in o.kv})


@pytest.fixture(scope="module")
def qwen_oracle_b1(qwen_q):
    prompt = synth.seeded_prompt("qwen25", 512, seed=SEED)
    _note("config 4: oracle 512 + 256")
    o = O.OracleModel(qwen_q, backend="c")
    rec = o.generate(prompt, 256)
    return prompt, rec, {L: o.kv[L] for L in o.kv}


def test_config4_qwen25_prefill512_decode256_b1(qwen_q, qwen_oracle_b1):
    prompt, want, kv = qwen_oracle_b1
    _note("config 4: GPU 512 + 256")
    g = G.GoldenModel(qwen_q)
    assert g.whole_prompt_prefill  # the default path: the 512 rows as one launch
    got = g.generate(prompt, 256)
    assert len(got["steps"]) == 512 // 16 + 256
    _assert_record_equal(got, want)
    _assert_kv_equal(g.kv, kv)


@pytest.fixture(scope="module")
def qwen_b16(qwen_q):
    """The batch-16 run: prompt b has seed SEED + b; prefill into slot b, then 256 decode launches of
    the 16 sequences together.  Keeps every sequence's decode record and KV snapshot."""
    prompts = [synth.seeded_prompt("qwen25", 512, seed=SEED + b) for b in range(16)]
    _note("config 4: GPU batch 16, 512 + 256")
    g = G.GoldenModel(qwen_q)
    pre = g.prefill_batch(prompts)
    first = [g.argmax(rows[-1], g.vocab) for rows in pre]
    toks, rows = g.decode_batch_loop(first, [512] * 16, 256)
    out = {}
    for b in B16_SEQS:
        prefill_rows = np.stack([np.asarray(pre[b][c * 16 + 15], np.int64)[:g.vocab] for c in range(32)])
        out[b] = (prompts[b], prefill_rows, first[b], toks[:, b].copy(), rows[:, b].copy(), g.kv_of(b))
    return out


@pytest.mark.parametrize("b", B16_SEQS)
def test_config4_qwen25_batch16_sequence(qwen_q, qwen_oracle_b1, qwen_b16, b):
    prompt, prefill_rows, first, toks, rows, kv = qwen_b16[b]
    if b == 0:  # sequence 0 has the batch-1 test's prompt: its oracle run is shared
        want, want_kv = qwen_oracle_b1[1], qwen_oracle_b1[2]
        assert qwen_oracle_b1[0] == prompt
    else:
        _note(f"config 4: oracle for batch sequence {b}")
        o = O.OracleModel(qwen_q, backend="c")
        want = o.generate(prompt, 256)
        want_kv = {L: o.kv[L] for L in o.kv}
    # the record: 32 prefill launches, then 256 decode launches at positions 512..767
    rec_rows = np.asarray(want["logits_last_rows"], np.int64)
    assert len(want["steps"]) == 32 + 256
    assert np.array_equal(prefill_rows, rec_rows[:32])
    assert first == want["argmax_per_step"][31]
    assert np.array_equal(rows.astype(np.int64), rec_rows[32:])
    assert toks.tolist() == want["argmax_per_step"][32:]
    assert [first] + toks[:255].tolist() == want["generated"]
    _assert_kv_equal(kv, want_kv)
