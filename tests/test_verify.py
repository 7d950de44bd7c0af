"""Record verification on the host (llaccel_amd.verify): the reference's compare_sim semantics
(python/llaccel/verify.py:80-104) on constructed records, and the host row checksum pinned
against plain Python integer arithmetic."""
from __future__ import annotations

import json

import numpy as np
import pytest

from llaccel_amd import verify as V


def _rec(n=3, vocab=5, seed=0):
    rng = np.random.default_rng(seed)
    rows = [[int(x) for x in rng.integers(-32768, 32768, vocab)] for _ in range(n)]
    argm = [int(np.argmax(r)) for r in rows]
    return {"prompt_tokens": [1, 2], "generated": argm[-2:], "argmax_per_step": argm, "logits_last_rows": rows}


def test_match_and_mismatch_messages():
    a, b = _rec(), _rec()
    ok, msg = V.compare_records(a, b)
    assert ok and msg == "MATCH: 2 tokens, 3 steps identical"
    c = _rec()
    c["logits_last_rows"][1][3] += 1
    ok, msg = V.compare_records(c, a)
    assert not ok and msg.startswith("MISMATCH in logits_last_rows at step 1: sim=")
    d = _rec()
    d["generated"] = d["generated"] + [7]
    assert V.compare_records(d, a) == (False, "MISMATCH: generated length sim=3 golden=2")
    e = _rec()
    e["argmax_per_step"][0] += 1
    ok, msg = V.compare_records(a, e)
    assert not ok and msg.startswith("MISMATCH in argmax_per_step at step 0:")


def test_malformed_records():
    a = _rec()
    for mutate, want in [
        (lambda r: r.pop("generated"), "MISMATCH: sim.json lacks an array 'generated'"),
        (lambda r: r["logits_last_rows"].pop(), "MISMATCH: sim.json logits/launch counts differ"),
        (lambda r: r["generated"].__setitem__(0, 1.0), "MISMATCH: sim.json token IDs must be integers"),
        (lambda r: r["generated"].__setitem__(0, True), "MISMATCH: sim.json token IDs must be integers"),
        (lambda r: r["logits_last_rows"].__setitem__(0, []), "MISMATCH: sim.json logits must be nonempty integer rows"),
        (lambda r: r["logits_last_rows"][0].__setitem__(0, 0.5),
         "MISMATCH: sim.json logits must be nonempty integer rows"),
    ]:
        s = _rec()
        mutate(s)
        assert V.compare_records(s, a) == (False, want)
    g = _rec()
    g.pop("argmax_per_step")
    assert V.compare_records(a, g) == (False, "MISMATCH: golden.json lacks an array 'argmax_per_step'")


def test_compare_sim_files_and_cli(tmp_path, capsys):
    a, b = _rec(seed=1), _rec(seed=1)
    pa, pb = tmp_path / "sim.json", tmp_path / "golden.json"
    pa.write_text(json.dumps(a))
    pb.write_text(json.dumps(b))
    assert V.compare_sim(pa, pb)[0]
    assert V.main(["--sim-json", str(pa), "--golden", str(pb)]) == 0
    assert capsys.readouterr().out.strip() == "MATCH: 2 tokens, 3 steps identical"
    b["logits_last_rows"][2][0] ^= 1
    pb.write_text(json.dumps(b))
    assert V.main(["--sim-json", str(pa), "--golden", str(pb)]) == 1


@pytest.mark.parametrize("n,cols", [(1, 1), (3, 7), (5, 151936 // 16)])
def test_host_checksum_is_the_stated_sum(n, cols):
    rng = np.random.default_rng(n * cols)
    rows = rng.integers(-32768, 32768, (n, cols))
    got = V.host_row_checksums(rows)
    for r in range(n):
        want = sum((c + 1) * (int(rows[r, c]) & 0xFFFF) for c in range(cols)) % (1 << 64)
        assert int(got[r]) == want
    # a swap of two unequal values changes the checksum
    if cols > 1 and rows[0, 0] != rows[0, 1]:
        sw = rows.copy()
        sw[0, [0, 1]] = sw[0, [1, 0]]
        assert V.host_row_checksums(sw)[0] != got[0]
