"""Device record verification (llhip_rows_first_mismatch_i16, llhip_rows_checksum_i16) against
numpy, and a decode run checked on the device against its own host record."""
from __future__ import annotations

import numpy as np
import pytest

from llaccel_amd import golden as G
from llaccel_amd import synth
from llaccel_amd import verify as V

pytestmark = pytest.mark.gpu


def _dev(a):
    import torch

    return torch.tensor(np.asarray(a, dtype=np.int16), device="cuda")


@pytest.mark.parametrize("rows,cols", [(1, 1), (3, 5), (64, 151936), (7, 1000)])
def test_first_mismatch_and_checksums(rows, cols):
    rng = np.random.default_rng(rows * 7 + cols)
    a = rng.integers(-32768, 32768, (rows, cols))
    ta, tb = _dev(a), _dev(a)
    assert V.first_mismatch(ta, tb) == -1
    assert np.array_equal(V.row_checksums(ta), V.host_row_checksums(a))
    # planted differences (host data): the first one in flat order is reported
    for flat in sorted(set(rng.integers(0, rows * cols, 3).tolist()), reverse=True):
        b = a.copy()
        b.flat[flat] = b.flat[flat] ^ 0x40
        tb = _dev(b)
        assert V.first_mismatch(ta, tb) == flat
        r = flat // cols
        cs = V.row_checksums(tb)
        assert cs[r] != V.host_row_checksums(a)[r] and np.array_equal(cs, V.host_row_checksums(b))


def test_strided_rows_and_errors():
    import torch

    rng = np.random.default_rng(3)
    a = rng.integers(-32768, 32768, (6, 40))
    wide = torch.zeros((6, 64), dtype=torch.int16, device="cuda")
    wide[:, :40] = _dev(a)
    assert V.first_mismatch(wide[:, :40], _dev(a)) == -1
    assert np.array_equal(V.row_checksums(wide[:, :40]), V.host_row_checksums(a))
    with pytest.raises(ValueError):
        V.first_mismatch(_dev(a), _dev(a[:5]))
    with pytest.raises(ValueError):
        V.row_checksums(torch.zeros((2, 3), dtype=torch.int32, device="cuda"))


def test_decode_run_checked_on_device(tmp_path):
    """A graph decode run's device ring equals the record of the same generate() run: one 8-byte
    download for the whole comparison, and the per-step checksums match the host record's."""
    import torch

    qdir = synth.build_qgraph(tmp_path / "q", "smol", seed=2, fusion=True)
    g = G.GoldenModel(qdir)
    prompt = synth.seeded_prompt("smol", 24, 2)
    rec = g.generate(prompt, 40)
    n_dec = len(rec["logits_last_rows"]) - 2  # prefill launches: ceil(24 / 16) = 2
    first = rec["argmax_per_step"][1]
    g.reset()
    g.prefill(prompt)
    g.decode_loop(first, 24, n_dec, sync=False)
    toks, rows = g.decode_ring(n_dec)
    want = np.array([r[:g.vocab] for r in rec["logits_last_rows"][2:]], dtype=np.int64)
    assert V.first_mismatch(rows, _dev(want)) == -1
    assert np.array_equal(V.row_checksums(rows), V.host_row_checksums(want))
    assert toks.cpu().numpy().tolist() == rec["argmax_per_step"][2:]
    # a single flipped logit is located exactly
    bad = want.copy()
    bad[17, 123] += 1
    assert V.first_mismatch(rows, _dev(bad)) == 17 * g.vocab + 123
    torch.cuda.synchronize()
