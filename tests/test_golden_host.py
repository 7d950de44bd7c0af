"""Host-side token-id handling of llaccel_amd.golden (no GPU): GoldenModel._token_rows follows the
numpy indexing that golden.py:369-373 applies to the embedding table -- negative ids count from the
end, and an out-of-range id raises numpy's own IndexError (message compared with numpy's)."""
from __future__ import annotations

import numpy as np
import pytest

from llaccel_amd.golden import GoldenModel


class _Table:
    def __init__(self, n):
        self.embed = np.arange(n * 2).reshape(n, 2)


def _numpy_rows(table, tokens):
    """What the reference's `embed[tokens]` selects, as row indices."""
    idx = np.arange(table.embed.shape[0])
    return idx[np.asarray(tokens, dtype=np.int64)] if len(tokens) else np.zeros(0, np.int64)


@pytest.mark.parametrize("tokens", [[0, 5, -1, 999], list(range(1000)) * 3, [], [-1000, 999],
                                    np.array([3, -2, 7], np.int32), np.array([4, 999], np.uint16)])
def test_rows_equal_numpy_indexing(tokens):
    t = _Table(1000)
    got = GoldenModel._token_rows(t, tokens)
    assert got.dtype == np.int32 and np.array_equal(got, _numpy_rows(t, list(np.asarray(tokens).reshape(-1))))


@pytest.mark.parametrize("tokens", [[1000], [-1001], [5, 7, 1200, -5000]])
def test_out_of_range_raises_numpys_error(tokens):
    t = _Table(1000)
    with pytest.raises(IndexError) as ours:
        GoldenModel._token_rows(t, tokens)
    with pytest.raises(IndexError) as theirs:
        t.embed[np.asarray(tokens)]
    assert str(ours.value) == str(theirs.value)


@pytest.mark.parametrize("tokens", [[5, 2**70], np.array([5, 2**63 + 5], np.uint64)])
def test_ids_beyond_int64_raise_index_error(tokens):
    with pytest.raises(IndexError, match="out of bounds for axis 0 with size 1000"):
        GoldenModel._token_rows(_Table(1000), tokens)
