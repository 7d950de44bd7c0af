"""CPU oracle of the quantizer's float -> integer conversions (the qgraph producer's weights).

TEST INFRASTRUCTURE ONLY.  Nothing in the product (`llaccel_amd`) may import this module; only
`tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` use it, and only as
the checker.

Restates, in float64 numpy as the reference computes them:
  llround        refquant.py:61-86   nearest integer, halves away from zero (C llround)
  row_scales     refquant.py:137-141 max|W[n,:]| / 127, an all-zero row -> 1
  quant_i8       refquant.py:119-125 llround(clip(v / scale, -128, 127))
  quant_i16      refquant.py:128-134 llround(clip(v * 2^-e, -32768, 32767))

Pinning: the reference's own known answers (test_refquant.py:18-33 llround and quant_i8/i16 ties
and saturation, :65-70 row scales and the 63.5 -> 64, 31.75 -> 32 weights), restated in
tests/test_quantize.py, plus the defining property of llround checked against Python's
`fractions.Fraction` rounding on random doubles.
"""
from __future__ import annotations

import numpy as np


def llround(x) -> np.ndarray:
    """refquant.py:75-86 -- elementwise; every input must be finite."""
    x = np.asarray(x, dtype=np.float64)
    if not np.all(np.isfinite(x)):
        raise ValueError("llround of a non-finite value")
    t = np.trunc(x)
    frac = x - t
    return np.where(frac >= 0.5, t + 1, np.where(frac <= -0.5, t - 1, t)).astype(np.int64)


def row_scales(w) -> np.ndarray:
    """refquant.py:137-141."""
    mx = np.abs(np.asarray(w, dtype=np.float64)).max(axis=1)
    return np.where(mx > 0.0, mx / 127.0, 1.0)


def quant_i8(v, scale) -> np.ndarray:
    """refquant.py:119-125 (scale broadcasts against v)."""
    v, scale = np.asarray(v, dtype=np.float64), np.asarray(scale, dtype=np.float64)
    with np.errstate(over="ignore"):
        return llround(np.clip(v / scale, -128, 127)).astype(np.int8)


def quant_rows_i8(w) -> tuple[np.ndarray, np.ndarray]:
    """Per-output-channel int8 weights and their scales (refquant.py:365-366)."""
    s = row_scales(w)
    return quant_i8(w, s[:, None]), s


def quant_i16(v, e: int) -> np.ndarray:
    """refquant.py:128-134."""
    v = np.asarray(v, dtype=np.float64)
    with np.errstate(over="ignore"):
        return llround(np.clip(np.ldexp(v, -int(e)), -32768, 32767)).astype(np.int16)
