"""Record verification: golden.json records compared bit for bit, on the host and on the device.

`compare_sim` / `compare_records` restate the reference's runtime-vs-golden check
(`python/llaccel/verify.py:80-104`): both records must carry the arrays `argmax_per_step`,
`generated` and `logits_last_rows` (one logits row per launch), token IDs and logits must be
integers, and the three arrays must be equal element by element; the result is
`(ok, message)` with the reference's MATCH / MISMATCH wording.  The reference's other mode
(integer model vs an fp32 checkpoint, `verify.py:28-77`) needs a trained float model and is not
part of this datapath.

On the device, `first_mismatch` and `row_checksums` (C ABI `llhip_rows_first_mismatch_i16`,
`llhip_rows_checksum_i16`) compare or fingerprint device-resident i16 logits rows, so a long
decode run (`GoldenModel.decode_loop` keeps its rows in a device ring) is checked against an
expected record with one 8-byte download, or n x 8 bytes of checksums, instead of n x vocab x 2
bytes.  `host_row_checksums` is the same checksum on the host.

    python -m llaccel_amd.verify --sim-json build/sim.json --golden build/golden.json
"""
from __future__ import annotations

import argparse
import ctypes
import json
import sys
from pathlib import Path

import numpy as np

from . import _lib

_KEYS = ("argmax_per_step", "generated", "logits_last_rows")


def _format_problem(record: dict) -> str | None:
    """The first way `record` departs from the record format (verify.py:86-95), or None: the three
    arrays present, one logits row per recorded argmax, integer tokens, nonempty integer rows."""
    missing = [k for k in _KEYS if not isinstance(record.get(k), list)]
    if missing:
        return f"lacks an array {missing[0]!r}"
    tokens, rows = record["argmax_per_step"] + record["generated"], record["logits_last_rows"]
    if len(rows) != len(record["argmax_per_step"]):
        return "logits/launch counts differ"
    if not all(type(t) is int for t in tokens):
        return "token IDs must be integers"
    if not all(isinstance(r, list) and r and all(type(v) is int for v in r) for r in rows):
        return "logits must be nonempty integer rows"
    return None


def _first_difference(a: list, b: list):
    """(index, a[i], b[i]) of the first unequal element of two equally long lists, or None."""
    return next(((i, x, y) for i, (x, y) in enumerate(zip(a, b)) if x != y), None)


def compare_records(sim: dict, gold: dict) -> tuple[bool, str]:
    """The record check of verify.py:80-104 on two loaded records: both well formed, then the three
    arrays equal element by element (the first difference is reported)."""
    for owner, record in (("sim", sim), ("golden", gold)):
        problem = _format_problem(record)
        if problem is not None:
            return False, f"MISMATCH: {owner}.json {problem}"
    for key in _KEYS:
        if len(sim[key]) != len(gold[key]):
            return False, f"MISMATCH: {key} length sim={len(sim[key])} golden={len(gold[key])}"
        diff = _first_difference(sim[key], gold[key])
        if diff is not None:
            step, left, right = diff
            return False, f"MISMATCH in {key} at step {step}: sim={left} golden={right}"
    return True, f"MATCH: {len(gold['generated'])} tokens, {len(gold['argmax_per_step'])} steps identical"


def compare_sim(sim_path: Path | str, golden_path: Path | str) -> tuple[bool, str]:
    """verify.py:80-104: the runtime's record file against the golden record file."""
    with open(sim_path) as f:
        sim = json.load(f)
    with open(golden_path) as f:
        gold = json.load(f)
    return compare_records(sim, gold)


# ---- device-side checks -----------------------------------------------------------------
def _torch():
    import torch

    return torch


def _as_i16_rows(t):
    torch = _torch()
    if not isinstance(t, torch.Tensor) or t.device.type != "cuda" or t.dtype != torch.int16 or t.dim() != 2:
        raise ValueError("expected a 2-D int16 tensor on the GPU")
    if t.stride(1) != 1:
        raise ValueError("rows must be contiguous")
    return t


def first_mismatch(a, b) -> int:
    """Smallest flat index r * cols + c where two device i16 row sets differ, or -1 (equal).
    Shapes must agree; row strides may differ."""
    torch = _torch()
    a, b = _as_i16_rows(a), _as_i16_rows(b)
    if a.shape != b.shape:
        raise ValueError(f"shape mismatch {tuple(a.shape)} vs {tuple(b.shape)}")
    out = torch.empty(1, dtype=torch.int64, device=a.device)
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.call("llhip_rows_first_mismatch_i16", ctypes.c_void_p(a.data_ptr()), a.stride(0), ctypes.c_void_p(b.data_ptr()),
              b.stride(0), a.shape[0], a.shape[1], ctypes.c_void_p(out.data_ptr()), s)
    return int(out.cpu()[0])


def row_checksums(x) -> np.ndarray:
    """Per-row sum_c (c + 1) * (uint16)x[r][c] mod 2^64 of device i16 rows, computed on the GPU."""
    torch = _torch()
    x = _as_i16_rows(x)
    out = torch.empty(max(x.shape[0], 1), dtype=torch.int64, device=x.device)
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.call("llhip_rows_checksum_i16", ctypes.c_void_p(x.data_ptr()), x.stride(0), x.shape[0], x.shape[1],
              ctypes.c_void_p(out.data_ptr()), s)
    return out[:x.shape[0]].cpu().numpy().view(np.uint64)


def host_row_checksums(rows) -> np.ndarray:
    """The same checksum of integer rows on the host (values taken modulo 2^16, as int16)."""
    r = np.asarray(rows, dtype=np.int64)
    if r.ndim != 2:
        raise ValueError("expected rows [n][cols]")
    u = (r & 0xFFFF).astype(np.uint64)
    w = np.arange(1, r.shape[1] + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return (u * w[None, :]).sum(axis=1, dtype=np.uint64)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="compare a runtime record with a golden.json record")
    ap.add_argument("--sim-json", required=True)
    ap.add_argument("--golden", default="build/golden.json")
    args = ap.parse_args(argv)
    ok, msg = compare_sim(Path(args.sim_json), Path(args.golden))
    print(msg)
    return 0 if ok else 1


if __name__ == "__main__":
    sys.exit(main())
