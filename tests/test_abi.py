"""CPU checks of the product boundary: the C-ABI library loads, exports every entry point
include/llhip.h declares, and its compiled-in LUTs are the reference's tables.  No compute
call is made (there may be no GPU)."""
from __future__ import annotations

import ctypes
import json
import re

import pytest

from llaccel_amd import _lib, luts


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    declared = _lib.declared_symbols()
    assert len(declared) >= 20
    for name in declared:
        assert hasattr(L, name), name
    assert set(declared) == set(_lib._SIGS), "ctypes signature table out of sync with include/llhip.h"


def test_library_resolves_every_symbol_at_load():
    """Every symbol the library references resolves when it is bound eagerly: a kernel template the
    host compilation pass failed to instantiate leaves its launch stub undefined, which a lazy load
    only reports at the first launch."""
    import os

    ctypes.CDLL(str(_lib.LIB_PATH), mode=os.RTLD_NOW | os.RTLD_LOCAL)


def test_abi_version_and_workspace():
    L = _lib.lib()
    assert L.llhip_abi_version() == 2
    assert L.llhip_workspace_bytes() >= 8 << 20


def test_header_declarations_cite_the_reference():
    text = _lib.HEADER.read_text()
    for name in _lib.declared_symbols():
        if name in ("llhip_abi_version", "llhip_last_error", "llhip_workspace_bytes"):
            continue
        # the comment block directly above each compute entry point cites the reference function it
        # replaces: golden.py:<lines> (the datapath), verify.py:<lines> (record verification),
        # refquant.py:<lines> (the qgraph producer), device.h:<lines> / funcsim.cpp:<lines> (the
        # instruction-set device), calibrate.py / smoothquant.py:<lines> (the float side); an entry
        # point with no reference counterpart says so and names the callers it is for
        idx = text.index(name + "(")
        before = text[:idx].rsplit(");", 1)[-1]
        assert (re.search(r"((golden|verify|refquant|calibrate|smoothquant)\.py|device\.h|funcsim\.cpp):\d+", before)
                or re.search(r"No counterpart in the reference: .* for callers", before, re.S)), name


def test_hip_luts_are_current_and_equal_reference(golden_dir):
    assert (luts.INC).read_text() == luts.hip_tables_text()
    ref = json.loads((golden_dir / "luts_ref.json").read_text())
    assert luts.sigmoid_lut().tolist() == ref["kSigmoidLut"]
    assert luts.exp_int_lut().tolist() == ref["kExpIntLut"]
    assert luts.exp_frac_lut().tolist() == ref["kExpFracLut"]


def test_errors_are_reported_without_a_gpu():
    """Argument validation happens before any HIP call: a bad shift returns -EINVAL and a message."""
    L = _lib.lib()
    rc = L.llhip_vquant_i64(None, 0, 1, 64, None, None)
    assert rc == -22
    assert b"shift" in L.llhip_last_error()
    with pytest.raises(ValueError, match="prob_bits"):
        _lib.call("llhip_attention", None, 1, 1, 1, 16, 16, 0, None, None, 0, None, None, 1, 1, 0, 1, 0, 9, None, 16, None,
                  None)


def test_product_does_not_import_the_oracle():
    from pathlib import Path

    pkg = Path(_lib.__file__).parent
    for f in list(pkg.rglob("*.py")) + list(pkg.rglob("*.hip")) + list(pkg.rglob("*.h")):
        text = f.read_text()
        assert "oracle" not in re.sub(r"#.*|//.*", "", text).replace("oracle/", ""), f
