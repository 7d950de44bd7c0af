from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))

GOLDEN = REPO / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C-ABI)")
    config.addinivalue_line("markers", "slow: larger CPU/GPU cases")


@pytest.fixture(scope="session")
def golden_dir() -> Path:
    return GOLDEN


@pytest.fixture(scope="session")
def ref_lib():
    """The reference's numerics.h compiled by oracle/Makefile into oracle/_ref (build container only)."""
    import ctypes

    path = REPO / "oracle" / "_ref" / "libllaccel_ref.so"
    if not path.exists():
        pytest.skip("oracle/_ref not built (reference tree absent)")
    lib = ctypes.CDLL(str(path))
    i64, u32, u64, p = ctypes.c_int64, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_void_p
    lib.ref_rshr.argtypes, lib.ref_rshr.restype = [i64, u32], i64
    lib.ref_mulshift.argtypes, lib.ref_mulshift.restype = [i64, u32, u32], i64
    lib.ref_isqrt48.argtypes, lib.ref_isqrt48.restype = [u64], u32
    lib.ref_udiv.argtypes, lib.ref_udiv.restype = [u64, u64], u32
    lib.ref_requant16.argtypes, lib.ref_requant16.restype = [ctypes.c_int32] * 3, i64
    lib.ref_requant8.argtypes, lib.ref_requant8.restype = [ctypes.c_int32] * 3, i64
    lib.ref_silu16.argtypes, lib.ref_silu16.restype = [i64, u32, u32, u32], i64
    lib.ref_vmul.argtypes, lib.ref_vmul.restype = [i64, i64, u32], i64
    lib.ref_vadd.argtypes, lib.ref_vadd.restype = [i64, i64, u32], i64
    lib.ref_vquant.argtypes, lib.ref_vquant.restype = [i64, u32, u32], i64
    lib.ref_rmsnorm.argtypes = [p, p, p, u32, u32, u32, u32]
    lib.ref_rope.argtypes = [p, p, u32, u32, p, p]
    lib.ref_attention_head.argtypes = [p, u32, u32, p, p, u32, u32, u32, u32, p, ctypes.c_int]
    lib.ref_luts.argtypes = [p, p, p]
    return lib


def gpu_available() -> bool:
    if os.environ.get("LLACCEL_FORCE_NO_GPU"):
        return False
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False
