"""Helpers of the GPU parity tests: device tensors and direct C-ABI calls."""
from __future__ import annotations

import ctypes

import numpy as np

from llaccel_amd import _lib

EPI = {"none": 0, "resadd": 1, "silu": 2, "mul": 3}


def torch():
    import torch as t

    assert t.cuda.is_available(), "GPU tests need a ROCm device"
    return t


def up(a, dtype):
    t = torch()
    return t.from_numpy(np.ascontiguousarray(a, dtype=dtype)).to("cuda")


def down(x) -> np.ndarray:
    return x.cpu().numpy().astype(np.int64)


def ptr(x):
    return None if x is None else ctypes.c_void_p(x.data_ptr())


def stream():
    return ctypes.c_void_p(torch().cuda.current_stream().cuda_stream)


_WS = {}


def workspace():
    t = torch()
    if "ws" not in _WS:
        _WS["ws"] = t.zeros(int(_lib.lib().llhip_workspace_bytes()), dtype=t.uint8, device="cuda")
    return _WS["ws"]


def gpu_linear(a, w, rq, bias=None, out_i8=False, epilogue="none", aux=None, aux_shift=0, silu=None, ws=True):
    """llhip_linear on host int arrays; returns int64 [M][N]."""
    t = torch()
    M, K = a.shape
    N = w.shape[0]
    ad, wd, rqd = up(a, np.int8), up(w, np.int8), up(rq, np.int32)
    bd = None if bias is None else up(bias, np.int32)
    auxd = None if aux is None else up(aux, np.int16)
    out = t.empty((M, N), dtype=t.int8 if out_i8 else t.int16, device="cuda")
    s = silu or {"Mi": 0, "Si": 0, "sh_out": 0}
    _lib.call("llhip_linear", ptr(ad), M, K, K, ptr(wd), N, ptr(rqd), ptr(bd), EPI[epilogue], ptr(auxd), N,
              aux_shift, s["Mi"], s["Si"], s["sh_out"], int(out_i8), ptr(out), N, ptr(workspace()) if ws else None,
              stream())
    return down(out)


def random_rq(rng, N, K, out_i8=True):
    """Per-channel (M, S) spanning the output range: M in [2^30, 2^31), S from the accumulator spread."""
    sigma = 73.0 * np.sqrt(K) * 73.0  # std of a sum of K products of uniform [-127,127] values
    target = 40.0 if out_i8 else 9000.0
    S = np.full(N, int(np.round(30 + np.log2(sigma / target))))
    S += rng.integers(-1, 2, N)
    M = rng.integers(1 << 30, 1 << 31, N)
    return np.stack([M, S], 1).astype(np.int32)
