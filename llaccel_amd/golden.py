"""Drop-in GPU twin of the reference's python/llaccel/golden.py.

Same names, signatures, argument meaning, records and error behaviour as the reference
module; every integer is computed by the gfx950 kernels of libllhip.so (include/llhip.h)
through ctypes.  PyTorch-ROCm only allocates device memory and supplies the stream.

    python -m llaccel_amd.golden --qgraph build/q/ --prompt-ids 1,2,3 --tokens 64 -o golden.json

Primitives (golden.py:35-180) take NumPy arrays / Python ints and return int64 NumPy
arrays (Python ints for isqrt48/udiv), like the reference.  Inputs of the datapath
primitives must fit the types NUMERICS.md gives them (rmsnorm/rope operands i16,
attention operands i8); the reference would also compute out-of-type values, this module
raises ValueError for them instead.

`GoldenModel` keeps the quantized weights, the KV caches and every activation resident in
HBM; `run_chunk` uploads the input rows and downloads the logits (and, when asked, every
activation).  `kv` returns host snapshots of the device caches; `set_kv` uploads one.
"""
from __future__ import annotations

import argparse
import contextlib
import ctypes
import gc
import json
import math
from collections.abc import Sequence
from pathlib import Path

import numpy as np

from . import _lib
from .luts import exp_frac_lut, exp_int_lut, sigmoid_lut

I64 = np.int64
SIG = sigmoid_lut().astype(I64)
EXPI = exp_int_lut().astype(I64)
EXPF = exp_frac_lut().astype(I64)
PREFILL_M = 16
DECODE_GRAPH_STEPS = 8  # decode launches per replay of the run graph (decode_loop)

_torch = None


def _t():
    global _torch
    if _torch is None:
        import torch

        if not torch.cuda.is_available():
            raise RuntimeError("llaccel_amd needs a ROCm GPU: torch.cuda.is_available() is False")
        _torch = torch
    return _torch


def _dev():
    torch = _t()
    return torch.device("cuda", torch.cuda.current_device())


def _stream():
    return ctypes.c_void_p(_t().cuda.current_stream().cuda_stream)


@contextlib.contextmanager
def capture_graph(graph):
    """torch.cuda.graph on a side stream with the Python garbage collector paused: a collection
    during capture could destroy an unreferenced graph or free device memory of an earlier model,
    runtime calls that are not permitted while a stream is being captured."""
    torch = _t()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    gc.collect()
    enabled = gc.isenabled()
    gc.disable()
    try:
        with torch.cuda.graph(graph, stream=side):
            yield
    finally:
        if enabled:
            gc.enable()
    torch.cuda.current_stream().wait_stream(side)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _up(a: np.ndarray, dtype=np.int64):
    """Host array -> contiguous device tensor of `dtype`."""
    torch = _t()
    return torch.from_numpy(np.ascontiguousarray(a, dtype=dtype)).to(_dev())


def _down(t) -> np.ndarray:
    return t.cpu().numpy()


def _check_range(a: np.ndarray, lo: int, hi: int, what: str) -> None:
    if a.size and (a.min() < lo or a.max() > hi):
        raise ValueError(f"{what} must lie in [{lo}, {hi}]")


def _check_shift(s, what="shift") -> None:
    s = np.asarray(s, dtype=I64)
    if s.size and (s.min() < 0 or s.max() > 63):
        raise ValueError(f"{what} must be in [0, 63]")


def _check_u32(v, what) -> None:
    v = np.asarray(v, dtype=I64)
    if v.size and (v.min() < 0 or v.max() > 0xFFFFFFFF):
        raise ValueError(f"{what} must be an unsigned 32-bit value")


def _elementwise(fn: str, arrays: list, *scalars) -> np.ndarray:
    """Broadcast int64 operands on the host, run one elementwise kernel, return int64."""
    arrs = np.broadcast_arrays(*[np.asarray(a, dtype=I64) for a in arrays])
    shape = arrs[0].shape
    n = int(np.prod(shape)) if shape else 1
    if n == 0:
        return np.zeros(shape, I64)
    dev = [_up(a.reshape(-1)) for a in arrs]
    out = _t().empty(n, dtype=_t().int64, device=_dev())
    ptrs = [_ptr(d) for d in dev]
    if fn in ("llhip_silu16_i64", "llhip_vquant_i64"):
        _lib.call(fn, ptrs[0], n, *scalars, _ptr(out), _stream())
    elif fn in ("llhip_vmul_i64", "llhip_vadd_i64"):
        _lib.call(fn, ptrs[0], ptrs[1], n, *scalars, _ptr(out), _stream())
    elif fn == "llhip_sat":
        _lib.call(fn, ptrs[0], n, *scalars, _ptr(out), _stream())
    elif fn == "llhip_requant":
        _lib.call(fn, ptrs[0], ptrs[1], ptrs[2], n, *scalars, _ptr(out), _stream())
    else:
        _lib.call(fn, *ptrs, n, _ptr(out), _stream())
    return _down(out).reshape(shape)


# --------------------------------------------------------------------------------------
# Primitives (golden.py:35-180)
# --------------------------------------------------------------------------------------
def rshr(v, s):
    """Round-half-up arithmetic right shift (golden.py:35-45); s in [0, 63]."""
    _check_shift(s)
    return _elementwise("llhip_rshr", [v, s])


def sat8(v):
    """golden.py:48-49"""
    return _elementwise("llhip_sat", [v], 0)


def satu8(v):
    """golden.py:52-53"""
    return _elementwise("llhip_sat", [v], 1)


def sat16(v):
    """golden.py:56-57"""
    return _elementwise("llhip_sat", [v], 2)


def satu16(v):
    """golden.py:60-61"""
    return _elementwise("llhip_sat", [v], 3)


def mulshift(v, M, S):
    """rshr(v*M, S) with a wrapping int64 product (golden.py:64-65)."""
    _check_shift(S)
    return _elementwise("llhip_mulshift", [v, M, S])


def isqrt48(t: int) -> int:
    """floor(sqrt(t)) for t < 2^48 (golden.py:68-81)."""
    t = int(t)
    if not 0 <= t < (1 << 48):
        raise ValueError(f"isqrt48 input out of range: {t}")
    return int(_elementwise("llhip_isqrt48", [np.array([t])])[0])


def udiv(a: int, b: int) -> int:
    """(a // max(b, 1)) & 0xFFFFFFFF (golden.py:84-88)."""
    a, b = int(a), int(b)
    if a < 0 or b < 0:
        raise ValueError("udiv operands must be unsigned")
    if a >= 1 << 63 or b >= 1 << 63:
        raise ValueError("udiv operands must fit int64")
    return int(_elementwise("llhip_udiv", [np.array([a]), np.array([b])])[0])


def requant16(acc, M, S):
    """golden.py:92-93"""
    _check_shift(S)
    return _elementwise("llhip_requant", [acc, M, S], 16)


def requant8(acc, M, S):
    """golden.py:96-97"""
    _check_shift(S)
    return _elementwise("llhip_requant", [acc, M, S], 8)


def silu16(x, Mi: int, Si: int, sh_out: int):
    """golden.py:101-107"""
    _check_shift(Si, "Si")
    _check_shift(sh_out, "sh_out")
    return _elementwise("llhip_silu16_i64", [x], int(Mi), int(Si), int(sh_out))


def vmul(a, b, sh: int):
    """golden.py:111-112"""
    _check_shift(sh)
    return _elementwise("llhip_vmul_i64", [a, b], int(sh))


def vadd(a, b, sh_b: int):
    """golden.py:115-116"""
    _check_shift(sh_b)
    return _elementwise("llhip_vadd_i64", [a, b], int(sh_b))


def vquant(x, M: int, S: int):
    """golden.py:119-120"""
    _check_shift(S)
    return _elementwise("llhip_vquant_i64", [x], int(M), int(S))


def rmsnorm(x, g, eps_t: int, C: int, sh_post: int):
    """Row-wise integer RMSNorm of x [rows][K] with gamma g [K] (golden.py:124-137)."""
    x = np.asarray(x, dtype=I64)
    g = np.asarray(g, dtype=I64).reshape(-1)
    if x.ndim != 2 or x.shape[1] != g.shape[0]:
        raise ValueError("rmsnorm: x must be [rows][K] with K = len(g)")
    _check_range(x, -32768, 32767, "rmsnorm input")
    _check_range(g, -32768, 32767, "rmsnorm gamma")
    _check_u32(eps_t, "eps_t")
    _check_u32(C, "C")
    _check_shift(sh_post, "sh_post")
    rows, K = x.shape
    if rows == 0:
        return np.zeros((0, K), I64)
    xd, gd = _up(x, np.int16), _up(g, np.int16)
    yd = _t().empty_like(xd)
    _lib.call("llhip_rmsnorm", _ptr(xd), rows, K, K, _ptr(gd), int(eps_t), int(C), int(sh_post), _ptr(yd), K, _stream())
    return _down(yd).astype(I64)


def rmsnorm_row(x, g, eps_t: int, C: int, sh_post: int):
    """golden.py:124-132"""
    return rmsnorm(np.asarray(x, dtype=I64)[None, :], g, eps_t, C, sh_post)[0]


def rope(x, H: int, D: int, cos_tab, sin_tab, pos: int):
    """x [M][H*D]; row m uses table row pos+m (golden.py:155-158)."""
    x = np.asarray(x, dtype=I64)
    cos_tab = np.asarray(cos_tab, dtype=I64)
    sin_tab = np.asarray(sin_tab, dtype=I64)
    H, D, pos = int(H), int(D), int(pos)
    if x.ndim != 2 or x.shape[1] != H * D or D % 2:
        raise ValueError("rope: x must be [M][H*D] with even D")
    if cos_tab.ndim != 2 or cos_tab.shape[1] != D // 2 or cos_tab.shape != sin_tab.shape:
        raise ValueError("rope: tables must be [rows][D/2]")
    if pos < 0 or pos + x.shape[0] > cos_tab.shape[0]:
        raise IndexError("rope: table rows pos..pos+M-1 out of range")
    for a, w in ((x, "rope input"), (cos_tab, "rope cos table"), (sin_tab, "rope sin table")):
        _check_range(a, -32768, 32767, w)
    M = x.shape[0]
    if M == 0:
        return np.zeros_like(x)
    xd = _up(x, np.int16)
    cd, sd = _up(cos_tab, np.int16), _up(sin_tab, np.int16)
    yd = _t().empty_like(xd)
    _lib.call("llhip_rope", _ptr(xd), M, H, D, H * D, _ptr(cd), _ptr(sd), cos_tab.shape[0], pos, None, None, _ptr(yd),
              H * D, _stream())
    return _down(yd).astype(I64)


def rope_row(x, H: int, D: int, cosv, sinv):
    """golden.py:141-152"""
    return rope(np.asarray(x, dtype=I64)[None, :], H, D, np.asarray(cosv)[None, :], np.asarray(sinv)[None, :], 0)[0]


def attention_head(q, keys, vals, Ms: int, Ss: int, Mo: int, So: int, prob_bits: int = 8):
    """q [D] i8; keys/vals [T][D] i8 -> out [D] (golden.py:162-180)."""
    if prob_bits not in (8, 15):
        raise ValueError("attention prob_bits must be 8 or 15")
    q = np.asarray(q, dtype=I64).reshape(-1)
    keys = np.asarray(keys, dtype=I64)
    vals = np.asarray(vals, dtype=I64)
    D = q.shape[0]
    if keys.ndim != 2 or keys.shape[1] != D or vals.shape != keys.shape or keys.shape[0] < 1:
        raise ValueError("attention_head: keys/vals must be [T][D], T >= 1")
    for a, w in ((q, "q"), (keys, "keys"), (vals, "vals")):
        _check_range(a, -128, 127, w)
    T = keys.shape[0]
    qd = _up(q[None, :], np.int8)
    kd, vd = _up(keys, np.int8), _up(vals, np.int8)
    out = _t().empty((1, D), dtype=_t().int8, device=_dev())
    _lib.call("llhip_attention", _ptr(qd), 1, 1, 1, D, D, T - 1, None, None, 0, _ptr(kd), _ptr(vd), T, int(Ms),
              int(Ss), int(Mo), int(So), int(prob_bits), _ptr(out), D, None, _stream())
    return _down(out)[0].astype(I64)


# --------------------------------------------------------------------------------------
# Quantized graph loading (golden.py:186-214)
# --------------------------------------------------------------------------------------
_DT = {"i8": (np.int8, 1), "i16": (np.dtype("<i2"), 2), "i32": (np.dtype("<i4"), 4), "rq": (np.dtype("<i4"), 8)}


class QGraph:
    """qgraph.json + memory-mapped qweights.bin (golden.py:189-214)."""

    def __init__(self, qdir: Path | str) -> None:
        self.dir = Path(qdir)
        with open(self.dir / "qgraph.json") as f:
            self.g = json.load(f)
        self.model = self.g["model"]
        self.ops = self.g["ops"]
        self.blob = np.memmap(self.dir / self.g["weights_file"], dtype=np.uint8, mode="r")
        self.tensors: dict[str, np.ndarray] = {}
        self.tensor_exp: dict[str, int] = {}
        self.specs: dict[str, dict] = {}
        for name, spec in self.g["tensors"].items():
            dt, _ = _DT[spec["dtype"]]
            count = int(np.prod(spec["shape"]))
            if spec["dtype"] == "rq":
                arr = np.frombuffer(self.blob, dtype=dt, count=2 * count, offset=spec["offset"]).reshape(count, 2)
            else:
                arr = np.frombuffer(self.blob, dtype=dt, count=count, offset=spec["offset"]).reshape(spec["shape"])
            self.tensors[name] = arr
            self.specs[name] = spec
            if "exp" in spec:
                self.tensor_exp[name] = spec["exp"]
        self.exps: dict[str, int] = dict(self.g.get("exps", {}))
        self.scales: dict[str, float] = dict(self.g.get("scales", {}))
        self.input_name = self.g.get("input", "input")
        self.output_name = self.g.get("output", "logits")


def exact_blas_matmul(a: np.ndarray, w: np.ndarray, chunk_rows: int = 1024) -> np.ndarray:
    """Exact integer A @ W.T (golden.py:217-240): same argument checks and errors as the
    reference, computed with integer arithmetic on the GPU (no floating point)."""
    if a.ndim != 2 or w.ndim != 2 or a.shape[1] != w.shape[1]:
        raise ValueError("invalid matrix dimensions")
    if a.dtype.kind not in "iu" or w.dtype.kind not in "iu" or chunk_rows < 1:
        raise ValueError("exact BLAS requires integer inputs and positive chunks")
    amax = max(abs(int(a.min(initial=0))), abs(int(a.max(initial=0))))
    wi = np.iinfo(w.dtype)
    wmax = max(abs(int(wi.min)), abs(int(wi.max)))
    if a.shape[1] * amax * wmax > (1 << 53):
        raise ValueError("integer dot product exceeds exact FP64 accumulation bound")
    M, K = a.shape
    N = w.shape[0]
    torch = _t()
    if w.dtype != np.int8 and (int(w.min(initial=0)) < -128 or int(w.max(initial=0)) > 127):
        # weights beyond int8 (any integer dtype, as the reference accepts): FP64 products and sums of
        # integers whose partial sums stay below 2^53 -- the bound checked above -- are exact, which is
        # the reference's own method (golden.py:226-240); here on the GPU through the library's FP64 GEMM
        af = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float64)).to(_dev())
        wf = torch.from_numpy(np.ascontiguousarray(w, dtype=np.float64)).to(_dev())
        out = torch.empty((M, N), dtype=torch.int64, device=_dev())
        for r0 in range(0, M, chunk_rows):
            out[r0:r0 + chunk_rows] = torch.matmul(af[r0:r0 + chunk_rows], wf.T.contiguous()).round().to(torch.int64)
        return _down(out)
    out = torch.empty((M, N), dtype=torch.int64, device=_dev())
    ad, wd = _up(a), _up(w, np.int8)  # int8-valued weights of a wider dtype convert exactly
    _lib.call("llhip_exact_matmul", _ptr(ad), M, K, _ptr(wd), N, _ptr(out), _stream())
    return _down(out)


# --------------------------------------------------------------------------------------
# Golden model
# --------------------------------------------------------------------------------------
_EPI = {"none": 0, "resadd": 1, "silu": 2, "mul": 3}
_TDT = {"i8": "int8", "i16": "int16"}


class _Deferred:
    """A graph error that the reference raises when the op executes; raised at the same point."""

    kind = "error"

    def __init__(self, exc: Exception) -> None:
        self.exc = exc

    def __call__(self, M, pos, pd=None):
        raise self.exc


class _RowPos:
    """Position context of a batch decode launch: row m is its own sequence, at the device position
    rows[m], with its K/V caches in slot m (`stride` elements after slot m - 1)."""

    def __init__(self, ptr, stride: int) -> None:
        self.ptr, self.stride = ptr, stride


class _SeqRows:
    """Position context of a batch prefill launch: the rows are M / rows sequences of `rows` rows
    each; row m is row m % rows of sequence m / rows, at position pos + m % rows, with its K/V caches
    in slot m / rows (`stride` elements after the slot before)."""

    def __init__(self, rows: int, stride: int) -> None:
        self.rows, self.stride = rows, stride


def _pos_args(pd):
    """(pos_dev, row_pos, slot_stride) kernel arguments of a step's position context."""
    if isinstance(pd, _RowPos):
        return None, pd.ptr, pd.stride
    if isinstance(pd, _SeqRows):
        return None, None, pd.stride
    return pd, None, 0


def _seq_rows(pd) -> int:
    """The rows per sequence of a batch prefill context (0 otherwise)."""
    return pd.rows if isinstance(pd, _SeqRows) else 0


class _Step:
    """One compiled op: `fn(M, pos, pos_dev)` launches its kernel(s); `bytes_fn(M)` gives the
    algorithmic HBM bytes of one launch (operands read once, results written once)."""

    def __init__(self, kind: str, fn, bytes_fn=None, name: str = "") -> None:
        self.kind, self.fn, self.bytes_fn, self.name = kind, fn, bytes_fn, name

    def __call__(self, M, pos, pd=None):
        self.fn(M, pos, pd)


class GoldenModel:
    """Device-resident twin of golden.py:246-440 (same attributes, methods and record)."""

    def __init__(self, qgraph_dir: Path | str, *, fast_matmul: bool = False, fuse: bool = True) -> None:
        self.fast_matmul = fast_matmul  # accepted for API parity: every path here is exact integer arithmetic
        self.fuse = fuse  # run matched op runs as fused launches (llaccel_amd.fusion); results are identical
        self.q = QGraph(qgraph_dir)
        m = self.q.model
        self.dim = int(m["dim"])
        self.n_layers = int(m["n_layers"])
        self.vocab = int(m["vocab"])
        self.vocab_padded = int(m.get("vocab_padded", self.vocab))
        self.max_seq = int(m["max_seq"])
        self.prefill_m = int(m.get("prefill_m", PREFILL_M))
        if not 1 <= self.prefill_m <= 16 or self.max_seq % self.prefill_m:
            raise ValueError("max_seq must be divisible by prefill_m in [1,16]")
        self.E_RES = int(m["E_RES"])
        self.E_LOGIT = int(m["E_LOGIT"])
        self.embed = self.q.tensors["embed"]
        self.rope_cos = self.q.tensors["rope_cos"]
        self.rope_sin = self.q.tensors["rope_sin"]
        torch = _t()
        self.device = _dev()
        # one upload of the whole weight blob; every tensor is a view of it
        self._blob = torch.from_numpy(np.array(self.q.blob, copy=True)).to(self.device)
        self._dt: dict[str, object] = {}
        for name, spec in self.q.specs.items():
            self._dt[name] = self._tensor_view(spec)
        self._ws = torch.zeros(int(_lib.lib().llhip_workspace_bytes()), dtype=torch.uint8, device=self.device)
        self._act: dict[str, object] = {}
        self._cap = 0
        self._lean = False  # set while a launch collects no activations (llaccel_amd.fusion)
        self._act_spec: dict[str, tuple[str, int]] = {}
        self._pf_graphs: dict = {}  # whole-prompt prefill graphs by (rows, prompt length, KV slot)
        self._pf_seen: dict = {}
        self._plan = self._compile()
        # one-row launches of a fused graph: three launches per layer (llaccel_amd.chain)
        self._chain = None
        if self.fuse:
            from . import chain

            self._chain = chain.build(self)
        self.use_chain = self._chain is not None
        self._ensure_capacity(self.prefill_m)
        self._graph = None
        self._ring_cap = 0
        self.use_graph = True
        self.whole_prompt_prefill = True
        self.reset()

    # ---- device tensors ---------------------------------------------------------------------
    def _tensor_view(self, spec: dict):
        torch = _t()
        dt = spec["dtype"]
        count = int(np.prod(spec["shape"]))
        nbytes = {"i8": 1, "i16": 2, "i32": 4, "rq": 8}[dt] * count
        raw = self._blob[int(spec["offset"]):int(spec["offset"]) + nbytes]
        tdt = {"i8": torch.int8, "i16": torch.int16, "i32": torch.int32, "rq": torch.int32}[dt]
        v = raw.view(tdt)
        return v.view(count, 2) if dt == "rq" else v.view(*spec["shape"]) if spec["shape"] else v

    def _buf(self, name: str):
        return self._act[name]

    def _kv_args(self, layer: int, pd):
        """(K cache, V cache, pos_dev, row_pos, slot_stride) kernel arguments of one layer."""
        kc, vc = self._kv[layer]
        if isinstance(pd, _RowPos):
            return _ptr(kc), _ptr(vc), None, pd.ptr, pd.stride
        if isinstance(pd, _SeqRows):
            return _ptr(kc), _ptr(vc), None, None, pd.stride
        return _ptr(kc[self._slot]), _ptr(vc[self._slot]), pd, None, 0

    def _ensure_capacity(self, M: int) -> None:
        if M <= self._cap:
            return
        torch = _t()
        cap = max(M, self.prefill_m)
        self._graph = None  # captured pointers would dangle
        self._graph_b = None
        self._pf_graphs.clear()
        for name, (dt, cols) in self._act_spec.items():
            self._act[name] = torch.zeros((cap, cols), dtype=getattr(torch, _TDT[dt]), device=self.device)
        self._cap = cap

    def reset(self) -> None:
        """Zero every layer's (Hkv, max_seq, D) int8 K and V caches (golden.py:266-272)."""
        torch = _t()
        if getattr(self, "_kv", None):
            for kc, vc in self._kv.values():  # in place: a captured decode graph holds these addresses
                kc.zero_()
                vc.zero_()
            return
        self._alloc_kv(1)

    def _alloc_kv(self, slots: int) -> None:
        """KV caches of `slots` independent sequences: per layer (slots, Hkv, max_seq, D) int8,
        zero-filled.  Single-sequence calls use slot `_slot` (0 unless a batch API selects one)."""
        torch = _t()
        self._graph = None
        self._graph_b = None
        getattr(self, "_pf_graphs", {}).clear()
        self._slot = 0
        self._kv_gen = getattr(self, "_kv_gen", 0) + 1  # new cache addresses (llaccel_amd.chain keys on it)
        self._kv: dict[int, tuple] = {}
        # every layer's K and V as views of ONE zero-filled allocation (one fill launch, not two per
        # layer); each view starts at a multiple of its (slots, Hkv, max_seq, D) size
        shapes = [(int(op["layer"]), (slots, int(op["Hkv"]), self.max_seq, int(op["D"])))
                  for op in self.q.ops if op["op"] == "kv_write"]
        sizes = [math.prod(sh) for _, sh in shapes]
        flat = torch.zeros(2 * sum(sizes), dtype=torch.int8, device=self.device)
        off = 0
        for (L, sh), n in zip(shapes, sizes):
            self._kv[L] = (flat[off:off + n].view(sh), flat[off + n:off + 2 * n].view(sh))
            off += 2 * n

    @property
    def kv(self) -> dict[int, tuple[np.ndarray, np.ndarray]]:
        """Host snapshots {layer: (K, V)} of the device caches, int8 (Hkv, max_seq, D)."""
        return self.kv_of(self._slot)

    def kv_of(self, slot: int) -> dict[int, tuple[np.ndarray, np.ndarray]]:
        """Host snapshots of the caches of KV slot `slot` (sequence `slot` of a batch run)."""
        n = next(iter(self._kv.values()))[0].shape[0] if self._kv else 0
        if not 0 <= slot < n:
            raise ValueError(f"KV slot {slot} outside the {n} allocated")
        return {L: (_down(k[slot]), _down(v[slot])) for L, (k, v) in self._kv.items()}

    def set_kv(self, layer: int, k: np.ndarray, v: np.ndarray) -> None:
        """Upload a (Hkv, max_seq, D) int8 K/V state for `layer` (preinitialised-state runs)."""
        kc, vc = self._kv[int(layer)]
        for src, dst in ((k, kc[self._slot]), (v, vc[self._slot])):
            a = np.asarray(src)
            if tuple(a.shape) != tuple(dst.shape):
                raise ValueError(f"KV shape {a.shape} != {tuple(dst.shape)}")
            dst.copy_(_up(a, np.int8))

    # ---- graph compilation ----------------------------------------------------------------
    def _compile(self) -> list:
        """Typecheck the op list and turn every op into one (or a few) kernel launches."""
        spec = self._act_spec
        spec[self.q.input_name] = ("i16", self.dim)
        plan = []
        T = self.q.tensors

        def need(name, dt=None):
            if name not in spec:
                raise ValueError(f"activation {name!r} is used before it is produced")
            if dt is not None and spec[name][0] != dt:
                raise ValueError(f"activation {name!r} is {spec[name][0]}, this op needs {dt}")
            return spec[name]

        for op in self.q.ops:
            k = op["op"]
            try:
                if k == "rmsnorm":
                    plan.append(_Step("rmsnorm", self._c_rmsnorm(op, need, T), name=op["out"]))
                elif k == "quant":
                    _, cols = need(op["in"], "i16")
                    _check_u32(op["M"], "quant M")
                    _check_shift(op["S"], "quant S")
                    spec[op["out"]] = ("i8", cols)
                    plan.append(_Step("quant", self._c_quant(op), name=op["out"]))
                elif k == "linear":
                    plan.append(_Step("linear", *self._c_linear(op, need, T), name=op["out"]))
                elif k == "rope":
                    _, cols = need(op["in"], "i16")
                    H, D = int(op["H"]), int(op["D"])
                    if cols != H * D or D % 2:
                        raise ValueError(f"rope {op['out']}: {cols} columns != H*D = {H * D}")
                    if self.rope_cos.shape[1] != D // 2:
                        raise ValueError("rope table width != D/2")
                    spec[op["out"]] = ("i16", cols)
                    plan.append(_Step("rope", self._c_rope(op), name=op["out"]))
                elif k == "kv_write":
                    plan.append(_Step("kv_write", self._c_kv_write(op, need), name=str(op["layer"])))
                elif k == "attention":
                    plan.append(_Step("attention", *self._c_attention(op, need), name=op["out"]))
                elif k in ("add", "mul"):
                    _, ca = need(op["a"], "i16")
                    _, cb = need(op["b"], "i16")
                    if ca != cb:
                        raise ValueError(f"{k} {op['out']}: operand widths differ")
                    _check_shift(op["sh_b" if k == "add" else "sh"], "shift")
                    spec[op["out"]] = ("i16", ca)
                    plan.append(_Step(k, self._c_binary(op, k), name=op["out"]))
                elif k == "silu":
                    _, cols = need(op["in"], "i16")
                    _check_u32(op["Mi"], "silu Mi")
                    _check_shift(op["Si"], "silu Si")
                    _check_shift(op["sh_out"], "silu sh_out")
                    spec[op["out"]] = ("i16", cols)
                    plan.append(_Step("silu", self._c_silu(op), name=op["out"]))
                else:
                    raise ValueError(f"unknown qgraph op {k!r}")
            except (ValueError, KeyError) as e:
                exc = e if isinstance(e, ValueError) else ValueError(f"missing tensor or field {e}")
                plan.append(_Deferred(exc))
                break
        if self.q.output_name not in spec and not any(isinstance(p, _Deferred) for p in plan):
            plan.append(_Deferred(ValueError(f"output {self.q.output_name!r} is never produced")))
        self._plan_unfused = plan
        if self.fuse:
            from . import fusion

            plan = fusion.fuse(self, self.q.ops, plan)
        return plan

    def _stream_handle(self):
        return _stream()

    def _c_rmsnorm(self, op, need, T):
        _, cols = need(op["in"], "i16")
        g = self._dt[op["gamma"]]
        K = int(g.shape[0])
        heads = int(op.get("heads", 1))
        if heads < 1 or cols != heads * K:
            raise ValueError("RMSNorm head geometry mismatch")
        _check_u32(op["eps_t"], "rmsnorm eps_t")
        _check_u32(op["C"], "rmsnorm C")
        _check_shift(op["sh_post"], "rmsnorm sh_post")
        self._act_spec[op["out"]] = ("i16", cols)
        src, dst = op["in"], op["out"]
        eps_t, C, sh = int(op["eps_t"]), int(op["C"]), int(op["sh_post"])

        def run(M, pos, pd=None):
            x, y = self._buf(src), self._buf(dst)
            _lib.call("llhip_rmsnorm", _ptr(x), M * heads, K, K, _ptr(g), eps_t, C, sh, _ptr(y), K, _stream())
        return run

    def _c_quant(self, op):
        src, dst, Mq, Sq = op["in"], op["out"], int(op["M"]), int(op["S"])
        cols = self._act_spec[src][1]

        def run(M, pos, pd=None):
            _lib.call("llhip_quant", _ptr(self._buf(src)), M * cols, Mq, Sq, _ptr(self._buf(dst)), _stream())
        return run

    def _c_linear(self, op, need, T):
        a_dt, a_cols = need(op["in"])
        w = T[op["w"]]
        rq = T[op["rq"]]
        N, K = int(op["N"]), int(op["K"])
        if tuple(w.shape) != (N, K) or a_cols != K:
            raise ValueError(f"linear {op['out']}: shapes A(M, {a_cols}) W{tuple(w.shape)} vs N={N} K={K}")
        if a_dt != "i8":
            raise ValueError(f"linear {op['out']}: input {op['in']!r} must be an i8 activation")
        if rq.shape != (N, 2):
            raise ValueError(f"linear {op['out']}: rq table shape {rq.shape}")
        if rq.size and (rq[:, 1].min() < 0 or rq[:, 1].max() > 63):
            raise ValueError(f"linear {op['out']}: rq shifts must be in [0, 63]")
        out_i8 = op.get("out_dtype", "i16") == "i8"
        ep = op.get("epilogue", "none") or "none"
        if out_i8 and ep != "none":
            raise ValueError("i8 output is only valid with epilogue none")
        if ep not in _EPI:
            raise ValueError(f"unknown epilogue {ep!r}")
        bias = self._dt[op["bias"]] if op.get("bias") else None
        if bias is not None and tuple(bias.shape) != (N,):
            raise ValueError(f"linear {op['out']}: bias shape {tuple(bias.shape)}")
        aux = None
        aux_shift = int(op.get("aux_shift", 0) or 0)
        if ep in ("resadd", "mul"):
            aux = op["aux"]
            _, c = need(aux, "i16")
            if c != N:
                raise ValueError(f"linear {op['out']}: aux width {c} != N={N}")
            if ep == "mul":
                _check_shift(aux_shift, "aux_shift")
        Mi = Si = sh = 0
        if ep == "silu":
            s = op["silu"]
            Mi, Si, sh = int(s["Mi"]), int(s["Si"]), int(s["sh_out"])
            _check_u32(Mi, "silu Mi")
            _check_shift(Si, "silu Si")
            _check_shift(sh, "silu sh_out")
        self._act_spec[op["out"]] = ("i8" if out_i8 else "i16", N)
        src, dst = op["in"], op["out"]
        wd, rqd = self._dt[op["w"]], self._dt[op["rq"]]
        epi = _EPI[ep]

        def run(M, pos, pd=None):
            a = self._buf(src)
            auxd = self._buf(aux) if aux is not None else None
            _lib.call("llhip_linear", _ptr(a), M, K, K, _ptr(wd), N, _ptr(rqd), _ptr(bias), epi, _ptr(auxd), N,
                      aux_shift, Mi, Si, sh, int(out_i8), _ptr(self._buf(dst)), N, _ptr(self._ws), _stream())

        def nbytes(M):
            # W + rq + bias + A + out (+ aux)  (linear(M,N,K) bytes of the measurement plan)
            return (N * K + 8 * N + (4 * N if bias is not None else 0) + M * K + M * N * (1 if out_i8 else 2)
                    + (2 * M * N if aux is not None else 0))
        return run, nbytes

    def _c_rope(self, op):
        src, dst, H, D = op["in"], op["out"], int(op["H"]), int(op["D"])
        cos_t, sin_t = self._dt["rope_cos"], self._dt["rope_sin"]
        rows = int(cos_t.shape[0])

        def run(M, pos, pd=None):
            if isinstance(pd, _SeqRows):
                raise ValueError("rope: no batch-prefill form (unfused graph)")
            pdev, rpos, _ = _pos_args(pd)
            _lib.call("llhip_rope", _ptr(self._buf(src)), M, H, D, H * D, _ptr(cos_t), _ptr(sin_t), rows, pos, pdev,
                      rpos, _ptr(self._buf(dst)), H * D, _stream())
        return run

    def _c_kv_write(self, op, need):
        Hkv, D = int(op["Hkv"]), int(op["D"])
        _, ck = need(op["k"], "i8")
        _, cv = need(op["v"], "i8")
        if ck < Hkv * D or cv < Hkv * D:
            raise ValueError("kv_write: K/V activations narrower than Hkv*D")
        layer = int(op["layer"])
        ksrc, vsrc = op["k"], op["v"]

        def run(M, pos, pd=None):
            if isinstance(pd, _SeqRows):
                raise ValueError("kv_write: no batch-prefill form (unfused graph)")
            kcp, vcp, pdev, rpos, stride = self._kv_args(layer, pd)
            _lib.call("llhip_kv_write", _ptr(self._buf(ksrc)), _ptr(self._buf(vsrc)), M, Hkv, D, ck, cv, pos, pdev,
                      rpos, stride, kcp, vcp, self.max_seq, _stream())
        return run

    def _c_attention(self, op, need):
        H, Hkv, D = int(op["H"]), int(op["Hkv"]), int(op["D"])
        _, cq = need(op["q"], "i8")
        if Hkv < 1 or H % Hkv:
            raise ValueError("attention: H must be a multiple of Hkv")
        if cq != H * D:
            raise ValueError(f"attention {op['out']}: q width {cq} != H*D")
        pb = op.get("prob_bits", 8)
        if pb not in (8, 15):
            raise ValueError("attention prob_bits must be 8 or 15")
        for f in ("Ms", "Mo"):
            _check_u32(op[f], f"attention {f}")
        for f in ("Ss", "So"):
            _check_shift(op[f], f"attention {f}")
        layer = int(op["layer"])
        self._act_spec[op["out"]] = ("i8", H * D)
        src, dst = op["q"], op["out"]
        Ms, Ss, Mo, So = (int(op[f]) for f in ("Ms", "Ss", "Mo", "So"))

        def run(M, pos, pd=None):
            if layer not in self._kv:
                raise KeyError(layer)
            kcp, vcp, pdev, rpos, stride = self._kv_args(layer, pd)
            if isinstance(pd, _SeqRows):
                _lib.call("llhip_attention_seqs", _ptr(self._buf(src)), M, pd.rows, H, Hkv, D, H * D, pos, kcp, vcp,
                          stride, self.max_seq, Ms, Ss, Mo, So, pb, _ptr(self._buf(dst)), H * D, _stream())
                return
            _lib.call("llhip_attention", _ptr(self._buf(src)), M, H, Hkv, D, H * D, pos, pdev, rpos, stride, kcp, vcp,
                      self.max_seq, Ms, Ss, Mo, So, pb, _ptr(self._buf(dst)), H * D, _ptr(self._ws), _stream())

        def nbytes(M, T):
            # K and V rows read once per GQA group + q in + out
            return 2 * Hkv * T * D + 2 * M * H * D
        return run, nbytes

    def _c_binary(self, op, kind):
        a, b, dst = op["a"], op["b"], op["out"]
        sh = int(op["sh_b"] if kind == "add" else op["sh"])
        cols = self._act_spec[a][1]
        fn = "llhip_vadd" if kind == "add" else "llhip_vmul"

        def run(M, pos, pd=None):
            _lib.call(fn, _ptr(self._buf(a)), _ptr(self._buf(b)), M * cols, sh, _ptr(self._buf(dst)), _stream())
        return run

    def _c_silu(self, op):
        src, dst = op["in"], op["out"]
        Mi, Si, sh = int(op["Mi"]), int(op["Si"]), int(op["sh_out"])
        cols = self._act_spec[src][1]

        def run(M, pos, pd=None):
            _lib.call("llhip_silu", _ptr(self._buf(src)), M * cols, Mi, Si, sh, _ptr(self._buf(dst)), _stream())
        return run

    # ---- one device launch --------------------------------------------------------------
    def _chained(self, M: int, pd=None) -> bool:
        return M == 1 and self.use_chain and self._chain is not None and not isinstance(pd, _RowPos)

    def _execute(self, M: int, pos: int, pd=None) -> None:
        if self._chained(M, pd):
            self._chain.run(pos, pd)
            return
        for step in self._plan:
            step(M, pos, pd)

    def _collect(self, M: int) -> dict:
        out = {}
        for name in self._act_spec:
            out[name] = _down(self._act[name][:M]).astype(I64)
        return out

    def run_chunk(self, rows: np.ndarray, pos: int, acts: dict | None = None) -> np.ndarray:
        """Execute the op list for `rows` [M][dim] (i16 at E_RES) at positions pos..pos+M-1
        (golden.py:275-314).  Returns logits [M][vocab_padded]; `acts` collects every activation."""
        rows = np.asarray(rows, dtype=I64)
        M = rows.shape[0]
        if pos < 0 or pos + M > self.max_seq:
            raise ValueError(f"positions {pos}..{pos + M - 1} exceed max_seq={self.max_seq}")
        if rows.ndim != 2 or rows.shape[1] != self.dim:
            raise ValueError(f"rows must be [M][{self.dim}]")
        _check_range(rows, -32768, 32767, "input rows")
        self._ensure_capacity(M)
        self._act[self.q.input_name][:M].copy_(_up(rows, np.int16))
        self._execute(M, int(pos))
        if acts is not None:
            got = self._collect(M)
            got[self.q.input_name] = rows
            acts.update(got)
        return _down(self._act[self.q.output_name][:M]).astype(I64)

    def linear(self, op: dict, act: dict) -> np.ndarray:
        """One gemm-engine op on host activations (golden.py:316-342)."""
        a = np.asarray(act[op["in"]], dtype=I64)
        w = self.q.tensors[op["w"]]
        N, K = int(op["N"]), int(op["K"])
        if w.shape != (N, K) or a.shape[1] != K:
            raise ValueError(f"linear {op['out']}: shapes A{a.shape} W{w.shape} vs N={N} K={K}")
        _check_range(a, -128, 127, "linear input")
        out_i8 = op.get("out_dtype", "i16") == "i8"
        ep = op.get("epilogue", "none") or "none"
        if out_i8 and ep != "none":
            raise ValueError("i8 output is only valid with epilogue none")
        if ep not in _EPI:
            raise ValueError(f"unknown epilogue {ep!r}")
        rq = self.q.tensors[op["rq"]]
        if rq.size and (rq[:, 1].min() < 0 or rq[:, 1].max() > 63):
            raise ValueError("rq shifts must be in [0, 63]")
        M = a.shape[0]
        ad = _up(a, np.int8)
        auxd = None
        if ep in ("resadd", "mul"):
            aux = np.asarray(act[op["aux"]], dtype=I64)
            _check_range(aux, -32768, 32767, "aux")
            auxd = _up(aux, np.int16)
        torch = _t()
        out = torch.empty((M, N), dtype=torch.int8 if out_i8 else torch.int16, device=self.device)
        s = op.get("silu") or {}
        bias = self._dt[op["bias"]] if op.get("bias") else None
        if M:
            _lib.call("llhip_linear", _ptr(ad), M, K, K, _ptr(self._dt[op["w"]]), N, _ptr(self._dt[op["rq"]]),
                      _ptr(bias), _EPI[ep], _ptr(auxd), N, int(op.get("aux_shift", 0) or 0), int(s.get("Mi", 0)),
                      int(s.get("Si", 0)), int(s.get("sh_out", 0)), int(out_i8), _ptr(out), N, _ptr(self._ws),
                      _stream())
        return _down(out).astype(I64)

    def kv_write(self, op: dict, act: dict, pos: int) -> None:
        """Write M rows of K/V into the caches at pos+m (golden.py:344-351)."""
        Hkv, D = int(op["Hkv"]), int(op["D"])
        k = np.asarray(act[op["k"]], dtype=I64)
        v = np.asarray(act[op["v"]], dtype=I64)
        _check_range(k, -128, 127, "k")
        _check_range(v, -128, 127, "v")
        kcp, vcp, _, _, _ = self._kv_args(int(op["layer"]), None)
        M = k.shape[0]
        kd, vd = _up(k, np.int8), _up(v, np.int8)
        _lib.call("llhip_kv_write", _ptr(kd), _ptr(vd), M, Hkv, D, k.shape[1], v.shape[1], pos, None, None, 0, kcp,
                  vcp, self.max_seq, _stream())

    def attention(self, op: dict, act: dict, pos: int) -> np.ndarray:
        """Causal GQA attention of host q rows over the device caches (golden.py:353-366)."""
        q = np.asarray(act[op["q"]], dtype=I64)
        _check_range(q, -128, 127, "q")
        H, Hkv, D = int(op["H"]), int(op["Hkv"]), int(op["D"])
        kcp, vcp, _, _, _ = self._kv_args(int(op["layer"]), None)
        M = q.shape[0]
        qd = _up(q, np.int8)
        out = _t().empty((M, H * D), dtype=_t().int8, device=self.device)
        _lib.call("llhip_attention", _ptr(qd), M, H, Hkv, D, q.shape[1], pos, None, None, 0, kcp, vcp, self.max_seq,
                  int(op["Ms"]), int(op["Ss"]), int(op["Mo"]), int(op["So"]), int(op.get("prob_bits", 8)), _ptr(out),
                  H * D, _ptr(self._ws), _stream())
        return _down(out).astype(I64)

    # ---- host side --------------------------------------------------------------------------
    def _token_rows(self, tokens) -> np.ndarray:
        """Embedding row of each token id, numpy indexing rules (golden.py:369-373 indexes the table
        with the ids: negative ids count from the end, out-of-range ids raise IndexError)."""
        n = self.embed.shape[0]
        arr = np.asarray(tokens)
        if arr.dtype.kind == "u" and arr.size and int(arr.max()) >= n:
            bad_u = arr.reshape(-1) >= n
            raise IndexError(f"index {int(arr.reshape(-1)[int(np.argmax(bad_u))])} is out of bounds for axis 0 with size {n}")
        if arr.dtype.kind in "iu":
            a = arr.astype(np.int64).reshape(-1)
        else:  # Python ints of any size, or values int() accepts
            try:
                a = np.asarray([int(t) for t in tokens], dtype=np.int64)
            except OverflowError:  # an id beyond int64: report it as numpy would
                for t in tokens:
                    if not -n <= int(t) < n:
                        raise IndexError(f"index {int(t)} is out of bounds for axis 0 with size {n}") from None
                raise
        bad = (a < -n) | (a >= n)
        if bad.any():
            raise IndexError(f"index {int(a[int(np.argmax(bad))])} is out of bounds for axis 0 with size {n}")
        return (a % n).astype(np.int32)

    def embed_rows(self, tokens, M: int) -> np.ndarray:
        """Embedding rows of `tokens`, zero pad rows up to M (golden.py:369-373)."""
        idx = self._token_rows(tokens)
        if len(idx) > M:
            raise ValueError(f"{len(idx)} tokens do not fit {M} rows")
        torch = _t()
        out = torch.empty((M, self.dim), dtype=torch.int16, device=self.device)
        td = _up(idx if len(idx) else np.zeros(1, np.int32), np.int32)
        _lib.call("llhip_embed_rows", _ptr(self._dt["embed"]), self.embed.shape[0], self.dim, _ptr(td), len(idx), M,
                  _ptr(out), _stream())
        return _down(out).astype(I64)

    @staticmethod
    def argmax(logits_row: np.ndarray, vocab: int) -> int:
        """First maximum over the first `vocab` logits (golden.py:376-377)."""
        row = np.asarray(logits_row, dtype=I64)[:vocab]
        if row.size == 0:
            raise ValueError("attempt to get argmax of an empty sequence")
        _check_range(row, -32768, 32767, "logits")
        d = _up(row[None, :], np.int16)
        idx = _t().empty(1, dtype=_t().int32, device=_dev())
        _lib.call("llhip_argmax_i16", _ptr(d), 1, row.size, row.size, _ptr(idx), _stream())
        return int(_down(idx)[0])

    def _launch_tokens(self, tokens, pos: int, M: int) -> None:
        """Embedding gather on the device + one launch (rows stay resident)."""
        idx = self._token_rows(tokens)
        if pos < 0 or pos + M > self.max_seq:
            raise ValueError(f"positions {pos}..{pos + M - 1} exceed max_seq={self.max_seq}")
        self._ensure_capacity(M)
        td = _up(idx if len(idx) else np.zeros(1, np.int32), np.int32)
        _lib.call("llhip_embed_rows", _ptr(self._dt["embed"]), self.embed.shape[0], self.dim, _ptr(td), len(idx), M,
                  _ptr(self._act[self.q.input_name]), _stream())
        self._execute(M, int(pos))

    PF_GRAPHS = 16  # whole-prompt prefill graphs kept (oldest dropped first)

    def _prefill_launch(self, tokens, M: int) -> None:
        """The whole-prompt prefill launch of `tokens` padded to M rows at positions 0..M-1.  Its
        ~300 kernel launches are enqueued by the host in about as long as the GPU runs them, so
        the second prefill of a (rows, prompt length, KV slot) shape captures them in a HIP graph
        and every later one replays it, after copying the token ids into the graph's buffer."""
        self._lean = True  # no activation is collected here: dead intermediates go unwritten
        try:
            self._prefill_launch_rows(tokens, M)
        finally:
            self._lean = False

    def _prefill_launch_rows(self, tokens, M: int) -> None:
        key = (M, len(tokens), self._slot)
        if not self.use_graph:
            self._launch_tokens(tokens, 0, M)
            return
        torch = _t()
        idx = self._token_rows(tokens)
        self._ensure_capacity(M)
        g = self._pf_graphs.get(key)
        if g is None:
            self._pf_seen[key] = self._pf_seen.get(key, 0) + 1
            if self._pf_seen[key] < 2:
                self._launch_tokens(tokens, 0, M)
                return
            tok = torch.zeros(max(len(idx), 1), dtype=torch.int32, device=self.device)
            graph = torch.cuda.CUDAGraph()
            with capture_graph(graph):
                _lib.call("llhip_embed_rows", _ptr(self._dt["embed"]), self.embed.shape[0], self.dim, _ptr(tok),
                          len(idx), M, _ptr(self._act[self.q.input_name]), _stream())
                self._execute(M, 0)
            while len(self._pf_graphs) >= self.PF_GRAPHS:
                self._pf_graphs.pop(next(iter(self._pf_graphs)))
            g = self._pf_graphs[key] = (graph, tok)
        graph, tok = g
        if len(idx):
            tok.copy_(torch.from_numpy(np.ascontiguousarray(idx, dtype=np.int32)), non_blocking=False)
        graph.replay()

    # ---- device-resident greedy decode ----------------------------------------------------
    def _decode_state(self, ring_cap: int) -> None:
        torch = _t()
        if ring_cap > self._ring_cap:
            cap = max(ring_cap, 64)
            self._ring_rows = torch.zeros((cap, self.vocab), dtype=torch.int16, device=self.device)
            self._ring_tok = torch.zeros(cap, dtype=torch.int32, device=self.device)
            self._ring_cap = cap
            self._graph = None
        if not hasattr(self, "_st"):
            self._st = torch.zeros(3, dtype=torch.int32, device=self.device)  # token, pos, step

    def _decode_launch(self) -> None:
        """One greedy decode launch at the device position.  Fused plan: embedding gather of the
        device token, the op list, greedy step.  Decode chain: the layers, the head and the greedy
        step, which also gathers the next launch's input row (the first one is gathered by
        decode_loop)."""
        st = self._st
        tok, pos, step = (ctypes.c_void_p(st.data_ptr() + 4 * i) for i in range(3))
        if self._chained(1):
            self._chain.run(0, pos, greedy=(tok, pos, step, _ptr(self._ring_rows), self.vocab, _ptr(self._ring_tok),
                                            self._ring_cap))
            return
        _lib.call("llhip_embed_rows", _ptr(self._dt["embed"]), self.embed.shape[0], self.dim, tok, 1, 1,
                  _ptr(self._act[self.q.input_name]), _stream())
        self._execute(1, 0, pos)
        _lib.call("llhip_greedy_step", _ptr(self._act[self.q.output_name]), self.vocab, tok, pos, step,
                  _ptr(self._ring_rows), self.vocab, _ptr(self._ring_tok), self._ring_cap, _ptr(self._ws), _stream())

    def _capture(self) -> None:
        """The decode graphs: one launch, and DECODE_GRAPH_STEPS launches in a row (each launch reads
        and advances the device position and step, so the copies run consecutive positions; one
        replay of the run graph instead of several saves the gaps between replays)."""
        torch = _t()
        g = torch.cuda.CUDAGraph()
        with capture_graph(g):
            self._decode_launch()
        run = torch.cuda.CUDAGraph()
        with capture_graph(run):
            for _ in range(DECODE_GRAPH_STEPS):
                self._decode_launch()
        self._graph, self._graph_run = g, run
        self._graph_chained = self._graph_key()

    def _graph_key(self):
        """What a captured decode graph depends on: the chain, and the decode step it launched."""
        ch = self._chain if self._chained(1) else None
        return (ch is not None, ch._step if ch is not None and ch.use_step else None)

    def decode_loop(self, token: int, pos: int, n: int, *, sync: bool = True):
        """Run `n` greedy M=1 decode launches from (token, pos) entirely on the device.

        Launch i decodes at pos + i; its argmax feeds launch i + 1.  Returns the n argmax tokens
        and the n recorded logits rows ([n][vocab] int16) -- the decode part of the golden.json
        record.  With `use_graph` each launch is one replay of a captured HIP graph.  With
        sync=False the device ring keeps its capacity (at least 64 launches) when that is smaller
        than n: the later launches run but are not recorded, and no graph is captured again."""
        if n <= 0:
            return np.zeros(0, np.int64), np.zeros((0, self.vocab), np.int16)
        if pos < 0 or pos + n > self.max_seq:
            raise ValueError(f"positions {pos}..{pos + n - 1} exceed max_seq={self.max_seq}")
        torch = _t()
        self._decode_state(n if sync else min(n, max(self._ring_cap, 64)))
        self._st.copy_(torch.tensor([int(self._token_rows([token])[0]), pos, 0], dtype=torch.int32))
        if self._chained(1):  # the chain's launches gather their next input row themselves
            _lib.call("llhip_embed_rows", _ptr(self._dt["embed"]), self.embed.shape[0], self.dim,
                      ctypes.c_void_p(self._st.data_ptr()), 1, 1, _ptr(self._act[self.q.input_name]), _stream())
        if self._chained(1):  # the decode step's handle and the head's panel are made outside any capture
            self._chain.step(ctypes.c_void_p(self._st.data_ptr() + 4))
            self._chain.prepare_head()
        if self.use_graph and (self._graph is None or self._graph_chained != self._graph_key()):
            self._capture()
        if self.use_graph:
            for _ in range(n // DECODE_GRAPH_STEPS):
                self._graph_run.replay()
            for _ in range(n % DECODE_GRAPH_STEPS):
                self._graph.replay()
        else:
            for _ in range(n):
                self._decode_launch()
        if not sync:
            return None
        if self._chained(1):
            self._chain.check_step()
        return _down(self._ring_tok[:n]).astype(np.int64), self._ring_rows[:n].cpu().numpy()

    def decode_ring(self, n: int):
        """Device tensors of the last decode_loop's record (valid until the next one): the argmax
        tokens (int32 [n]) and logits rows (int16 [n][vocab]) -- for checks on the device
        (llaccel_amd.verify.first_mismatch / row_checksums) without downloading the rows."""
        if not 0 <= n <= self._ring_cap:
            raise ValueError(f"the decode ring holds {self._ring_cap} steps")
        return self._ring_tok[:n], self._ring_rows[:n]

    # ---- batch decode: B independent sequences, one per row -------------------------------
    def _batch_state(self, B: int, ring_cap: int) -> None:
        torch = _t()
        if self._kv and next(iter(self._kv.values()))[0].shape[0] < B:
            raise ValueError(f"{B} sequences need {B} KV slots (generate_batch allocates them)")
        if getattr(self, "_b_rows", None) != B or ring_cap > self._b_cap:
            cap = max(ring_cap, 64)
            self._b_ring_rows = torch.zeros((cap, B, self.vocab), dtype=torch.int16, device=self.device)
            self._b_ring_tok = torch.zeros((cap, B), dtype=torch.int32, device=self.device)
            self._b_st = torch.zeros(3 * B, dtype=torch.int32, device=self.device)  # tokens, positions, base
            self._b_rows, self._b_cap = B, cap
            self._graph_b = None

    def _decode_batch_launch(self) -> None:
        """Embedding gather of the B device tokens, the op list with one sequence per row, greedy step."""
        B = self._b_rows
        st = self._b_st
        tok, posp, base = (ctypes.c_void_p(st.data_ptr() + 4 * B * i) for i in range(3))
        _lib.call("llhip_embed_rows", _ptr(self._dt["embed"]), self.embed.shape[0], self.dim, tok, B, B,
                  _ptr(self._act[self.q.input_name]), _stream())
        kc0 = next(iter(self._kv.values()))[0]
        self._execute(B, 0, _RowPos(posp, kc0[0].numel()))
        out = self._act[self.q.output_name]
        _lib.call("llhip_greedy_rows", _ptr(out), B, out.shape[1], self.vocab, tok, posp, base,
                  _ptr(self._b_ring_rows), self.vocab, _ptr(self._b_ring_tok), self._b_cap, _stream())

    def decode_batch_loop(self, tokens, positions, n: int, *, sync: bool = True):
        """Run `n` greedy decode launches of B = len(tokens) sequences together: row b is sequence b,
        at position positions[b] + i in launch i, with its KV caches in slot b.  Every row is
        computed exactly as its own single-sequence decode launch.  Returns tokens [n][B] and
        logits rows [n][B][vocab].  With sync=False the ring keeps its capacity (at least 64
        launches), as in decode_loop."""
        B = len(tokens)
        if B < 1 or len(positions) != B:
            raise ValueError("tokens and positions must be nonempty and of equal length")
        if n <= 0:
            return np.zeros((0, B), np.int64), np.zeros((0, B, self.vocab), np.int16)
        pos = [int(p) for p in positions]
        if min(pos) < 0 or max(pos) + n > self.max_seq:
            raise ValueError(f"positions up to {max(pos) + n - 1} exceed max_seq={self.max_seq}")
        torch = _t()
        self._ensure_capacity(B)
        self._batch_state(B, n if sync else min(n, max(getattr(self, "_b_cap", 0), 64)))
        idx = [int(t) for t in self._token_rows(tokens)]
        self._b_st.copy_(torch.tensor(idx + pos + pos, dtype=torch.int32))
        if self.use_graph and self._graph_b is None:
            g = torch.cuda.CUDAGraph()
            with capture_graph(g):
                self._decode_batch_launch()
            self._graph_b = g
        for _ in range(n):
            if self.use_graph:
                self._graph_b.replay()
            else:
                self._decode_batch_launch()
        if not sync:
            return None
        return (_down(self._b_ring_tok[:n]).astype(np.int64), self._b_ring_rows[:n].cpu().numpy())

    def prefill_batch(self, prompts) -> list[Sequence]:
        """Reallocate the KV caches with B = len(prompts) slots and prefill prompt b into slot b
        (golden.py:379-390 per prompt); returns each prompt's prefill logits rows.

        Prompts of one length run as ONE launch of B x padded rows: sequence b's rows (its prompt,
        then the zero pad rows of its last chunk) at positions 0.. in slot b, each row seeing only
        its own sequence's keys -- the whole-prompt prefill of every prompt at once, so the logits
        and the KV state equal B separate prefill() calls (a GPU test checks it), with the GEMMs at
        M = B x padded rows.  Otherwise (other lengths, a graph with unfused rope or kv_write ops)
        one prefill() per prompt."""
        prompts = [[int(t) for t in p] for p in prompts]
        self._alloc_kv(len(prompts))
        B = len(prompts)
        L = len(prompts[0]) if prompts else 0
        Lp = -(-L // self.prefill_m) * self.prefill_m
        if (B > 1 and L > self.prefill_m and all(len(p) == L for p in prompts) and self.whole_prompt_prefill
                and Lp % 16 == 0 and Lp <= self.max_seq
                and not any(st.kind in ("rope", "kv_write") for st in self._plan)):
            rows = self._prefill_seqs(prompts, Lp)
            return [DeviceRows(rows[b * Lp:b * Lp + L]) for b in range(B)]
        out = []
        for b, p in enumerate(prompts):
            self._slot = b
            out.append(self.prefill(p))
        self._slot = 0
        return out

    def _prefill_seqs(self, prompts, Lp: int):
        """The one-launch batch prefill: embedding gathers of every prompt into its Lp rows (pad rows
        zero), then the op list over B x Lp rows in the sequence-major position context.  Returns the
        B x Lp logits rows: a buffer of their own that the lm_head writes directly (no device copy of
        the B x Lp x vocab rows; this launch is not captured, so the output buffer may change)."""
        torch = _t()
        B = len(prompts)
        M = B * Lp
        self._ensure_capacity(M)
        x = self._act[self.q.input_name]
        # every prompt's token rows in one upload (alive until the gathers ran); prompts that fill
        # their Lp rows exactly are gathered by one launch, else one launch per prompt pads its rows
        L = len(prompts[0])
        toks = _up(np.concatenate([self._token_rows(p) for p in prompts]), np.int32)
        if L == Lp:
            _lib.call("llhip_embed_rows", _ptr(self._dt["embed"]), self.embed.shape[0], self.dim, _ptr(toks), M, M,
                      _ptr(x), _stream())
        else:
            for b in range(B):
                _lib.call("llhip_embed_rows", _ptr(self._dt["embed"]), self.embed.shape[0], self.dim,
                          ctypes.c_void_p(toks.data_ptr() + 4 * b * L), L, Lp, _ptr(x[b * Lp]), _stream())
        kc0 = next(iter(self._kv.values()))[0]
        out_name = self.q.output_name
        shared = self._act[out_name]
        rows = torch.empty((M, shared.shape[1]), dtype=shared.dtype, device=self.device)
        self._act[out_name] = rows
        self._lean = True  # no activation is collected: dead intermediates go unwritten
        try:
            self._execute(M, 0, _SeqRows(Lp, kc0[0].numel()))
        finally:
            self._lean = False
            self._act[out_name] = shared
        # freed in stream order: the caching allocator reuses the token buffers only after the gathers
        del toks
        return rows

    def generate_batch(self, prompts, n_tokens: int) -> list[dict]:
        """Greedy generation of B = len(prompts) independent sequences of one prompt length: each
        prompt is prefilled into its own KV-cache slot, then every decode launch runs the B
        sequences together as B rows.  Record b equals generate(prompts[b], n_tokens) run alone
        (the same golden.json record).  Reallocates the KV caches with B slots."""
        if not isinstance(n_tokens, int) or n_tokens < 0:
            raise ValueError("n_tokens must be a nonnegative integer")
        prompts = [[int(t) for t in p] for p in prompts]
        if not prompts or any(not p for p in prompts):
            raise ValueError("empty prompt")
        L = len(prompts[0])
        if any(len(p) != L for p in prompts):
            raise ValueError("generate_batch needs prompts of one length")
        if L + n_tokens > self.max_seq:
            raise ValueError(f"prompt + tokens = {L + n_tokens} exceeds max_seq={self.max_seq}")
        B = len(prompts)
        recs = [self._chunk_records(rows, L) for rows in self.prefill_batch(prompts)]
        nxt = [argm[-1] for _, argm, _ in recs]
        n_dec = min(n_tokens, self.max_seq - L - 1)
        toks = rows_dev = None
        if n_dec > 0:
            toks, rows_dev = self.decode_batch_loop(nxt, [L] * B, n_dec)
        out = []
        for b, (steps, argm, lrows) in enumerate(recs):
            generated, cur = [], nxt[b]
            for i in range(n_tokens):
                generated.append(cur)
                if L + i + 1 >= self.max_seq:
                    break
                steps.append({"kind": "decode", "pos": L + i, "rows": 1, "valid_rows": 1})
                argm.append(int(toks[i][b]))
                lrows.append(rows_dev[i][b].tolist())
                cur = int(toks[i][b])
            out.append({"prompt_tokens": prompts[b], "generated": generated, "argmax_per_step": argm,
                        "logits_last_rows": lrows, "steps": steps,
                        "model": {"vocab": self.vocab, "vocab_padded": self.vocab_padded, "E_LOGIT": self.E_LOGIT,
                                  "E_RES": self.E_RES, "max_seq": self.max_seq}})
        return out

    # ---- measurement aids ------------------------------------------------------------------
    def capture_steps(self, kinds, pos: int):
        """HIP graph of the M=1 launches of the plan steps whose kind is in `kinds`, reading the
        position from the device decode state (set to `pos`).  Used to time kernel families."""
        torch = _t()
        self._decode_state(1)
        self._st.copy_(torch.tensor([0, pos, 0], dtype=torch.int32))
        pd = ctypes.c_void_p(self._st.data_ptr() + 4)
        g = torch.cuda.CUDAGraph()
        with capture_graph(g):
            for st in self._plan:
                if st.kind in kinds:
                    st(1, 0, pd)
        return g

    def step_bytes(self, kind: str, M: int = 1, T: int = 1) -> int:
        """Algorithmic HBM bytes of all plan steps of `kind` for one launch of M rows at context T."""
        total = 0
        for st in self._plan:
            if st.kind != kind or st.bytes_fn is None:
                continue
            total += st.bytes_fn(M, T) if kind == "attention" else st.bytes_fn(M)
        return total

    def count_steps(self, kind: str) -> int:
        return sum(1 for st in self._plan if st.kind == kind)

    def _chunk_records(self, rows, L: int) -> tuple[list, list, list]:
        """The prefill part of the launch record (golden.py:411-431): one entry per prompt chunk, its
        argmax and logits row taken from row (L - 1) mod prefill_m of the last chunk and row
        prefill_m - 1 of the others.  Rows still on the device are gathered there, their argmax
        computed there and only those rows downloaded."""
        P = self.prefill_m
        lasts = [min(L, (c + 1) * P) - 1 for c in range(math.ceil(L / P))]
        steps = [{"kind": "prefill", "pos": c * P, "rows": P, "valid_rows": last + 1 - c * P}
                 for c, last in enumerate(lasts)]
        if isinstance(rows, DeviceRows):
            torch = _t()
            sel = rows._rows[torch.tensor(lasts, device=self.device)]
            idx = torch.empty(len(lasts), dtype=torch.int32, device=self.device)
            _lib.call("llhip_argmax_i16", _ptr(sel), len(lasts), sel.shape[1], self.vocab, _ptr(idx), _stream())
            return steps, [int(v) for v in idx.cpu()], sel[:, :self.vocab].cpu().numpy().tolist()
        return (steps, [self.argmax(rows[i], self.vocab) for i in lasts],
                [[int(v) for v in rows[i][:self.vocab]] for i in lasts])

    def prefill(self, tokens, acts: list | None = None) -> Sequence:
        """Prefill with the launch structure of golden.py:379-390 (chunks of prefill_m rows).

        Without `acts` (and with `whole_prompt_prefill`) the chunks run as ONE launch of all
        ceil(L/prefill_m)*prefill_m rows at positions 0..: every row depends only on itself and
        on keys at earlier positions, and the zero pad rows of the last chunk sit at the same
        positions as in the chunked run, so logits and the KV state are identical (a GPU test
        checks it) while the GEMMs run at M = padded prompt length on the MFMA tiled kernel.  That
        path returns the rows as a DeviceRows sequence (each row an int64 array when read), the
        chunked one as a list."""
        tokens = [int(t) for t in tokens]
        L = len(tokens)
        padded = -(-L // self.prefill_m) * self.prefill_m
        if acts is None and self.whole_prompt_prefill and L > self.prefill_m and padded <= self.max_seq:
            self._prefill_launch(tokens, padded)
            # a device copy of the L rows; each row crosses to the host when it is read
            return DeviceRows(self._act[self.q.output_name][:L].clone())
        rows_out = []
        for start in range(0, len(tokens), self.prefill_m):
            chunk = tokens[start:start + self.prefill_m]
            self._launch_tokens(chunk, start, self.prefill_m)
            if acts is not None:
                acts.append({"kind": "prefill", "pos": start, "rows": self.prefill_m, "valid_rows": len(chunk),
                             "acts": self._collect(self.prefill_m)})
            logits = _down(self._act[self.q.output_name][:len(chunk)]).astype(I64)
            rows_out.extend(logits)
        return rows_out

    def decode(self, token: int, pos: int, acts: list | None = None) -> np.ndarray:
        """One M=1 launch (golden.py:392-397)."""
        self._launch_tokens([token], pos, 1)
        if acts is not None:
            acts.append({"kind": "decode", "pos": pos, "rows": 1, "valid_rows": 1, "acts": self._collect(1)})
        return _down(self._act[self.q.output_name][0]).astype(I64)

    def generate(self, prompt_tokens, n_tokens: int, acts: list | None = None) -> dict:
        """Greedy generation with the launch sequence of golden.py:399-440; returns the golden.json record."""
        if not isinstance(n_tokens, int) or n_tokens < 0:
            raise ValueError("n_tokens must be a nonnegative integer")
        prompt_tokens = [int(t) for t in prompt_tokens]
        if not prompt_tokens:
            raise ValueError("empty prompt")
        if len(prompt_tokens) + n_tokens > self.max_seq:
            raise ValueError(f"prompt + tokens = {len(prompt_tokens) + n_tokens} exceeds max_seq={self.max_seq}")
        self.reset()

        def record(kind: str, pos: int, valid: int, row: np.ndarray) -> int:
            steps.append({"kind": kind, "pos": pos, "rows": self.prefill_m if kind == "prefill" else 1,
                          "valid_rows": valid})
            argmax_per_step.append(self.argmax(row, self.vocab))
            logits_rows.append([int(v) for v in row[:self.vocab]])
            return argmax_per_step[-1]

        L = len(prompt_tokens)
        steps, argmax_per_step, logits_rows = self._chunk_records(self.prefill(prompt_tokens, acts), L)
        nxt = argmax_per_step[-1]
        generated: list[int] = []
        n_dec = min(n_tokens, self.max_seq - L - 1)
        if acts is None and self.use_graph and n_dec > 0:
            # device-resident decode: one captured graph per launch, the record kept in a device ring
            toks, rows_dev = self.decode_loop(nxt, L, n_dec)
            for i in range(n_tokens):
                generated.append(nxt)
                if L + i + 1 >= self.max_seq:
                    break
                steps.append({"kind": "decode", "pos": L + i, "rows": 1, "valid_rows": 1})
                argmax_per_step.append(int(toks[i]))
                logits_rows.append(rows_dev[i].tolist())
                nxt = int(toks[i])
        else:
            for i in range(n_tokens):
                generated.append(nxt)
                if L + i + 1 >= self.max_seq:
                    break
                nxt = record("decode", L + i, 1, self.decode(nxt, L + i, acts))
        return {"prompt_tokens": prompt_tokens, "generated": generated, "argmax_per_step": argmax_per_step,
                "logits_last_rows": logits_rows, "steps": steps,
                "model": {"vocab": self.vocab, "vocab_padded": self.vocab_padded, "E_LOGIT": self.E_LOGIT,
                          "E_RES": self.E_RES, "max_seq": self.max_seq}}


class DeviceRows(Sequence):
    """The logits rows of a whole-prompt prefill, kept on the device: row i is an int64 numpy array
    (the values golden.py:379-390 returns), downloaded when it is read.  Callers that read a few
    rows -- generate() reads one per prompt chunk -- move a few rows instead of L x vocab_padded
    values; `numpy()` downloads them all at once."""

    def __init__(self, rows) -> None:
        self._rows = rows  # int16 [L][vocab_padded] device tensor owned by this object

    def __len__(self) -> int:
        return int(self._rows.shape[0])

    def __getitem__(self, i):
        if isinstance(i, slice):
            return list(self.numpy()[i])
        n = len(self)
        i = int(i)
        if not -n <= i < n:
            raise IndexError("prefill row index out of range")
        return self._rows[i].cpu().numpy().astype(I64)

    def numpy(self) -> np.ndarray:
        """All rows as one int64 [L][vocab_padded] array."""
        return self._rows.cpu().numpy().astype(I64)


def dump_acts(acts: list, out_dir: Path) -> int:
    """step{i:03d}_{kind}_pos{P}_{name}.npy as int32 for every activation (golden.py:443-450)."""
    out_dir = Path(out_dir)
    out_dir.mkdir(parents=True, exist_ok=True)
    n = 0
    for i, step in enumerate(acts):
        for name, arr in step["acts"].items():
            np.save(out_dir / f"step{i:03d}_{step['kind']}_pos{step['pos']}_{name}.npy", np.asarray(arr).astype(np.int32))
            n += 1
    return n


def main(argv=None) -> None:
    """CLI of golden.py:453-477.  A char-level tokenizer.json ({"itos": [...]}) next to the qgraph
    is used as in the reference; --prompt-ids bypasses it with explicit token ids."""
    ap = argparse.ArgumentParser(description="GPU golden model (integer datapath on MI355X)")
    ap.add_argument("--qgraph", required=True)
    ap.add_argument("--prompt", default="ROMEO:")
    ap.add_argument("--prompt-ids", default=None, help="comma-separated token ids (instead of --prompt)")
    ap.add_argument("--tokens", type=int, default=64)
    ap.add_argument("--tokenizer", default=None, help="tokenizer.json (default: <qgraph>/tokenizer.json)")
    ap.add_argument("-o", "--out", default="build/golden.json")
    ap.add_argument("--dump-acts", default=None)
    args = ap.parse_args(argv)
    itos = None
    if args.prompt_ids is not None:
        prompt = [int(t) for t in args.prompt_ids.split(",") if t.strip()]
    else:
        tok_path = Path(args.tokenizer) if args.tokenizer else Path(args.qgraph) / "tokenizer.json"
        itos = json.loads(Path(tok_path).read_text())["itos"]
        stoi = {c: i for i, c in enumerate(itos)}
        prompt = [stoi[c] for c in args.prompt]
    g = GoldenModel(args.qgraph)
    acts = [] if args.dump_acts else None
    rec = g.generate(prompt, args.tokens, acts)
    if itos is not None:
        rec["prompt"] = args.prompt
        rec["text"] = "".join(itos[t] for t in rec["generated"])
    Path(args.out).parent.mkdir(parents=True, exist_ok=True)
    with open(args.out, "w") as f:
        json.dump(rec, f)
    print(f"wrote {args.out}: {len(rec['steps'])} launches, {len(rec['generated'])} tokens")
    if itos is not None:
        print(args.prompt + rec["text"])
    if acts is not None:
        n = dump_acts(acts, Path(args.dump_acts))
        print(f"dumped {n} activation arrays to {args.dump_acts}")


if __name__ == "__main__":
    main()
