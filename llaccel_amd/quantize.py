"""qgraph producer: a model export directory -> qgraph.json + qweights.bin, the datapath's input.

The contract is the reference quantizer's (python/llaccel/refquant.py): the same export directory
gives the same op list, tensor names, integer parameters and blob bytes (tests/golden/refquant/
holds graphs the reference wrote; tests/test_quantize.py and tests/test_gpu_quantize.py compare).
What is fixed by that contract is kept: the parameter formulas of docs/NUMERICS.md's "Compiler:"
lines (refquant.py:89-241), the op order of a decoder layer (refquant.py:403-490), the tensor
names, the blob layout (refquant.py:244-270) and the error messages.  One extension: head_dim 128
and 256 are accepted (refquant.py:411 stops at 64), with Q/K RMSNorm.

The design here is a data pipeline rather than an emitter class:

* `Formats` picks every activation's number format from the calibration (i16 exponent or i8
  scale; the first choice of a name is final, ties are explicit);
* `LAYER_TEMPLATE` lists a decoder layer's steps as data, `Graph` expands it per layer and
  writes the op dicts, each step kind one small function in `STEP_KINDS`;
* `Pack` owns qweights.bin: weight matrices are converted on the GPU (`llhip_quant_rows_i8`:
  int8 rows and their scales; `llhip_quant_i16` for the embedding and gammas) as they are
  packed; requant pairs and biases follow from the returned scales in float64 numpy.

    python -m llaccel_amd.quantize EXPORT_DIR -o OUT_DIR [--fusion]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import re
from pathlib import Path

import numpy as np

from . import _lib

INT32_MIN, INT32_MAX = -(2**31), 2**31 - 1
HEAD_DIMS = (16, 32, 64, 128, 256)


# ---- rounding and multiplier pairs -----------------------------------------------------------
def llround(x: float) -> int:
    """The C library's llround (refquant.py:61-72): nearest integer, halves away from zero."""
    x = float(x)
    if not math.isfinite(x):
        raise ValueError(f"llround of {x}")
    whole, part = divmod(abs(x), 1.0)  # float divmod by 1 is exact
    n = int(whole) + (part >= 0.5)
    return n if x >= 0 else -n


def llround_vec(x) -> np.ndarray:
    """llround of every element (refquant.py:75-86); finite values below 2^63 only."""
    a = np.asarray(x, dtype=np.float64)
    if not np.isfinite(a).all():
        raise ValueError("llround of a non-finite value")
    if (np.abs(a) >= 2.0**63).any():
        raise ValueError("llround input exceeds int64 range")
    mag = np.abs(a)
    whole = np.floor(mag)
    n = whole.astype(np.int64) + (mag - whole >= 0.5)  # mag - whole is exact
    return np.where(a < 0, -n, n)


def mulshift_pairs(r) -> tuple[np.ndarray, np.ndarray]:
    """(M, S) with M * 2^-S ~= r (refquant.py:89-104): M is the frexp mantissa of r rounded to 31
    bits, so M is in [2^30, 2^31); a mantissa rounding up to 2^31 becomes 2^30 with S one lower;
    S past 63 is held at 63 with M = llround(r * 2^63)."""
    r = np.asarray(r, dtype=np.float64)
    if not (np.isfinite(r).all() and (r > 0.0).all()):
        raise ValueError("normalize_mulshift: ratio must be positive and finite")
    mant, ex = np.frexp(r)
    M = llround_vec(np.ldexp(mant, 31))
    S = 31 - ex.astype(np.int64)
    carried = M == 1 << 31
    M, S = np.where(carried, 1 << 30, M), np.where(carried, S - 1, S)
    if (S < 0).any():
        raise ValueError(f"normalize_mulshift: ratio {float(r[S < 0][0])} too large (S < 0)")
    pinned = S > 63
    if pinned.any():
        M = np.where(pinned, llround_vec(np.where(pinned, np.ldexp(r, 63), 0.0)), M)
        S = np.minimum(S, 63)
    return M.astype(np.int64), S.astype(np.int64)


def mulshift_pair(r: float) -> tuple[int, int]:
    M, S = mulshift_pairs([r])
    return int(M[0]), int(S[0])


# ---- number formats and per-op parameters (NUMERICS.md "Compiler:" lines) ---------------------
def i16_exponent(absmax: float) -> int:
    """e = max(ceil(log2(absmax / 32767)), -15) (refquant.py:107-111)."""
    return max(int(math.ceil(math.log2(absmax) - math.log2(32767.0))), -15) if absmax > 0.0 else -15


def i8_scale(absmax: float) -> float:
    """s = absmax / 127, 1 for an all-zero tensor (refquant.py:114-116)."""
    return absmax / 127.0 if absmax > 0.0 else 1.0


def gemm_rq_rows(s_a: float, s_w: np.ndarray, out_i8: bool, e_out: int, s_out: float) -> np.ndarray:
    """Per-output-channel requant pairs (refquant.py:143-146): s_a * s_w[n] over s_out (i8 output)
    or 2^e_out (i16 output), as int32 [N][2]."""
    target = s_out if out_i8 else math.ldexp(1.0, int(e_out))
    return np.column_stack(mulshift_pairs(s_a * np.asarray(s_w, dtype=np.float64) / target))


def gemm_bias_rows(b: np.ndarray, s_a: float, s_w: np.ndarray) -> np.ndarray:
    """i32 bias per output channel (refquant.py:149-151): llround(b / (s_a * s_w[n])) clamped."""
    with np.errstate(divide="ignore", over="ignore", invalid="ignore"):
        x = np.asarray(b, dtype=np.float64) / (s_a * np.asarray(s_w, dtype=np.float64))
    if not np.isfinite(x).all():
        raise ValueError("gemm bias: non-finite quotient")
    # beyond +-2^40 the result is the clamp either way; bounding first keeps llround in int64
    return np.clip(llround_vec(np.clip(x, -(2.0**40), 2.0**40)), INT32_MIN, INT32_MAX).astype(np.int32)


def quant_params(e_x: int, s_y: float) -> tuple[int, int]:
    """QUANT i16 -> i8 (refquant.py:154-156): M * 2^-S ~= 2^e_x / s_y."""
    return mulshift_pair(math.ldexp(1.0, int(e_x)) / s_y)


def _rms_shift(K: int, r_typ: float) -> tuple[int, int]:
    """(R, C): the largest R <= 31 whose C = llround(2^R sqrt K) fits u32 and keeps C / r_typ
    below 65535 / 4 (refquant.py:177-183); None when no R does."""
    root = math.sqrt(float(K))
    feasible = ((R, llround(math.ldexp(root, R))) for R in range(31, -1, -1))
    return next(((R, C) for R, C in feasible if C < 2**32 and math.floor(C / r_typ) < 65535.0 / 4.0), None)


def rmsnorm_params(K: int, eps: float, e_x: int, e_g: int, e_y: int, absmax_x: float, name: str,
                   rms_min: float | None = None) -> dict:
    """RMSNorm parameters (refquant.py:159-186): eps_t = llround(eps K 2^-2e_x); the typical row
    inverse uses rms_min when the calibration has it, else absmax/4; sh_post = R - e_g + e_y."""
    if rms_min is not None and not (math.isfinite(rms_min) and 0 <= rms_min <= absmax_x):
        raise ValueError(f"rmsnorm {name}: rms_min must be finite and in [0, absmax]")
    eps_t = llround(eps * float(K) * math.ldexp(1.0, -2 * int(e_x)))
    if not 0 <= eps_t < 2**32:
        raise ValueError(f"rmsnorm {name}: eps_t does not fit the ISA u32 operand")
    rms = (absmax_x / 4.0 if rms_min is None else rms_min) / math.ldexp(1.0, int(e_x))
    picked = _rms_shift(K, max(1.0, math.floor(math.sqrt(float(K) * rms * rms + float(eps_t)))))
    if picked is None:
        raise ValueError(f"rmsnorm {name}: no R in [0,31] keeps inv below 65535/4 "
                         f"(input abs-max {absmax_x} too small for e_x)")
    R, C = picked
    sh_post = R - e_g + e_y
    if not 0 <= sh_post <= 63:
        raise ValueError(f"rmsnorm {name}: sh_post = {sh_post} outside [0, 63]")
    return {"eps_t": eps_t, "C": C, "R": R, "sh_post": sh_post}


def _shift(value: int, what: str) -> int:
    if not 0 <= value <= 63:
        raise ValueError(f"{what} = {value} outside [0, 63]")
    return value


def silu_params(e_x: int, e_y: int, name: str) -> dict:
    """SiLU (refquant.py:189-196): Mi = 2^30, Si = 18 - e_x, sh_out = 16 + e_y - e_x."""
    return {"Mi": 1 << 30, "Si": _shift(30 - (e_x + 12), f"silu {name}: Si"),
            "sh_out": _shift(16 + e_y - e_x, f"silu {name}: sh_out")}


def mul_shift(e_a: int, e_b: int, e_y: int, name: str) -> int:
    """MUL (refquant.py:199-209): the product's exponent e_a + e_b brought to e_y."""
    return _shift(e_y - e_a - e_b, f"mul {name}: sh")


def add_shift(e_a: int, e_b: int, name: str) -> int:
    """ADD (refquant.py:212-218): b brought to a's (coarser) exponent."""
    sh = e_a - e_b
    if not 0 <= sh <= 63:
        raise ValueError(f"add {name}: sh_b = {sh} outside [0, 63] (b must not have a larger exponent than a)")
    return sh


def attn_params(s_q: float, s_k: float, s_v: float, s_out: float, D: int) -> dict:
    """Attention (refquant.py:221-224): the score scale 256 s_q s_k / sqrt(D), the output scale
    s_v / (256 s_out)."""
    (Ms, Ss), (Mo, So) = mulshift_pair(256.0 * s_q * s_k / math.sqrt(float(D))), mulshift_pair(s_v / (256.0 * s_out))
    return {"Ms": Ms, "Ss": Ss, "Mo": Mo, "So": So}


def rope_tables(max_seq: int, D: int, base: float) -> tuple[np.ndarray, np.ndarray]:
    """Q1.14 RoPE tables [max_seq][D/2] (refquant.py:227-238): the angle of position p and pair i is
    p * base^(-2i/D); values are llround(16384 cos), llround(16384 sin) capped at 32767, with the C
    library's cos and sin per element."""
    freqs = [math.pow(base, -2.0 * float(i) / float(D)) for i in range(D // 2)]

    def q14(v: float) -> int:
        return min(llround(16384.0 * v), 32767)

    angles = [[float(p) * f for f in freqs] for p in range(max_seq)]
    cos_t = np.array([[q14(math.cos(a)) for a in row] for row in angles], dtype=np.int16).reshape(max_seq, D // 2)
    sin_t = np.array([[q14(math.sin(a)) for a in row] for row in angles], dtype=np.int16).reshape(max_seq, D // 2)
    return cos_t, sin_t


# ---- device conversions ----------------------------------------------------------------------
class _Device:
    """The GPU conversions: f32 weight rows -> int8 + float64 scales, f32 values -> i16."""

    def __init__(self):
        import torch

        if not torch.cuda.is_available():
            raise RuntimeError("llaccel_amd.quantize converts weights on the GPU; no GPU is available")
        _lib.lib()  # raises LibraryNotBuilt when the HIP library is missing
        self.torch = torch
        self.status = torch.zeros(1, dtype=torch.int32, device="cuda")

    def _run(self, fn: str, what: str, *args) -> None:
        self.status.zero_()
        _lib.call(fn, *args, ctypes.c_void_p(self.status.data_ptr()),
                  ctypes.c_void_p(self.torch.cuda.current_stream().cuda_stream))
        if int(self.status.item()):
            raise ValueError(f"{what}: non-finite value")

    def rows_i8(self, w: np.ndarray, n_rows: int | None = None) -> tuple[np.ndarray, np.ndarray]:
        """int8 rows and scales of w [N][K]; rows w.shape[0] .. n_rows - 1 are zero padding."""
        t = self.torch
        w = np.require(w, dtype=np.float32, requirements=["C", "W"])  # a read-only view is copied
        N, K = (w.shape[0] if n_rows is None else int(n_rows)), w.shape[1]
        src = t.zeros((N, K), dtype=t.float32, device="cuda")
        src[: w.shape[0]].copy_(t.from_numpy(w))
        q = t.empty((N, K), dtype=t.int8, device="cuda")
        s = t.empty(N, dtype=t.float64, device="cuda")
        ptr = lambda x: ctypes.c_void_p(x.data_ptr())  # noqa: E731
        self._run("llhip_quant_rows_i8", "quant_i8", ptr(src), N, K, K, ptr(q), K, ptr(s))
        return q.cpu().numpy(), s.cpu().numpy()

    def i16(self, x: np.ndarray, e: int) -> np.ndarray:
        t = self.torch
        x = np.array(x, dtype=np.float32)  # a writable copy for torch
        src = t.from_numpy(x.reshape(-1)).cuda()
        y = t.empty(x.size, dtype=t.int16, device="cuda")
        self._run("llhip_quant_i16", "quant_i16", ctypes.c_void_p(src.data_ptr()), x.size, int(e),
                  ctypes.c_void_p(y.data_ptr()))
        return y.cpu().numpy().reshape(x.shape)


# ---- qweights.bin ----------------------------------------------------------------------------
_BLOB_TYPES = {"i8": "<i1", "i16": "<i2", "i32": "<i4", "rq": "<i4"}
BLOB_ALIGN = 64


class Pack:
    """The tensors of qweights.bin in packing order, each starting on a 64-byte boundary
    (refquant.py:244-270); weight matrices go through the device conversions as they are packed."""

    def __init__(self, device) -> None:
        self.device = device
        self.chunks: list[bytes] = []
        self.tensors: dict[str, dict] = {}
        self.size = 0

    def put(self, name: str, arr: np.ndarray, dtype: str, exp: int | None = None) -> None:
        if name in self.tensors:
            raise ValueError(f"duplicate tensor {name}")
        raw = np.asarray(arr).astype(_BLOB_TYPES[dtype]).tobytes()
        shape = arr.shape[:-1] if dtype == "rq" else arr.shape  # rq tensors list N pairs
        self.tensors[name] = {"dtype": dtype, "shape": [int(d) for d in shape], "offset": self.size}
        if exp is not None:
            self.tensors[name]["exp"] = int(exp)
        padded = raw.ljust(-(-len(raw) // BLOB_ALIGN) * BLOB_ALIGN, b"\0")
        self.chunks.append(padded)
        self.size += len(padded)

    def weight(self, name: str, w: np.ndarray, n_rows: int) -> np.ndarray:
        """Per-output-channel int8 weights (GPU); returns the row scales."""
        q, scales = self.device.rows_i8(w, n_rows)
        self.put(name, q, "i8")
        return scales

    def i16(self, name: str, x: np.ndarray, e: int) -> None:
        self.put(name, self.device.i16(x, e), "i16", e)

    def bytes(self) -> bytes:
        return b"".join(self.chunks)


# ---- export directory (refquant.py:275-301) -----------------------------------------------------
_ATTR = re.compile(r"(\w+)\s*=\s*([-+0-9.eE]+)\s*:\s*(i64|f64)")


def parse_model_attrs(mlir: str) -> dict:
    """The `llaccel.model = {name = value : i64|f64, ...}` attribute of model.mlir."""
    block = re.search(r"llaccel\.model\s*=\s*\{(.*?)\}\}", mlir, re.S)
    if block is None:
        raise ValueError("model.mlir: llaccel.model attribute not found")
    return {key: int(val) if kind == "i64" else float(val) for key, val, kind in _ATTR.findall(block.group(1))}


def load_export(export_dir) -> tuple[dict, dict[str, np.ndarray], dict[str, float]]:
    """(model attributes, {weight name: f32 array}, {activation: abs-max}) of an export directory.
    The weights stay f32 (each is exactly a double; the conversions widen them exactly)."""
    root = Path(export_dir)
    blob = (root / "weights.bin").read_bytes()
    weights = {e["name"]: np.frombuffer(blob, dtype="<f4", count=int(np.prod(e["shape"])), offset=e["offset"])
               .reshape(e["shape"]) for e in json.loads((root / "weights.json").read_text())}
    return (parse_model_attrs((root / "model.mlir").read_text()), weights,
            json.loads((root / "calib.json").read_text()))


# ---- number formats of the activations -------------------------------------------------------
class Formats:
    """i16 exponents and i8 scales of named activations, chosen from the calibration abs-max (or a
    selected `.i16_absmax` / `.i8_absmax` bound, refquant.py:312-338).  The first choice of a name is
    kept; `fix` sets one explicitly (RoPE ties, residual branches)."""

    def __init__(self, calib: dict[str, float]) -> None:
        self.calib = calib
        self.exps: dict[str, int] = {}
        self.scales: dict[str, float] = {}

    def absmax(self, name: str) -> float:
        if name not in self.calib:
            raise KeyError(f"calib.json has no entry for activation {name!r}")
        v = float(self.calib[name])
        if not (math.isfinite(v) and v >= 0):
            raise ValueError(f"calibration for {name!r} must be finite and nonnegative")
        return v

    def optional(self, name: str) -> float | None:
        return self.absmax(name) if name in self.calib else None

    def bound(self, name: str, bits: int) -> float:
        raw = self.absmax(name)
        sel = self.optional(f"{name}.i{bits}_absmax")
        if sel is None:
            return raw
        if sel > raw or (raw > 0 and sel == 0):
            raise ValueError(f"invalid selected quantization bound for {name!r}")
        return sel

    def calib_exp(self, name: str) -> int:
        return i16_exponent(self.bound(name, 16))

    def e16(self, name: str) -> int:
        if name not in self.exps:
            self.exps[name] = self.calib_exp(name)
        return self.exps[name]

    def s8(self, name: str, src: str | None = None) -> float:
        if name not in self.scales:
            self.scales[name] = i8_scale(self.bound(src or name.removesuffix(".q"), 8))
        return self.scales[name]

    def fix(self, exp: int, *names: str) -> None:
        for n in names:
            self.exps[n] = exp


# ---- the graph ---------------------------------------------------------------------------------
# One decoder layer as data: (step kind, operand names) with {p} = the layer prefix l<i>, {r} = the
# layer's residual input, {q}/{k} = the tensors RoPE reads (q/k, or qn/kn after Q/K RMSNorm).  The
# order is the reference's (refquant.py:426-487); kinds are the STEP_KINDS below.
LAYER_TEMPLATE = (
    ("norm", "{r}", "{p}_attn_norm", "{p}.h"),
    ("quant", "{p}.h"),
    ("rope_formats", "{q}", "{p}.qr", "{k}", "{p}.kr"),
    ("proj", "{p}.h.q", "{p}_wq", "{p}_bq", "{p}.q", "i16"),
    ("proj", "{p}.h.q", "{p}_wk", "{p}_bk", "{p}.k", "i16"),
    ("proj", "{p}.h.q", "{p}_wv", "{p}_bv", "{p}.v", "i8"),
    ("head_norms", "{p}"),
    ("rope", "{q}", "{p}.qr", "H"),
    ("rope", "{k}", "{p}.kr", "Hkv"),
    ("quant", "{p}.qr"),
    ("quant", "{p}.kr"),
    ("kv_write", "{p}.kr.q", "{p}.v"),
    ("attention", "{p}.qr.q", "{p}.kr.q", "{p}.v", "{p}.a"),
    ("residual", "{p}.a", "{p}_wo", "{p}_bo", "{p}.o", "{r}", "{p}.x1"),
    ("norm", "{p}.x1", "{p}_ffn_norm", "{p}.h2"),
    ("quant", "{p}.h2"),
    ("gate_up", "{p}"),
    ("quant", "{p}.f"),
    ("residual", "{p}.f.q", "{p}_wd", "{p}_bd", "{p}.d", "{p}.x1", "{p}.x2"),
)


class Graph:
    """Expands LAYER_TEMPLATE over the layers of an export and packs the tensors."""

    def __init__(self, cfg: dict, weights: dict[str, np.ndarray], calib: dict[str, float], fusion: bool,
                 device=None) -> None:
        self.cfg, self.W, self.fusion = cfg, weights, fusion
        self.fmt = Formats(calib)
        self.pack = Pack(device or _Device())
        self.ops: list[dict] = []
        shape = {k: int(cfg[k]) for k in ("dim", "n_layers", "n_heads", "n_kv_heads", "head_dim", "ffn", "vocab",
                                          "max_seq")}
        self.dim, self.L, self.H, self.Hkv = shape["dim"], shape["n_layers"], shape["n_heads"], shape["n_kv_heads"]
        self.D, self.ffn, self.vocab, self.max_seq = shape["head_dim"], shape["ffn"], shape["vocab"], shape["max_seq"]
        self.vocab_padded = -(-self.vocab // 16) * 16
        self.layer = 0

    # -- packed operands ------------------------------------------------------------------------
    def _gamma(self, name: str) -> tuple[int, int]:
        """The gamma i16 at its own exponent; returns (K, e_g)."""
        g = self.W[name]
        e_g = i16_exponent(float(np.abs(g.astype(np.float64)).max()))
        self.pack.i16(name, g, e_g)
        return int(g.shape[0]), e_g

    def _linear(self, a: str, w: str, b: str | None, y: str, out_dtype: str, *, e_rq: int | None = None,
                n_rows: int | None = None, epilogue: str = "none", aux: str | None = None, aux_shift: int = 0,
                silu: dict | None = None) -> None:
        wf = self.W[w]
        N, K = int(n_rows if n_rows is not None else wf.shape[0]), int(wf.shape[1])
        s_w = self.pack.weight(w, wf, N)
        s_a = self.fmt.s8(a)
        if out_dtype == "i8" and epilogue != "none":
            raise ValueError(f"linear {y}: i8 output is only valid with epilogue none")
        if out_dtype not in ("i8", "i16"):
            raise ValueError(out_dtype)
        rq = (gemm_rq_rows(s_a, s_w, True, 0, self.fmt.s8(y)) if out_dtype == "i8" else
              gemm_rq_rows(s_a, s_w, False, self.fmt.e16(y) if e_rq is None else e_rq, 0.0))
        self.pack.put(w + ".rq", rq, "rq")
        bias = b if b is not None and b in self.W else None
        if bias is not None:
            bf = np.zeros(N)
            bf[: self.W[b].shape[0]] = self.W[b]
            self.pack.put(b, gemm_bias_rows(bf, s_a, s_w), "i32")
        self.ops.append({"op": "linear", "in": a, "w": w, "rq": w + ".rq", "bias": bias, "out": y, "N": N, "K": K,
                         "out_dtype": out_dtype, "epilogue": epilogue, "aux": aux, "aux_shift": aux_shift,
                         "silu": silu})

    # -- step kinds ------------------------------------------------------------------------------
    def norm(self, x: str, gamma: str, y: str, heads: int = 1) -> None:
        e_x, e_y = self.fmt.e16(x), self.fmt.e16(y)
        K, e_g = self._gamma(gamma)
        prm = rmsnorm_params(K, self.cfg["rms_eps"], e_x, e_g, e_y, self.fmt.absmax(x), y,
                             self.fmt.optional(x + ".rms_min"))
        op = {"op": "rmsnorm", "in": x, "gamma": gamma, "out": y, "K": K, "eps_t": prm["eps_t"], "C": prm["C"],
              "sh_post": prm["sh_post"]}
        if heads != 1:
            op["heads"] = heads
        self.ops.append(op)

    def quant(self, x: str) -> None:
        y = x + ".q"
        M, S = quant_params(self.fmt.e16(x), self.fmt.s8(y, x))
        self.ops.append({"op": "quant", "in": x, "out": y, "M": M, "S": S})

    def rope_formats(self, q: str, qr: str, k: str, kr: str) -> None:
        """RoPE keeps the exponent: a tensor and its rotation share the coarser of their two."""
        for a, b in ((q, qr), (k, kr)):
            self.fmt.fix(max(self.fmt.calib_exp(a), self.fmt.calib_exp(b)), a, b)

    def proj(self, a: str, w: str, b: str, y: str, out_dtype: str) -> None:
        self._linear(a, w, b, y, out_dtype)

    def head_norms(self, p: str) -> None:
        if f"{p}_q_norm" in self.W:
            self.norm(f"{p}.q", f"{p}_q_norm", f"{p}.qn", heads=self.H)
            self.norm(f"{p}.k", f"{p}_k_norm", f"{p}.kn", heads=self.Hkv)

    def rope(self, x: str, y: str, heads: str) -> None:
        self.ops.append({"op": "rope", "in": x, "out": y, "H": getattr(self, heads), "D": self.D})

    def kv_write(self, kq: str, v: str) -> None:
        self.ops.append({"op": "kv_write", "layer": self.layer, "k": kq, "v": v, "Hkv": self.Hkv, "D": self.D})

    def attention(self, qq: str, kq: str, v: str, out: str) -> None:
        prm = attn_params(self.fmt.s8(qq), self.fmt.s8(kq), self.fmt.s8(v), self.fmt.s8(out), self.D)
        self.ops.append({"op": "attention", "q": qq, "layer": self.layer, "out": out, "H": self.H, "Hkv": self.Hkv,
                         "D": self.D, "prob_bits": 15, **prm})

    def residual(self, a: str, w: str, b: str, branch: str, resid: str, out: str) -> None:
        """A branch projection added to the residual (refquant.py:387-401).  The branch and the sum
        share an exponent with room for the add; with --fusion and no shift needed the add becomes
        the linear's resadd epilogue, else it is an explicit add with the coarser operand first."""
        e_res = self.fmt.e16(resid)
        e_sum = max(self.fmt.e16(branch), self.fmt.e16(out), e_res, self.fmt.calib_exp(resid))
        self.fmt.fix(e_sum, branch, out)
        if self.fusion and e_sum == e_res:
            self._linear(a, w, b, out, "i16", e_rq=e_sum, epilogue="resadd", aux=resid, aux_shift=0)
            return
        self._linear(a, w, b, branch, "i16")
        first, second = (resid, branch) if e_res == e_sum else (branch, resid)
        self.ops.append({"op": "add", "a": first, "b": second, "out": out,
                         "sh_b": add_shift(self.fmt.e16(first), self.fmt.e16(second), out)})

    def gate_up(self, p: str) -> None:
        """silu(gate) * up, as silu/mul epilogues of the two linears (--fusion) or as four ops."""
        e_g, e_u, e_sg, e_f = (self.fmt.e16(f"{p}.{n}") for n in ("g", "u", "sg", "f"))
        silu = silu_params(e_g, e_sg, f"{p}.sg")
        sh = mul_shift(e_sg, e_u, e_f, f"{p}.f")
        x = f"{p}.h2.q"
        if self.fusion:
            self._linear(x, f"{p}_wg", f"{p}_bg", f"{p}.sg", "i16", e_rq=e_g, epilogue="silu", silu=silu)
            self._linear(x, f"{p}_wu", f"{p}_bu", f"{p}.f", "i16", e_rq=e_u, epilogue="mul", aux=f"{p}.sg",
                         aux_shift=sh)
            return
        self._linear(x, f"{p}_wg", f"{p}_bg", f"{p}.g", "i16")
        self._linear(x, f"{p}_wu", f"{p}_bu", f"{p}.u", "i16")
        self.ops.append({"op": "silu", "in": f"{p}.g", "out": f"{p}.sg", **silu})
        self.ops.append({"op": "mul", "a": f"{p}.sg", "b": f"{p}.u", "out": f"{p}.f", "sh": sh})

    # -- the whole graph ---------------------------------------------------------------------------
    def _check_shape(self) -> None:
        for what, val in (("dim", self.dim), ("ffn", self.ffn), ("n_kv_heads*head_dim", self.Hkv * self.D)):
            if val % 16:
                raise ValueError(f"{what} = {val} must be a multiple of 16")
        if self.D not in HEAD_DIMS:
            raise ValueError(f"head_dim {self.D} not in {HEAD_DIMS}")

    def _tables(self) -> None:
        """Embedding (padded to vocab_padded rows) at E_RES, then the RoPE tables: static ones from the
        export when present, else computed."""
        emb = np.zeros((self.vocab_padded, self.dim), dtype=np.float32)
        emb[: self.vocab] = self.W["embed"]
        self.pack.i16("embed", emb, self.fmt.e16("input"))
        names = ("rope_cos_input", "rope_sin_input")
        if any(n in self.W for n in names):
            for n, out in zip(names, ("rope_cos", "rope_sin")):
                t = np.asarray(self.W[n], dtype=np.float64)
                bad = (t.shape != (self.max_seq, self.D // 2) or not np.isfinite(t).all()
                       or ((t < -2.0) | (t > 32767.0 / 16384.0)).any())
                if bad:
                    raise ValueError(f"invalid static RoPE table {n}")
                self.pack.put(out, llround_vec(t * 16384.0).astype(np.int16), "i16")
            return
        for out, tab in zip(("rope_cos", "rope_sin"), rope_tables(self.max_seq, self.D, float(self.cfg["rope_base"]))):
            self.pack.put(out, tab, "i16")

    def build(self) -> dict:
        self._check_shape()
        E_RES = self.fmt.e16("input")
        E_LOGIT = self.fmt.calib_exp("logits")
        self.fmt.fix(E_LOGIT, "logits")
        self._tables()
        resid = "input"
        for i in range(self.L):
            p = f"l{i}"
            if (f"{p}_q_norm" in self.W) != (f"{p}_k_norm" in self.W):
                raise ValueError("Q/K normalization must be paired")
            qk = f"{p}_q_norm" in self.W
            names = {"p": p, "r": resid, "q": f"{p}.qn" if qk else f"{p}.q", "k": f"{p}.kn" if qk else f"{p}.k"}
            self.layer = i
            for kind, *args in LAYER_TEMPLATE:
                getattr(self, kind)(*[a.format(**names) if "{" in a else a for a in args])
            resid = f"{p}.x2"
        self.norm(resid, "norm", "hn")
        self.quant("hn")
        self._linear("hn.q", "lm_head", "lm_head_bias", "logits", "i16", n_rows=self.vocab_padded)
        return {"model": {"dim": self.dim, "n_layers": self.L, "n_heads": self.H, "n_kv_heads": self.Hkv,
                          "head_dim": self.D, "ffn": self.ffn, "vocab": self.vocab, "vocab_padded": self.vocab_padded,
                          "max_seq": self.max_seq, "E_RES": E_RES, "E_LOGIT": E_LOGIT},
                "weights_file": "qweights.bin", "tensors": self.pack.tensors, "ops": self.ops,
                "input": "input", "output": "logits", "exps": self.fmt.exps, "scales": self.fmt.scales,
                "fusion": self.fusion}


STEP_KINDS = tuple(sorted({kind for kind, *_ in LAYER_TEMPLATE}))


def quantize_export(export_dir, out_dir, fusion: bool = False, device=None) -> dict:
    """export_dir -> out_dir/{qgraph.json, qweights.bin} (+ a tokenizer.json the export carries);
    the reference's quantize_export (refquant.py:493-506).  Returns the qgraph."""
    export_dir, out_dir = Path(export_dir), Path(out_dir)
    graph = Graph(*load_export(export_dir), fusion, device)
    qgraph = graph.build()
    out_dir.mkdir(parents=True, exist_ok=True)
    (out_dir / "qweights.bin").write_bytes(graph.pack.bytes())
    (out_dir / "qgraph.json").write_text(json.dumps(qgraph, indent=1))
    tok = export_dir / "tokenizer.json"
    if tok.exists():
        (out_dir / "tokenizer.json").write_bytes(tok.read_bytes())
    return qgraph


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="export directory -> qgraph.json + qweights.bin (weights converted "
                                             "on the GPU)")
    ap.add_argument("export_dir")
    ap.add_argument("-o", "--out", default="build/q-ref/")
    ap.add_argument("--fusion", "--fuse", dest="fusion", action="store_true", help="emit epilogue-fused linears")
    args = ap.parse_args(argv)
    g = quantize_export(args.export_dir, args.out, fusion=args.fusion)
    kinds = sorted({op["op"] for op in g["ops"]})
    size = sum(p.stat().st_size for p in Path(args.out).glob("qweights.bin"))
    print(f"{args.out}: {len(g['ops'])} ops ({', '.join(kinds)}), {len(g['tensors'])} tensors in {size} bytes; "
          f"E_RES {g['model']['E_RES']}, E_LOGIT {g['model']['E_LOGIT']}, {'fused' if args.fusion else 'unfused'}")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
