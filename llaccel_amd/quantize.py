"""qgraph producer: a model export directory -> qgraph.json + qweights.bin, the datapath's input.

Restates the decisions of the reference quantizer (python/llaccel/refquant.py): the graph it emits
(`RefQuantizer.run`, refquant.py:403-490, with its emitters :341-401), the tensor blob (:244-270),
the export-directory reader (:275-301) and the integer-parameter formulas (:89-241, the "Compiler:"
lines of docs/NUMERICS.md).  Same names, same op list, same integers; one extension: head_dim 128
and 256 are accepted (refquant.py:411 stops at 64, while the datapath handles both, with Q/K
RMSNorm, which the reference's run() already emits).

The export directory holds `model.mlir` (only its `llaccel.model = {...}` attribute is read),
`weights.bin` + `weights.json` (little-endian f32 tensors and their name/shape/offset index) and
`calib.json` (abs-max per named activation, optional `.i16_absmax` / `.i8_absmax` selected bounds
and `.rms_min` row statistics).  `llaccel_amd.synth.write_export` writes one from a seeded float
model.

Device work: every weight matrix becomes per-output-channel int8 with its row scales on the GPU
(`llhip_quant_rows_i8`), the embedding and RMSNorm gammas become i16 there too
(`llhip_quant_i16`); there is no host fallback.  The per-row requant pairs and biases are float64
numpy evaluated in the reference's order, the per-op parameters float64 Python scalars.

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


# ---- C rounding and (M, S) pairs -------------------------------------------------------------
def llround(x: float) -> int:
    """C llround (refquant.py:61-72): nearest integer, halves away from zero."""
    x = float(x)
    if not math.isfinite(x):
        raise ValueError(f"llround of {x}")
    t = math.trunc(x)
    f = x - t
    return t + 1 if f >= 0.5 else (t - 1 if f <= -0.5 else t)


def llround_vec(x) -> np.ndarray:
    """Elementwise llround of finite doubles (refquant.py:75-86)."""
    x = np.asarray(x, dtype=np.float64)
    if not np.all(np.isfinite(x)):
        raise ValueError("llround of a non-finite value")
    if np.any(np.abs(x) >= 2.0**63):
        raise ValueError("llround input exceeds int64 range")
    t = np.trunc(x)
    f = x - t
    return (t + (f >= 0.5) - (f <= -0.5)).astype(np.int64)


def mulshift_pair(r: float) -> tuple[int, int]:
    """(M, S), M * 2^-S ~= r with M in [2^30, 2^31) (refquant.py:89-104)."""
    M, S = mulshift_pairs(np.array([r], dtype=np.float64))
    return int(M[0]), int(S[0])


def mulshift_pairs(r) -> tuple[np.ndarray, np.ndarray]:
    """Vector form of refquant.py:89-104: frexp mantissa rounded to 31 bits; a mantissa that rounds
    up to 1.0 becomes 2^30 one exponent lower; S above 63 is pinned at 63 with a smaller M."""
    r = np.asarray(r, dtype=np.float64)
    if not np.all(np.isfinite(r)) or np.any(r <= 0.0):
        raise ValueError("normalize_mulshift: ratio must be positive and finite")
    f, e = np.frexp(r)
    M = llround_vec(np.ldexp(f, 31))
    S = 31 - e.astype(np.int64)
    up = M >= 1 << 31
    M = np.where(up, 1 << 30, M)
    S = np.where(up, S - 1, S)
    if np.any(S < 0):
        raise ValueError(f"normalize_mulshift: ratio {float(r[S < 0][0])} too large (S < 0)")
    deep = S > 63
    if np.any(deep):
        M = np.where(deep, llround_vec(np.where(deep, np.ldexp(r, 63), 0.0)), M)
        S = np.where(deep, 63, S)
    return M.astype(np.int64), S.astype(np.int64)


# ---- activation formats and per-op parameters (refquant.py:107-241) ---------------------------
def i16_exponent(absmax: float) -> int:
    if not absmax > 0.0:
        return -15
    return max(int(math.ceil(math.log2(absmax) - math.log2(32767.0))), -15)


def i8_scale(absmax: float) -> float:
    return absmax / 127.0 if absmax > 0.0 else 1.0


def gemm_rq_rows(s_a: float, s_w: np.ndarray, out_i8: bool, e_out: int, s_out: float) -> np.ndarray:
    """refquant.py:143-146 for every output channel: rq[n] = (M, S) of s_a*s_w[n] / (s_out or 2^e_out)."""
    den = s_out if out_i8 else math.ldexp(1.0, int(e_out))
    M, S = mulshift_pairs(s_a * np.asarray(s_w, dtype=np.float64) / den)
    return np.stack([M, S], axis=1)


def gemm_bias_rows(b: np.ndarray, s_a: float, s_w: np.ndarray) -> np.ndarray:
    """refquant.py:149-151 for every output channel: clamp(llround(b / (s_a * s_w)), int32)."""
    with np.errstate(divide="ignore", over="ignore", invalid="ignore"):
        x = np.asarray(b, dtype=np.float64) / (s_a * np.asarray(s_w, dtype=np.float64))
    if not np.all(np.isfinite(x)):
        raise ValueError("gemm bias: non-finite quotient")
    # quotients beyond +-2^40 clamp to the int32 range either way; bounding them first keeps the
    # vector rounding inside int64
    v = llround_vec(np.clip(x, -(2.0**40), 2.0**40))
    return np.clip(v, INT32_MIN, INT32_MAX).astype(np.int32)


def quant_params(e_x: int, s_y: float) -> tuple[int, int]:
    """refquant.py:154-156: QUANT i16 -> i8, M*2^-S ~= 2^e_x / s_y."""
    return mulshift_pair(math.ldexp(1.0, int(e_x)) / s_y)


def rmsnorm_params(K: int, eps: float, e_x: int, e_g: int, e_y: int, absmax_x: float, name: str,
                   rms_min: float | None = None) -> dict:
    """refquant.py:159-186: eps_t = llround(eps K 2^-2e_x); R is the largest shift <= 31 whose
    C = llround(2^R sqrt K) fits u32 and keeps the typical inverse (from rms_min, else absmax/4)
    below 65535/4; sh_post = R - e_g + e_y."""
    if rms_min is not None and (not math.isfinite(rms_min) or not 0 <= rms_min <= absmax_x):
        raise ValueError(f"rmsnorm {name}: rms_min must be finite and in [0, absmax]")
    eps_t = llround(eps * float(K) * math.ldexp(1.0, int(-2 * e_x)))
    if not 0 <= eps_t < 2**32:
        raise ValueError(f"rmsnorm {name}: eps_t does not fit the ISA u32 operand")
    rms_q = (absmax_x / 4.0 if rms_min is None else rms_min) / math.ldexp(1.0, int(e_x))
    r_typ = max(1.0, math.floor(math.sqrt(float(K) * rms_q * rms_q + float(eps_t))))
    for R in range(31, -1, -1):
        C = llround(math.ldexp(math.sqrt(float(K)), R))
        if C < 4294967296 and math.floor(C / r_typ) < 65535.0 / 4.0:
            break
    else:
        raise ValueError(f"rmsnorm {name}: no R in [0,31] keeps inv below 65535/4 "
                         f"(input abs-max {absmax_x} too small for e_x)")
    sh_post = R - e_g + e_y
    if not 0 <= sh_post <= 63:
        raise ValueError(f"rmsnorm {name}: sh_post = {sh_post} outside [0, 63]")
    return {"eps_t": eps_t, "C": C, "R": R, "sh_post": sh_post}


def silu_params(e_x: int, e_y: int, name: str) -> dict:
    """refquant.py:189-196: Mi = 2^30, Si = 30 - (e_x + 12), sh_out = 16 + e_y - e_x."""
    p = {"Mi": 1 << 30, "Si": 30 - (e_x + 12), "sh_out": 16 + e_y - e_x}
    for k in ("Si", "sh_out"):
        if not 0 <= p[k] <= 63:
            raise ValueError(f"silu {name}: {k} = {p[k]} outside [0, 63]")
    return p


def mul_shift(e_a: int, e_b: int, e_y: int, name: str) -> int:
    """refquant.py:199-209: the right shift of a*b (exponent e_a + e_b) to e_y."""
    sh = e_y - e_a - e_b
    if not 0 <= sh <= 63:
        raise ValueError(f"mul {name}: sh = {sh} outside [0, 63]")
    return sh


def add_shift(e_a: int, e_b: int, name: str) -> int:
    """refquant.py:212-218: b brought from e_b to e_a (the coarser operand comes first)."""
    sh = e_a - e_b
    if not 0 <= sh <= 63:
        raise ValueError(f"add {name}: sh_b = {sh} outside [0, 63] (b must not have a larger exponent than a)")
    return sh


def attn_params(s_q: float, s_k: float, s_v: float, s_out: float, D: int) -> dict:
    """refquant.py:221-224."""
    Ms, Ss = mulshift_pair(256.0 * s_q * s_k / math.sqrt(float(D)))
    Mo, So = mulshift_pair(s_v / (256.0 * s_out))
    return {"Ms": Ms, "Ss": Ss, "Mo": Mo, "So": So}


def rope_tables(max_seq: int, D: int, base: float) -> tuple[np.ndarray, np.ndarray]:
    """refquant.py:227-238: Q1.14 cos/sin of p * base^(-2i/D), computed with the C library's
    cos/sin per element as the reference does."""
    half = D // 2
    cos_t = np.zeros((max_seq, half), dtype=np.int16)
    sin_t = np.zeros((max_seq, half), dtype=np.int16)
    for i in range(half):
        theta = math.pow(base, -2.0 * float(i) / float(D))
        for p in range(max_seq):
            ang = float(p) * theta
            cos_t[p, i] = min(llround(16384.0 * math.cos(ang)), 32767)
            sin_t[p, i] = min(llround(16384.0 * math.sin(ang)), 32767)
    return cos_t, sin_t


# ---- device conversions -----------------------------------------------------------------------
class _Device:
    """The GPU side of the producer: f32 tensors in, int8 rows + scales / i16 values out."""

    def __init__(self):
        import torch

        if not torch.cuda.is_available():
            raise RuntimeError("llaccel_amd.quantize converts weights on the GPU; no GPU is available")
        _lib.lib()  # raises LibraryNotBuilt when the HIP library is missing
        self.torch = torch
        self.status = torch.zeros(1, dtype=torch.int32, device="cuda")

    def _stream(self):
        return ctypes.c_void_p(self.torch.cuda.current_stream().cuda_stream)

    def _check(self, what: str):
        if int(self.status.item()) != 0:
            raise ValueError(f"{what}: non-finite value")

    def rows_i8(self, w: np.ndarray, n_rows: int | None = None) -> tuple[np.ndarray, np.ndarray]:
        """int8 rows and float64 scales of w [N][K] (rows past w.shape[0], up to n_rows, are zero)."""
        torch = self.torch
        w = np.ascontiguousarray(w, dtype=np.float32)
        N = w.shape[0] if n_rows is None else int(n_rows)
        K = w.shape[1]
        src = torch.zeros((N, K), dtype=torch.float32, device="cuda")
        src[: w.shape[0]].copy_(torch.from_numpy(w))
        q = torch.empty((N, K), dtype=torch.int8, device="cuda")
        s = torch.empty(N, dtype=torch.float64, device="cuda")
        self.status.zero_()
        _lib.call("llhip_quant_rows_i8", ctypes.c_void_p(src.data_ptr()), N, K, K, ctypes.c_void_p(q.data_ptr()), K,
                  ctypes.c_void_p(s.data_ptr()), ctypes.c_void_p(self.status.data_ptr()), self._stream())
        self._check("quant_i8")
        return q.cpu().numpy(), s.cpu().numpy()

    def i16(self, x: np.ndarray, e: int) -> np.ndarray:
        torch = self.torch
        x = np.ascontiguousarray(x, dtype=np.float32)
        src = torch.from_numpy(x.reshape(-1)).cuda()
        y = torch.empty(x.size, dtype=torch.int16, device="cuda")
        self.status.zero_()
        _lib.call("llhip_quant_i16", ctypes.c_void_p(src.data_ptr()), x.size, int(e), ctypes.c_void_p(y.data_ptr()),
                  ctypes.c_void_p(self.status.data_ptr()), self._stream())
        self._check("quant_i16")
        return y.cpu().numpy().reshape(x.shape)


# ---- qweights.bin ----------------------------------------------------------------------------
class Blob:
    """refquant.py:244-270: tensors back to back, each padded to 64 bytes, and their index."""

    _NP = {"i8": "<i1", "i16": "<i2", "i32": "<i4", "rq": "<i4"}

    def __init__(self) -> None:
        self.parts: list[bytes] = []
        self.off = 0
        self.tensors: dict[str, dict] = {}

    def add(self, name: str, arr: np.ndarray, dtype: str, exp: int | None = None) -> None:
        if name in self.tensors:
            raise ValueError(f"duplicate tensor {name}")
        data = np.asarray(arr).astype(self._NP[dtype]).tobytes()
        shape = arr.shape[:-1] if dtype == "rq" else arr.shape
        spec = {"dtype": dtype, "shape": [int(s) for s in shape], "offset": self.off}
        if exp is not None:
            spec["exp"] = int(exp)
        self.tensors[name] = spec
        pad = -len(data) % 64
        self.parts.append(data + b"\0" * pad)
        self.off += len(data) + pad

    def bytes(self) -> bytes:
        return b"".join(self.parts)


# ---- export directory (refquant.py:275-301) ------------------------------------------------------
def parse_model_attrs(mlir: str) -> dict:
    m = re.search(r"llaccel\.model\s*=\s*\{(.*?)\}\}", mlir, re.S)
    if not m:
        raise ValueError("model.mlir: llaccel.model attribute not found")
    return {k: (int(v) if ty == "i64" else float(v))
            for k, v, ty in re.findall(r"(\w+)\s*=\s*([-+0-9.eE]+)\s*:\s*(i64|f64)", m.group(1))}


def load_export(export_dir) -> tuple[dict, dict[str, np.ndarray], dict[str, float]]:
    """(model attributes, {weight: f32 array}, {activation: abs-max}).  The weights stay f32: every
    f32 is exactly a double, and the device conversions widen them exactly."""
    export_dir = Path(export_dir)
    cfg = parse_model_attrs((export_dir / "model.mlir").read_text())
    blob = (export_dir / "weights.bin").read_bytes()
    index = json.loads((export_dir / "weights.json").read_text())
    weights = {}
    for e in index:
        n = int(np.prod(e["shape"]))
        weights[e["name"]] = np.frombuffer(blob, dtype="<f4", count=n, offset=e["offset"]).reshape(e["shape"])
    calib = json.loads((export_dir / "calib.json").read_text())
    return cfg, weights, calib


# ---- the producer ----------------------------------------------------------------------------
class Quantizer:
    """refquant.py:304-490 (`RefQuantizer`): same emitters, same graph, same integers."""

    HEAD_DIMS = (16, 32, 64, 128, 256)

    def __init__(self, cfg: dict, weights: dict[str, np.ndarray], calib: dict[str, float], fusion: bool,
                 device: _Device | None = None) -> None:
        self.cfg, self.W, self.calib, self.fusion = cfg, weights, calib, fusion
        self.dev = device or _Device()
        self.blob = Blob()
        self.ops: list[dict] = []
        self.exps: dict[str, int] = {}
        self.scales: dict[str, float] = {}

    # activation formats (refquant.py:312-338)
    def absmax(self, name: str) -> float:
        if name not in self.calib:
            raise KeyError(f"calib.json has no entry for activation {name!r}")
        v = float(self.calib[name])
        if not math.isfinite(v) or v < 0:
            raise ValueError(f"calibration for {name!r} must be finite and nonnegative")
        return v

    def quant_absmax(self, name: str, bits: int) -> float:
        raw = self.absmax(name)
        key = f"{name}.i{bits}_absmax"
        bound = self.absmax(key) if key in self.calib else raw
        if bound > raw or (raw > 0 and bound == 0):
            raise ValueError(f"invalid selected quantization bound for {name!r}")
        return bound

    def e16(self, name: str) -> int:
        if name not in self.exps:
            self.exps[name] = i16_exponent(self.quant_absmax(name, 16))
        return self.exps[name]

    def s8(self, name: str, src: str | None = None) -> float:
        if name not in self.scales:
            self.scales[name] = i8_scale(self.quant_absmax(src or name.removesuffix(".q"), 8))
        return self.scales[name]

    # emitters (refquant.py:341-401)
    def rmsnorm(self, x: str, gamma: str, y: str, heads: int = 1) -> None:
        e_x, e_y = self.e16(x), self.e16(y)
        g = self.W[gamma]
        e_g = i16_exponent(float(np.abs(g.astype(np.float64)).max()))
        self.blob.add(gamma, self.dev.i16(g, e_g), "i16", e_g)
        K = int(g.shape[0])
        rms_min = self.absmax(x + ".rms_min") if x + ".rms_min" in self.calib else None
        p = rmsnorm_params(K, self.cfg["rms_eps"], e_x, e_g, e_y, self.absmax(x), y, rms_min)
        op = {"op": "rmsnorm", "in": x, "gamma": gamma, "out": y, "K": K, "eps_t": p["eps_t"], "C": p["C"],
              "sh_post": p["sh_post"]}
        if heads != 1:
            op["heads"] = heads
        self.ops.append(op)

    def quant(self, x: str) -> str:
        y = x + ".q"
        M, S = quant_params(self.e16(x), self.s8(y, x))
        self.ops.append({"op": "quant", "in": x, "out": y, "M": M, "S": S})
        return y

    def linear(self, a: str, w: str, b: str | None, y: str, out_dtype: str, *, e_rq: int | None = None,
               n_pad: int | None = None, epilogue: str = "none", aux: str | None = None, aux_shift: int = 0,
               silu: dict | None = None) -> None:
        wf = self.W[w]
        N, K = (int(n_pad) if n_pad is not None else int(wf.shape[0])), int(wf.shape[1])
        q, s_w = self.dev.rows_i8(wf, N)
        self.blob.add(w, q, "i8")
        s_a = self.s8(a)
        if out_dtype == "i16":
            rq = gemm_rq_rows(s_a, s_w, False, self.e16(y) if e_rq is None else e_rq, 0.0)
        elif out_dtype == "i8":
            if epilogue != "none":
                raise ValueError(f"linear {y}: i8 output is only valid with epilogue none")
            rq = gemm_rq_rows(s_a, s_w, True, 0, self.s8(y))
        else:
            raise ValueError(out_dtype)
        self.blob.add(w + ".rq", rq, "rq")
        bias = None
        if b is not None and b in self.W:
            bf = np.zeros(N)
            bf[: self.W[b].shape[0]] = self.W[b]
            self.blob.add(b, gemm_bias_rows(bf, s_a, s_w), "i32")
            bias = b
        self.ops.append({"op": "linear", "in": a, "w": w, "rq": w + ".rq", "bias": bias, "out": y, "N": N, "K": K,
                         "out_dtype": out_dtype, "epilogue": epilogue, "aux": aux, "aux_shift": aux_shift,
                         "silu": silu})

    def residual_linear(self, a: str, w: str, bias: str, branch: str, residual: str, out: str) -> None:
        """The branch GEMM targets an exponent with room for this ADD; fused into a RESADD epilogue
        when no shift is needed, else an explicit add with the coarser operand first."""
        e_res = self.e16(residual)
        e_branch = max(self.e16(branch), self.e16(out), e_res, i16_exponent(self.quant_absmax(residual, 16)))
        self.exps[branch] = self.exps[out] = e_branch
        if self.fusion and e_branch == e_res:
            self.linear(a, w, bias, out, "i16", e_rq=e_branch, epilogue="resadd", aux=residual, aux_shift=0)
            return
        self.linear(a, w, bias, branch, "i16")
        first, second = (residual, branch) if e_res == e_branch else (branch, residual)
        self.ops.append({"op": "add", "a": first, "b": second, "out": out,
                         "sh_b": add_shift(self.e16(first), self.e16(second), out)})

    # the graph (refquant.py:403-490)
    def run(self) -> dict:
        c = self.cfg
        dim, L, H, Hkv, D, ffn, vocab, max_seq = (int(c[k]) for k in ("dim", "n_layers", "n_heads", "n_kv_heads",
                                                                    "head_dim", "ffn", "vocab", "max_seq"))
        vocab_padded = (vocab + 15) // 16 * 16
        for what, val in (("dim", dim), ("ffn", ffn), ("n_kv_heads*head_dim", Hkv * D)):
            if val % 16:
                raise ValueError(f"{what} = {val} must be a multiple of 16")
        if D not in self.HEAD_DIMS:
            raise ValueError(f"head_dim {D} not in {self.HEAD_DIMS}")

        E_RES = self.e16("input")  # the embedding's exponent; later residuals carry their own
        E_LOGIT = i16_exponent(self.quant_absmax("logits", 16))
        self.exps["logits"] = E_LOGIT

        emb = np.zeros((vocab_padded, dim), dtype=np.float32)
        emb[:vocab] = self.W["embed"]
        self.blob.add("embed", self.dev.i16(emb, E_RES), "i16", E_RES)
        if "rope_cos_input" in self.W or "rope_sin_input" in self.W:
            tables = []
            for name in ("rope_cos_input", "rope_sin_input"):
                t = np.asarray(self.W[name], dtype=np.float64)
                if t.shape != (max_seq, D // 2) or not np.isfinite(t).all() or ((t < -2.0) | (t > 32767.0 / 16384.0)).any():
                    raise ValueError(f"invalid static RoPE table {name}")
                tables.append(llround_vec(t * 16384.0).astype(np.int16))
            cos_t, sin_t = tables
        else:
            cos_t, sin_t = rope_tables(max_seq, D, float(c["rope_base"]))
        self.blob.add("rope_cos", cos_t, "i16")
        self.blob.add("rope_sin", sin_t, "i16")

        residual = "input"
        for i in range(L):
            p = f"l{i}"
            self.rmsnorm(residual, f"{p}_attn_norm", f"{p}.h")
            hq = self.quant(f"{p}.h")
            qk_norm = f"{p}_q_norm" in self.W
            if qk_norm != (f"{p}_k_norm" in self.W):
                raise ValueError("Q/K normalization must be paired")
            q_src, k_src = (f"{p}.qn", f"{p}.kn") if qk_norm else (f"{p}.q", f"{p}.k")
            for a, b in ((q_src, f"{p}.qr"), (k_src, f"{p}.kr")):  # RoPE keeps the exponent
                self.exps[a] = self.exps[b] = max(i16_exponent(self.quant_absmax(a, 16)),
                                                  i16_exponent(self.quant_absmax(b, 16)))
            self.linear(hq, f"{p}_wq", f"{p}_bq", f"{p}.q", "i16")
            self.linear(hq, f"{p}_wk", f"{p}_bk", f"{p}.k", "i16")
            self.linear(hq, f"{p}_wv", f"{p}_bv", f"{p}.v", "i8")
            if qk_norm:
                self.rmsnorm(f"{p}.q", f"{p}_q_norm", q_src, heads=H)
                self.rmsnorm(f"{p}.k", f"{p}_k_norm", k_src, heads=Hkv)
            self.ops.append({"op": "rope", "in": q_src, "out": f"{p}.qr", "H": H, "D": D})
            self.ops.append({"op": "rope", "in": k_src, "out": f"{p}.kr", "H": Hkv, "D": D})
            qq, kq = self.quant(f"{p}.qr"), self.quant(f"{p}.kr")
            self.ops.append({"op": "kv_write", "layer": i, "k": kq, "v": f"{p}.v", "Hkv": Hkv, "D": D})
            self.ops.append({"op": "attention", "q": qq, "layer": i, "out": f"{p}.a", "H": H, "Hkv": Hkv, "D": D,
                             "prob_bits": 15,
                             **attn_params(self.s8(qq), self.s8(kq), self.s8(f"{p}.v"), self.s8(f"{p}.a"), D)})
            self.residual_linear(f"{p}.a", f"{p}_wo", f"{p}_bo", f"{p}.o", residual, f"{p}.x1")
            self.rmsnorm(f"{p}.x1", f"{p}_ffn_norm", f"{p}.h2")
            h2q = self.quant(f"{p}.h2")
            e_g, e_u, e_sg, e_f = (self.e16(f"{p}.{n}") for n in ("g", "u", "sg", "f"))
            silu = silu_params(e_g, e_sg, f"{p}.sg")
            sh_mul = mul_shift(e_sg, e_u, e_f, f"{p}.f")
            if self.fusion:
                self.linear(h2q, f"{p}_wg", f"{p}_bg", f"{p}.sg", "i16", e_rq=e_g, epilogue="silu", silu=silu)
                self.linear(h2q, f"{p}_wu", f"{p}_bu", f"{p}.f", "i16", e_rq=e_u, epilogue="mul", aux=f"{p}.sg",
                            aux_shift=sh_mul)
            else:
                self.linear(h2q, f"{p}_wg", f"{p}_bg", f"{p}.g", "i16")
                self.linear(h2q, f"{p}_wu", f"{p}_bu", f"{p}.u", "i16")
                self.ops.append({"op": "silu", "in": f"{p}.g", "out": f"{p}.sg", **silu})
                self.ops.append({"op": "mul", "a": f"{p}.sg", "b": f"{p}.u", "out": f"{p}.f", "sh": sh_mul})
            fq = self.quant(f"{p}.f")
            self.residual_linear(fq, f"{p}_wd", f"{p}_bd", f"{p}.d", f"{p}.x1", f"{p}.x2")
            residual = f"{p}.x2"
        self.rmsnorm(residual, "norm", "hn")
        hnq = self.quant("hn")
        self.linear(hnq, "lm_head", "lm_head_bias", "logits", "i16", n_pad=vocab_padded)
        return {
            "model": {"dim": dim, "n_layers": L, "n_heads": H, "n_kv_heads": Hkv, "head_dim": D, "ffn": ffn,
                      "vocab": vocab, "vocab_padded": vocab_padded, "max_seq": max_seq, "E_RES": E_RES,
                      "E_LOGIT": E_LOGIT},
            "weights_file": "qweights.bin",
            "tensors": self.blob.tensors,
            "ops": self.ops,
            "input": "input", "output": "logits",
            "exps": self.exps, "scales": self.scales,
            "fusion": self.fusion,
        }


def quantize_export(export_dir, out_dir, fusion: bool = False) -> dict:
    """refquant.py:493-506: `export_dir` -> `out_dir/{qgraph.json, qweights.bin}` (+ tokenizer.json)."""
    export_dir, out_dir = Path(export_dir), Path(out_dir)
    cfg, W, calib = load_export(export_dir)
    q = Quantizer(cfg, W, calib, fusion)
    graph = q.run()
    out_dir.mkdir(parents=True, exist_ok=True)
    (out_dir / "qweights.bin").write_bytes(q.blob.bytes())
    (out_dir / "qgraph.json").write_text(json.dumps(graph, indent=1))
    tok = export_dir / "tokenizer.json"
    if tok.exists():
        (out_dir / "tokenizer.json").write_bytes(tok.read_bytes())
    return graph


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="export directory -> qgraph.json + qweights.bin (reference recipe)")
    ap.add_argument("export_dir")
    ap.add_argument("-o", "--out", default="build/q-ref/")
    ap.add_argument("--fusion", "--fuse", dest="fusion", action="store_true", help="emit epilogue-fused linears")
    args = ap.parse_args(argv)
    g = quantize_export(args.export_dir, args.out, fusion=args.fusion)
    counts: dict[str, int] = {}
    for op in g["ops"]:
        counts[op["op"]] = counts.get(op["op"], 0) + 1
    print(f"wrote {args.out}: {len(g['ops'])} ops {counts}, {len(g['tensors'])} tensors, E_RES={g['model']['E_RES']} "
          f"E_LOGIT={g['model']['E_LOGIT']} fusion={args.fusion}")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
