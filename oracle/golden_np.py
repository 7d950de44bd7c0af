"""CPU oracle: a numpy restatement of the reference's bit-exact integer datapath.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (`llaccel_amd`) may import this
module; only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of
`bench.py` use it, and only as the checker.

Every function restates the semantics of `python/llaccel/golden.py` in the
reference (citations are `golden.py:<line>` there) and of `docs/NUMERICS.md`.
Arithmetic is int64 numpy or Python int, as in the reference; numpy's int64
multiply wraps modulo 2^64 exactly like the reference's does.

Heavy ops (`linear`, `attention`) can optionally run through the C restatement
in `oracle/numerics.c` (`backend="c"`), which is checked against this numpy
path on small cases by the test-suite.  The numpy path (`backend="np"`) is the
structure the reference uses (`a @ w.T` in int64, a Python loop per
(row, head) for attention) and is what `bench.py` times as the CPU baseline.

Pinning (what checks each function against something other than itself):
  rshr/sat*/mulshift : closed forms over the integers (Python big ints), the
                       reference KATs (test_golden_primitives.py:16-36), full
                       i64 domain (test_rounding_boundaries.py:5-16) and the
                       reference numerics.h built into oracle/_ref.
  isqrt48            : math.isqrt; numerics.h.
  udiv               : Python floor division; KATs test_golden_primitives.py:45-49.
  LUTs               : constants committed in the reference's include/llaccel/luts.h
                       (fixture tests/golden/luts_ref.json).
  silu16, vmul, vadd, vquant, rmsnorm, rope, attention_head:
                       KATs/invariants of test_golden_primitives.py and
                       test_rounding_boundaries.py, and numerics.h (oracle/_ref).
  linear             : brute-force integer matmul + the scalar epilogue.
  GoldenModel composition : golden.json/KV fixtures written by the reference
                       golden.py itself (tests/golden/), plus the invariants of
                       the reference's test_golden_e2e.py.
"""
from __future__ import annotations

import ctypes
import json
import math
import os
from pathlib import Path

import numpy as np

I64 = np.int64
_HERE = Path(__file__).resolve().parent


# --------------------------------------------------------------------------------------
# LUTs (luts.py:18-29; NUMERICS.md "SiLU" and "Attention"): Python round = half-even.
# --------------------------------------------------------------------------------------
def sigmoid_table() -> np.ndarray:
    """SIG[j] = round(65536 * sigmoid(-8 + j/16)), j = 0..256, capped at 65535 (luts.py:18-21)."""
    out = []
    for j in range(257):
        x = -8.0 + j / 16.0
        out.append(min(65535, round(65536.0 / (1.0 + math.exp(-x)))))
    return np.array(out, dtype=np.uint16)


def exp_int_table() -> np.ndarray:
    """EXPI[i] = round(65535 * e^-i), i = 0..15 (luts.py:24-25)."""
    return np.array([round(65535 * math.exp(-i)) for i in range(16)], dtype=np.uint16)


def exp_frac_table() -> np.ndarray:
    """EXPF[f] = round(65535 * e^(-f/256)), f = 0..255 (luts.py:28-29)."""
    return np.array([round(65535 * math.exp(-f / 256.0)) for f in range(256)], dtype=np.uint16)


SIG = sigmoid_table().astype(I64)
EXPI = exp_int_table().astype(I64)
EXPF = exp_frac_table().astype(I64)


# --------------------------------------------------------------------------------------
# Primitives (golden.py:35-120)
# --------------------------------------------------------------------------------------
def rshr(v, s):
    """Round-half-up arithmetic right shift (golden.py:35-45, NUMERICS.md:15-18).

    s == 0 leaves v unchanged; otherwise (v >> s) + bit (s-1) of v.  `s` may be a
    scalar or an array broadcast against v."""
    v = np.asarray(v, dtype=I64)
    s = np.asarray(s, dtype=I64)
    s1 = np.maximum(s, I64(1))
    shifted = (v >> s1) + ((v >> (s1 - I64(1))) & I64(1))
    out = np.where(s == 0, v, shifted)
    return out.astype(I64)


def sat8(v):
    """Clamp to [-128, 127] (golden.py:48-49)."""
    return np.clip(np.asarray(v, dtype=I64), -128, 127)


def satu8(v):
    """Clamp to [0, 255] (golden.py:52-53)."""
    return np.clip(np.asarray(v, dtype=I64), 0, 255)


def sat16(v):
    """Clamp to [-32768, 32767] (golden.py:56-57)."""
    return np.clip(np.asarray(v, dtype=I64), -32768, 32767)


def satu16(v):
    """Clamp to [0, 65535] (golden.py:60-61)."""
    return np.clip(np.asarray(v, dtype=I64), 0, 65535)


def mulshift(v, M, S):
    """rshr(v * M, S) with the product in wrapping int64 (golden.py:64-65)."""
    return rshr(np.asarray(v, dtype=I64) * np.asarray(M, dtype=I64), S)


def isqrt48(t: int) -> int:
    """floor(sqrt(t)) for 0 <= t < 2^48 by the restoring bit-serial method, two bits per
    step for 24 steps (golden.py:68-81).  Out-of-range input raises ValueError."""
    t = int(t)
    if t < 0 or t >= 1 << 48:
        raise ValueError(f"isqrt48 input out of range: {t}")
    remainder = 0
    root = 0
    for step in range(24):
        shift = 2 * (23 - step)
        remainder = (remainder << 2) | ((t >> shift) & 3)
        candidate = (root << 2) | 1          # (2*root)*2 + 1 = trial divisor for the next root bit
        root <<= 1
        if candidate <= remainder:
            remainder -= candidate
            root |= 1
    return root


def udiv(a: int, b: int) -> int:
    """floor(a / max(b, 1)) truncated to u32; negative operands raise (golden.py:84-88)."""
    a, b = int(a), int(b)
    if a < 0 or b < 0:
        raise ValueError("udiv operands must be unsigned")
    return (a // max(b, 1)) & 0xFFFFFFFF


def requant16(acc, M, S):
    """sat16(mulshift(acc, M, S)) (golden.py:92-93)."""
    return sat16(mulshift(acc, M, S))


def requant8(acc, M, S):
    """sat8(mulshift(acc, M, S)) (golden.py:96-97)."""
    return sat8(mulshift(acc, M, S))


def silu16(x, Mi: int, Si: int, sh_out: int):
    """LUT SiLU with linear interpolation (golden.py:101-107, NUMERICS.md "SiLU")."""
    x = np.asarray(x, dtype=I64)
    u = sat16(mulshift(x, Mi, Si))            # Q3.12
    j = (u >> 8) + 128                        # 0..255
    frac = u & 255
    lo = SIG[j]
    hi = SIG[j + 1]
    sg = lo + (((hi - lo) * frac) >> 8)
    return sat16(rshr(x * sg, sh_out))


def vmul(a, b, sh: int):
    """sat16(rshr(a*b, sh)) (golden.py:111-112)."""
    return sat16(rshr(np.asarray(a, dtype=I64) * np.asarray(b, dtype=I64), sh))


def vadd(a, b, sh_b: int):
    """sat16(a + rshr(b, sh_b)) (golden.py:115-116)."""
    return sat16(np.asarray(a, dtype=I64) + rshr(b, sh_b))


def vquant(x, M: int, S: int):
    """sat8(mulshift(x, M, S)) (golden.py:119-120)."""
    return sat8(mulshift(x, M, S))


def rmsnorm_row(x, g, eps_t: int, C: int, sh_post: int):
    """Integer RMSNorm of one row (golden.py:124-132, NUMERICS.md "RMSNorm")."""
    x = np.asarray(x, dtype=I64)
    g = np.asarray(g, dtype=I64)
    ss = int((x * x).sum())
    r = isqrt48(ss + int(eps_t))
    inv = min(65535, udiv(C, max(r, 1)))
    return sat16(rshr((x * g) * I64(inv), sh_post))


def rmsnorm(x, g, eps_t: int, C: int, sh_post: int):
    """Row-wise RMSNorm over a [rows][K] matrix (golden.py:135-137)."""
    x = np.asarray(x, dtype=I64)
    out = np.empty_like(x)
    for i in range(x.shape[0]):
        out[i] = rmsnorm_row(x[i], g, eps_t, C, sh_post)
    return out


def rope_row(x, H: int, D: int, cosv, sinv):
    """rotate_half RoPE of one row of H heads (golden.py:141-152, NUMERICS.md "RoPE")."""
    x = np.asarray(x, dtype=I64).reshape(H, D)
    c = np.asarray(cosv, dtype=I64)
    s = np.asarray(sinv, dtype=I64)
    half = D // 2
    a, b = x[:, :half], x[:, half:]
    first = sat16(rshr(a * c - b * s, 14))
    second = sat16(rshr(b * c + a * s, 14))
    return np.concatenate([first, second], axis=1).reshape(H * D)


def rope(x, H: int, D: int, cos_tab, sin_tab, pos: int):
    """Row m uses table row pos + m (golden.py:155-158)."""
    x = np.asarray(x, dtype=I64)
    return np.stack([rope_row(x[m], H, D, cos_tab[pos + m], sin_tab[pos + m]) for m in range(x.shape[0])])


def attention_head(q, keys, vals, Ms: int, Ss: int, Mo: int, So: int, prob_bits: int = 8):
    """Integer softmax attention for one query row and one head (golden.py:162-180).

    Three global reductions, in order: max score, sum of LUT exponentials, then the
    probability-weighted value sum."""
    q = np.asarray(q, dtype=I64)
    keys = np.asarray(keys, dtype=I64)
    vals = np.asarray(vals, dtype=I64)
    s = keys @ q
    z = mulshift(I64(int(s.max())) - s, Ms, Ss)
    zc = np.minimum(z, 4095)
    p = np.where(z < 4096, (EXPI[zc >> 8] * EXPF[zc & 255] + (1 << 15)) >> 16, I64(0))
    inv = udiv(1 << 31, int(p.sum()))
    if prob_bits not in (8, 15):
        raise ValueError("attention prob_bits must be 8 or 15")
    pn = np.minimum(rshr(p * I64(inv), 31 - prob_bits), (1 << prob_bits) - 1)
    o = pn @ vals
    if prob_bits == 15:
        o = rshr(o, 7)
    return sat8(mulshift(o, Mo, So))


# --------------------------------------------------------------------------------------
# C restatement (oracle/numerics.c) for the heavy ops
# --------------------------------------------------------------------------------------
_CLIB = None


def c_oracle():
    """ctypes handle of oracle/liboracle.so (built by oracle/Makefile), or None."""
    global _CLIB
    if _CLIB is None:
        path = _HERE / "liboracle.so"
        if not path.exists():
            return None
        lib = ctypes.CDLL(str(path))
        p = ctypes.c_void_p
        i64 = ctypes.c_int64
        lib.orc_linear.argtypes = [p, i64, i64, p, i64, p, p, i64, p, i64, i64, i64, i64, i64, p]
        lib.orc_linear.restype = ctypes.c_int
        lib.orc_attention.argtypes = [p, i64, i64, i64, i64, i64, p, p, i64, i64, i64, i64, i64, i64, p]
        lib.orc_attention.restype = ctypes.c_int
        lib.orc_set_threads.argtypes = [ctypes.c_int]
        lib.orc_set_threads.restype = ctypes.c_int
        lib.orc_set_luts.argtypes = [p, p, p]
        lib.orc_rshr.argtypes = [i64, i64]
        lib.orc_rshr.restype = i64
        lib.orc_mulshift.argtypes = [i64, i64, i64]
        lib.orc_mulshift.restype = i64
        lib.orc_isqrt48.argtypes = [ctypes.c_uint64]
        lib.orc_isqrt48.restype = i64
        lib.orc_silu16.argtypes = [i64, i64, i64, i64]
        lib.orc_silu16.restype = i64
        lib.orc_rmsnorm_row.argtypes = [p, p, i64, i64, i64, i64, p]
        lib.orc_rmsnorm_row.restype = ctypes.c_int
        lib.orc_rope_row.argtypes = [p, i64, i64, p, p, p]
        lib.orc_attention_head.argtypes = [p, p, p, i64, i64, i64, i64, i64, i64, i64, p]
        lib.orc_attention_head.restype = ctypes.c_int
        tables = [np.ascontiguousarray(t, dtype=np.uint16) for t in (SIG, EXPI, EXPF)]
        lib.orc_set_luts(*[_ptr(t) for t in tables])
        lib._keep = tables
        _CLIB = lib
    return _CLIB


def _ptr(a: np.ndarray):
    return ctypes.c_void_p(a.ctypes.data) if a is not None else None


_EPI = {"none": 0, "resadd": 1, "silu": 2, "mul": 3}


def linear_c(a, w, rq, bias, out_i8: bool, epilogue: str, aux, aux_shift: int, silu: dict | None):
    """C twin of OracleModel.linear's arithmetic: i8 A x i8 W^T, bias, requant, epilogue."""
    lib = c_oracle()
    a8 = np.ascontiguousarray(a, dtype=np.int8)
    w8 = np.ascontiguousarray(w, dtype=np.int8)
    rq32 = np.ascontiguousarray(rq, dtype=np.int32)
    M, K = a8.shape
    N = w8.shape[0]
    b32 = None if bias is None else np.ascontiguousarray(bias, dtype=np.int32)
    aux16 = None if aux is None else np.ascontiguousarray(aux, dtype=np.int16)
    out = np.empty((M, N), dtype=np.int64)
    Mi, Si, sh = (0, 0, 0) if silu is None else (int(silu["Mi"]), int(silu["Si"]), int(silu["sh_out"]))
    rc = lib.orc_linear(_ptr(a8), M, K, _ptr(w8), N, _ptr(rq32), _ptr(b32), int(out_i8), _ptr(aux16),
                        int(aux_shift), _EPI[epilogue], Mi, Si, sh, _ptr(out))
    if rc != 0:
        raise ValueError(f"orc_linear failed ({rc})")
    return out


def attention_c(q, kc, vc, pos: int, H: int, Hkv: int, D: int, Ms, Ss, Mo, So, prob_bits):
    lib = c_oracle()
    q8 = np.ascontiguousarray(q, dtype=np.int8)
    M = q8.shape[0]
    out = np.empty((M, H * D), dtype=np.int64)
    rc = lib.orc_attention(_ptr(q8), M, H, Hkv, D, pos, _ptr(kc), _ptr(vc), kc.shape[1],
                           int(Ms), int(Ss), int(Mo), int(So), int(prob_bits), _ptr(out))
    if rc != 0:
        raise ValueError(f"orc_attention failed ({rc})")
    return out


# --------------------------------------------------------------------------------------
# qgraph loading (golden.py:186-214; DIALECT.md section 2)
# --------------------------------------------------------------------------------------
_DTYPES = {"i8": (np.dtype("i1"), 1), "i16": (np.dtype("<i2"), 1), "i32": (np.dtype("<i4"), 1), "rq": (np.dtype("<i4"), 2)}


class OracleQGraph:
    """qgraph.json + qweights.bin reader; tensors are zero-copy views of the blob (golden.py:189-214)."""

    def __init__(self, qdir) -> None:
        self.dir = Path(qdir)
        self.g = json.loads((self.dir / "qgraph.json").read_text())
        self.model = self.g["model"]
        self.ops = self.g["ops"]
        self.blob = np.memmap(self.dir / self.g["weights_file"], dtype=np.uint8, mode="r")
        self.tensors: dict[str, np.ndarray] = {}
        for name, spec in self.g["tensors"].items():
            dt, per = _DTYPES[spec["dtype"]]
            shape = [int(d) for d in spec["shape"]]
            n = int(np.prod(shape)) if shape else 1
            arr = np.frombuffer(self.blob, dtype=dt, count=n * per, offset=int(spec["offset"]))
            self.tensors[name] = arr.reshape(n, 2) if spec["dtype"] == "rq" else arr.reshape(shape)
        self.input_name = self.g.get("input", "input")
        self.output_name = self.g.get("output", "logits")


# --------------------------------------------------------------------------------------
# the model (golden.py:246-440)
# --------------------------------------------------------------------------------------
def exact_blas_matmul(a: np.ndarray, w: np.ndarray, chunk_rows: int = 1024) -> np.ndarray:
    """Integer A @ W.T through FP64 BLAS, exact because every product and partial sum stays below
    2^53 (golden.py:217-240): the same checks and errors, W converted chunk_rows rows at a time."""
    if a.ndim != 2 or w.ndim != 2 or a.shape[1] != w.shape[1]:
        raise ValueError("invalid matrix dimensions")
    if a.dtype.kind not in "iu" or w.dtype.kind not in "iu" or chunk_rows < 1:
        raise ValueError("exact BLAS requires integer inputs and positive chunks")
    amax = max(abs(int(a.min(initial=0))), abs(int(a.max(initial=0))))
    info = np.iinfo(w.dtype)
    if a.shape[1] * amax * max(abs(int(info.min)), abs(int(info.max))) > (1 << 53):
        raise ValueError("integer dot product exceeds exact FP64 accumulation bound")
    af = a.astype(np.float64)
    out = np.empty((a.shape[0], w.shape[0]), dtype=I64)
    for lo in range(0, w.shape[0], chunk_rows):
        hi = min(lo + chunk_rows, w.shape[0])
        out[:, lo:hi] = (af @ w[lo:hi].astype(np.float64).T).astype(I64)
    return out


class OracleModel:
    """CPU restatement of GoldenModel.  `backend` is "np" (reference structure: int64 a @ w.T and a
    Python loop per (row, head) for attention), "blas" (the reference's fast_matmul path: the
    GEMMs through exact_blas_matmul, golden.py:217-240, with all BLAS threads) or "c"
    (oracle/numerics.c, OpenMP)."""

    def __init__(self, qdir, backend: str = "np") -> None:
        if backend not in ("np", "blas", "c"):
            raise ValueError(f"unknown oracle backend {backend!r}")
        if backend == "c" and c_oracle() is None:
            raise RuntimeError("oracle/liboracle.so is not built (make -C oracle)")
        self.backend = backend
        self.q = OracleQGraph(qdir)
        m = self.q.model
        self.dim = int(m["dim"])
        self.n_layers = int(m["n_layers"])
        self.vocab = int(m["vocab"])
        self.vocab_padded = int(m.get("vocab_padded", self.vocab))
        self.max_seq = int(m["max_seq"])
        self.prefill_m = int(m.get("prefill_m", 16))
        if not (1 <= self.prefill_m <= 16) or self.max_seq % self.prefill_m != 0:
            raise ValueError("max_seq must be divisible by prefill_m in [1,16]")
        self.E_RES = int(m["E_RES"])
        self.E_LOGIT = int(m["E_LOGIT"])
        self.embed = self.q.tensors["embed"]
        self.rope_cos = self.q.tensors["rope_cos"]
        self.rope_sin = self.q.tensors["rope_sin"]
        self.reset()

    def reset(self) -> None:
        """Zeroed (Hkv, max_seq, D) int8 K and V per layer (golden.py:266-272)."""
        self.kv = {}
        for op in self.q.ops:
            if op["op"] == "kv_write":
                shape = (int(op["Hkv"]), self.max_seq, int(op["D"]))
                self.kv[int(op["layer"])] = (np.zeros(shape, np.int8), np.zeros(shape, np.int8))

    def run_chunk(self, rows, pos: int, acts: dict | None = None) -> np.ndarray:
        """Op interpreter (golden.py:275-314)."""
        rows = np.asarray(rows, dtype=I64)
        M = rows.shape[0]
        if pos < 0 or pos + M > self.max_seq:
            raise ValueError(f"positions {pos}..{pos + M - 1} exceed max_seq={self.max_seq}")
        env = {self.q.input_name: rows}
        T = self.q.tensors
        for op in self.q.ops:
            kind = op["op"]
            if kind == "rmsnorm":
                x = env[op["in"]]
                g = T[op["gamma"]]
                heads = int(op.get("heads", 1))
                if heads < 1 or x.shape[1] != heads * len(g):
                    raise ValueError("RMSNorm head geometry mismatch")
                y = rmsnorm(x.reshape(-1, len(g)), g, op["eps_t"], op["C"], op["sh_post"])
                env[op["out"]] = y.reshape(x.shape)
            elif kind == "quant":
                env[op["out"]] = vquant(env[op["in"]], op["M"], op["S"])
            elif kind == "linear":
                env[op["out"]] = self.linear(op, env)
            elif kind == "rope":
                env[op["out"]] = rope(env[op["in"]], op["H"], op["D"], self.rope_cos, self.rope_sin, pos)
            elif kind == "kv_write":
                self.kv_write(op, env, pos)
            elif kind == "attention":
                env[op["out"]] = self.attention(op, env, pos)
            elif kind == "add":
                env[op["out"]] = vadd(env[op["a"]], env[op["b"]], op["sh_b"])
            elif kind == "mul":
                env[op["out"]] = vmul(env[op["a"]], env[op["b"]], op["sh"])
            elif kind == "silu":
                env[op["out"]] = silu16(env[op["in"]], op["Mi"], op["Si"], op["sh_out"])
            else:
                raise ValueError(f"unknown qgraph op {kind!r}")
        if acts is not None:
            acts.update(env)
        return env[self.q.output_name]

    def linear(self, op: dict, env: dict) -> np.ndarray:
        """gemm engine: acc = A W^T (+bias), requant, epilogue (golden.py:316-342)."""
        a = env[op["in"]]
        w = self.q.tensors[op["w"]]
        rq = self.q.tensors[op["rq"]]
        N, K = int(op["N"]), int(op["K"])
        if w.shape != (N, K) or a.shape[1] != K:
            raise ValueError(f"linear {op['out']}: shapes A{a.shape} W{w.shape} vs N={N} K={K}")
        out_i8 = op.get("out_dtype", "i16") == "i8"
        ep = op.get("epilogue", "none")
        if out_i8 and ep != "none":
            raise ValueError("i8 output is only valid with epilogue none")
        if ep not in _EPI:
            raise ValueError(f"unknown epilogue {ep!r}")
        bias = self.q.tensors[op["bias"]] if op.get("bias") else None
        aux = env[op["aux"]] if ep in ("resadd", "mul") else None
        if self.backend == "c":
            return linear_c(a, w, rq, bias, out_i8, ep, aux, int(op.get("aux_shift", 0)), op.get("silu"))
        acc = exact_blas_matmul(a, w) if self.backend == "blas" else a @ w.astype(I64).T
        if bias is not None:
            acc = acc + bias.astype(I64)[None, :]
        Mn = rq[:, 0].astype(I64)[None, :]
        Sn = rq[:, 1].astype(I64)[None, :]
        if out_i8:
            return requant8(acc, Mn, Sn)
        t = requant16(acc, Mn, Sn)
        if ep == "none":
            return t
        if ep == "resadd":
            return sat16(t + aux)
        if ep == "silu":
            s = op["silu"]
            return silu16(t, s["Mi"], s["Si"], s["sh_out"])
        return sat16(rshr(t * aux, op["aux_shift"]))

    def kv_write(self, op: dict, env: dict, pos: int) -> None:
        """Row m, KV head h -> cache[h, pos+m] (golden.py:344-351)."""
        kc, vc = self.kv[int(op["layer"])]
        Hkv, D = int(op["Hkv"]), int(op["D"])
        k, v = env[op["k"]], env[op["v"]]
        M = k.shape[0]
        kc[:, pos:pos + M, :] = k.reshape(M, Hkv, D).transpose(1, 0, 2)
        vc[:, pos:pos + M, :] = v.reshape(M, Hkv, D).transpose(1, 0, 2)

    def attention(self, op: dict, env: dict, pos: int) -> np.ndarray:
        """Causal GQA attention: row m sees keys 0..pos+m; head h reads KV head h // (H/Hkv)
        (golden.py:353-366)."""
        q = env[op["q"]]
        kc, vc = self.kv[int(op["layer"])]
        H, Hkv, D = int(op["H"]), int(op["Hkv"]), int(op["D"])
        pb = op.get("prob_bits", 8)
        if self.backend == "c":
            if pb not in (8, 15):
                raise ValueError("attention prob_bits must be 8 or 15")
            return attention_c(q, kc, vc, pos, H, Hkv, D, op["Ms"], op["Ss"], op["Mo"], op["So"], pb)
        group = H // Hkv
        M = q.shape[0]
        out = np.zeros((M, H * D), I64)
        for m in range(M):
            T = pos + m + 1
            for h in range(H):
                g = h // group
                out[m, h * D:(h + 1) * D] = attention_head(q[m, h * D:(h + 1) * D], kc[g, :T], vc[g, :T],
                                                           op["Ms"], op["Ss"], op["Mo"], op["So"], pb)
        return out

    def embed_rows(self, tokens, M: int) -> np.ndarray:
        """Embedding rows for `tokens`, zero pad rows up to M (golden.py:369-373)."""
        rows = np.zeros((M, self.dim), I64)
        for i, t in enumerate(tokens):
            rows[i] = self.embed[int(t)]
        return rows

    @staticmethod
    def argmax(logits_row, vocab: int) -> int:
        """First maximum over the first `vocab` logits (golden.py:376-377)."""
        return int(np.argmax(np.asarray(logits_row)[:vocab]))

    def prefill(self, tokens, acts: list | None = None) -> list:
        """Chunks of prefill_m rows at positions start.. (golden.py:379-390)."""
        tokens = [int(t) for t in tokens]
        out = []
        for start in range(0, len(tokens), self.prefill_m):
            chunk = tokens[start:start + self.prefill_m]
            a = {} if acts is not None else None
            logits = self.run_chunk(self.embed_rows(chunk, self.prefill_m), start, a)
            if acts is not None:
                acts.append({"kind": "prefill", "pos": start, "rows": self.prefill_m, "valid_rows": len(chunk), "acts": a})
            out.extend(logits[:len(chunk)])
        return out

    def decode(self, token: int, pos: int, acts: list | None = None) -> np.ndarray:
        """One M=1 launch (golden.py:392-397)."""
        a = {} if acts is not None else None
        logits = self.run_chunk(self.embed_rows([token], 1), pos, a)
        if acts is not None:
            acts.append({"kind": "decode", "pos": pos, "rows": 1, "valid_rows": 1, "acts": a})
        return logits[0]

    def generate(self, prompt_tokens, n_tokens: int, acts: list | None = None, *, max_decode_launches=None) -> dict:
        """Greedy generation and the golden.json record (golden.py:399-440).

        `max_decode_launches` (oracle-only) stops after that many decode launches, so a
        bounded CPU sample of a long run can be timed or compared; None = the full run."""
        if not isinstance(n_tokens, int) or n_tokens < 0:
            raise ValueError("n_tokens must be a nonnegative integer")
        prompt = [int(t) for t in prompt_tokens]
        if not prompt:
            raise ValueError("empty prompt")
        if len(prompt) + n_tokens > self.max_seq:
            raise ValueError(f"prompt + tokens = {len(prompt) + n_tokens} exceeds max_seq={self.max_seq}")
        self.reset()
        steps, amax, rows_rec = [], [], []

        def record(kind, pos, valid, row):
            steps.append({"kind": kind, "pos": pos, "rows": self.prefill_m if kind == "prefill" else 1, "valid_rows": valid})
            amax.append(self.argmax(row, self.vocab))
            rows_rec.append([int(v) for v in row[:self.vocab]])
            return amax[-1]

        rows = self.prefill(prompt, acts)
        L = len(prompt)
        nxt = -1
        for c in range((L + self.prefill_m - 1) // self.prefill_m):
            last = min(L, (c + 1) * self.prefill_m) - 1
            nxt = record("prefill", c * self.prefill_m, last + 1 - c * self.prefill_m, rows[last])
        generated = []
        for i in range(n_tokens):
            generated.append(nxt)
            if L + i + 1 >= self.max_seq:
                break
            if max_decode_launches is not None and i >= max_decode_launches:
                break
            nxt = record("decode", L + i, 1, self.decode(nxt, L + i, acts))
        return {"prompt_tokens": prompt, "generated": generated, "argmax_per_step": amax,
                "logits_last_rows": rows_rec, "steps": steps,
                "model": {"vocab": self.vocab, "vocab_padded": self.vocab_padded, "E_LOGIT": self.E_LOGIT,
                          "E_RES": self.E_RES, "max_seq": self.max_seq}}


def set_threads(n: int) -> None:
    lib = c_oracle()
    if lib is not None:
        lib.orc_set_threads(int(n))


if os.environ.get("LLACCEL_ORACLE_THREADS"):
    set_threads(int(os.environ["LLACCEL_ORACLE_THREADS"]))
