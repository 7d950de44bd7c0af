"""Seeded synthetic quantized graphs (qgraph.json + qweights.bin) for the benchmark configs.

Produces the input format of the integer datapath (reference docs/DIALECT.md section 2,
read by python/llaccel/golden.py:189-214) from a random-init float Llama/Qwen decoder:

1. float weights: N(0, 0.02) linears and embedding, RMSNorm gamma 1 (Q/K-norm gamma
   uniform [0.75, 1.25]), optional QKV bias uniform +-0.03;
2. a float forward over a seeded calibration sequence records the abs-max of every named
   activation (the role of the reference's calib.json);
3. integer parameters follow the "Compiler:" lines of the reference's docs/NUMERICS.md:
   per-channel int8 weights (max|w[n,:]|/127), i16 exponents
   e = max(ceil(log2(absmax/32767)), -15), (M, S) pairs normalised to M in [2^30, 2^31),
   RMSNorm (eps_t, C, sh_post), SiLU (Mi, Si, sh_out), MUL/ADD shifts, attention
   (Ms, Ss, Mo, So) and Q1.14 RoPE tables.

Residual-stream values (input, o, x1, d, x2) share one exponent E_RES so every residual
ADD has sh_b = 0 and the v2 (fused) graph can use the RESADD epilogue; the v1 graph keeps
explicit add/silu/mul ops.  Both are bit-identical by the datapath's definition.

Unlike the reference's quantizer this producer accepts head_dim 128/256, Q/K-norm and
widths that are not multiples of 16 (the datapath itself has no such restriction).
"""
from __future__ import annotations

import dataclasses
import json
import math
from pathlib import Path

import numpy as np


@dataclasses.dataclass(frozen=True)
class ModelConfig:
    name: str
    dim: int
    n_layers: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    ffn: int
    vocab: int
    max_seq: int
    qkv_bias: bool = False
    qk_norm: bool = False
    rope_base: float = 10000.0
    rms_eps: float = 1e-5
    prefill_m: int = 16

    @property
    def vocab_padded(self) -> int:
        return (self.vocab + 15) // 16 * 16


# BASELINE.json configs 1, 3, 4, 5 (config 2 is the isolated GEMM sweep).
CONFIGS = {
    "tiny": ModelConfig("tiny", 64, 2, 4, 2, 16, 172, 256, 64),
    "smol": ModelConfig("smol", 576, 30, 9, 3, 64, 1536, 49152, 256),
    "qwen25": ModelConfig("qwen25", 896, 24, 14, 2, 64, 4864, 151936, 1024, qkv_bias=True, rope_base=1e6, rms_eps=1e-6),
    "qwen3": ModelConfig("qwen3", 1024, 28, 16, 8, 128, 3072, 151936, 4096, qk_norm=True, rope_base=1e6, rms_eps=1e-6),
}


# --------------------------------------------------------------------------------------
# float -> integer parameter rules (docs/NUMERICS.md "Compiler:" lines)
# --------------------------------------------------------------------------------------
def round_away(x):
    """Nearest integer, ties away from zero (the compiler's float->int rounding, NUMERICS.md)."""
    x = np.asarray(x, dtype=np.float64)
    return (np.sign(x) * np.floor(np.abs(x) + 0.5)).astype(np.int64)


def mulshift_pair(r):
    """(M, S) with M * 2^-S ~= r, M in [2^30, 2^31), 0 <= S <= 63 (vectorised; r > 0)."""
    r = np.asarray(r, dtype=np.float64)
    if np.any(~np.isfinite(r)) or np.any(r <= 0):
        raise ValueError("mulshift ratio must be positive and finite")
    f, e = np.frexp(r)
    M = round_away(np.ldexp(f, 31))
    S = 31 - e.astype(np.int64)
    top = M >= (1 << 31)
    M = np.where(top, 1 << 30, M)
    S = np.where(top, S - 1, S)
    if np.any(S < 0):
        raise ValueError("mulshift ratio too large")
    tiny = S > 63
    if np.any(tiny):
        M = np.where(tiny, round_away(np.ldexp(r, 63)), M)
        S = np.where(tiny, 63, S)
    return M.astype(np.int64), S.astype(np.int64)


def scalar_pair(r: float) -> tuple[int, int]:
    M, S = mulshift_pair(np.array([r]))
    return int(M[0]), int(S[0])


def i16_exp(absmax: float) -> int:
    if not absmax > 0:
        return -15
    return max(int(math.ceil(math.log2(absmax) - math.log2(32767.0))), -15)


def i8_scale(absmax: float) -> float:
    return absmax / 127.0 if absmax > 0 else 1.0


def quant_rows_i8(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Per-output-channel symmetric int8: s[n] = max|w[n,:]|/127 (zero rows -> 1)."""
    mx = np.abs(w).max(axis=1).astype(np.float64)
    s = np.where(mx > 0, mx / 127.0, 1.0)
    q = np.clip(round_away(w.astype(np.float64) / s[:, None]), -128, 127).astype(np.int8)
    return q, s


def quant_i16(x: np.ndarray, e: int) -> np.ndarray:
    return np.clip(round_away(np.ldexp(np.asarray(x, dtype=np.float64), -e)), -32768, 32767).astype(np.int16)


def rope_tables_q14(max_seq: int, D: int, base: float):
    half = D // 2
    theta = base ** (-2.0 * np.arange(half, dtype=np.float64) / D)
    ang = np.arange(max_seq, dtype=np.float64)[:, None] * theta[None, :]
    c = np.minimum(round_away(16384.0 * np.cos(ang)), 32767).astype(np.int16)
    s = np.minimum(round_away(16384.0 * np.sin(ang)), 32767).astype(np.int16)
    return c, s


def rmsnorm_int_params(K: int, eps: float, e_x: int, e_g: int, e_y: int, absmax_x: float) -> dict:
    """eps_t = round(eps K 2^-2e_x); largest R <= 31 with C = round(2^R sqrt K) < 2^32 and the
    typical reciprocal floor(C / r) below 65535/4 (r from rms ~ absmax/4); sh_post = R - e_g + e_y."""
    eps_t = int(round_away(eps * K * 2.0 ** (-2 * e_x)))
    if not 0 <= eps_t < 2**32:
        raise ValueError("rmsnorm eps_t does not fit u32")
    rms_q = (absmax_x / 4.0) / 2.0**e_x
    r_typ = max(1.0, math.floor(math.sqrt(K * rms_q * rms_q + eps_t)))
    for R in range(31, -1, -1):
        C = int(round_away(math.ldexp(math.sqrt(K), R)))
        if C < 2**32 and math.floor(C / r_typ) < 65535.0 / 4.0:
            sh = R - e_g + e_y
            if not 0 <= sh <= 63:
                raise ValueError(f"rmsnorm sh_post {sh} out of range")
            return {"eps_t": eps_t, "C": C, "sh_post": sh}
    raise ValueError("rmsnorm: no R keeps the reciprocal in range")


# --------------------------------------------------------------------------------------
# float model + calibration
# --------------------------------------------------------------------------------------
def float_weights(cfg: ModelConfig, seed: int) -> dict[str, np.ndarray]:
    rng = np.random.default_rng(seed)
    W: dict[str, np.ndarray] = {}

    def normal(*shape):
        return (rng.standard_normal(shape, dtype=np.float32) * np.float32(0.02))

    dim, H, Hkv, D, F = cfg.dim, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.ffn
    W["embed"] = normal(cfg.vocab, dim)
    for i in range(cfg.n_layers):
        p = f"l{i}"
        W[f"{p}_attn_norm"] = np.ones(dim, np.float32)
        W[f"{p}_wq"] = normal(H * D, dim)
        W[f"{p}_wk"] = normal(Hkv * D, dim)
        W[f"{p}_wv"] = normal(Hkv * D, dim)
        if cfg.qkv_bias:
            for b, n in (("bq", H * D), ("bk", Hkv * D), ("bv", Hkv * D)):
                W[f"{p}_{b}"] = rng.uniform(-0.03, 0.03, n).astype(np.float32)
        if cfg.qk_norm:
            W[f"{p}_q_norm"] = rng.uniform(0.75, 1.25, D).astype(np.float32)
            W[f"{p}_k_norm"] = rng.uniform(0.75, 1.25, D).astype(np.float32)
        W[f"{p}_wo"] = normal(dim, H * D)
        W[f"{p}_ffn_norm"] = np.ones(dim, np.float32)
        W[f"{p}_wg"] = normal(F, dim)
        W[f"{p}_wu"] = normal(F, dim)
        W[f"{p}_wd"] = normal(dim, F)
    W["norm"] = np.ones(dim, np.float32)
    W["lm_head"] = normal(cfg.vocab, dim)
    return W


def _rms(x, g, eps):
    return x / np.sqrt(np.mean(x.astype(np.float64) ** 2, axis=-1, keepdims=True) + eps).astype(np.float32) * g


def _rope_f(x, H, D, pos0, base):
    T = x.shape[0]
    half = D // 2
    theta = base ** (-2.0 * np.arange(half) / D)
    ang = (np.arange(pos0, pos0 + T)[:, None] * theta[None, :]).astype(np.float32)
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    xh = x.reshape(T, H, D)
    a, b = xh[..., :half], xh[..., half:]
    return np.concatenate([a * c - b * s, b * c + a * s], -1).reshape(T, H * D)


def calibrate(cfg: ModelConfig, W: dict, tokens: list[int]) -> dict[str, float]:
    """Float forward; returns abs-max per named activation."""
    amax: dict[str, float] = {}

    def rec(name, v):
        amax[name] = max(amax.get(name, 0.0), float(np.abs(v).max()))
        return v

    dim, H, Hkv, D = cfg.dim, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
    T = len(tokens)
    x = rec("input", W["embed"][np.asarray(tokens)])
    causal = np.triu(np.full((T, T), -np.inf, np.float32), 1)
    for i in range(cfg.n_layers):
        p = f"l{i}"
        h = rec(f"{p}.h", _rms(x, W[f"{p}_attn_norm"], cfg.rms_eps))
        q = h @ W[f"{p}_wq"].T
        k = h @ W[f"{p}_wk"].T
        v = h @ W[f"{p}_wv"].T
        if cfg.qkv_bias:
            q, k, v = q + W[f"{p}_bq"], k + W[f"{p}_bk"], v + W[f"{p}_bv"]
        rec(f"{p}.q", q)
        rec(f"{p}.k", k)
        rec(f"{p}.v", v)
        if cfg.qk_norm:
            q = rec(f"{p}.qn", _rms(q.reshape(T, H, D), W[f"{p}_q_norm"], cfg.rms_eps).reshape(T, H * D))
            k = rec(f"{p}.kn", _rms(k.reshape(T, Hkv, D), W[f"{p}_k_norm"], cfg.rms_eps).reshape(T, Hkv * D))
        qr = rec(f"{p}.qr", _rope_f(q, H, D, 0, cfg.rope_base))
        kr = rec(f"{p}.kr", _rope_f(k, Hkv, D, 0, cfg.rope_base))
        rep = H // Hkv
        qh = qr.reshape(T, H, D).transpose(1, 0, 2)
        kh = np.repeat(kr.reshape(T, Hkv, D).transpose(1, 0, 2), rep, axis=0)
        vh = np.repeat(v.reshape(T, Hkv, D).transpose(1, 0, 2), rep, axis=0)
        sc = qh @ kh.transpose(0, 2, 1) / np.float32(math.sqrt(D)) + causal
        sc = np.exp(sc - sc.max(-1, keepdims=True))
        sc /= sc.sum(-1, keepdims=True)
        a = rec(f"{p}.a", (sc @ vh).transpose(1, 0, 2).reshape(T, H * D))
        o = rec(f"{p}.o", a @ W[f"{p}_wo"].T)
        x1 = rec(f"{p}.x1", x + o)
        h2 = rec(f"{p}.h2", _rms(x1, W[f"{p}_ffn_norm"], cfg.rms_eps))
        g = rec(f"{p}.g", h2 @ W[f"{p}_wg"].T)
        u = rec(f"{p}.u", h2 @ W[f"{p}_wu"].T)
        sg = rec(f"{p}.sg", g / (1 + np.exp(-g)))
        f = rec(f"{p}.f", sg * u)
        d = rec(f"{p}.d", f @ W[f"{p}_wd"].T)
        x = rec(f"{p}.x2", x1 + d)
    hn = rec("hn", _rms(x, W["norm"], cfg.rms_eps))
    rec("logits", hn @ W["lm_head"].T)
    return amax


# --------------------------------------------------------------------------------------
# qweights.bin writer + op emission
# --------------------------------------------------------------------------------------
class _Blob:
    """Tensors concatenated at 64-byte aligned offsets (DIALECT.md section 2 layout)."""

    def __init__(self):
        self.chunks: list[bytes] = []
        self.size = 0
        self.tensors: dict[str, dict] = {}

    def put(self, name: str, arr: np.ndarray, dtype: str, exp: int | None = None):
        if name in self.tensors:
            raise ValueError(f"duplicate tensor {name}")
        np_dt = {"i8": "<i1", "i16": "<i2", "i32": "<i4", "rq": "<i4"}[dtype]
        data = np.ascontiguousarray(arr).astype(np_dt, copy=False).tobytes()
        shape = list(arr.shape[:-1]) if dtype == "rq" else list(arr.shape)
        spec = {"dtype": dtype, "shape": [int(s) for s in shape], "offset": self.size}
        if exp is not None:
            spec["exp"] = int(exp)
        self.tensors[name] = spec
        self.chunks.append(data)
        self.size += len(data)
        pad = -len(data) % 64
        if pad:
            self.chunks.append(bytes(pad))
            self.size += pad


def build_qgraph(out_dir, cfg: ModelConfig | str, *, seed: int = 0, fusion: bool = True, calib_len: int = 32,
                 weights: dict | None = None) -> Path:
    """Write `out_dir/qgraph.json` and `out_dir/qweights.bin`; returns out_dir."""
    if isinstance(cfg, str):
        cfg = CONFIGS[cfg]
    out = Path(out_dir)
    out.mkdir(parents=True, exist_ok=True)
    W = weights if weights is not None else float_weights(cfg, seed)
    crng = np.random.default_rng(seed + 1000)
    amax = calibrate(cfg, W, crng.integers(0, cfg.vocab, min(calib_len, cfg.max_seq)).tolist())

    dim, L, H, Hkv, D, F = cfg.dim, cfg.n_layers, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.ffn
    blob = _Blob()
    ops: list[dict] = []
    exps: dict[str, int] = {}
    scales: dict[str, float] = {}

    res_names = ["input"] + [f"l{i}.{n}" for i in range(L) for n in ("o", "x1", "d", "x2")]
    E_RES = max(i16_exp(amax[n]) for n in res_names)
    for n in res_names:
        exps[n] = E_RES

    def e16(name):
        if name not in exps:
            exps[name] = i16_exp(amax[name])
        return exps[name]

    def s8(name, src=None):
        if name not in scales:
            scales[name] = i8_scale(amax[src or name.removesuffix(".q")])
        return scales[name]

    def rmsnorm(x, gamma, y, heads=1):
        g = W[gamma]
        e_g = i16_exp(float(np.abs(g).max()))
        blob.put(gamma, quant_i16(g, e_g), "i16", e_g)
        K = int(g.shape[0])
        prm = rmsnorm_int_params(K, cfg.rms_eps, e16(x), e_g, e16(y), amax[x])
        op = {"op": "rmsnorm", "in": x, "gamma": gamma, "out": y, "K": K, **prm}
        if heads != 1:
            op["heads"] = heads
        ops.append(op)

    def quant(x):
        y = x + ".q"
        M, S = scalar_pair(2.0 ** e16(x) / s8(y, x))
        ops.append({"op": "quant", "in": x, "out": y, "M": M, "S": S})
        return y

    def linear(a, w, b, y, out_dtype, *, e_rq=None, n_pad=None, epilogue="none", aux=None, aux_shift=0, silu=None):
        wf = W[w]
        if n_pad is not None and n_pad != wf.shape[0]:
            wf = np.concatenate([wf, np.zeros((n_pad - wf.shape[0], wf.shape[1]), wf.dtype)])
        N, K = wf.shape
        wq, sw = quant_rows_i8(wf)
        blob.put(w, wq, "i8")
        sa = s8(a)
        if out_dtype == "i16":
            r = sa * sw / 2.0 ** (e16(y) if e_rq is None else e_rq)
        else:
            r = sa * sw / s8(y)
        M, S = mulshift_pair(r)
        blob.put(w + ".rq", np.stack([M, S], 1), "rq")
        bias = None
        if b is not None and b in W:
            bf = np.zeros(N)
            bf[:W[b].shape[0]] = W[b]
            bq = np.clip(round_away(bf / (sa * sw)), -(2**31), 2**31 - 1)
            blob.put(b, bq, "i32")
            bias = b
        ops.append({"op": "linear", "in": a, "w": w, "rq": w + ".rq", "bias": bias, "out": y, "N": int(N), "K": int(K),
                    "out_dtype": out_dtype, "epilogue": epilogue, "aux": aux, "aux_shift": int(aux_shift), "silu": silu})

    emb = np.zeros((cfg.vocab_padded, dim), np.float32)
    emb[:cfg.vocab] = W["embed"]
    blob.put("embed", quant_i16(emb, E_RES), "i16", E_RES)
    cos_t, sin_t = rope_tables_q14(cfg.max_seq, D, cfg.rope_base)
    blob.put("rope_cos", cos_t, "i16")
    blob.put("rope_sin", sin_t, "i16")

    resid = "input"
    for i in range(L):
        p = f"l{i}"
        rmsnorm(resid, f"{p}_attn_norm", f"{p}.h")
        hq = quant(f"{p}.h")
        qs, ks = (f"{p}.qn", f"{p}.kn") if cfg.qk_norm else (f"{p}.q", f"{p}.k")
        for src, dst in ((qs, f"{p}.qr"), (ks, f"{p}.kr")):   # RoPE keeps the exponent
            exps[src] = exps[dst] = max(i16_exp(amax[src]), i16_exp(amax[dst]))
        linear(hq, f"{p}_wq", f"{p}_bq", f"{p}.q", "i16")
        linear(hq, f"{p}_wk", f"{p}_bk", f"{p}.k", "i16")
        linear(hq, f"{p}_wv", f"{p}_bv", f"{p}.v", "i8")
        if cfg.qk_norm:
            rmsnorm(f"{p}.q", f"{p}_q_norm", qs, heads=H)
            rmsnorm(f"{p}.k", f"{p}_k_norm", ks, heads=Hkv)
        ops.append({"op": "rope", "in": qs, "out": f"{p}.qr", "H": H, "D": D})
        ops.append({"op": "rope", "in": ks, "out": f"{p}.kr", "H": Hkv, "D": D})
        qq, kq = quant(f"{p}.qr"), quant(f"{p}.kr")
        ops.append({"op": "kv_write", "layer": i, "k": kq, "v": f"{p}.v", "Hkv": Hkv, "D": D})
        Ms, Ss = scalar_pair(256.0 * s8(qq) * s8(kq) / math.sqrt(D))
        Mo, So = scalar_pair(s8(f"{p}.v") / (256.0 * s8(f"{p}.a")))
        ops.append({"op": "attention", "q": qq, "layer": i, "out": f"{p}.a", "H": H, "Hkv": Hkv, "D": D,
                    "prob_bits": 15, "Ms": Ms, "Ss": Ss, "Mo": Mo, "So": So})
        if fusion:
            linear(f"{p}.a", f"{p}_wo", None, f"{p}.x1", "i16", e_rq=E_RES, epilogue="resadd", aux=resid)
        else:
            linear(f"{p}.a", f"{p}_wo", None, f"{p}.o", "i16")
            ops.append({"op": "add", "a": resid, "b": f"{p}.o", "out": f"{p}.x1", "sh_b": 0})
        rmsnorm(f"{p}.x1", f"{p}_ffn_norm", f"{p}.h2")
        h2q = quant(f"{p}.h2")
        e_g, e_u, e_sg, e_f = (e16(f"{p}.{n}") for n in ("g", "u", "sg", "f"))
        Si, sh_out = 30 - (e_g + 12), 16 + e_sg - e_g
        sh_mul = e_f - e_sg - e_u
        for what, val in (("Si", Si), ("sh_out", sh_out), ("mul sh", sh_mul)):
            if not 0 <= val <= 63:
                raise ValueError(f"{p}: {what} = {val} out of range")
        silu = {"Mi": 1 << 30, "Si": Si, "sh_out": sh_out}
        if fusion:
            linear(h2q, f"{p}_wg", None, f"{p}.sg", "i16", e_rq=e_g, epilogue="silu", silu=silu)
            linear(h2q, f"{p}_wu", None, f"{p}.f", "i16", e_rq=e_u, epilogue="mul", aux=f"{p}.sg", aux_shift=sh_mul)
        else:
            linear(h2q, f"{p}_wg", None, f"{p}.g", "i16")
            linear(h2q, f"{p}_wu", None, f"{p}.u", "i16")
            ops.append({"op": "silu", "in": f"{p}.g", "out": f"{p}.sg", **silu})
            ops.append({"op": "mul", "a": f"{p}.sg", "b": f"{p}.u", "out": f"{p}.f", "sh": sh_mul})
        fq = quant(f"{p}.f")
        if fusion:
            linear(fq, f"{p}_wd", None, f"{p}.x2", "i16", e_rq=E_RES, epilogue="resadd", aux=f"{p}.x1")
        else:
            linear(fq, f"{p}_wd", None, f"{p}.d", "i16")
            ops.append({"op": "add", "a": f"{p}.x1", "b": f"{p}.d", "out": f"{p}.x2", "sh_b": 0})
        resid = f"{p}.x2"
    rmsnorm(resid, "norm", "hn")
    hnq = quant("hn")
    exps["logits"] = E_LOGIT = i16_exp(amax["logits"])
    linear(hnq, "lm_head", None, "logits", "i16", n_pad=cfg.vocab_padded)

    qgraph = {"model": {"dim": dim, "n_layers": L, "n_heads": H, "n_kv_heads": Hkv, "head_dim": D, "ffn": F,
                        "vocab": cfg.vocab, "vocab_padded": cfg.vocab_padded, "max_seq": cfg.max_seq,
                        "prefill_m": cfg.prefill_m, "E_RES": E_RES, "E_LOGIT": E_LOGIT},
              "weights_file": "qweights.bin", "tensors": blob.tensors, "ops": ops, "input": "input",
              "output": "logits", "exps": exps, "scales": scales, "fusion": fusion,
              "synthetic": {"config": cfg.name, "seed": seed}}
    with open(out / "qweights.bin", "wb") as f:
        for c in blob.chunks:
            f.write(c)
    (out / "qgraph.json").write_text(json.dumps(qgraph))
    return out


def write_export(out_dir, cfg: ModelConfig | str, *, seed: int = 0, calib_len: int = 32,
                 weights: dict | None = None) -> Path:
    """A model export directory in the reference's format (read by refquant.py:275-301 and by
    llaccel_amd.quantize.load_export) for the seeded float model of `cfg`: `model.mlir` with the
    `llaccel.model` attribute and the weight declarations, `weights.bin` (little-endian f32) +
    `weights.json` (name, shape, byte offset), and `calib.json` (abs-max of every named activation
    over the seeded calibration sequence).  Returns out_dir."""
    if isinstance(cfg, str):
        cfg = CONFIGS[cfg]
    out = Path(out_dir)
    out.mkdir(parents=True, exist_ok=True)
    W = weights if weights is not None else float_weights(cfg, seed)
    crng = np.random.default_rng(seed + 1000)
    amax = calibrate(cfg, W, crng.integers(0, cfg.vocab, min(calib_len, cfg.max_seq)).tolist())
    attrs = {"dim": cfg.dim, "n_layers": cfg.n_layers, "n_heads": cfg.n_heads, "n_kv_heads": cfg.n_kv_heads,
             "head_dim": cfg.head_dim, "ffn": cfg.ffn, "vocab": cfg.vocab, "max_seq": cfg.max_seq}
    body = ", ".join(f"{k} = {v} : i64" for k, v in attrs.items())
    body += f", rope_base = {float(cfg.rope_base)!r} : f64, rms_eps = {float(cfg.rms_eps)!r} : f64"
    lines = [f"module attributes {{llaccel.model = {{{body}}}}} {{"]
    index, off = [], 0
    with open(out / "weights.bin", "wb") as f:
        for name, arr in W.items():
            a = np.ascontiguousarray(arr, dtype="<f4")
            lines.append(f"  llaccel.weight @{name} : tensor<{'x'.join(str(s) for s in a.shape)}xf32>")
            index.append({"name": name, "shape": [int(s) for s in a.shape], "offset": off})
            f.write(a.tobytes())
            off += a.nbytes
    lines.append("}")
    (out / "model.mlir").write_text("\n".join(lines) + "\n")
    (out / "weights.json").write_text(json.dumps(index, indent=1))
    (out / "calib.json").write_text(json.dumps(amax, indent=1))
    return out


def seeded_prompt(cfg: ModelConfig | str, length: int, seed: int = 0) -> list[int]:
    """Prompt ids uniform over [0, vocab) from numpy's default_rng(seed)."""
    if isinstance(cfg, str):
        cfg = CONFIGS[cfg]
    return np.random.default_rng(seed).integers(0, cfg.vocab, length).tolist()
