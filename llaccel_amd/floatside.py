"""The float side on the GPU: activation calibration and SmoothQuant of an fp32 Llama/Qwen2-architecture
decoder, the producer of the calibration record (calib.json) that the qgraph producer quantizes with.

* `FloatModel` holds the fp32 parameters on the GPU under the export's weight names (`embed`,
  `l{i}_wq`, ..., `norm`, `lm_head`; python/llaccel/export.py:790-866), loaded from an export
  directory (weights.bin + weights.json), from the reference's TinyLlama state dict
  (python/llaccel/model.py:150-190 names) or from a dict of arrays.  Its forward is the TinyLlama
  forward (model.py:70-178): RMSNorm x * rsqrt(mean(x^2) + eps) * w, HF rotate-half RoPE with the
  tables of rope.py:64-99, causal GQA attention, SwiGLU.  The float GEMMs and attention run through
  the ROCm libraries (hipBLASLt); what calibration and smoothing add -- the per-tensor and
  per-channel abs-max records, the row-RMS minima, the objective of the alpha search and the in-place
  rescaling of the parameters -- runs in this library's kernels (llhip_f32_*), and the records stay
  on the GPU until one download at the end.
* `calibrate_tokens` (calibrate.py:80-118): max |x| of every named activation (`input`, `l{i}.h`,
  `l{i}.q`, ..., `hn`, `logits`; export.py:762-866), `<name>.rms_min` for the inputs of every
  RMSNorm, and with optimize_quantization the clipping bounds of calibration_bounds.py.
* `smooth_model` (smoothquant.py:19-272): SmoothQuant's equivalent reparameterisation of the
  RMSNorm -> projection groups (gamma / s, W[:, j] * s[j]), and optionally of value/output and
  up/down, with a fixed alpha or the calibration-weighted alpha search; returns the reference's
  metadata record.

The product path fails loudly without the HIP library and a GPU (`_lib.call`).
"""
from __future__ import annotations

import ctypes
import json
import math
from dataclasses import asdict, dataclass
from pathlib import Path

import numpy as np

from . import _lib


# ---- configuration ---------------------------------------------------------------------------
@dataclass
class FloatConfig:
    """The model shape of model.py:27-44 (same field names and checks)."""
    dim: int = 128
    n_layers: int = 4
    n_heads: int = 4
    n_kv_heads: int = 2
    head_dim: int = 32
    ffn: int = 384
    vocab: int = 65
    max_seq: int = 256
    rope_base: float = 10000.0
    rms_eps: float = 1e-5
    qkv_bias: bool = False
    o_bias: bool = False
    mlp_bias: bool = False
    qk_norm: bool = False
    rope_scaling: dict | None = None

    def __post_init__(self) -> None:
        for name in ("dim", "n_layers", "n_heads", "n_kv_heads", "head_dim", "ffn", "vocab", "max_seq"):
            value = getattr(self, name)
            if type(value) is not int or value <= 0:
                raise ValueError(f"{name} must be a positive integer")
        if not math.isfinite(self.rope_base) or self.rope_base <= 0:
            raise ValueError("rope_base must be positive and finite")
        if not math.isfinite(self.rms_eps) or self.rms_eps <= 0:
            raise ValueError("rms_eps must be positive and finite")
        for name in ("qkv_bias", "o_bias", "mlp_bias", "qk_norm"):
            if type(getattr(self, name)) is not bool:
                raise ValueError(f"{name} must be boolean")
        if self.n_heads % self.n_kv_heads != 0:
            raise ValueError("n_heads must be a multiple of n_kv_heads")
        if self.head_dim % 2 != 0:
            raise ValueError("head_dim must be even (rotate_half)")

    def to_dict(self) -> dict:
        return asdict(self)

    @classmethod
    def from_dict(cls, d: dict) -> "FloatConfig":
        return cls(**{k: d[k] for k in cls.__dataclass_fields__ if k in d})


def _torch():
    import torch

    return torch


def rope_tables(cfg: FloatConfig):
    """cos, sin [max_seq][head_dim] float32 as rope.py:64-99 builds them (torch fp32 on the host, the
    same operations in the same order: default, linear, llama3 and yarn scaling)."""
    torch = _torch()
    p = cfg.rope_scaling or {"rope_type": "default", "rope_theta": cfg.rope_base}
    d = cfg.head_dim
    inv = p["rope_theta"] ** (-torch.arange(0, d, 2, dtype=torch.float32) / d)
    amplitude = 1.0
    kind = p["rope_type"]
    if kind == "linear":
        inv = inv / p["factor"]
    elif kind == "llama3":
        wave = 2 * math.pi / inv
        n0 = p["original_max_position_embeddings"]
        low_wave, high_wave = n0 / p["low_freq_factor"], n0 / p["high_freq_factor"]
        scaled = torch.where(wave > low_wave, inv / p["factor"], inv)
        smooth = (n0 / wave - p["low_freq_factor"]) / (p["high_freq_factor"] - p["low_freq_factor"])
        blended = (1 - smooth) * scaled / p["factor"] + smooth * scaled
        inv = torch.where((wave >= high_wave) & (wave <= low_wave), blended, scaled)
    elif kind == "yarn":
        n0, theta = p["original_max_position_embeddings"], p["rope_theta"]

        def correction(rotations):
            return d * math.log(n0 / (rotations * 2 * math.pi)) / (2 * math.log(theta))
        low, high = correction(p["beta_fast"]), correction(p["beta_slow"])
        if p["truncate"]:
            low, high = math.floor(low), math.ceil(high)
        low, high = max(low, 0), min(high, d - 1)
        if low == high:
            high += 0.001
        ramp = ((torch.arange(d // 2, dtype=torch.float32) - low) / (high - low)).clamp(0, 1)
        frequency = theta ** (torch.arange(0, d, 2, dtype=torch.float32) / d)
        inv = (1 / (p["factor"] * frequency)) * ramp + (1 / frequency) * (1 - ramp)
        amplitude = p["attention_factor"]
    elif kind != "default":
        raise ValueError(f"unsupported RoPE type {kind}")
    angles = torch.outer(torch.arange(cfg.max_seq, dtype=torch.float32), inv)
    angles = torch.cat((angles, angles), dim=-1)
    return angles.cos() * amplitude, angles.sin() * amplitude


# ---- parameter names -------------------------------------------------------------------------
# export weight name -> TinyLlama state-dict name (export.py:790-866 <- model.py:70-190)
_LAYER_NAMES = {"attn_norm": "input_layernorm.weight", "wq": "self_attn.q_proj.weight",
                "bq": "self_attn.q_proj.bias", "wk": "self_attn.k_proj.weight", "bk": "self_attn.k_proj.bias",
                "wv": "self_attn.v_proj.weight", "bv": "self_attn.v_proj.bias", "q_norm": "self_attn.q_norm.weight",
                "k_norm": "self_attn.k_norm.weight", "wo": "self_attn.o_proj.weight", "bo": "self_attn.o_proj.bias",
                "ffn_norm": "post_attention_layernorm.weight", "wg": "mlp.gate_proj.weight",
                "bg": "mlp.gate_proj.bias", "wu": "mlp.up_proj.weight", "bu": "mlp.up_proj.bias",
                "wd": "mlp.down_proj.weight", "bd": "mlp.down_proj.bias"}


def state_dict_name(name: str) -> str:
    """The TinyLlama state-dict name of an export weight name."""
    if name == "embed":
        return "embed_tokens.weight"
    if name in ("norm", "lm_head"):
        return f"{name}.weight"
    layer, _, role = name.partition("_")
    return f"layers.{int(layer[1:])}.{_LAYER_NAMES[role]}"


def export_name(sd_name: str) -> str:
    """The export weight name of a TinyLlama state-dict name."""
    if sd_name == "embed_tokens.weight":
        return "embed"
    if sd_name in ("norm.weight", "lm_head.weight"):
        return sd_name.split(".")[0]
    parts = sd_name.split(".", 2)
    rest = {v: k for k, v in _LAYER_NAMES.items()}[parts[2]]
    return f"l{int(parts[1])}_{rest}"


def _expected_shapes(cfg: FloatConfig) -> dict[str, tuple]:
    H, Hkv, D, dim, F = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.dim, cfg.ffn
    s = {"embed": (cfg.vocab, dim), "norm": (dim,), "lm_head": (cfg.vocab, dim)}
    for i in range(cfg.n_layers):
        p = f"l{i}_"
        s.update({p + "attn_norm": (dim,), p + "wq": (H * D, dim), p + "wk": (Hkv * D, dim), p + "wv": (Hkv * D, dim),
                  p + "wo": (dim, H * D), p + "ffn_norm": (dim,), p + "wg": (F, dim), p + "wu": (F, dim),
                  p + "wd": (dim, F)})
        if cfg.qkv_bias:
            s.update({p + "bq": (H * D,), p + "bk": (Hkv * D,), p + "bv": (Hkv * D,)})
        if cfg.o_bias:
            s[p + "bo"] = (dim,)
        if cfg.mlp_bias:
            s.update({p + "bg": (F,), p + "bu": (F,), p + "bd": (dim,)})
        if cfg.qk_norm:
            s.update({p + "q_norm": (D,), p + "k_norm": (D,)})
    return s


# ---- the model -------------------------------------------------------------------------------
class FloatModel:
    """fp32 parameters on the GPU (export weight names) and the TinyLlama forward over them."""

    def __init__(self, cfg: FloatConfig, params: dict, *, tied: bool = False, device: str = "cuda"):
        torch = _torch()
        _lib.lib()  # the product path needs the HIP library
        if not torch.cuda.is_available():
            raise RuntimeError("FloatModel needs a GPU")
        self.cfg = cfg
        want = _expected_shapes(cfg)
        if tied:
            want.pop("lm_head")
        missing = sorted(set(want) - set(params))
        extra = sorted(set(params) - set(want) - ({"lm_head"} if tied else set()))
        if missing or extra:
            raise ValueError(f"parameters do not match the model: missing {missing}, unexpected {extra}")
        self.p = {}
        for name, shape in want.items():
            t = torch.as_tensor(np.asarray(params[name]) if not isinstance(params[name], torch.Tensor) else params[name])
            if tuple(t.shape) != shape:
                raise ValueError(f"{name}: shape {tuple(t.shape)}, expected {shape}")
            if t.dtype != torch.float32:
                raise ValueError(f"{name}: smoothing and calibration take fp32 parameters")
            self.p[name] = t.to(device).contiguous().clone()
        self.tied = tied
        if tied:
            self.p["lm_head"] = self.p["embed"]  # one tensor, as TinyLlama's tied head
        cos, sin = rope_tables(cfg)
        self.cos, self.sin = cos.to(device), sin.to(device)

    # -- constructors --
    @classmethod
    def from_state_dict(cls, cfg: FloatConfig | dict, state_dict: dict, **kw) -> "FloatModel":
        """From TinyLlama's state dict (model.py names); a head that shares the embedding's storage, or
        is absent, is tied."""
        cfg = cfg if isinstance(cfg, FloatConfig) else FloatConfig.from_dict(cfg)
        params = {export_name(k): v for k, v in state_dict.items()}
        head, emb = state_dict.get("lm_head.weight"), state_dict.get("embed_tokens.weight")
        tied = head is None or (hasattr(head, "data_ptr") and head.data_ptr() == emb.data_ptr())
        if tied:
            params.pop("lm_head", None)
        return cls(cfg, params, tied=tied, **kw)

    @classmethod
    def from_export(cls, export_dir, **kw) -> "FloatModel":
        """From an export directory (model.mlir attributes, weights.bin + weights.json)."""
        from .quantize import parse_model_attrs

        d = Path(export_dir)
        attrs = parse_model_attrs((d / "model.mlir").read_text())
        index = json.loads((d / "weights.json").read_text())
        blob = np.fromfile(d / "weights.bin", dtype="<f4")
        params = {e["name"]: blob[e["offset"] // 4:e["offset"] // 4 + int(np.prod(e["shape"]))].reshape(e["shape"])
                  for e in index}
        names = set(params)
        cfg = FloatConfig(dim=attrs["dim"], n_layers=attrs["n_layers"], n_heads=attrs["n_heads"],
                          n_kv_heads=attrs["n_kv_heads"], head_dim=attrs["head_dim"], ffn=attrs["ffn"],
                          vocab=attrs["vocab"], max_seq=attrs["max_seq"], rope_base=float(attrs["rope_base"]),
                          rms_eps=float(attrs["rms_eps"]), qkv_bias="l0_bq" in names, o_bias="l0_bo" in names,
                          mlp_bias="l0_bg" in names, qk_norm="l0_q_norm" in names)
        return cls(cfg, params, tied="lm_head" not in names, **kw)

    def state_dict(self) -> dict:
        """TinyLlama state dict (model.py names) of the current parameters, as host float32 arrays."""
        out = {state_dict_name(k): v.detach().cpu().numpy() for k, v in self.p.items() if k != "lm_head"}
        out["lm_head.weight"] = self.p["lm_head"].detach().cpu().numpy()
        return out

    def untie_head(self) -> None:
        if self.tied:
            self.p["lm_head"] = self.p["embed"].clone()
            self.tied = False

    # -- forward --
    def _rms(self, x, w):
        torch = _torch()
        return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + self.cfg.rms_eps) * w

    def _lin(self, x, w, b=None):
        y = x @ w.t()
        return y + b if b is not None else y

    def _rope(self, x, T):
        torch = _torch()
        half = x.shape[-1] // 2
        rot = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
        return x * self.cos[:T, None, :] + rot * self.sin[:T, None, :]

    def forward(self, ids, rec=None, *, head: bool = True):
        """Logits [T][vocab] of one sequence (or None with head=False, which stops after the final norm);
        rec(name, tensor [T][cols] or [T*heads][width]) sees every named activation."""
        torch = _torch()
        F = torch.nn.functional
        cfg, p = self.cfg, self.p
        H, Hkv, D = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
        idx = torch.as_tensor(list(ids), dtype=torch.long, device=p["embed"].device)
        T = idx.numel()
        r = rec or (lambda name, t: None)
        g = p.get
        with torch.no_grad():
            x = p["embed"].index_select(0, idx)
            r("input", x)
            for i in range(cfg.n_layers):
                L = f"l{i}"
                h = self._rms(x, p[f"{L}_attn_norm"])
                r(f"{L}.h", h)
                q = self._lin(h, p[f"{L}_wq"], g(f"{L}_bq"))
                k = self._lin(h, p[f"{L}_wk"], g(f"{L}_bk"))
                v = self._lin(h, p[f"{L}_wv"], g(f"{L}_bv"))
                r(f"{L}.q", q)
                r(f"{L}.k", k)
                r(f"{L}.v", v)
                q, k = q.view(T, H, D), k.view(T, Hkv, D)
                if cfg.qk_norm:
                    q = self._rms(q, p[f"{L}_q_norm"])
                    k = self._rms(k, p[f"{L}_k_norm"])
                    r(f"{L}.qn", q.reshape(T, H * D))
                    r(f"{L}.kn", k.reshape(T, Hkv * D))
                q, k = self._rope(q, T), self._rope(k, T)
                r(f"{L}.qr", q.reshape(T, H * D))
                r(f"{L}.kr", k.reshape(T, Hkv * D))
                qh, kh, vh = q.transpose(0, 1), k.transpose(0, 1), v.view(T, Hkv, D).transpose(0, 1)
                if H != Hkv:
                    kh = kh.repeat_interleave(H // Hkv, dim=0)
                    vh = vh.repeat_interleave(H // Hkv, dim=0)
                a = F.scaled_dot_product_attention(qh.unsqueeze(0).contiguous(), kh.unsqueeze(0).contiguous(),
                                                   vh.unsqueeze(0).contiguous(), is_causal=True)
                a = a[0].transpose(0, 1).reshape(T, H * D)
                r(f"{L}.a", a)
                o = self._lin(a, p[f"{L}_wo"], g(f"{L}_bo"))
                r(f"{L}.o", o)
                x1 = x + o
                r(f"{L}.x1", x1)
                h2 = self._rms(x1, p[f"{L}_ffn_norm"])
                r(f"{L}.h2", h2)
                gt = self._lin(h2, p[f"{L}_wg"], g(f"{L}_bg"))
                up = self._lin(h2, p[f"{L}_wu"], g(f"{L}_bu"))
                r(f"{L}.g", gt)
                r(f"{L}.u", up)
                sg = F.silu(gt)
                r(f"{L}.sg", sg)
                f = sg * up
                r(f"{L}.f", f)
                d = self._lin(f, p[f"{L}_wd"], g(f"{L}_bd"))
                r(f"{L}.d", d)
                x = x1 + d
                r(f"{L}.x2", x)
            hn = self._rms(x, p["norm"])
            r("hn", hn)
            if not head:
                return None
            logits = hn @ p["lm_head"].t()
            r("logits", logits)
            return logits


# ---- device records --------------------------------------------------------------------------
def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(_torch().cuda.current_stream().cuda_stream)


class _Records:
    """Running abs-max records of named tensors on the GPU (per tensor, optionally per column), row-RMS
    minima and non-finite counts, downloaded once by `host()`."""

    def __init__(self, device):
        self.torch = _torch()
        self.device = device
        self.names: list[str] = []
        self.slot: dict[str, int] = {}
        self.cols: dict[str, object] = {}
        self.rms: dict[str, object] = {}
        self._amax_parts = []
        self._bad_parts = []

    def _slot(self, name):
        if name not in self.slot:
            self.slot[name] = len(self.names)
            self.names.append(name)
            self._amax_parts.append(self.torch.zeros(1, dtype=self.torch.float32, device=self.device))
            self._bad_parts.append(self.torch.zeros(1, dtype=self.torch.int32, device=self.device))
        return self.slot[name]

    def absmax(self, name, t, col_name=None):
        """max |t| into the record `name`; with col_name, also per column into that vector."""
        if t.dim() != 2 or t.stride(1) != 1:
            t = t.reshape(-1, t.shape[-1]).contiguous()
        i = self._slot(name)
        colv = None
        if col_name is not None:
            if col_name not in self.cols:
                self.cols[col_name] = self.torch.zeros(t.shape[1], dtype=self.torch.float32, device=self.device)
            colv = self.cols[col_name]
        _lib.call("llhip_f32_absmax", _ptr(t), t.shape[0], t.shape[1], t.stride(0),
                  _ptr(colv) if colv is not None else None, _ptr(self._amax_parts[i]), _ptr(self._bad_parts[i]),
                  _stream())

    def rms_min(self, name, t, width):
        t = t.contiguous()
        if name not in self.rms:
            self.rms[name] = self.torch.full((1,), math.inf, dtype=self.torch.float64, device=self.device)
        _lib.call("llhip_f32_rms_min", _ptr(t), t.numel() // width, width, _ptr(self.rms[name]), _stream())

    def host(self):
        """(abs-max by name, per-column maxima by name, rms minima by name, non-finite counts by name)"""
        torch = self.torch
        amax = torch.cat(self._amax_parts).cpu().numpy() if self.names else np.zeros(0, np.float32)
        bad = torch.cat(self._bad_parts).cpu().numpy() if self.names else np.zeros(0, np.int32)
        return ({n: float(amax[i]) for i, n in enumerate(self.names)},
                {n: v for n, v in self.cols.items()},
                {n: float(v.cpu()[0]) for n, v in self.rms.items()},
                {n: int(bad[i]) for i, n in enumerate(self.names)})


def _check_sequences(cfg: FloatConfig, sequences, min_len: int, message: str) -> None:
    for ids in sequences:
        if not min_len <= len(ids) <= cfg.max_seq:
            raise ValueError(message)
        if any(type(i) is not int or not 0 <= i < cfg.vocab for i in ids):
            raise ValueError("calibration token IDs must be integers within vocabulary")


def _rmsnorm_inputs(cfg: FloatConfig) -> dict[str, int]:
    """Named input of every RMSNorm and its row width (calibrate.py:95-96: cols // heads)."""
    out = {}
    for i in range(cfg.n_layers):
        out["input" if i == 0 else f"l{i - 1}.x2"] = cfg.dim
        out[f"l{i}.x1"] = cfg.dim
        if cfg.qk_norm:
            out[f"l{i}.q"] = cfg.head_dim
            out[f"l{i}.k"] = cfg.head_dim
    out[f"l{cfg.n_layers - 1}.x2"] = cfg.dim
    return out


class _QuantSamples:
    """calibration_bounds.py:13-32 QuantizationSamples.add on the GPU: per sequence, n values at the
    linspace indices of the flattened activation and its extreme (first largest |x|), kept on the GPU."""

    def __init__(self, per_sequence: int):
        self.per = per_sequence
        self.parts = []

    def add(self, t):
        torch = _torch()
        flat = t.reshape(-1)
        n = min(self.per, flat.numel())
        idx = torch.as_tensor(np.linspace(0, flat.numel() - 1, n, dtype=np.int64), device=flat.device)
        extreme = flat[torch.argmax(flat.abs())]
        self.parts.append((flat.index_select(0, idx), flat.numel() / n, extreme.reshape(1)))

    def select(self, absmax: float, bits: int) -> dict:
        """calibration_bounds.py:34-57 on the downloaded samples."""
        if not math.isfinite(absmax) or absmax < 0 or bits not in (8, 16) or not self.parts:
            raise ValueError("invalid calibration range, bit width, or empty samples")
        values = np.concatenate([p[0].cpu().numpy() for p in self.parts]).astype(np.float64)
        weights = np.concatenate([np.full(len(p[0]), p[1]) for p in self.parts])
        values = np.concatenate([values, np.asarray([float(p[2].cpu()[0]) for p in self.parts])])
        weights = np.concatenate([weights, np.ones(len(self.parts))])
        if absmax == 0:
            return {"absmax": 0.0, "mse": 0.0, "unclipped_mse": 0.0, "sampled_values": len(values)}
        qmax = (1 << (bits - 1)) - 1
        if bits == 8:
            candidates = [(absmax * f, absmax * f / qmax)
                          for f in (1, .999, .995, .99, .98, .95, .9, .85, .8, .7, .6, .5)]
        else:
            top = max(math.ceil(math.log2(absmax) - math.log2(qmax)), -15)
            candidates = [(min(absmax, qmax * 2.0 ** e), 2.0 ** e) for e in range(top, max(top - 4, -15) - 1, -1)]
        scored = []
        for bound, step in candidates:
            q = np.clip(np.floor(values / step + .5), -qmax - 1, qmax) * step
            scored.append((float(np.average((q - values) ** 2, weights=weights)), bound))
        mse, bound = min(scored, key=lambda s: s[0])
        return {"absmax": float(bound), "mse": mse, "unclipped_mse": scored[0][0], "sampled_values": len(values)}


def calibrate_tokens(model: FloatModel, sequences: list[list[int]], *, optimize_quantization: bool = False,
                     sample_budget: int = 32768) -> dict[str, float]:
    """calibrate.py:80-118 on the GPU: abs-max of every named activation over the sequences,
    `<name>.rms_min` of every RMSNorm input, and with optimize_quantization the
    `<name>.i{8,16}_{absmax,mse,unclipped_mse}` clipping bounds."""
    if not sequences:
        raise ValueError("calibration requires at least one token sequence")
    if type(optimize_quantization) is not bool or type(sample_budget) is not int or sample_budget < 1:
        raise ValueError("invalid quantization calibration options")
    if optimize_quantization and len(sequences) > sample_budget:
        raise ValueError("sample_budget must cover at least one value per sequence")
    cfg = model.cfg
    _check_sequences(cfg, sequences, 2, "calibration sequence length must be in [2,max_seq]")
    rms_w = _rmsnorm_inputs(cfg)
    rec = _Records(model.p["embed"].device)
    per = max(1, sample_budget // len(sequences)) if optimize_quantization else 0
    samples: dict[str, _QuantSamples] = {}

    def record(name, t):
        rec.absmax(name, t)
        if name in rms_w:
            rec.rms_min(name, t, rms_w[name])
        if per:
            samples.setdefault(name, _QuantSamples(per)).add(t)

    for ids in sequences:
        model.forward(ids, record)
    amax, _, rms, bad = rec.host()
    nonfinite = [n for n in rec.names if bad[n]]
    if nonfinite:
        raise ValueError(f"nonfinite calibration activation {nonfinite[0]!r}")
    out = dict(amax) | {f"{n}.rms_min": v for n, v in rms.items()}
    if optimize_quantization:
        for name, s in samples.items():
            for bits in (8, 16):
                sel = s.select(amax[name], bits)
                out[f"{name}.i{bits}_absmax"] = sel["absmax"]
                out[f"{name}.i{bits}_mse"] = sel["mse"]
                out[f"{name}.i{bits}_unclipped_mse"] = sel["unclipped_mse"]
    return out


# ---- SmoothQuant -----------------------------------------------------------------------------
def _groups(cfg: FloatConfig, smooth_lm_head: bool):
    """(group name, norm weight, [linear weights], activation record) of smoothquant.py:62-69."""
    out = []
    for i in range(cfg.n_layers):
        out.append((f"layers.{i}.input_layernorm", f"l{i}_attn_norm", [f"l{i}_wq", f"l{i}_wk", f"l{i}_wv"], f"l{i}.h"))
        out.append((f"layers.{i}.post_attention_layernorm", f"l{i}_ffn_norm", [f"l{i}_wg", f"l{i}_wu"],
                    f"l{i}.h2"))
    if smooth_lm_head:
        out.append(("norm", "norm", ["lm_head"], "hn"))
    return out


def _transfers(cfg: FloatConfig, smooth_values: bool, smooth_ffn: bool):
    """(name, source weight, source bias, target weight, repeat, activation record) of
    smoothquant.py:71-81: value/output (V rows and bias / s, O columns * s over the GQA repeat) and
    product/down (up rows and bias / s, down columns * s)."""
    out = []
    for i in range(cfg.n_layers):
        if smooth_values:
            out.append((f"layers.{i}.value_output", f"l{i}_wv", f"l{i}_bv", f"l{i}_wo", cfg.n_heads // cfg.n_kv_heads,
                        f"l{i}.v"))
        if smooth_ffn:
            out.append((f"layers.{i}.mlp_product_down", f"l{i}_wu", f"l{i}_bu", f"l{i}_wd", 1, f"l{i}.f"))
    return out


def smooth_model(model: FloatModel, sequences: list[list[int]], alpha: float = 0.5, *, smooth_lm_head: bool = True,
                 smooth_values: bool = True, smooth_ffn: bool = True, row_chunk: int = 1024,
                 auto_alpha: bool = False, sample_rows: int = 128) -> dict:
    """smoothquant.py:19-272 on the GPU: the same groups, scales, alpha search, checks and order of
    the in-place updates, and the same metadata record.  Every check completes before a parameter
    changes.  row_chunk bounds the reference's temporary memory and is validated, not needed here."""
    torch = _torch()
    if isinstance(alpha, bool) or not isinstance(alpha, (int, float)) or not math.isfinite(alpha) or not 0 <= alpha <= 1:
        raise ValueError("alpha must be finite and in [0,1]")
    if type(sample_rows) is not int or sample_rows < 1:
        raise ValueError("sample_rows must be positive")
    if type(auto_alpha) is not bool:
        raise ValueError("auto_alpha must be boolean")
    if type(row_chunk) is not int or row_chunk <= 0:
        raise ValueError("row_chunk must be a positive integer")
    for flag in (smooth_lm_head, smooth_values, smooth_ffn):
        if type(flag) is not bool:
            raise ValueError("smoothing options must be boolean")
    if not isinstance(model, FloatModel):
        raise TypeError("smooth_model requires a FloatModel")
    if not sequences:
        raise ValueError("smoothing requires at least one calibration sequence")
    cfg, p = model.cfg, model.p
    _check_sequences(cfg, sequences, 1, "calibration sequence length must be in [1,max_seq]")
    dev = p["embed"].device
    groups, transfers = _groups(cfg, smooth_lm_head), _transfers(cfg, smooth_values, smooth_ffn)
    # activation record -> maxima name (the reference's group names)
    wanted = {g[3]: g[0] for g in groups} | {t[5]: t[0] for t in transfers}
    rec = _Records(dev)
    samples = {name: [] for name in wanted.values()}
    counts = {name: 0 for name in wanted.values()}
    n_sampled = min(len(sequences), (sample_rows + 1) // 2)
    sampled = ({0} if n_sampled == 1 else
               {round(i * (len(sequences) - 1) / (n_sampled - 1)) for i in range(n_sampled)})
    collect = False

    def record(act, t):
        name = wanted.get(act)
        if name is None:
            return
        rec.absmax(name, t, col_name=name)
        if auto_alpha and collect and counts[name] < sample_rows:
            count = min(2, t.shape[0], sample_rows - counts[name])
            sel = np.linspace(0, t.shape[0] - 1, count).astype(np.int64)
            samples[name].append(t[torch.as_tensor(sel, device=dev)].clone())
            counts[name] += count

    for si, ids in enumerate(sequences):
        collect = si in sampled
        model.forward(ids, record, head=False)  # the hidden states only (smoothquant.py:117-124)
    _, maxima_dev, _, bad = rec.host()
    for name in rec.names:
        if bad[name]:
            raise ValueError(f"nonfinite calibration activation: {name}")
    maxima = {k: v.double().cpu() for k, v in maxima_dev.items()}

    def column_max(wnames, name):
        """max |W[:, j]| over the weights, with the non-finite check of smoothquant.py:206-210"""
        colv = torch.zeros(p[wnames[0]].shape[1], dtype=torch.float32, device=dev)
        bad = torch.zeros(1, dtype=torch.int32, device=dev)
        for w in wnames:
            W = p[w]
            _lib.call("llhip_f32_absmax", _ptr(W), W.shape[0], W.shape[1], W.shape[1], _ptr(colv), None, _ptr(bad),
                      _stream())
        if int(bad.cpu()[0]):
            raise ValueError(f"nonfinite weight in {name}")
        return colv.cpu()

    minimum, limit = 1e-5, torch.finfo(torch.float32).max
    candidates = sorted({0.0, 0.25, 0.5, 0.75, 0.9, 1.0, float(alpha)})
    selected, objectives = {}, {}

    def objective(name, scales, wnames, repeat):
        """smoothquant.py:142-163: the activation terms on the sampled rows, the weight terms in
        llhip_f32_smooth_objective"""
        x = torch.cat(samples[name])
        s_dev = scales.to(dev)
        mx = maxima_dev[name]
        if repeat > 1:
            Hk, D = cfg.n_kv_heads, cfg.head_dim
            x = x.reshape(len(x), Hk, D).repeat_interleave(repeat, dim=1).reshape(len(x), -1)
            s_dev = s_dev.reshape(Hk, D).repeat_interleave(repeat, dim=0).flatten()
            mx = mx.reshape(Hk, D).repeat_interleave(repeat, dim=0).flatten()
        smoothed = x / s_dev
        step = (mx / s_dev).max().clamp_min(1e-30) / 127
        quantized = (smoothed / step).round().clamp(-128, 127) * step
        act_err = (quantized - smoothed).square().mean(dim=0).contiguous()
        act_energy = smoothed.square().mean(dim=0).contiguous()
        s_dev = s_dev.contiguous()
        acc = torch.zeros(2, dtype=torch.float64, device=dev)
        for w in wnames:
            W = p[w]
            _lib.call("llhip_f32_smooth_objective", _ptr(W), W.shape[0], W.shape[1], _ptr(s_dev), _ptr(act_err),
                      _ptr(act_energy), _ptr(acc), _stream())
        return float(acc.sum().cpu())

    def scales_for(name, colmax, wnames, repeat=1):
        """smoothquant.py:165-185: s = exp(alpha log max|x| - (1 - alpha) log max|W|), clamped"""
        act = maxima[name]
        best, scores = None, []
        for cand in (candidates if auto_alpha else [float(alpha)]):
            logs = cand * act.clamp_min(minimum).log()
            logs -= (1 - cand) * colmax.double().clamp_min(minimum).log()
            scales = logs.exp().clamp_min(minimum).float()
            if not torch.isfinite(scales).all().item() or not (scales > 0).all().item():
                raise ValueError(f"nonfinite or nonpositive smoothing scale: {name}")
            err = objective(name, scales, wnames, repeat) if auto_alpha else 0.0
            if not math.isfinite(err):
                raise ValueError(f"nonfinite calibration objective: {name}")
            scores.append({"alpha": cand, "weighted_error": err})
            if best is None or err < best[0]:
                best = (err, cand, scales)
        selected[name] = best[1]
        objectives[name] = scores
        return best[2]

    def report(name, scales, colmax):
        act = maxima_dev[name].cpu()
        return {"group": name, "selected_alpha": selected[name], "alpha_objective": objectives[name],
                "scale_min": scales.min().item(), "scale_max": scales.max().item(), "scales": scales.tolist(),
                "activation_max_before": act.max().item(), "activation_max_after": (act / scales).max().item(),
                "weight_max_before": colmax.max().item(),
                "weight_max_after": (colmax.double() * scales.double()).max().item()}

    def check_range(t, name):
        if not torch.isfinite(t).all().item() or (t.abs() > limit).any().item():
            raise ValueError(f"smoothing would overflow fp32 parameters: {name}")

    plans, stats, input_scales = [], [], {}
    for name, norm, wnames, _ in groups:
        colmax = column_max(wnames, name)
        scales = scales_for(name, colmax, wnames)
        check_range(p[norm].double().cpu() / scales.double(), name)
        check_range(colmax.double() * scales.double(), name)
        plans.append((norm, wnames, scales))
        for w in wnames:
            input_scales[w] = scales
        stats.append(report(name, scales, colmax))
    transfer_plans = []
    for name, src, src_b, dst, repeat, _ in transfers:
        colmax = column_max([dst], name)
        if name.endswith(".value_output"):
            grouped = colmax.reshape(cfg.n_kv_heads, repeat, cfg.head_dim).amax(dim=1).flatten()
            scales = scales_for(name, grouped, [dst], repeat)
            dst_scales = scales.reshape(cfg.n_kv_heads, 1, cfg.head_dim).expand(-1, repeat, -1).reshape(-1)
        else:
            grouped = colmax
            scales = scales_for(name, grouped, [dst])
            dst_scales = scales
        check_range(colmax.double() * dst_scales.double(), name)
        sd = scales.double().to(dev)
        composed = p[src].double() * input_scales[src].double().to(dev).unsqueeze(0) / sd.unsqueeze(1)
        check_range(composed, name)
        del composed
        if src_b in p:
            check_range(p[src_b].double() / sd, name)
        transfer_plans.append((src, src_b, dst, scales, dst_scales))
        stats.append(report(name, scales, grouped))

    # every check passed: the in-place updates, in the reference's order
    untie = smooth_lm_head and model.tied
    if untie:
        model.untie_head()

    def rescale(t, col_mul=None, col_div=None, row_div=None):
        rows, cols = (1, t.shape[0]) if t.dim() == 1 else t.shape
        keep = [v.to(dev).contiguous() if v is not None else None for v in (col_mul, col_div, row_div)]
        _lib.call("llhip_f32_rescale", _ptr(t), rows, cols, cols, *[_ptr(v) if v is not None else None for v in keep],
                  _stream())

    for norm, wnames, scales in plans:
        rescale(p[norm], col_div=scales)
        for w in wnames:
            rescale(p[w], col_mul=scales)
    for src, src_b, dst, scales, dst_scales in transfer_plans:
        rescale(p[src], row_div=scales)
        if src_b in p:
            rescale(p[src_b], col_div=scales)
        rescale(p[dst], col_mul=dst_scales)
    torch.cuda.synchronize()
    return {"algorithm": "SmoothQuant equivalent RMSNorm, value/output and FFN reparameterization",
            "alpha": float(alpha), "auto_alpha": auto_alpha, "sample_rows_limit": sample_rows,
            "calibration_sequences": len(sequences), "calibration_tokens": sum(map(len, sequences)),
            "smooth_lm_head": smooth_lm_head, "untied_lm_head": bool(untie), "minimum_scale": minimum,
            "smooth_values": smooth_values, "smooth_ffn": smooth_ffn, "groups": stats}


def main(argv=None) -> int:
    """Calibrate (and optionally smooth) an export directory's float model on the GPU and write its
    calib.json (and smoothed weights.bin) in place."""
    import argparse

    ap = argparse.ArgumentParser(description="GPU calibration / SmoothQuant of an export directory")
    ap.add_argument("export_dir")
    ap.add_argument("--tokens", required=True, help="JSON list of token-ID sequences")
    ap.add_argument("--smooth-alpha", type=float, default=None, help="apply SmoothQuant first")
    ap.add_argument("--auto-alpha", action="store_true")
    ap.add_argument("--optimize-quantization", action="store_true")
    args = ap.parse_args(argv)
    d = Path(args.export_dir)
    seqs = json.loads(Path(args.tokens).read_text())
    model = FloatModel.from_export(d)
    if args.smooth_alpha is not None:
        meta = smooth_model(model, seqs, args.smooth_alpha, auto_alpha=args.auto_alpha)
        (d / "smoothquant.json").write_text(json.dumps(meta, indent=1))
        index = json.loads((d / "weights.json").read_text())
        with open(d / "weights.bin", "r+b") as f:
            for e in index:
                f.seek(e["offset"])
                f.write(np.ascontiguousarray(model.p[e["name"]].cpu().numpy(), dtype="<f4").tobytes())
    calib = calibrate_tokens(model, seqs, optimize_quantization=args.optimize_quantization)
    (d / "calib.json").write_text(json.dumps(calib, indent=1))
    print(f"calibrated {len(calib)} records over {len(seqs)} sequences -> {d / 'calib.json'}")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
