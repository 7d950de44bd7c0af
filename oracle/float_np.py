"""CPU restatement of the float side in float64 numpy -- test infrastructure only.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this module, as the checker
of llaccel_amd.floatside (the GPU product); nothing in the product imports it.

* `forward` is TinyLlama's forward (python/llaccel/model.py:70-178: RMSNorm, rotate-half RoPE with
  the rope.py:64-99 tables, causal GQA softmax attention, SwiGLU) in float64, calling rec(name, x) at
  the activations export.py:762-866 names.
* `calibrate_tokens` restates calibrate.py:80-126 without the clipping bounds: abs-max per name and
  `<name>.rms_min` of every RMSNorm input (calibrate.py:104).
* `smooth_model` restates smoothquant.py:19-272 (groups, transfers, scales, the auto-alpha objective
  of :142-163, the range checks and the update order) on a dict of float64 parameters.

Pinned by tests/test_floatside_oracle.py against vectors the reference's own TinyLlama and
smooth_model wrote (tests/golden/float/, written by tests/golden/make_float_fixtures.py), and by
properties the reparameterisation fixes: the smoothed model's logits equal the original's; with
alpha = 1/2 every group's largest scaled activation equals its largest scaled weight column.
"""
from __future__ import annotations

import math

import numpy as np

F64 = np.float64


def rope_tables(cfg) -> tuple[np.ndarray, np.ndarray]:
    """rope.py:64-99 for the default and linear kinds, in float32 as the reference builds them
    (inv_freq by a float32 power, the angles as a float32 outer product)."""
    p = cfg.rope_scaling or {"rope_type": "default", "rope_theta": cfg.rope_base}
    d = cfg.head_dim
    expo = (-np.arange(0, d, 2, dtype=np.float32) / np.float32(d)).astype(np.float32)
    inv = np.power(np.float32(p["rope_theta"]), expo).astype(np.float32)
    if p["rope_type"] == "linear":
        inv = (inv / np.float32(p["factor"])).astype(np.float32)
    elif p["rope_type"] != "default":
        raise ValueError("the oracle restates the default and linear RoPE tables")
    ang = np.outer(np.arange(cfg.max_seq, dtype=np.float32), inv).astype(np.float32)
    ang = np.concatenate([ang, ang], -1)
    return np.cos(ang.astype(F64)), np.sin(ang.astype(F64))


def _rms(x, w, eps):
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * w


def _lin(x, p, w, b):
    y = x @ p[w].T
    return y + p[b] if b in p else y


def forward(cfg, p: dict, ids, rec=None, head: bool = True):
    """Logits [T][vocab] (float64) of one sequence; rec(name, x) sees the named activations."""
    r = rec or (lambda n, x: None)
    H, Hkv, D = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
    cos, sin = rope_tables(cfg)
    ids = np.asarray(ids, dtype=np.int64)
    T = len(ids)
    c, s = cos[:T, None, :], sin[:T, None, :]

    def rope(x):
        half = D // 2
        return x * c + np.concatenate([-x[..., half:], x[..., :half]], -1) * s

    x = p["embed"][ids].astype(F64)
    r("input", x)
    mask = np.triu(np.full((T, T), -np.inf), 1)
    for i in range(cfg.n_layers):
        L = f"l{i}"
        h = _rms(x, p[f"{L}_attn_norm"], cfg.rms_eps)
        r(f"{L}.h", h)
        q, k, v = (_lin(h, p, f"{L}_w{n}", f"{L}_b{n}") for n in "qkv")
        r(f"{L}.q", q)
        r(f"{L}.k", k)
        r(f"{L}.v", v)
        q, k = q.reshape(T, H, D), k.reshape(T, Hkv, D)
        if cfg.qk_norm:
            q = _rms(q, p[f"{L}_q_norm"], cfg.rms_eps)
            k = _rms(k, p[f"{L}_k_norm"], cfg.rms_eps)
            r(f"{L}.qn", q.reshape(T, -1))
            r(f"{L}.kn", k.reshape(T, -1))
        q, k = rope(q), rope(k)
        r(f"{L}.qr", q.reshape(T, -1))
        r(f"{L}.kr", k.reshape(T, -1))
        rep = H // Hkv
        kh = np.repeat(k.transpose(1, 0, 2), rep, axis=0)
        vh = np.repeat(v.reshape(T, Hkv, D).transpose(1, 0, 2), rep, axis=0)
        sc = q.transpose(1, 0, 2) @ kh.transpose(0, 2, 1) / math.sqrt(D) + mask
        sc = np.exp(sc - sc.max(-1, keepdims=True))
        sc /= sc.sum(-1, keepdims=True)
        a = (sc @ vh).transpose(1, 0, 2).reshape(T, H * D)
        r(f"{L}.a", a)
        o = _lin(a, p, f"{L}_wo", f"{L}_bo")
        r(f"{L}.o", o)
        x1 = x + o
        r(f"{L}.x1", x1)
        h2 = _rms(x1, p[f"{L}_ffn_norm"], cfg.rms_eps)
        r(f"{L}.h2", h2)
        g = _lin(h2, p, f"{L}_wg", f"{L}_bg")
        u = _lin(h2, p, f"{L}_wu", f"{L}_bu")
        r(f"{L}.g", g)
        r(f"{L}.u", u)
        sg = g / (1.0 + np.exp(-g))
        r(f"{L}.sg", sg)
        f = sg * u
        r(f"{L}.f", f)
        d = _lin(f, p, f"{L}_wd", f"{L}_bd")
        r(f"{L}.d", d)
        x = x1 + d
        r(f"{L}.x2", x)
    hn = _rms(x, p["norm"], cfg.rms_eps)
    r("hn", hn)
    if not head:
        return None
    logits = hn @ p.get("lm_head", p["embed"]).T
    r("logits", logits)
    return logits


def rmsnorm_inputs(cfg) -> dict[str, int]:
    """calibrate.py:104: the input of every RMSNorm and its row width"""
    out = {}
    for i in range(cfg.n_layers):
        out["input" if i == 0 else f"l{i - 1}.x2"] = cfg.dim
        out[f"l{i}.x1"] = cfg.dim
        if cfg.qk_norm:
            out[f"l{i}.q"] = cfg.head_dim
            out[f"l{i}.k"] = cfg.head_dim
    out[f"l{cfg.n_layers - 1}.x2"] = cfg.dim
    return out


def calibrate_tokens(cfg, p: dict, sequences) -> dict[str, float]:
    """calibrate.py:80-126 (abs-max and rms_min records) in float64."""
    amax: dict[str, float] = {}
    rms = {n: math.inf for n in rmsnorm_inputs(cfg)}
    widths = rmsnorm_inputs(cfg)

    def rec(name, x):
        amax[name] = max(amax.get(name, 0.0), float(np.abs(x).max()))
        if name in widths:
            rows = x.reshape(-1, widths[name])
            rms[name] = min(rms[name], float(np.sqrt(np.mean(rows * rows, -1)).min()))

    for ids in sequences:
        forward(cfg, p, ids, rec)
    return amax | {f"{n}.rms_min": v for n, v in rms.items()}


def smooth_model(cfg, p: dict, sequences, alpha: float = 0.5, *, smooth_lm_head=True, smooth_values=True,
                 smooth_ffn=True, auto_alpha=False, sample_rows=128) -> dict:
    """smoothquant.py:19-272 on float64 parameters (p is updated in place; a missing lm_head is the
    tied embedding and is untied first).  Returns {group: scales} and the selected alphas."""
    groups = []
    for i in range(cfg.n_layers):
        groups.append((f"layers.{i}.input_layernorm", f"l{i}_attn_norm", [f"l{i}_wq", f"l{i}_wk", f"l{i}_wv"],
                       f"l{i}.h"))
        groups.append((f"layers.{i}.post_attention_layernorm", f"l{i}_ffn_norm", [f"l{i}_wg", f"l{i}_wu"], f"l{i}.h2"))
    if smooth_lm_head:
        groups.append(("norm", "norm", ["lm_head"], "hn"))
    transfers = []
    for i in range(cfg.n_layers):
        if smooth_values:
            transfers.append((f"layers.{i}.value_output", f"l{i}_wv", f"l{i}_bv", f"l{i}_wo",
                              cfg.n_heads // cfg.n_kv_heads, f"l{i}.v"))
        if smooth_ffn:
            transfers.append((f"layers.{i}.mlp_product_down", f"l{i}_wu", f"l{i}_bu", f"l{i}_wd", 1, f"l{i}.f"))
    if smooth_lm_head and "lm_head" not in p:
        p["lm_head"] = p["embed"].copy()
    wanted = {g[3]: g[0] for g in groups} | {t[5]: t[0] for t in transfers}
    maxima: dict[str, np.ndarray] = {}
    samples = {n: [] for n in wanted.values()}
    counts = {n: 0 for n in wanted.values()}
    n_sampled = min(len(sequences), (sample_rows + 1) // 2)
    sampled = {0} if n_sampled == 1 else {round(i * (len(sequences) - 1) / (n_sampled - 1)) for i in range(n_sampled)}
    state = {"collect": False}

    def rec(act, x):
        name = wanted.get(act)
        if name is None:
            return
        cm = np.abs(x).max(0)
        maxima[name] = cm if name not in maxima else np.maximum(maxima[name], cm)
        if auto_alpha and state["collect"] and counts[name] < sample_rows:
            count = min(2, x.shape[0], sample_rows - counts[name])
            samples[name].append(x[np.linspace(0, x.shape[0] - 1, count).astype(np.int64)])
            counts[name] += count

    for si, ids in enumerate(sequences):
        state["collect"] = si in sampled
        forward(cfg, p, ids, rec, head=False)

    minimum = 1e-5
    cands = sorted({0.0, 0.25, 0.5, 0.75, 0.9, 1.0, float(alpha)})

    def objective(name, s, wnames, repeat):
        x = np.concatenate(samples[name])
        mx = maxima[name]
        if repeat > 1:
            Hk, D = cfg.n_kv_heads, cfg.head_dim
            x = np.repeat(x.reshape(len(x), Hk, D), repeat, axis=1).reshape(len(x), -1)
            s = np.repeat(s.reshape(Hk, D), repeat, axis=0).reshape(-1)
            mx = np.repeat(mx.reshape(Hk, D), repeat, axis=0).reshape(-1)
        sm = x / s
        step = max((mx / s).max(), 1e-30) / 127
        qa = np.clip(np.round(sm / step), -128, 127) * step
        a_err, a_en = ((qa - sm) ** 2).mean(0), (sm ** 2).mean(0)
        err = 0.0
        for w in wnames:
            W = p[w] * s[None, :]
            ws = np.maximum(np.abs(W).max(1, keepdims=True), 1e-30) / 127
            qw = np.clip(np.round(W / ws), -128, 127) * ws
            err += float((W * W * a_err[None, :]).sum()) + float(((qw - W) ** 2 * a_en[None, :]).sum())
        return err

    def scales_for(name, colmax, wnames, repeat=1):
        best = None
        errors = {}
        for a in (cands if auto_alpha else [float(alpha)]):
            logs = a * np.log(np.maximum(maxima[name], minimum)) - (1 - a) * np.log(np.maximum(colmax, minimum))
            s = np.maximum(np.exp(logs), minimum)
            e = objective(name, s, wnames, repeat) if auto_alpha else 0.0
            errors[a] = e
            if best is None or e < best[0]:
                best = (e, a, s)
        return best[2], best[1], errors

    out = {"scales": {}, "alpha": {}, "objective": {}}
    plans, input_scales = [], {}
    for name, norm, wnames, _ in groups:
        colmax = np.max([np.abs(p[w]).max(0) for w in wnames], axis=0)
        s, a, e = scales_for(name, colmax, wnames)
        plans.append((norm, wnames, s))
        for w in wnames:
            input_scales[w] = s
        out["scales"][name], out["alpha"][name], out["objective"][name] = s, a, e
    tplans = []
    for name, src, src_b, dst, repeat, _ in transfers:
        colmax = np.abs(p[dst]).max(0)
        if name.endswith(".value_output"):
            grouped = colmax.reshape(cfg.n_kv_heads, repeat, cfg.head_dim).max(1).reshape(-1)
            s, a, e = scales_for(name, grouped, [dst], repeat)
            ds = np.repeat(s.reshape(cfg.n_kv_heads, 1, cfg.head_dim), repeat, axis=1).reshape(-1)
        else:
            s, a, e = scales_for(name, colmax, [dst])
            ds = s
        tplans.append((src, src_b, dst, s, ds))
        out["scales"][name], out["alpha"][name], out["objective"][name] = s, a, e
    for norm, wnames, s in plans:
        p[norm] = p[norm] / s
        for w in wnames:
            p[w] = p[w] * s[None, :]
    for src, src_b, dst, s, ds in tplans:
        p[src] = p[src] / s[:, None]
        if src_b in p:
            p[src_b] = p[src_b] / s
        p[dst] = p[dst] * ds[None, :]
    out["maxima"] = maxima
    return out
