"""Writes tests/golden/float/ (run in the build container only): vectors of the reference's float side
-- its TinyLlama (python/llaccel/model.py) and smooth_model (python/llaccel/smoothquant.py:19) -- on
small seeded models.  They pin oracle/float_np.py (tests/test_floatside_oracle.py) and the GPU float
side llaccel_amd.floatside (tests/test_gpu_floatside.py).

For each case: the model config and its state dict before smoothing (case.npz, float32, `sd.<name>`),
the calibration sequences, the named activations' abs-max and rms_min as calibrate.py:80-126 records
them (taken with forward hooks at the modules whose outputs the exported graph names, and around
apply_rotary for the RoPE outputs; case.json), the clipping bounds calibration_bounds.py selects from
those activations with a 64-value budget, the logits of every sequence (`logits.<i>`), and for
each smoothing option set the smoothed state dict (`sm<k>.<name>`) and the metadata record
smooth_model returns (case.json); and rope.npz / rope.json, the cos/sin tables of every RoPE scaling
kind.  The reference is read from /root/reference, which exists only in
the build container; the fixtures travel with the repository.
"""
from __future__ import annotations

import json
import math
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REF = Path("/root/reference")

CASES = {
    # the reference test's fixture (tests/python/test_smoothquant.py:10-21) with bias, untied and tied
    "bias": dict(cfg=dict(dim=32, n_layers=2, n_heads=2, n_kv_heads=1, head_dim=16, ffn=48, vocab=80, max_seq=32,
                          qkv_bias=True), seed=72, tied=False, bias_std=0.1,
                 seqs=[list(range(16)), list(range(16, 32))],
                 smooth=[dict(alpha=0.5), dict(alpha=0.25, auto_alpha=True, sample_rows=4, row_chunk=13),
                         dict(alpha=0.75, smooth_values=False, smooth_ffn=True)]),
    "tied": dict(cfg=dict(dim=32, n_layers=2, n_heads=2, n_kv_heads=1, head_dim=16, ffn=48, vocab=80, max_seq=32),
                 seed=72, tied=True, bias_std=0.0, seqs=[list(range(16)), list(range(16, 32)), [5, 3, 1]],
                 smooth=[dict(alpha=0.5), dict(alpha=1.0, smooth_lm_head=False)]),
    # GQA groups, Q/K norm, output and MLP biases (test_smoothquant.py:113-190)
    "gqa_qknorm": dict(cfg=dict(dim=64, n_layers=1, n_heads=4, n_kv_heads=2, head_dim=16, ffn=96, vocab=80,
                                max_seq=32, qkv_bias=True, o_bias=True, mlp_bias=True, qk_norm=True),
                       seed=724, tied=False, bias_std=-0.2, seqs=[list(range(16)), list(range(16, 32))],
                       smooth=[dict(alpha=0.5, auto_alpha=True, row_chunk=7), dict(alpha=0.5)]),
}


def build(torch, TinyLlama, ModelConfig, case):
    torch.manual_seed(case["seed"])
    model = TinyLlama(ModelConfig(**case["cfg"])).eval()
    with torch.no_grad():
        for name, prm in model.named_parameters():
            if name.endswith(".bias"):
                if case["bias_std"] > 0:
                    prm.normal_(0, case["bias_std"])
                elif case["bias_std"] < 0:
                    prm.uniform_(case["bias_std"], -case["bias_std"])
    if case["tied"]:
        model.lm_head.weight = model.embed_tokens.weight
    return model


def record(torch, model, seqs, cfg):
    """abs-max per exported name and rms_min of every RMSNorm input over the sequences, and the logits"""
    import llaccel.model as M

    amax, rms, acts = {}, {}, {}
    widths = {}
    for i in range(cfg.n_layers):
        widths["input" if i == 0 else f"l{i - 1}.x2"] = cfg.dim
        widths[f"l{i}.x1"] = cfg.dim
        if cfg.qk_norm:
            widths[f"l{i}.q"] = cfg.head_dim
            widths[f"l{i}.k"] = cfg.head_dim
    widths[f"l{cfg.n_layers - 1}.x2"] = cfg.dim

    def put(name, x):
        x = x.detach()
        amax[name] = max(amax.get(name, 0.0), float(x.abs().max()))
        acts.setdefault(name, []).append(x.numpy().copy())
        if name in widths:
            v = x.double().reshape(-1, widths[name])
            rms[name] = min(rms.get(name, math.inf), v.square().mean(dim=-1).sqrt().min().item())

    hooks = []

    def out_hook(name):
        return lambda _m, _i, o: put(name, o)

    def in_hook(name):
        return lambda _m, i: put(name, i[0])

    hooks.append(model.embed_tokens.register_forward_hook(out_hook("input")))
    for i, layer in enumerate(model.layers):
        L = f"l{i}"
        at, mlp = layer.self_attn, layer.mlp
        hooks.append(layer.input_layernorm.register_forward_hook(out_hook(f"{L}.h")))
        for proj, n in ((at.q_proj, "q"), (at.k_proj, "k"), (at.v_proj, "v")):
            hooks.append(proj.register_forward_hook(out_hook(f"{L}.{n}")))
        if cfg.qk_norm:
            hooks.append(at.q_norm.register_forward_hook(out_hook(f"{L}.qn")))
            hooks.append(at.k_norm.register_forward_hook(out_hook(f"{L}.kn")))
        hooks.append(at.o_proj.register_forward_pre_hook(in_hook(f"{L}.a")))
        hooks.append(at.o_proj.register_forward_hook(out_hook(f"{L}.o")))
        hooks.append(layer.post_attention_layernorm.register_forward_pre_hook(in_hook(f"{L}.x1")))
        hooks.append(layer.post_attention_layernorm.register_forward_hook(out_hook(f"{L}.h2")))
        hooks.append(mlp.gate_proj.register_forward_hook(out_hook(f"{L}.g")))
        hooks.append(mlp.gate_proj.register_forward_hook(
            lambda _m, _i, o, L=L: put(f"{L}.sg", torch.nn.functional.silu(o))))
        hooks.append(mlp.up_proj.register_forward_hook(out_hook(f"{L}.u")))
        hooks.append(mlp.down_proj.register_forward_pre_hook(in_hook(f"{L}.f")))
        hooks.append(mlp.down_proj.register_forward_hook(out_hook(f"{L}.d")))
        hooks.append(layer.register_forward_hook(out_hook(f"{L}.x2")))
    hooks.append(model.norm.register_forward_hook(out_hook("hn")))
    hooks.append(model.lm_head.register_forward_hook(out_hook("logits")))
    rot = M.apply_rotary
    state = {"layer": 0, "n": 0}

    def rotary(x, cos, sin):  # q then k, once per layer
        y = rot(x, cos, sin)
        L = f"l{state['n'] // 2}"
        put(f"{L}.qr" if state["n"] % 2 == 0 else f"{L}.kr", y.transpose(1, 2).reshape(y.shape[0], y.shape[2], -1))
        state["n"] += 1
        return y

    M.apply_rotary = rotary
    logits = []
    try:
        with torch.no_grad():
            for ids in seqs:
                state["n"] = 0
                logits.append(model(torch.tensor([ids])).numpy()[0])
    finally:
        M.apply_rotary = rot
        for h in hooks:
            h.remove()
    return amax, rms, logits, acts


def bounds(acts, amax, n_seqs, budget):
    """calibrate.py:107-125 with optimize_quantization: calibration_bounds.QuantizationSamples of every
    named activation, max(1, budget // sequences) values per sequence, selected for 8 and 16 bits"""
    from llaccel.calibration_bounds import QuantizationSamples

    out = {}
    for name, parts in acts.items():
        qs = QuantizationSamples(max(1, budget // n_seqs))
        for a in parts:
            qs.add(a)
        for bits in (8, 16):
            sel = qs.select(amax[name], bits)
            out[f"{name}.i{bits}_absmax"] = sel["absmax"]
            out[f"{name}.i{bits}_mse"] = sel["mse"]
            out[f"{name}.i{bits}_unclipped_mse"] = sel["unclipped_mse"]
    return out


# RoPE scalings of rope.py:64-99, each with a head_dim and context where they differ from the default
ROPE = {
    "default": dict(head_dim=32, max_seq=64, rope_base=10000.0, rope_scaling=None),
    "linear": dict(head_dim=64, max_seq=96, rope_base=1e6, rope_scaling={"rope_type": "linear", "rope_theta": 1e6,
                                                                          "factor": 4.0}),
    "llama3": dict(head_dim=64, max_seq=96, rope_base=5e5,
                   rope_scaling={"rope_type": "llama3", "rope_theta": 5e5, "factor": 8.0, "low_freq_factor": 1.0,
                                 "high_freq_factor": 4.0, "original_max_position_embeddings": 16}),
    "yarn": dict(head_dim=64, max_seq=96, rope_base=1e4,
                 rope_scaling={"rope_type": "yarn", "rope_theta": 1e4, "factor": 4.0, "original_max_position_embeddings": 32,
                               "attention_factor": 1.1386, "beta_fast": 32.0, "beta_slow": 1.0, "truncate": True}),
}


def rope_fixture(out) -> None:
    """cos/sin tables the reference's build_rope_tables (rope.py:64-99) writes for every scaling kind"""
    from llaccel.model import ModelConfig
    from llaccel.rope import build_rope_tables

    arrays, cfgs = {}, {}
    for name, kw in ROPE.items():
        cfg = ModelConfig(dim=kw["head_dim"] * 2, n_layers=1, n_heads=2, n_kv_heads=1, head_dim=kw["head_dim"], ffn=64,
                          vocab=16, max_seq=kw["max_seq"], rope_base=kw["rope_base"], rope_scaling=kw["rope_scaling"])
        cos, sin = build_rope_tables(cfg)
        arrays[f"{name}.cos"], arrays[f"{name}.sin"] = cos.numpy(), sin.numpy()
        cfgs[name] = cfg.to_dict()
    np.savez_compressed(out / "rope.npz", **arrays)
    (out / "rope.json").write_text(json.dumps(cfgs))


def main() -> None:
    sys.path.insert(0, str(REF / "python"))
    import torch
    from llaccel.model import ModelConfig, TinyLlama  # noqa: E402  (the reference, build container only)
    from llaccel.smoothquant import smooth_model  # noqa: E402

    out = HERE / "float"
    out.mkdir(exist_ok=True)
    rope_fixture(out)
    for name, case in CASES.items():
        model = build(torch, TinyLlama, ModelConfig, case)
        cfg = model.cfg
        arrays = {f"sd.{k}": v.detach().numpy().copy() for k, v in model.state_dict().items()}
        amax, rms, logits, acts = record(torch, model, case["seqs"], cfg)
        for i, lg in enumerate(logits):
            arrays[f"logits.{i}"] = lg
        meta = {"cfg": cfg.to_dict(), "tied": case["tied"], "seqs": case["seqs"], "amax": amax,
                "rms_min": rms, "bounds_budget": 64, "bounds": bounds(acts, amax, len(case["seqs"]), 64),
                "smooth": []}
        for k, opts in enumerate(case["smooth"]):
            m = build(torch, TinyLlama, ModelConfig, case)
            md = smooth_model(m, case["seqs"], **opts)
            for pn, v in m.state_dict().items():
                arrays[f"sm{k}.{pn}"] = v.detach().numpy().copy()
            with torch.no_grad():
                arrays[f"sm{k}.logits.0"] = m(torch.tensor([case["seqs"][0]])).numpy()[0]
            meta["smooth"].append({"options": opts, "metadata": md})
        np.savez_compressed(out / f"{name}.npz", **arrays)
        (out / f"{name}.json").write_text(json.dumps(meta))
        print(name, len(arrays), "arrays", sum(a.nbytes for a in arrays.values()), "bytes")


if __name__ == "__main__":
    main()
