"""Writes the golden-vector fixtures of tests/golden/ (run in the build container only).

Two kinds of data are produced:

* luts_ref.json -- the LUT constants the reference commits in include/llaccel/luts.h
  (parsed from that header as data).
* ref_tiny_*/   -- a config-1 (tiny Llama) qgraph written by llaccel_amd.synth, plus the
  outputs of the reference's own python/llaccel/golden.py on it: the golden.json record
  of GoldenModel.generate, the final KV caches and every activation of selected launches.
* ref_qwen2_bias/, ref_qwen3_qknorm_d128/, ref_d256/ -- the same outputs on three tiny
  graphs for the compositions the Llama fixtures leave open: q/k/v bias (golden.py:324-325),
  the per-head Q/K RMSNorm of Qwen3 (golden.py:287-293, heads > 1) at head_dim 128, and one
  layer at head_dim 256.
  The composition GoldenModel.run_chunk/prefill/decode/generate has no golden vectors in
  the reference (no golden.json is committed there, and its C++ runtime twin does not
  build here), so these fixtures are the reference-executed evidence for it.

The reference tree is read from /root/reference, which exists only in the build
container; the fixtures are small and travel with the repository.
"""
from __future__ import annotations

import json
import re
import shutil
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
REF = Path("/root/reference")


def lut_fixture() -> None:
    text = (REF / "include" / "llaccel" / "luts.h").read_text()
    tables = {}
    for name in ("kSigmoidLut", "kExpIntLut", "kExpFracLut"):
        body = re.search(name + r"\s*=\s*\{(.*?)\};", text, re.S).group(1)
        tables[name] = [int(v) for v in re.findall(r"\d+", body)]
    (HERE / "luts_ref.json").write_text(json.dumps(tables))


def run_reference(qdir: Path, prompt: list[int], n_tokens: int, acts_steps: tuple[int, ...], out: Path) -> None:
    sys.path.insert(0, str(REF / "python"))
    from llaccel import golden as G  # the reference implementation, run here only

    g = G.GoldenModel(qdir)
    acts: list = []
    rec = g.generate(prompt, n_tokens, acts)
    (out / "record.json").write_text(json.dumps(rec))
    kv = {}
    for layer, (k, v) in g.kv.items():
        kv[f"k{layer}"] = k
        kv[f"v{layer}"] = v
    np.savez_compressed(out / "kv_final.npz", **kv)
    sel = {}
    for i in acts_steps:
        for name, arr in acts[i]["acts"].items():
            sel[f"step{i}/{name}"] = np.asarray(arr).astype(np.int32)
    np.savez_compressed(out / "acts.npz", **sel)
    meta = {"prompt": prompt, "n_tokens": n_tokens, "acts_steps": list(acts_steps),
            "steps": [{k: a[k] for k in ("kind", "pos", "rows", "valid_rows")} for a in acts]}
    (out / "meta.json").write_text(json.dumps(meta))


def main(only: list[str]) -> None:
    """Writes every fixture, or only the cases named on the command line."""
    sys.path.insert(0, str(REPO))
    from llaccel_amd import synth

    # tiny graphs of the Qwen compositions (name, config, prompt length, prompt seed, tokens, activation steps)
    qwen_cases = [
        ("ref_qwen2_bias", synth.ModelConfig("tiny_qwen2", 64, 2, 4, 2, 16, 172, 256, 64, qkv_bias=True,
                                             rope_base=1e6, rms_eps=1e-6), 20, 7, 10, (0, 1, 2)),
        ("ref_qwen3_qknorm_d128", synth.ModelConfig("tiny_qwen3", 128, 2, 2, 1, 128, 256, 256, 64, qk_norm=True,
                                                    rope_base=1e6, rms_eps=1e-6), 18, 11, 8, (0, 1, 2)),
        ("ref_d256", synth.ModelConfig("tiny_d256", 256, 1, 2, 1, 256, 256, 256, 64), 17, 13, 6, (0, 1, 2)),
    ]

    if not only:
        lut_fixture()
    cases = [
        # name, fusion, prefill_m, prompt length, prompt seed, tokens, steps whose activations are kept
        ("ref_tiny_v2", True, 16, 16, 0, 32, (0, 1, 32)),
        ("ref_tiny_v1", False, 16, 16, 0, 32, (0, 1)),
        ("ref_tiny_v2_pad", True, 16, 20, 3, 12, (0, 1, 2)),
        ("ref_tiny_v2_m4", True, 4, 9, 5, 6, (2, 3)),
    ]
    for name, fusion, pm, plen, pseed, ntok, steps in cases:
        if only and name not in only:
            continue
        out = HERE / name
        if out.exists():
            shutil.rmtree(out)
        qdir = out / "qgraph"
        synth.build_qgraph(qdir, "tiny", seed=0, fusion=fusion)
        if pm != 16:
            g = json.loads((qdir / "qgraph.json").read_text())
            g["model"]["prefill_m"] = pm
            (qdir / "qgraph.json").write_text(json.dumps(g))
        prompt = synth.seeded_prompt("tiny", plen, pseed)
        run_reference(qdir, prompt, ntok, steps, out)
        print("wrote", out)
    for name, cfg, plen, pseed, ntok, steps in qwen_cases:
        if only and name not in only:
            continue
        out = HERE / name
        if out.exists():
            shutil.rmtree(out)
        qdir = out / "qgraph"
        synth.build_qgraph(qdir, cfg, seed=0, fusion=True)
        prompt = synth.seeded_prompt(cfg, plen, pseed)
        run_reference(qdir, prompt, ntok, steps, out)
        print("wrote", out)


if __name__ == "__main__":
    main(sys.argv[1:])
