"""Writes tests/golden/refquant_*/ (run in the build container only): qgraphs written by the
reference's own quantizer, python/llaccel/refquant.py (`quantize_export`, refquant.py:493-506), on
small seeded export directories.  They pin llaccel_amd.quantize: the same export must give the same
qgraph.json and byte-identical qweights.bin (tests/test_quantize.py, tests/test_gpu_quantize.py).

Layout: tests/golden/refquant/export_<model>/ (model.mlir, weights.bin, weights.json, calib.json,
written by llaccel_amd.synth.write_export -- committed, so the inputs do not depend on the float BLAS
of the machine that runs the tests) and tests/golden/refquant/q_<model>_<v1|v2>/ (the reference
quantizer's qgraph.json + qweights.bin without and with --fusion).  The reference tree is read from
/root/reference, which exists only in the build container; the fixtures travel with the repository.
"""
from __future__ import annotations

import shutil
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
REF = Path("/root/reference")

# shapes the reference quantizer accepts (dim, ffn and Hkv*D multiples of 16, head_dim <= 64)
MODELS = {
    # Llama-like, vocab padded 200 -> 208
    "llama": (dict(name="rq_llama", dim=64, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=16, ffn=176, vocab=200,
                   max_seq=64), 11),
    # Qwen-like with QKV bias
    "qwen": (dict(name="rq_qwen", dim=64, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=16, ffn=128, vocab=256,
                  max_seq=64, qkv_bias=True, rope_base=1e6, rms_eps=1e-6), 12),
}
GRAPHS = {"llama_v2": ("llama", True), "qwen_v1": ("qwen", False), "qwen_v2": ("qwen", True)}


def main() -> None:
    sys.path.insert(0, str(REPO))
    sys.path.insert(0, str(REF / "python"))
    from llaccel import refquant  # noqa: E402  (the reference, build container only)

    from llaccel_amd import synth

    out = HERE / "refquant"
    if out.exists():
        shutil.rmtree(out)
    for model, (shape, seed) in MODELS.items():
        synth.write_export(out / f"export_{model}", synth.ModelConfig(**shape), seed=seed, calib_len=24)
    for name, (model, fusion) in GRAPHS.items():
        refquant.quantize_export(out / f"export_{model}", out / f"q_{name}", fusion=fusion)
        print(f"{name}: {sorted(p.name for p in (out / f'q_{name}').iterdir())}")


if __name__ == "__main__":
    main()
