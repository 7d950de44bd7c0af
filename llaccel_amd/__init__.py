"""llaccel_amd: MI355X-native (gfx950) kernels for llaccel's bit-exact integer decoder datapath.

`llaccel_amd.golden` is the drop-in twin of the reference's python/llaccel/golden.py;
`llaccel_amd.synth` writes seeded synthetic qgraphs of the benchmark configurations.
"""
__all__ = ["golden", "luts", "synth"]
