"""ctypes binding of libllhip.so (C ABI declared in include/llhip.h).

There is no fallback: if the shared object is missing the import of any compute entry
point raises, naming the build command.
"""
from __future__ import annotations

import ctypes
import errno
import re
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libllhip.so"
HEADER = PKG.parent / "include" / "llhip.h"

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int

# name -> argument types (pointers as void*, integers as int64 unless the header says int)
_SIGS = {
    "llhip_abi_version": [],
    "llhip_last_error": [],
    "llhip_workspace_bytes": [],
    "llhip_rshr": [_p, _p, _i64, _p, _p],
    "llhip_sat": [_p, _i64, _i32, _p, _p],
    "llhip_mulshift": [_p, _p, _p, _i64, _p, _p],
    "llhip_requant": [_p, _p, _p, _i64, _i32, _p, _p],
    "llhip_isqrt48": [_p, _i64, _p, _p],
    "llhip_udiv": [_p, _p, _i64, _p, _p],
    "llhip_silu16_i64": [_p, _i64, _i64, _i64, _i64, _p, _p],
    "llhip_vmul_i64": [_p, _p, _i64, _i64, _p, _p],
    "llhip_vadd_i64": [_p, _p, _i64, _i64, _p, _p],
    "llhip_vquant_i64": [_p, _i64, _i64, _i64, _p, _p],
    "llhip_rmsnorm": [_p, _i64, _i64, _i64, _p, _i64, _i64, _i64, _p, _i64, _p],
    "llhip_quant": [_p, _i64, _i64, _i64, _p, _p],
    "llhip_silu": [_p, _i64, _i64, _i64, _i64, _p, _p],
    "llhip_vmul": [_p, _p, _i64, _i64, _p, _p],
    "llhip_vadd": [_p, _p, _i64, _i64, _p, _p],
    "llhip_rope": [_p, _i64, _i64, _i64, _i64, _p, _p, _i64, _i64, _p, _p, _p, _i64, _p],
    "llhip_linear": [_p, _i64, _i64, _i64, _p, _i64, _p, _p, _i32, _p, _i64, _i64, _i64, _i64, _i64, _i32, _p,
                     _i64, _p, _p],
    "llhip_linear_norm": [_p, _i64, _i64, _i64, _p, _i64, _p, _p, _p, _i64, _p, _i64, _p, _p, _p],
    "llhip_exact_matmul": [_p, _i64, _i64, _p, _i64, _p, _p],
    "llhip_kv_write": [_p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p, _i64, _p, _p, _i64, _p],
    "llhip_attention": [_p, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p, _i64, _p, _p, _i64, _i64, _i64, _i64, _i64,
                        _i64, _p, _i64, _p, _p],
    "llhip_attention_seqs": [_p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64,
                             _i64, _p, _i64, _p],
    "llhip_attention_noalloc": [_p, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p, _i64, _p, _p, _i64, _i64, _i64, _i64,
                                _i64, _i64, _p, _i64, _p],
    "llhip_embed_rows": [_p, _i64, _i64, _p, _i64, _i64, _p, _p],
    "llhip_argmax_i16": [_p, _i64, _i64, _i64, _p, _p],
    "llhip_greedy_step": [_p, _i64, _p, _p, _p, _p, _i64, _p, _i64, _p, _p],
    "llhip_greedy_rows": [_p, _i64, _i64, _i64, _p, _p, _p, _p, _i64, _p, _i64, _p],
    "llhip_rows_first_mismatch_i16": [_p, _i64, _p, _i64, _i64, _i64, _p, _p],
    "llhip_rows_checksum_i16": [_p, _i64, _i64, _i64, _p, _p],
    "llhip_linear_group": [_p, _i64, _i64, _i64, _i64, _p, _p, _p],
    "llhip_gate_up": [_p, _p],
    "llhip_rope_quant": [_p, _i64, _i64, _i64, _i64, _p, _p, _i64, _i64, _p, _p, _p, _p, _i64, _i64, _p, _p, _i64, _p,
                         _i64, _i64, _p],
    "llhip_rope_quant2": [_p, _p, _p],
    "llhip_quant_rows_i8": [_p, _i64, _i64, _i64, _p, _i64, _p, _p, _p],
    "llhip_f32_absmax": [_p, _i64, _i64, _i64, _p, _p, _p, _p],
    "llhip_f32_rms_min": [_p, _i64, _i64, _p, _p],
    "llhip_f32_rescale": [_p, _i64, _i64, _i64, _p, _p, _p, _p],
    "llhip_f32_smooth_objective": [_p, _i64, _i64, _p, _p, _p, _p, _p],
    "llhip_quant_i16": [_p, _i64, _i64, _p, _p, _p],
    "llhip_rmsnorm_quant": [_p, _i64, _p],
    "llhip_dev_create": [ctypes.c_uint64, _i32],
    "llhip_dev_destroy": [_p],
    "llhip_dev_dram_write": [_p, ctypes.c_uint64, _p, ctypes.c_uint64],
    "llhip_dev_dram_read": [_p, ctypes.c_uint64, _p, ctypes.c_uint64],
    "llhip_dev_dram_size": [_p],
    "llhip_dev_run": [_p, ctypes.c_uint32, ctypes.c_uint32, _p],
    "llhip_dev_sram_snapshot": [_p, _p],
    "llhip_dev_max_attention_head_dim": [],
    "llhip_dev_set_interleave": [_p, ctypes.c_uint32],
    "llhip_dev_dram_ptr": [_p],
}
_RESTYPES = {"llhip_last_error": ctypes.c_char_p, "llhip_workspace_bytes": _i64, "llhip_dev_create": _p,
             "llhip_dev_destroy": None, "llhip_dev_dram_size": ctypes.c_uint64,
             "llhip_dev_max_attention_head_dim": ctypes.c_uint32, "llhip_dev_dram_ptr": _p}

_LIB = None


class LibraryNotBuilt(RuntimeError):
    pass


def declared_symbols() -> list[str]:
    """Every entry point declared in include/llhip.h."""
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(llhip_\w+)\s*\(", text)))


def lib():
    """The loaded library (raises LibraryNotBuilt if it has not been built)."""
    global _LIB
    if _LIB is None:
        try:  # load PyTorch's HIP runtime first so the library binds to the same runtime instance
            import torch  # noqa: F401
        except ImportError:
            pass
        if not LIB_PATH.exists():
            raise LibraryNotBuilt(f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; "
                                  f"g.build()'` (make -C llaccel_amd/csrc)")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, args in _SIGS.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = _RESTYPES.get(name, ctypes.c_int)
        _LIB = L
    return _LIB


def check(rc: int, what: str) -> None:
    """Map a negative errno return code to the exception the reference raises."""
    if rc == 0:
        return
    msg = (lib().llhip_last_error() or b"").decode()
    if rc in (-errno.EINVAL, -errno.ERANGE):
        raise ValueError(msg or what)
    raise RuntimeError(f"{what} failed ({rc}): {msg}")


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)


# ---- descriptors of the fused entry points (include/llhip.h) -------------------------------
class NormQuantDesc(ctypes.Structure):
    _fields_ = [("x", _p), ("gamma", _p), ("h_out", _p), ("hq_out", _p), ("ldx", _i64), ("K", _i64), ("eps_t", _i64),
                ("C", _i64), ("sh_post", _i64), ("Mq", _i64), ("Sq", _i64), ("prequant", _i64)]


class GateUpDesc(ctypes.Structure):
    _fields_ = [("A", _p), ("M", _i64), ("K", _i64), ("lda", _i64), ("Wg", _p), ("rqg", _p), ("bg", _p), ("Wu", _p),
                ("rqu", _p), ("bu", _p), ("N", _i64), ("ld", _i64), ("silu_Mi", _i64), ("silu_Si", _i64),
                ("silu_sh", _i64), ("mul_sh", _i64), ("fq_M", _i64), ("fq_S", _i64), ("sg_out", _p), ("f_out", _p),
                ("fq_out", _p)]


class RopeQuantDesc(ctypes.Structure):
    """llhip_rope_quant_desc: the arguments of one llhip_rope_quant call."""
    _fields_ = [("x", _p), ("M", _i64), ("H", _i64), ("D", _i64), ("ldx", _i64), ("cos_tab", _p), ("sin_tab", _p),
                ("table_rows", _i64), ("pos", _i64), ("pos_dev", _p), ("row_pos", _p), ("y", _p), ("yq", _p),
                ("qM", _i64), ("qS", _i64), ("kc", _p), ("v", _p), ("ldv", _i64), ("vc", _p), ("max_seq", _i64),
                ("slot_stride", _i64), ("seq_rows", _i64)]


class LinearProblem(ctypes.Structure):
    _fields_ = [("W", _p), ("N", _i64), ("rq", _p), ("bias", _p), ("out", _p), ("ldo", _i64), ("out_i8", _i64)]


class AttnInDesc(ctypes.Structure):
    _fields_ = [("pre", NormQuantDesc), ("W", _p * 3), ("rq", _p * 3), ("bias", _p * 3), ("lin_out", _p * 3),
                ("nrm_gamma", _p * 2), ("nrm_out", _p * 2), ("nrm_eps", _i64 * 2), ("nrm_C", _i64 * 2),
                ("nrm_sh", _i64 * 2), ("cos_tab", _p), ("sin_tab", _p), ("pos_dev", _p), ("rope_out", _p * 2),
                ("quant_out", _p * 2), ("quant_M", _i64 * 2), ("quant_S", _i64 * 2), ("kc", _p), ("vc", _p),
                ("max_seq", _i64), ("M", _i64), ("H", _i64), ("Hkv", _i64), ("D", _i64), ("pos", _i64),
                ("has_norm", _i64), ("row_pos", _p), ("slot_stride", _i64)]


class MlpInDesc(ctypes.Structure):
    _fields_ = [("pre", NormQuantDesc), ("Wg", _p), ("Wu", _p), ("rqg", _p), ("rqu", _p), ("bg", _p), ("bu", _p),
                ("g_out", _p), ("u_out", _p), ("sg_out", _p), ("f_out", _p), ("fq_out", _p), ("silu_Mi", _i64),
                ("silu_Si", _i64), ("silu_sh", _i64), ("mul_sh", _i64), ("fq_M", _i64), ("fq_S", _i64), ("M", _i64),
                ("N", _i64)]


class NormLinearDesc(ctypes.Structure):
    _fields_ = [("pre", NormQuantDesc), ("W", _p), ("rq", _p), ("bias", _p), ("aux", _p), ("out", _p),
                ("epilogue", _i64), ("aux_shift", _i64), ("silu_Mi", _i64), ("silu_Si", _i64), ("silu_sh", _i64),
                ("out_i8", _i64), ("M", _i64), ("N", _i64)]


_SIGS.update({
    "llhip_attn_in": [ctypes.POINTER(AttnInDesc), _p],
    "llhip_mlp_in": [ctypes.POINTER(MlpInDesc), _p],
    "llhip_norm_linear": [ctypes.POINTER(NormLinearDesc), _p],
})


# ---- decode chain (include/llhip.h: llhip_dec_*) ------------------------------------------
class ResidDesc(ctypes.Structure):
    _fields_ = [("acc", _p), ("R", _i64), ("rq", _p), ("bias", _p), ("aux", _p), ("x_out", _p)]


class DecAttnDesc(ctypes.Structure):
    _fields_ = [("q", _p), ("kc", _p), ("vc", _p), ("out", _p), ("pos_dev", _p), ("pos", _i64), ("H", _i64),
                ("Hkv", _i64), ("D", _i64), ("max_seq", _i64), ("Ms", _i64), ("Ss", _i64), ("Mo", _i64), ("So", _i64),
                ("prob_bits", _i64), ("wo_panel", _p), ("N", _i64), ("acc", _p), ("zero", _p), ("zero_n", _i64),
                ("state", _p), ("state_bytes", _i64)]


_SIGS.update({
    "llhip_dec_attn_in": [ctypes.POINTER(AttnInDesc), ctypes.POINTER(ResidDesc), _p, _i64, _p],
    "llhip_dec_attention": [ctypes.POINTER(DecAttnDesc), _p, _p],
    "llhip_dec_attn_state_bytes": [_i64, _i64],
    "llhip_dec_attn_status": [_p, ctypes.POINTER(_i64), ctypes.POINTER(_i64)],
    "llhip_dec_mlp": [ctypes.POINTER(MlpInDesc), ctypes.POINTER(ResidDesc), _p, _p, _i64, _i64, _p],
    "llhip_dec_finish": [ctypes.POINTER(NormQuantDesc), ctypes.POINTER(ResidDesc), _p],
    "llhip_dec_head": [ctypes.POINTER(NormLinearDesc), _i64, _p, _p, _p, _i64, _i64, _p],
    "llhip_dec_head_keys": [_i64],
    "llhip_dec_greedy": [_p, _i64, _p, _p, _p, _p, _i64, _p, _i64, _p, _p],
    "llhip_dec_logits": [ctypes.POINTER(NormLinearDesc), _p, ctypes.POINTER(ResidDesc), _i64, _p, _p, _p, _p, _p, _i64, _p, _i64, _p, _i64, _p, _p],
    "llhip_dec_logits_keys": [],
    "llhip_dec_logits_panel": [_p, _i64, _i64, _p, _p],
    "llhip_linear_group_rope": [_p, _i64, _i64, _i64, _p, ctypes.POINTER(RopeQuantDesc),
                                ctypes.POINTER(RopeQuantDesc), _p, _p],
})
_RESTYPES["llhip_dec_head_keys"] = _i64
_RESTYPES["llhip_dec_logits_keys"] = _i64
_RESTYPES["llhip_dec_attn_state_bytes"] = _i64


# ---- decode step (include/llhip.h: llhip_dec_step_*) -------------------------------------
class StepLayer(ctypes.Structure):
    _fields_ = [("g1", _p), ("eps1", _i64), ("C1", _i64), ("sh1", _i64), ("Mq1", _i64), ("Sq1", _i64),
                ("W", _p * 3), ("rq", _p * 3), ("bias", _p * 3), ("quant_M", _i64 * 2), ("quant_S", _i64 * 2),
                ("kc", _p), ("vc", _p), ("Ms", _i64), ("Ss", _i64), ("Mo", _i64), ("So", _i64), ("prob_bits", _i64),
                ("wo_panel", _p), ("rq_o", _p), ("bias_o", _p), ("g2", _p), ("eps2", _i64), ("C2", _i64),
                ("sh2", _i64), ("Mq2", _i64), ("Sq2", _i64), ("Wg", _p), ("Wu", _p), ("rqg", _p), ("rqu", _p),
                ("bg", _p), ("bu", _p), ("silu_Mi", _i64), ("silu_Si", _i64), ("silu_sh", _i64), ("mul_sh", _i64),
                ("fq_M", _i64), ("fq_S", _i64), ("wd_panel", _p), ("rq_d", _p), ("bias_d", _p)]


class DecStepDesc(ctypes.Structure):
    _fields_ = [("layers", ctypes.POINTER(StepLayer)), ("L", _i64), ("dim", _i64), ("H", _i64), ("Hkv", _i64),
                ("D", _i64), ("F", _i64), ("max_seq", _i64), ("x_in", _p), ("cos_tab", _p), ("sin_tab", _p),
                ("pos_dev", _p)]


_SIGS.update({
    "llhip_dec_step_create": [ctypes.POINTER(DecStepDesc)],
    "llhip_dec_step_run": [_p, _p],
    "llhip_dec_step_outputs": [_p, ctypes.POINTER(_p), ctypes.POINTER(_p)],
    "llhip_dec_step_status": [_p, ctypes.POINTER(_i64), ctypes.POINTER(_i64)],
    "llhip_dec_step_destroy": [_p],
})
_RESTYPES["llhip_dec_step_create"] = _p
_RESTYPES["llhip_dec_step_destroy"] = None
