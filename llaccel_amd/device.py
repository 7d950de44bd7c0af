"""The reference accelerator's instruction set on MI355X: a device that runs `.llbin` programs.

`GpuDevice` mirrors `llaccel::Device` (runtime/include/llaccel/device.h:15-29) -- `name`,
`max_attention_head_dim`, `dram_write`, `dram_read`, `dram_size`, `run(pc, pos)` returning the 27
performance counters, `sram_snapshot` -- with the semantics of the reference's functional simulator
(runtime/src/funcsim.cpp: its sequential policy, or its random legal interleaving of the engine
queues for a seed): the ISA's DRAM and 1 MiB SRAM live in GPU memory and
every instruction runs as GPU kernels (`llaccel_amd/csrc/device.hip`, C ABI `llhip_dev_*`).  Errors
are `RuntimeError`s carrying the simulator's messages, as its `std::runtime_error`s.

`Llbin` mirrors the container reader (runtime/include/llaccel/llbin.h, runtime/src/llbin.cpp): the
DRAM image, the programs by row count M with their entry PCs, and the META JSON, with the same
validation and messages.
"""
from __future__ import annotations

import ctypes
import json
import struct
from dataclasses import dataclass, field
from pathlib import Path

from . import _lib

NUM_PERF = 27
# include/llaccel/isa.h:142-149
PERF_NAMES = ("cycles", "instr_issued", "cp_stall_wait", "cp_stall_qfull", "cp_stall_fetch", "gemm_busy",
              "gemm_mac_cycles", "gemm_sram_stall", "gemm_epilogue_cycles", "vec_busy", "vec_sram_stall", "attn_busy",
              "attn_sram_stall", "attn_mac_cycles", "dma_busy", "dma_sram_stall", "dma_dram_wait", "sram_rd_bytes",
              "sram_wr_bytes", "dram_rd_bytes", "dram_wr_bytes", "gemm_idle_qempty", "vec_idle_qempty",
              "attn_idle_qempty", "attn_dram_wait", "attn_dram_rd_bytes", "attn_dram_wr_bytes")
SRAM_BYTES = 1 << 20
INSTR_BYTES = 64
GEMM_TM = 16
ATTN_TMAX = 4096
LLBIN_MAGIC = 0x4E424C4C  # "LLBN"
LLBIN_VERSION = 2
SEC_DRAM_IMAGE, SEC_PROGRAM, SEC_META_JSON = 1, 2, 3


def _err() -> str:
    return (_lib.lib().llhip_last_error() or b"").decode()


class GpuDevice:
    """`llaccel::Device` on the GPU (device.h:15-29; funcsim.cpp semantics and counters).

    `dram_bytes` = 0 sizes the DRAM to 1 MiB (it grows with writes, as the simulator's);
    `epilogue_fusion` selects the v2 target whose GEMM runs epilogues; `interleave_seed` != 0 runs
    the engine queues in the simulator's random legal order for that seed (DeviceOptions,
    device.h:31-39)."""

    def __init__(self, dram_bytes: int = 0, epilogue_fusion: bool = False, interleave_seed: int = 0):
        L = _lib.lib()
        self._h = L.llhip_dev_create(int(dram_bytes), int(bool(epilogue_fusion)))
        if not self._h:
            raise RuntimeError(_err())
        self.epilogue_fusion = bool(epilogue_fusion)
        self.interleave_seed = int(interleave_seed)
        if self.interleave_seed and L.llhip_dev_set_interleave(self._h, self.interleave_seed):
            raise RuntimeError(_err())

    def name(self) -> str:
        return "mi355x (interleaved)" if self.interleave_seed else "mi355x"

    def max_attention_head_dim(self) -> int:
        return int(_lib.lib().llhip_dev_max_attention_head_dim())

    def dram_write(self, addr: int, data) -> None:
        b = bytes(data)
        buf = ctypes.create_string_buffer(b, len(b))
        if _lib.lib().llhip_dev_dram_write(self._h, int(addr), buf, len(b)):
            raise RuntimeError(_err())

    def dram_read(self, addr: int, n: int) -> bytes:
        buf = ctypes.create_string_buffer(int(n))
        if _lib.lib().llhip_dev_dram_read(self._h, int(addr), buf, int(n)):
            raise RuntimeError(_err())
        return buf.raw

    def dram_size(self) -> int:
        return int(_lib.lib().llhip_dev_dram_size(self._h))

    def run(self, pc: int, pos: int) -> list[int]:
        """Runs the program at `pc` until HALT with the POS register at `pos`; returns the 27
        counters of this launch (device.h:25-26)."""
        perf = (ctypes.c_uint64 * NUM_PERF)()
        if _lib.lib().llhip_dev_run(self._h, int(pc), int(pos), perf):
            raise RuntimeError(_err())
        return list(perf)

    def sram_snapshot(self) -> bytes:
        buf = ctypes.create_string_buffer(SRAM_BYTES)
        if _lib.lib().llhip_dev_sram_snapshot(self._h, buf):
            raise RuntimeError(_err())
        return buf.raw

    def close(self) -> None:
        if getattr(self, "_h", None):
            _lib.lib().llhip_dev_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


@dataclass
class Program:
    """llbin.h:13-17: the rows M a program was compiled for, its entry PC and its instructions
    (16 little-endian u32 words each)."""
    M: int
    pc: int = 0
    instrs: list = field(default_factory=list)


@dataclass
class Llbin:
    """The `.llbin` container (llbin.h:19-27)."""
    dram_image: bytes
    programs: list
    meta: dict

    @staticmethod
    def load(path) -> "Llbin":
        """llbin.cpp:9-125: reads and validates a container."""
        try:
            data = Path(path).read_bytes()
        except OSError:
            raise RuntimeError(f"cannot open {path}") from None
        return Llbin.parse(data)

    @staticmethod
    def parse(data: bytes) -> "Llbin":
        if len(data) < 12:
            raise RuntimeError("llbin too small")
        magic, version, nsec = struct.unpack_from("<III", data, 0)
        if magic != LLBIN_MAGIC:
            raise RuntimeError("bad llbin magic")
        if version != LLBIN_VERSION:
            raise RuntimeError(f"unsupported llbin version {version}")
        if nsec > (len(data) - 12) // 24:
            raise RuntimeError("truncated section table")
        dram = None
        meta = None
        programs: list[Program] = []
        shapes: set[int] = set()
        off = 12
        for _ in range(nsec):
            if off + 24 > len(data):
                raise RuntimeError("truncated section table")
            kind, flags, s_off, s_size = struct.unpack_from("<IIQQ", data, off)
            off += 24
            if s_off > len(data) or s_size > len(data) - s_off:
                raise RuntimeError("section out of range")
            body = data[s_off:s_off + s_size]
            if kind == SEC_DRAM_IMAGE:
                if dram is not None:
                    raise RuntimeError("duplicate DRAM section")
                dram = body
            elif kind == SEC_PROGRAM:
                if flags == 0 or flags > GEMM_TM or flags in shapes or s_size == 0:
                    raise RuntimeError("invalid or duplicate program shape")
                shapes.add(flags)
                if s_size % INSTR_BYTES:
                    raise RuntimeError("program size not a multiple of 64")
                programs.append(Program(flags, 0, [list(struct.unpack_from("<16I", body, k))
                                                   for k in range(0, s_size, INSTR_BYTES)]))
            elif kind == SEC_META_JSON:
                if meta is not None:
                    raise RuntimeError("duplicate META section")
                meta = json.loads(body.decode())
            else:
                raise RuntimeError(f"unknown section kind {kind}")
        if not dram:
            raise RuntimeError("llbin has no DRAM image")
        if meta is None or "programs" not in meta:
            raise RuntimeError("llbin META has no programs")
        if not programs or not isinstance(meta["programs"], list) or len(meta["programs"]) != len(programs):
            raise RuntimeError("program metadata count mismatch")
        model = meta.get("model")
        if isinstance(model, dict) and "head_dim" in model:
            def positive(f):
                v = model[f]
                if not isinstance(v, int) or isinstance(v, bool) or v <= 0:
                    raise RuntimeError(f"invalid model geometry field {f}")
                return v
            D, H, Hkv = positive("head_dim"), positive("n_heads"), positive("n_kv_heads")
            if D not in (16, 32, 64, 128, 256) or H > 255 or Hkv > 255 or H % Hkv or positive("max_seq") > ATTN_TMAX:
                raise RuntimeError("model attention geometry exceeds ISA limits")
            dim = positive("dim")
            if dim % 16 or dim > 0xFFFFFFFF // 32:
                raise RuntimeError("model hidden width exceeds ISA limits")
        mapped: set[int] = set()
        for pj in meta["programs"]:
            shape, pc = int(pj["M"]), int(pj["pc"])
            if shape > GEMM_TM or shape not in shapes or shape in mapped or pc > 0xFFFFFFFF or pc % INSTR_BYTES:
                raise RuntimeError("invalid program entry metadata")
            mapped.add(shape)
            prog = next(p for p in programs if p.M == shape)
            size = len(prog.instrs) * INSTR_BYTES
            if pc > len(dram) or size > len(dram) - pc:
                raise RuntimeError("program entry outside DRAM image")
            if dram[pc:pc + size] != b"".join(struct.pack("<16I", *w) for w in prog.instrs):
                raise RuntimeError("program section differs from executable DRAM image")
            prog.pc = pc
        if len(dram) > (1 << 32):
            raise RuntimeError("DRAM image exceeds 32-bit device address space")
        kv = meta.get("dram", {}).get("kv_cache") if isinstance(meta.get("dram"), dict) else None
        if kv is not None:
            if not isinstance(kv, list):
                raise RuntimeError("DRAM KV metadata must be an array")
            regions, total = [], 0
            for item in kv:
                base, size = item["addr"], item["bytes"]
                if not (isinstance(base, int) and base >= 0 and isinstance(size, int) and size >= 0):
                    raise RuntimeError("DRAM KV addresses/sizes must be unsigned integers")
                if base % 64 or not size or size % 16 or base > len(dram) or size > len(dram) - base:
                    raise RuntimeError("DRAM KV region out of range or misaligned")
                if any(base < e and s < base + size for s, e in regions):
                    raise RuntimeError("overlapping DRAM KV regions")
                if any(base < p.pc + len(p.instrs) * INSTR_BYTES and p.pc < base + size for p in programs):
                    raise RuntimeError("DRAM KV region overlaps executable program")
                if any(dram[base:base + size]):
                    raise RuntimeError("DRAM KV image must be zero-initialized")
                regions.append((base, base + size))
                total += size
            if int(meta["dram"]["kv_cache_bytes"]) != total:
                raise RuntimeError("DRAM KV metadata byte count mismatch")
        return Llbin(dram, programs, meta)

    def program_for_m(self, M: int) -> Program:
        """llbin.cpp:128-132."""
        for p in self.programs:
            if p.M == M:
                return p
        raise RuntimeError(f"no program compiled for M={M}")
