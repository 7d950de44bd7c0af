"""CPU restatement of the reference's functional simulator -- TEST INFRASTRUCTURE ONLY.

Only tests/, `__graft_entry__.smoke()` and bench.py's CPU-baseline leg may import this module; the
product (llaccel_amd.device, csrc/device.hip) never does.

`FuncSimNp` executes programs of the reference accelerator's instruction set (docs/ISA.md, binary
version 2) as runtime/src/funcsim.cpp does under its sequential policy (funcsim.cpp:84-87: the engine
queues drain before the next instruction issues, i.e. program order): the same checks and messages,
the same performance counters, and the datapath arithmetic of oracle/golden_np.py (the NUMERICS.md
primitives the simulator calls through include/llaccel/numerics.h).  It is pinned against the
simulator itself, compiled from the reference sources into oracle/_ref (tests/test_isa_oracle.py).
"""
from __future__ import annotations

import numpy as np

from . import golden_np as O

SRAM = 1 << 20
INSTR = 64
NUM_SEM = 32
NO_SEM = 0xFF
GEMM_TM = 16
ATTN_TMAX = 4096
BEAT = 64
NUM_PERF = 27
(P_CYCLES, P_INSTR, P_CP_WAIT, P_CP_QFULL, P_CP_FETCH, P_GEMM_BUSY, P_GEMM_MAC, P_GEMM_STALL, P_GEMM_EPI, P_VEC_BUSY,
 P_VEC_STALL, P_ATTN_BUSY, P_ATTN_STALL, P_ATTN_MAC, P_DMA_BUSY, P_DMA_STALL, P_DMA_WAIT, P_SRAM_RD, P_SRAM_WR,
 P_DRAM_RD, P_DRAM_WR, P_GEMM_IDLE, P_VEC_IDLE, P_ATTN_IDLE, P_ATTN_WAIT, P_ATTN_DRAM_RD, P_ATTN_DRAM_WR) = range(27)
OP_NAMES = {0x00: "NOP", 0x01: "HALT", 0x10: "DMA_LOAD", 0x11: "DMA_STORE", 0x20: "GEMM", 0x30: "VEC_RMSNORM",
            0x31: "VEC_ROPE", 0x32: "VEC_SILU", 0x33: "VEC_MUL", 0x34: "VEC_ADD", 0x35: "VEC_QUANT", 0x40: "ATTN",
            0x41: "KV_WRITE"}


def engine_of(op: int) -> int:
    """include/llaccel/isa.h:49-56."""
    return 0 if op < 0x10 else 1 if op < 0x20 else 2 if op < 0x30 else 3 if op < 0x40 else 4


class FuncSimNp:
    """funcsim.cpp:22-403 (sequential policy) over bytearray DRAM and SRAM."""

    def __init__(self, dram_bytes: int = 0, epilogue_fusion: bool = False):
        self.dram = bytearray(max(dram_bytes, 1 << 20))
        self.sram = bytearray(SRAM)
        self.fusion = epilogue_fusion
        self.pos = 0
        self.perf = [0] * NUM_PERF

    # ---- Device interface (funcsim.cpp:29-39) ----
    def dram_write(self, addr: int, data) -> None:
        data = bytes(data)
        self._ensure(addr + len(data))
        self.dram[addr:addr + len(data)] = data

    def dram_read(self, addr: int, n: int) -> bytes:
        if addr > len(self.dram) or n > len(self.dram) - addr:
            raise RuntimeError("dramRead out of range")
        return bytes(self.dram[addr:addr + n])

    def dram_size(self) -> int:
        return len(self.dram)

    def sram_snapshot(self) -> bytes:
        return bytes(self.sram)

    def _ensure(self, n: int) -> None:
        if n > len(self.dram):
            self.dram.extend(bytes(n - len(self.dram)))

    # ---- run (funcsim.cpp:41-107) ----
    def run(self, pc: int, pos: int) -> list[int]:
        self.perf = [0] * NUM_PERF
        sem = [0] * NUM_SEM
        self.pos = pos
        fetch, issued = pc, 0
        while True:
            if fetch + INSTR > len(self.dram):
                raise RuntimeError("instruction fetch out of DRAM range")
            w = [int(v) for v in np.frombuffer(bytes(self.dram[fetch:fetch + INSTR]), "<u4")]
            op, ws, ss = w[0] & 0xFF, (w[0] >> 16) & 0xFF, (w[0] >> 24) & 0xFF
            if (ws != NO_SEM and ws >= NUM_SEM) or (ss != NO_SEM and ss >= NUM_SEM):
                raise RuntimeError("invalid semaphore index")
            if engine_of(op) == 0 and op not in (0x00, 0x01):
                raise RuntimeError("invalid command processor opcode")
            if ws != NO_SEM and sem[ws] < w[1]:
                raise RuntimeError(f"deadlock at pc=0x{fetch:x} ({OP_NAMES.get(op, '?')} waits sem {ws} >= {w[1]}, "
                                   f"current {sem[ws]})")
            fetch += INSTR
            self.perf[P_INSTR] += 1
            self.perf[P_DRAM_RD] += INSTR
            issued += 1
            if op == 0x01:
                break
            if op != 0x00:
                self._execute(w)
            if ss != NO_SEM:
                sem[ss] += 1
        return list(self.perf)

    # ---- memory helpers (funcsim.cpp:124-137) ----
    def _chk(self, addr, n, what):
        if addr + n > SRAM:
            raise RuntimeError(f"SRAM access out of range in {what} @0x{addr:x}")

    def _chk_dram(self, addr, n, what):
        if addr > len(self.dram) or n > len(self.dram) - addr or addr > 0xFFFFFFFF or n > (1 << 32) - addr:
            raise RuntimeError(f"DRAM access out of range in {what} @0x{addr:x}")

    def _i16(self, addr, n):
        return np.frombuffer(bytes(self.sram[addr:addr + 2 * n]), "<i2").astype(np.int64)

    def _i8(self, addr, n):
        return np.frombuffer(bytes(self.sram[addr:addr + n]), np.int8).astype(np.int64)

    def _put16(self, addr, v):
        b = np.asarray(v, np.int64).astype("<i2").tobytes()
        self.sram[addr:addr + len(b)] = b

    def _put8(self, addr, v):
        b = np.asarray(v, np.int64).astype(np.int8).tobytes()
        self.sram[addr:addr + len(b)] = b

    def _execute(self, w):
        """funcsim.cpp:130-154: shift operands checked first, then the op."""
        op = w[0] & 0xFF

        def shift(s):
            if s > 63:
                raise RuntimeError("shift outside [0,63]")
        if op == 0x20:
            shift((w[11] >> 8) & 0xFF), shift(w[13] & 255), shift((w[13] >> 8) & 255)
        elif op == 0x30:
            shift(w[9])
        elif op == 0x32:
            shift(w[6]), shift(w[7])
        elif op in (0x33, 0x34, 0x35):
            shift(w[6])
        elif op == 0x40:
            shift(w[12]), shift(w[14])
        fn = {0x10: lambda: self._dma(w, True), 0x11: lambda: self._dma(w, False), 0x20: lambda: self._gemm(w),
              0x30: lambda: self._rmsnorm(w), 0x31: lambda: self._rope(w), 0x32: lambda: self._elementwise(w, 0),
              0x33: lambda: self._elementwise(w, 1), 0x34: lambda: self._elementwise(w, 2),
              0x35: lambda: self._elementwise(w, 3), 0x40: lambda: self._attn(w), 0x41: lambda: self._kv_write(w)}
        if op not in fn:
            raise RuntimeError(f"unexpected opcode {op}")
        fn[op]()

    def _dma(self, w, load):
        """funcsim.cpp:156-190."""
        sramA, dramA, rows, rowBytes, srcStride, dstStride = w[2:8]
        if rowBytes % 16 or sramA % 16:
            raise RuntimeError("DMA row/addr not 16-B aligned")
        beats = sram_rd = 0
        for r in range(rows):
            dram_row = dramA + r * (srcStride if load else dstStride)
            beats += ((dram_row % 64) + rowBytes + 63) // 64 if rowBytes else 0
            if not load:
                copied = 0
                while copied < rowBytes:
                    useful = min(64 - ((dram_row + copied) % 64), rowBytes - copied)
                    source = sramA + r * srcStride + copied
                    sram_rd += ((source % 64 + useful + 63) // 64) * 64
                    copied += useful
            if load:
                s, d = dramA + r * srcStride, sramA + r * dstStride
                if s + rowBytes > len(self.dram):
                    raise RuntimeError("DMA_LOAD source out of DRAM range")
                self._chk(d, rowBytes, "DMA_LOAD")
                self.sram[d:d + rowBytes] = self.dram[s:s + rowBytes]
            else:
                s, d = sramA + r * srcStride, dramA + r * dstStride
                self._chk(s, rowBytes, "DMA_STORE")
                self._ensure(d + rowBytes)
                self.dram[d:d + rowBytes] = self.sram[s:s + rowBytes]
        self.perf[P_SRAM_WR if load else P_SRAM_RD] += rows * rowBytes if load else sram_rd
        self.perf[P_DRAM_RD if load else P_DRAM_WR] += beats * 64
        self.perf[P_DMA_BUSY] += beats

    def _gemm(self, w):
        """funcsim.cpp:192-241: 16x16 weight tiles, i32 accumulation, bias, per-channel requant and the
        epilogue of each output."""
        a, wa, out, rq, bias, aux, M, N, K, ep, siluMi = w[2:13]
        siluSi, siluSh = w[13] & 0xFF, (w[13] >> 8) & 0xFF
        has_bias = bool((w[0] >> 8) & 1)
        mode, out_i8, aux_shift = ep & 0xF, bool((ep >> 4) & 1), (ep >> 8) & 0xFF
        if M == 0 or M > GEMM_TM or N % 16 or K % 16 or N == 0 or K == 0:
            raise RuntimeError("GEMM bad shape")
        if wa % 256:
            raise RuntimeError("GEMM weight address not 256-B aligned")
        if out_i8 and mode != 0:
            raise RuntimeError("GEMM i8 output with epilogue")
        if mode != 0 and not self.fusion:
            raise RuntimeError("GEMM epilogue used on a target without EPILOGUE_FUSION")
        NT, KT = N // 16, K // 16
        out_row = N if out_i8 else 2 * N
        self._chk(a, M * K, "GEMM A")
        self._chk(wa, NT * KT * 256, "GEMM W")
        self._chk(rq, N * 8, "GEMM rq")
        self._chk(out, M * out_row, "GEMM out")
        if has_bias:
            self._chk(bias, N * 4, "GEMM bias")
        use_aux = mode in (1, 3)
        if use_aux:
            self._chk(aux, M * 2 * N, "GEMM aux")
        A = self._i8(a, M * K).reshape(M, K)
        tiles = self._i8(wa, NT * KT * 256).reshape(NT, KT, 16, 16)   # [nt][kt][n][k]
        W = tiles.transpose(0, 2, 1, 3).reshape(N, K)
        acc = A @ W.T                                                   # |acc| < 2^31 for K <= 65535
        tab = np.frombuffer(bytes(self.sram[rq:rq + 8 * N]), "<i4").astype(np.int64).reshape(N, 2)
        v = acc + (np.frombuffer(bytes(self.sram[bias:bias + 4 * N]), "<i4").astype(np.int64) if has_bias else 0)
        if (tab[:, 0] < 0).any() or (tab[:, 1] < 0).any() or (tab[:, 1] > 63).any():
            raise RuntimeError("invalid requantization table entry")
        if out_i8:
            y = O.sat8(O.mulshift(v, tab[:, 0], tab[:, 1]))
        else:
            t = O.sat16(O.mulshift(v, tab[:, 0], tab[:, 1]))
            if mode == 0:
                y = t
            elif mode == 1:
                y = O.sat16(t + self._i16(aux, M * N).reshape(M, N))
            elif mode == 2:
                y = O.silu16(t, siluMi, siluSi, siluSh)
            elif mode == 3:
                y = O.sat16(O.rshr(t * self._i16(aux, M * N).reshape(M, N), aux_shift))
            else:
                raise RuntimeError("GEMM bad epilogue mode")
        # output rows are written tile by tile in the simulator; without overlap the order is moot
        for m in range(M):
            (self._put8 if out_i8 else self._put16)(out + m * out_row, y[m])
        p = self.perf
        p[P_SRAM_RD] += NT * KT * (256 + M * 16) + NT * (128 + (64 if has_bias else 0)) + (NT * M * 32 if use_aux else 0)
        p[P_GEMM_MAC] += NT * KT * M
        p[P_SRAM_WR] += NT * M * (16 if out_i8 else 32)
        p[P_GEMM_EPI] += NT * M
        p[P_GEMM_BUSY] += NT * KT * (1 + M) + NT * M

    def _rmsnorm(self, w):
        """funcsim.cpp:243-258."""
        src, gamma, dst, M, K, epsT, C, shPost = w[2:10]
        if K % 16 or K == 0:
            raise RuntimeError("RMSNORM K not a multiple of 16")
        self._chk(src, M * K * 2, "RMSNORM src")
        self._chk(gamma, K * 2, "RMSNORM gamma")
        self._chk(dst, M * K * 2, "RMSNORM dst")
        g = self._i16(gamma, K)
        for m in range(M):
            self._put16(dst + m * K * 2, O.rmsnorm_row(self._i16(src + m * K * 2, K), g, epsT, C, shPost))
        self.perf[P_SRAM_RD] += M * (2 * K * 2 + K * 2)
        self.perf[P_SRAM_WR] += M * K * 2
        self.perf[P_VEC_BUSY] += M * (2 * K // 16 + 24 + 32)

    def _rope(self, w):
        """funcsim.cpp:260-283."""
        src, dst, M, H, D, table, stride = w[2:9]
        if D not in (16, 32, 64, 128, 256):
            raise RuntimeError("ROPE bad D")
        if M == 0 or M > GEMM_TM or H == 0 or H > 255 or self.pos >= ATTN_TMAX or M > ATTN_TMAX - self.pos \
                or stride < 2 * D:
            raise RuntimeError("ROPE invalid row/head/context dimensions")
        row = H * D
        self._chk(src, M * row * 2, "ROPE src")
        self._chk(dst, M * row * 2, "ROPE dst")
        for m in range(M):
            p = self.pos + m
            self._chk(table + p * stride, 2 * D, "ROPE table")
            c = self._i16(table + p * stride, D // 2)
            s = self._i16(table + p * stride + D, D // 2)
            self._put16(dst + m * row * 2, O.rope_row(self._i16(src + m * row * 2, row), H, D, c, s))
        self.perf[P_SRAM_RD] += M * (row * 2 + H * 2 * D)
        self.perf[P_SRAM_WR] += M * row * 2
        self.perf[P_VEC_BUSY] += M * H * (D // 2 // 16 + 1)

    def _elementwise(self, w, kind):
        """funcsim.cpp:285-314: 0 SILU, 1 MUL, 2 ADD, 3 QUANT."""
        if kind in (0, 3):
            src, dst, count, p0, p1, p2 = w[2:8]
            if count % 16:
                raise RuntimeError("VEC count not a multiple of 16")
            self._chk(src, count * 2, "VEC src")
            self._chk(dst, count * (1 if kind == 3 else 2), "VEC dst")
            x = self._i16(src, count)
            if kind == 0:
                self._put16(dst, O.silu16(x, p0, p1, p2))
            else:
                self._put8(dst, O.vquant(x, p0, p1))
            self.perf[P_SRAM_RD] += count * 2
            self.perf[P_SRAM_WR] += count * (1 if kind == 3 else 2)
        else:
            a, b, dst, count, sh = w[2:7]
            if count % 16:
                raise RuntimeError("VEC count not a multiple of 16")
            self._chk(a, count * 2, "VEC a")
            self._chk(b, count * 2, "VEC b")
            self._chk(dst, count * 2, "VEC dst")
            x, y = self._i16(a, count), self._i16(b, count)
            self._put16(dst, O.vmul(x, y, sh) if kind == 1 else O.vadd(x, y, sh))
            self.perf[P_SRAM_RD] += count * 4
            self.perf[P_SRAM_WR] += count * 2
        self.perf[P_VEC_BUSY] += count // 16

    def _attn(self, w):
        """funcsim.cpp:316-375."""
        q, out, kbase, vbase, M, H, Hkv, D, kvs, Ms, Ss, Mo, So = w[2:15]
        wide = bool((w[0] >> 8) & 2)
        if D not in (16, 32, 64, 128, 256):
            raise RuntimeError("ATTN bad D")
        if M == 0 or M > GEMM_TM or H == 0 or H > 255 or Hkv == 0 or Hkv > 255 or H % Hkv:
            raise RuntimeError("ATTN invalid row/head dimensions")
        if self.pos >= ATTN_TMAX or M > ATTN_TMAX - self.pos or (self.pos + M) * D > kvs or kvs % 16 or kbase % 16 \
                or vbase % 16:
            raise RuntimeError("ATTN invalid context/DRAM cache stride")
        row, grp = H * D, H // Hkv
        self._chk(q, M * row, "ATTN q")
        self._chk(out, M * row, "ATTN out")

        def row_beats(base, T):
            return sum((D // 16) if ((base + t * D) % BEAT + D > BEAT) else 1 for t in range(T))
        for m in range(M):
            T = self.pos + m + 1
            for h in range(H):
                kvh = h // grp
                kb, vb = kbase + kvh * kvs, vbase + kvh * kvs
                self._chk_dram(kb, T * D, "ATTN K")
                self._chk_dram(vb, T * D, "ATTN V")
                keys = np.frombuffer(bytes(self.dram[kb:kb + T * D]), np.int8).reshape(T, D)
                vals = np.frombuffer(bytes(self.dram[vb:vb + T * D]), np.int8).reshape(T, D)
                o = O.attention_head(self._i8(q + m * row + h * D, D), keys, vals, Ms, Ss, Mo, So, 15 if wide else 8)
                self._put8(out + m * row + h * D, o)
                kv_read = (3 * row_beats(kb, T) + row_beats(vb, T)) * BEAT
                p = self.perf
                p[P_SRAM_RD] += D
                p[P_DRAM_RD] += kv_read
                p[P_ATTN_DRAM_RD] += kv_read
                p[P_SRAM_WR] += D
                p[P_ATTN_MAC] += 4 * T
                p[P_ATTN_BUSY] += 7 * T + 32

    def _kv_write(self, w):
        """funcsim.cpp:377-400."""
        src, base, M, Hkv, D, kvs = w[2:8]
        if D not in (16, 32, 64, 128, 256) or M == 0 or M > GEMM_TM or Hkv == 0 or Hkv > 255 \
                or self.pos >= ATTN_TMAX or M > ATTN_TMAX - self.pos or (self.pos + M) * D > kvs or kvs % 16 \
                or base % 16:
            raise RuntimeError("KV_WRITE invalid dimensions/DRAM cache stride")
        row = Hkv * D
        self._chk(src, M * row, "KV_WRITE src")
        for m in range(M):
            for kvh in range(Hkv):
                d = base + kvh * kvs + (self.pos + m) * D
                self._chk_dram(d, D, "KV_WRITE dst")
                s = src + m * row + kvh * D
                self.dram[d:d + D] = self.sram[s:s + D]
                wr = ((D // 16) if (d % BEAT + D > BEAT) else 1) * BEAT
                self.perf[P_DRAM_WR] += wr
                self.perf[P_ATTN_DRAM_WR] += wr
        self.perf[P_SRAM_RD] += M * row
        self.perf[P_ATTN_BUSY] += M * Hkv
