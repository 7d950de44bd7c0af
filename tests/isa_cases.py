"""Seeded programs of the reference accelerator's instruction set (docs/ISA.md), shared by the
CPU tests (oracle/isa_np.py against the reference's own simulator) and the GPU tests (the GPU
device against the oracle).  Each case is a DRAM image: the program at address 0, operand blobs
from DATA on; programs DMA their operands into SRAM, run the instructions under test and store the
results back to DRAM."""
from __future__ import annotations

import struct

import numpy as np

DATA = 0x10000
NO = 0xFF
OPS = dict(NOP=0x00, HALT=0x01, DMA_LOAD=0x10, DMA_STORE=0x11, GEMM=0x20, RMSNORM=0x30, ROPE=0x31, SILU=0x32,
           MUL=0x33, ADD=0x34, QUANT=0x35, ATTN=0x40, KV_WRITE=0x41)


def ins(op: str, *operands, flags=0, wait=(NO, 0), signal=NO) -> bytes:
    """One 64-byte instruction: word0 = opcode | flags<<8 | wait_sem<<16 | signal_sem<<24,
    word1 = wait_val, words 2.. the operands in ISA order."""
    w = [0] * 16
    w[0] = OPS[op] | (flags << 8) | (wait[0] << 16) | (signal << 24)
    w[1] = wait[1]
    for i, v in enumerate(operands):
        w[2 + i] = int(v) & 0xFFFFFFFF
    return struct.pack("<16I", *w)


class Builder:
    def __init__(self):
        self.code = []
        self.data = bytearray()

    def blob(self, b, align=256) -> int:
        pad = (-len(self.data)) % align
        self.data.extend(bytes(pad))
        addr = DATA + len(self.data)
        self.data.extend(bytes(b))
        return addr

    def load(self, sram, b, rows=1):
        """DMA_LOAD of a blob into SRAM (rows of equal length)."""
        b = bytes(b)
        addr = self.blob(b)
        rb = len(b) // rows
        self.code.append(ins("DMA_LOAD", sram, addr, rows, rb, rb, rb))

    def store(self, sram, n) -> int:
        addr = self.blob(bytes(n))
        self.code.append(ins("DMA_STORE", sram, addr, 1, n, n, n))
        return addr

    def emit(self, *a, **k):
        self.code.append(ins(*a, **k))

    def image(self) -> bytes:
        self.code.append(ins("HALT"))
        code = b"".join(self.code)
        assert len(code) <= DATA
        return code + bytes(DATA - len(code)) + bytes(self.data)


def _i16(x):
    return np.asarray(x, np.int64).astype("<i2").tobytes()


def _i8(x):
    return np.asarray(x, np.int64).astype(np.int8).tobytes()


def _i32(x):
    return np.asarray(x, np.int64).astype("<i4").tobytes()


def tile_w(W: np.ndarray) -> bytes:
    """Row-major W [N][K] into the ISA's 16x16 tiles: tile (nt, kt) at (nt*K/16 + kt)*256, byte
    n*16 + k = W[nt*16 + n][kt*16 + k]."""
    N, K = W.shape
    return W.reshape(N // 16, 16, K // 16, 16).transpose(0, 2, 1, 3).astype(np.int8).tobytes()


def gemm_case(rng, M, N, K, mode, out_i8=False, bias=True, inplace=False):
    b = Builder()
    A = rng.integers(-128, 128, (M, K))
    W = rng.integers(-128, 128, (N, K))
    rq = np.stack([rng.integers(1 << 20, 1 << 30, N), rng.integers(18, 34, N)], 1)
    bz = rng.integers(-(1 << 20), 1 << 20, N)
    aux = rng.integers(-32768, 32768, (M, N))
    a_s, w_s, rq_s, b_s, aux_s, out_s = 0x0, 0x10000, 0x90000, 0x98000, 0xA0000, 0xC0000
    b.load(a_s, _i8(A))
    b.load(w_s, tile_w(W))
    b.load(rq_s, _i32(rq))
    b.load(b_s, _i32(bz))
    b.load(aux_s, _i16(aux))
    if inplace:
        out_s = aux_s
    ep = mode | (int(out_i8) << 4) | ((11 if mode == 3 else 0) << 8)
    b.emit("GEMM", a_s, w_s, out_s, rq_s, b_s, aux_s, M, N, K, ep, 1 << 30, 30 | (16 << 8), flags=int(bias))
    b.store(out_s, M * N * (1 if out_i8 else 2))
    return b.image()


def vec_case(rng, kind, count, inplace=False):
    b = Builder()
    x = rng.integers(-32768, 32768, count)
    y = rng.integers(-32768, 32768, count)
    b.load(0x0, _i16(x))
    b.load(0x40000, _i16(y))
    dst = 0x0 if inplace else 0x80000
    if kind == "SILU":
        b.emit("SILU", 0x0, dst, count, 1 << 30, 30, 16)
    elif kind == "QUANT":
        b.emit("QUANT", 0x0, dst, count, int(rng.integers(1 << 20, 1 << 30)), 25)
    else:
        b.emit(kind, 0x0, 0x40000, dst, count, 9)
    b.store(dst, count * (1 if kind == "QUANT" else 2))
    return b.image()


def rmsnorm_case(rng, M, K, inplace=False):
    b = Builder()
    x = rng.integers(-4000, 4000, (M, K))
    g = rng.integers(-20000, 20000, K)
    b.load(0x0, _i16(x))
    b.load(0x40000, _i16(g))
    dst = 0x0 if inplace else 0x80000
    b.emit("RMSNORM", 0x0, 0x40000, dst, M, K, 1000, 1 << 30, 22)
    b.store(dst, M * K * 2)
    return b.image()


def rope_case(rng, M, H, D, pos, pad=0, inplace=False):
    b = Builder()
    stride = 2 * D + pad
    rows = pos + M
    tab = bytearray()
    for _ in range(rows):
        tab += _i16(rng.integers(-16384, 16385, D)) + bytes(pad)
    x = rng.integers(-32768, 32768, (M, H * D))
    b.load(0x0, _i16(x))
    b.load(0x40000, bytes(tab))
    dst = 0x0 if inplace else 0x80000
    b.emit("ROPE", 0x0, dst, M, H, D, 0x40000, stride)
    b.store(dst, M * H * D * 2)
    return b.image()


def attn_case(rng, M, H, Hkv, D, pos, wide, max_seq=None, inplace=False):
    """K/V caches in DRAM at a 64-byte-aligned base, filled for keys 0..pos+M-1; a KV_WRITE of the
    M new rows first, then ATTN."""
    b = Builder()
    max_seq = max_seq or pos + M + 5
    kvs = max_seq * D
    T = pos + M
    kc = np.zeros((Hkv, max_seq, D), np.int64)
    vc = np.zeros((Hkv, max_seq, D), np.int64)
    kc[:, :T] = rng.integers(-128, 128, (Hkv, T, D))
    vc[:, :T] = rng.integers(-128, 128, (Hkv, T, D))
    kbase = b.blob(_i8(kc), 64)
    vbase = b.blob(_i8(vc), 64)
    knew = rng.integers(-128, 128, (M, Hkv * D))
    q = rng.integers(-128, 128, (M, H * D))
    b.load(0x0, _i8(q))
    b.load(0x40000, _i8(knew))
    b.emit("KV_WRITE", 0x40000, kbase, M, Hkv, D, kvs)
    out = 0x0 if inplace else 0x80000
    b.emit("ATTN", 0x0, out, kbase, vbase, M, H, Hkv, D, kvs, int(rng.integers(1 << 28, 1 << 30)), 30,
           int(rng.integers(1 << 28, 1 << 30)), 36 if wide else 29, flags=2 if wide else 0)
    b.store(out, M * H * D)
    return b.image(), pos


def dma_case(rng):
    """DRAM-side addresses off the 16-byte grid, a strided gather, destination rows that overlap
    (later rows win) and a store that grows the DRAM."""
    b = Builder()
    src = b.blob(rng.integers(0, 256, 4096).astype(np.uint8).tobytes())
    b.emit("DMA_LOAD", 0x100, src + 3, 5, 48, 100, 64)
    b.emit("DMA_LOAD", 0x1000, src + 7, 4, 64, 64, 32)   # overlapping destination rows
    b.emit("DMA_STORE", 0x100, DATA + 0x3000 + 5, 3, 32, 64, 80)
    b.emit("DMA_STORE", 0x1000, (1 << 21) + 9, 2, 96, 96, 112)   # past the initial DRAM size
    return b.image()


def dma_chain_case(rng):
    """Consecutive aligned DMAs that depend on each other (the GPU device batches independent
    ones): store of what a load just wrote, load of what a store just wrote, two loads into
    overlapping SRAM (the later wins), and more than eight independent loads in a row."""
    b = Builder()
    a = b.blob(rng.integers(0, 256, 2048).astype(np.uint8).tobytes())
    c = b.blob(rng.integers(0, 256, 2048).astype(np.uint8).tobytes())
    scratch = b.blob(bytes(4096))
    b.emit("DMA_LOAD", 0x0, a, 4, 256, 256, 256)
    b.emit("DMA_STORE", 0x0, scratch, 2, 512, 512, 512)
    b.emit("DMA_LOAD", 0x2000, scratch + 256, 1, 512, 512, 512)
    b.emit("DMA_LOAD", 0x3000, a, 1, 1024, 1024, 1024)
    b.emit("DMA_LOAD", 0x3200, c, 1, 1024, 1024, 1024)
    for i in range(10):
        b.emit("DMA_LOAD", 0x8000 + 0x400 * i, c + 128 * i, 2, 64, 64, 128)
    b.emit("DMA_STORE", 0x3000, scratch + 1024, 1, 1536, 1536, 1536)
    return b.image()


def self_modifying_case():
    """A program that stores over one of its own later instructions (a NOP becomes a VEC_ADD) before
    reaching it: the stored instruction runs."""
    b = Builder()
    b.load(0x0, _i16(np.arange(64) - 32))
    b.load(0x4000, ins("ADD", 0x0, 0x0, 0x200, 64, 1))
    b.code.append(None)  # the DMA_STORE below, whose target is the NOP after it
    b.emit("NOP")
    b.store(0x200, 128)
    i = b.code.index(None)
    b.code[i] = ins("DMA_STORE", 0x4000, 64 * (i + 1), 1, 64, 64, 64)
    return b.image()


def sem_case(ok=True):
    """NOPs and ops that signal and wait on semaphores; ok=False waits for a count never reached."""
    b = Builder()
    b.load(0x0, _i16(np.arange(64) - 32))
    b.emit("NOP", signal=3)
    b.emit("NOP", signal=3)
    b.emit("SILU", 0x0, 0x200, 64, 1 << 30, 30, 16, wait=(3, 2), signal=4)
    b.emit("ADD", 0x0, 0x200, 0x400, 64, 2, wait=(4, 1 if ok else 2))
    b.store(0x400, 128)
    return b.image()


def chain_case(rng):
    """One decoder-style chain on SRAM: rmsnorm, quant, GEMM (resadd in place on the residual),
    silu, mul, add."""
    b = Builder()
    K, N, M = 64, 64, 3
    x = rng.integers(-3000, 3000, (M, K))
    g = rng.integers(-20000, 20000, K)
    W = rng.integers(-128, 128, (N, K))
    rq = np.stack([rng.integers(1 << 24, 1 << 28, N), rng.integers(20, 30, N)], 1)
    b.load(0x0, _i16(x))
    b.load(0x1000, _i16(g))
    b.load(0x2000, tile_w(W))
    b.load(0x4000, _i32(rq))
    b.emit("RMSNORM", 0x0, 0x1000, 0x5000, M, K, 77, 1 << 30, 22)
    b.emit("QUANT", 0x5000, 0x6000, M * K, 1 << 28, 24)
    b.emit("GEMM", 0x6000, 0x2000, 0x0, 0x4000, 0, 0x0, M, N, K, 1, 0, 0)
    b.emit("SILU", 0x0, 0x7000, M * N, 1 << 30, 30, 16)
    b.emit("MUL", 0x7000, 0x0, 0x8000, M * N, 11)
    b.emit("ADD", 0x8000, 0x0, 0x8000, M * N, 1)
    b.store(0x0, M * N * 2)
    b.store(0x8000, M * N * 2)
    return b.image()


def cases():
    """(id, dram image, pos, epilogue_fusion) of every parity case."""
    rng = np.random.default_rng(20261201)
    out = []
    for M, N, K in [(1, 16, 16), (5, 48, 64), (16, 128, 896), (3, 896, 128)]:
        for mode, i8 in [(0, True), (0, False), (1, False), (2, False), (3, False)]:
            out.append((f"gemm-{M}x{N}x{K}-m{mode}{'i8' if i8 else ''}", gemm_case(rng, M, N, K, mode, i8, bias=mode != 2),
                        0, True))
    out.append(("gemm-resadd-inplace", gemm_case(rng, 4, 64, 128, 1, inplace=True), 0, True))
    for kind in ("SILU", "QUANT", "MUL", "ADD"):
        out.append((f"vec-{kind}", vec_case(rng, kind, 4096), 0, False))
        out.append((f"vec-{kind}-inplace", vec_case(rng, kind, 1024, inplace=True), 0, False))
    out.append(("rmsnorm", rmsnorm_case(rng, 7, 896), 0, False))
    out.append(("rmsnorm-inplace", rmsnorm_case(rng, 2, 64, inplace=True), 0, False))
    for M, H, D, pos, pad in [(1, 14, 64, 37, 0), (4, 2, 128, 0, 32), (3, 3, 16, 100, 16), (2, 1, 256, 5, 0)]:
        out.append((f"rope-{M}x{H}x{D}@{pos}", rope_case(rng, M, H, D, pos, pad), pos, False))
    out.append(("rope-inplace", rope_case(rng, 2, 2, 32, 3, inplace=True), 3, False))
    for M, H, Hkv, D, pos, wide in [(1, 14, 2, 64, 37, True), (5, 4, 4, 16, 0, False), (3, 4, 1, 128, 300, True),
                                    (16, 2, 2, 64, 70, False), (1, 2, 1, 256, 12, True)]:
        img, p = attn_case(rng, M, H, Hkv, D, pos, wide)
        out.append((f"attn-{M}x{H}/{Hkv}x{D}@{pos}{'w' if wide else ''}", img, p, False))
    img, p = attn_case(rng, 2, 2, 2, 64, 9, True, inplace=True)
    out.append(("attn-inplace", img, p, False))
    out.append(("dma", dma_case(rng), 0, False))
    out.append(("dma-chain", dma_chain_case(rng), 0, False))
    out.append(("self-modifying", self_modifying_case(), 0, False))
    out.append(("semaphores", sem_case(True), 0, False))
    out.append(("chain", chain_case(rng), 0, True))
    return out


def error_cases():
    """(id, dram image, pos, fusion, message) of programs the simulator rejects."""
    b = Builder()
    b.emit("GEMM", 0, 0, 0, 0, 0, 0, 17, 16, 16, 0, 0, 0)
    gemm_shape = b.image()
    b = Builder()
    b.emit("GEMM", 0, 0x180, 0x1000, 0x2000, 0, 0, 1, 16, 16, 0, 0, 0)
    gemm_align = b.image()
    b = Builder()
    b.emit("GEMM", 0, 0, 0x1000, 0x2000, 0, 0, 1, 16, 16, 1, 0, 0)
    no_fusion = b.image()
    b = Builder()
    b.emit("SILU", 0, 0x100, 16, 1, 64, 0)
    bad_shift = b.image()
    b = Builder()
    b.emit("QUANT", 0xFFFF0, 0, 32, 1, 1)
    oob = b.image()
    b = Builder()
    b.load(0x2000, _i32(np.array([[1 << 20, 64]] * 16)))
    b.emit("GEMM", 0, 0, 0x1000, 0x2000, 0, 0, 1, 16, 16, 0, 0, 0)
    bad_rq = b.image()
    b = Builder()
    b.code.append(struct.pack("<16I", 0x05 | (NO << 16) | (NO << 24), *([0] * 15)))
    bad_cp = b.image()
    return [("gemm-shape", gemm_shape, 0, True, "GEMM bad shape"),
            ("gemm-w-align", gemm_align, 0, True, "GEMM weight address not 256-B aligned"),
            ("gemm-no-fusion", no_fusion, 0, False, "GEMM epilogue used on a target without EPILOGUE_FUSION"),
            ("shift", bad_shift, 0, False, "shift outside [0,63]"),
            ("sram-oob", oob, 0, False, "SRAM access out of range in VEC src @0xffff0"),
            ("bad-rq", bad_rq, 0, False, "invalid requantization table entry"),
            ("cp-opcode", bad_cp, 0, False, "invalid command processor opcode"),
            ("deadlock", sem_case(False), 0, False, "deadlock at pc=0x")]


def partial_error_cases():
    """(id, dram image, pos, fusion, message, sram_exact) of failing programs whose DRAM (and, where
    sram_exact, SRAM) after the error the device must leave as the simulator does: a DMA or KV_WRITE
    that fails at a later row writes the rows before it; an invalid requant entry stops the program
    before a later DMA_STORE, and a later failing instruction does not replace its message."""
    rng = np.random.default_rng(21)
    out = []
    b = Builder()
    b.load(0x100, _i8(rng.integers(-128, 128, 64)))
    b.load(0x2000, _i32(np.array([[1 << 20, 64]] * 16)))
    b.emit("GEMM", 0, 0, 0x1000, 0x2000, 0, 0, 1, 16, 16, 0, 0, 0)
    b.store(0x100, 64)
    b.emit("QUANT", 0xFFFF0, 0, 32, 1, 1)
    out.append(("rq-then-store", b.image(), 0, False, "invalid requantization table entry", False))
    # DMA_STORE rows at SRAM 0xFFF00 + r * 0x80: row 2 starts past the SRAM
    b = Builder()
    b.load(0xFFF00, _i8(rng.integers(-128, 128, 256)))
    dst = b.blob(bytes(4 * 64))
    b.emit("DMA_STORE", 0xFFF00, dst, 4, 64, 0x80, 64)
    out.append(("dma-store-rows", b.image(), 0, False, "SRAM access out of range in DMA_STORE", True))
    # DMA_LOAD rows from the last 192 bytes of a 1 MiB DRAM, stride 64: row 3 ends past it
    b = Builder()
    b.emit("DMA_LOAD", 0x400, (1 << 20) - 192, 4, 64, 64, 64)
    img = b.image()
    img = img + bytes((1 << 20) - 192 - len(img)) + _i8(rng.integers(-128, 128, 192))
    out.append(("dma-load-rows", img, 0, False, "DMA_LOAD source out of DRAM range", True))
    # KV_WRITE of 2 rows x 2 heads (D = 16, head stride 64) ending at the 1 MiB DRAM's end: the pair
    # (row 1, head 1) is out of range, row 0 and (row 1, head 0) are written
    b = Builder()
    b.load(0x0, _i8(rng.integers(-128, 128, 64)))
    b.emit("KV_WRITE", 0x0, (1 << 20) - 80, 2, 2, 16, 64)
    out.append(("kv-write-rows", b.image(), 0, False, "DRAM access out of range in KV_WRITE dst", True))
    return out


def toy_llbin(seed=5) -> bytes:
    """A .llbin of a one-head toy model (vocab 48, dim 64, max_seq 32) with programs for M = 4 and
    M = 1: input rows -> quant -> K/V cache write -> attention over the cache -> lm_head GEMM ->
    logits rows, with the META entries the host loop reads (host.cpp:47-100)."""
    rng = np.random.default_rng(seed)
    V, Dm, S = 48, 64, 32
    emb, inp, lg, wa, rqa, kc, vc = 0x4000, 0x6000, 0x7000, 0x8000, 0x9000, 0xA000, 0xA800
    kvs = S * Dm

    def program(M):
        c = [ins("DMA_LOAD", 0x0, inp, M, 128, 128, 128),
             ins("DMA_LOAD", 0x10000, wa, 1, V * Dm, V * Dm, V * Dm),
             ins("DMA_LOAD", 0x20000, rqa, 1, V * 8, V * 8, V * 8),
             ins("QUANT", 0x0, 0x1000, M * Dm, 1 << 28, 22),
             ins("KV_WRITE", 0x1000, kc, M, 1, Dm, kvs),
             ins("KV_WRITE", 0x1000, vc, M, 1, Dm, kvs),
             ins("ATTN", 0x1000, 0x2000, kc, vc, M, 1, 1, Dm, kvs, 1 << 29, 30, 1 << 29, 36, flags=2),
             ins("GEMM", 0x2000, 0x10000, 0x3000, 0x20000, 0, 0, M, V, Dm, 0, 0, 0),
             ins("DMA_STORE", 0x3000, lg, M, V * 2, V * 2, 128),
             ins("HALT")]
        return b"".join(c)
    p4, p1 = program(4), program(1)
    dram = bytearray(0xB000)
    dram[0:len(p4)] = p4
    dram[0x1000:0x1000 + len(p1)] = p1
    dram[emb:emb + V * 128] = _i16(rng.integers(-3000, 3000, (V, 64)))
    dram[wa:wa + V * Dm] = tile_w(rng.integers(-128, 128, (V, Dm)))
    dram[rqa:rqa + V * 8] = _i32(np.stack([rng.integers(1 << 24, 1 << 28, V), rng.integers(18, 26, V)], 1))
    meta = {"programs": [{"M": 4, "pc": 0}, {"M": 1, "pc": 0x1000}],
            "model": {"vocab": V, "dim": Dm, "max_seq": S, "head_dim": Dm, "n_heads": 1, "n_kv_heads": 1},
            "dram": {"embedding": {"addr": emb, "row_bytes": 128}, "input": {"addr": inp, "row_bytes": 128},
                     "logits": {"addr": lg, "row_bytes": 128},
                     "kv_cache": [{"addr": kc, "bytes": kvs}, {"addr": vc, "bytes": kvs}], "kv_cache_bytes": 2 * kvs}}
    import json
    secs = [(1, 0, bytes(dram)), (2, 4, p4), (2, 1, p1), (3, 0, json.dumps(meta).encode())]
    off = 12 + 24 * len(secs)
    table, body = b"", b""
    for kind, flags, data in secs:
        table += struct.pack("<IIQQ", kind, flags, off + len(body), len(data))
        body += data
    return struct.pack("<III", 0x4E424C4C, 2, len(secs)) + table + body
