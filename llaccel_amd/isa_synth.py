"""Synthetic programs of the reference accelerator's instruction set (docs/ISA.md) in the shape the
reference compiler gives a decoder step: per layer RMSNorm + quant, the q/k/v projections, RoPE,
KV_WRITE of the new K/V rows into DRAM caches, attention over the cache, the output projection with
the residual add, RMSNorm + quant, gate (SiLU epilogue) and up (mul epilogue) projections, quant and
the down projection with the residual add; then the final RMSNorm and the lm_head.  Weights stay
in DRAM in the ISA's 16x16-tile layout and stream into SRAM with DMA_LOAD in N-chunks that fit the
1 MiB SRAM beside the activations, one GEMM per chunk, as a compiler for this SRAM must.  Values
are seeded random integers (requant tables and normalisation constants in the ranges the quantizer
produces), so the programs measure the device and check it against the CPU restatement; they are not
a trained model.
"""
from __future__ import annotations

import struct

import numpy as np

NO = 0xFF
_OPS = dict(HALT=0x01, DMA_LOAD=0x10, DMA_STORE=0x11, GEMM=0x20, RMSNORM=0x30, ROPE=0x31, SILU=0x32, MUL=0x33,
            ADD=0x34, QUANT=0x35, ATTN=0x40, KV_WRITE=0x41)
# SRAM map (bytes): activations below 0x40000, weight chunks from WBUF, rq/bias of a chunk after them
X, H16, HQ, Q16, K16, QQ, KQ, VQ, ATT, AUX, G16, F16, FQ, GAM, ROPE_T = (
    0x0, 0x4000, 0x8000, 0xA000, 0xE000, 0xF000, 0x10000, 0x11000, 0x12000, 0x14000, 0x18000, 0x24000, 0x30000,
    0x36000, 0x38000)
WBUF, WMAX, RQB = 0x40000, 0xA0000, 0xE8000


def ins(op: str, *operands, flags=0) -> bytes:
    w = [0] * 16
    w[0] = _OPS[op] | (flags << 8) | (NO << 16) | (NO << 24)
    for i, v in enumerate(operands):
        w[2 + i] = int(v) & 0xFFFFFFFF
    return struct.pack("<16I", *w)


def _tile(W: np.ndarray) -> bytes:
    N, K = W.shape
    return W.reshape(N // 16, 16, K // 16, 16).transpose(0, 2, 1, 3).astype(np.int8).tobytes()


class _Image:
    def __init__(self, base: int):
        self.base, self.data = base, bytearray()

    def put(self, b: bytes, align: int = 256) -> int:
        self.data.extend(bytes((-len(self.data)) % align))
        addr = self.base + len(self.data)
        self.data.extend(b)
        return addr


def decoder_program(dim=896, heads=14, kv_heads=2, head_dim=64, ffn=4864, vocab=151936, layers=24, max_seq=1024,
                    pos=512, seed=0):
    """(DRAM image, entry pc, POS, meta) of one M = 1 decode step; meta gives the instruction count
    and the logits buffer's DRAM address and length.  The K/V caches hold seeded keys and values for
    every position."""
    rng = np.random.default_rng(seed)
    D, Hq, Hkv = head_dim, heads, kv_heads
    code: list[bytes] = []
    img = _Image(0x100000)   # programs below 1 MiB, data above
    kvs = max_seq * D

    def rq(n, s0=18, s1=26):
        return np.stack([rng.integers(1 << 24, 1 << 28, n), rng.integers(s0, s1, n)], 1).astype("<i4").tobytes()

    def linear(W_addr, rq_addr, bias_addr, N, K, a, out, ep=0, aux=0, out_i8=False, silu=(0, 0)):
        """DMA_LOAD of each N-chunk's tiles, requant table and bias, then its GEMM."""
        rows = max(16, (WMAX // K) // 16 * 16)
        for n0 in range(0, N, rows):
            n = min(rows, N - n0)
            wb = n * K
            code.append(ins("DMA_LOAD", WBUF, W_addr + n0 * K, 1, wb, wb, wb))
            code.append(ins("DMA_LOAD", RQB, rq_addr + n0 * 8, 1, n * 8, n * 8, n * 8))
            if bias_addr:
                code.append(ins("DMA_LOAD", RQB + 0x8000, bias_addr + n0 * 4, 1, n * 4, n * 4, n * 4))
            # a chunk's outputs land at column n0 of [1][N]; aux the same columns
            osz = 1 if out_i8 else 2
            e = ep | (int(out_i8) << 4) | ((11 if ep == 3 else 0) << 8)
            code.append(ins("GEMM", a, WBUF, out + n0 * osz, RQB, RQB + 0x8000, aux + n0 * 2, 1, n, K, e, silu[0],
                            silu[1], flags=1 if bias_addr else 0))

    def weights(N, K):
        # tiles of each 16-row block are contiguous, so an N-chunk of whole 16-row blocks is one range
        return img.put(_tile(rng.integers(-128, 128, (N, K)))), img.put(rq(N)), img.put(
            rng.integers(-(1 << 16), 1 << 16, N).astype("<i4").tobytes())

    x0 = img.put(rng.integers(-3000, 3000, dim).astype("<i2").tobytes())
    rope_rows = img.put(rng.integers(-16384, 16385, (max_seq, D)).astype("<i2").tobytes())
    logits = img.put(bytes(vocab * 2))
    code.append(ins("DMA_LOAD", X, x0, 1, dim * 2, dim * 2, dim * 2))
    code.append(ins("DMA_LOAD", ROPE_T, rope_rows + pos * 2 * D, 1, 2 * D, 2 * D, 2 * D))
    for _ in range(layers):
        g = img.put(rng.integers(8000, 24000, dim).astype("<i2").tobytes())
        wq, wk, wv, wo = weights(Hq * D, dim), weights(Hkv * D, dim), weights(Hkv * D, dim), weights(dim, Hq * D)
        wg, wu, wd = weights(ffn, dim), weights(ffn, dim), weights(dim, ffn)
        kc = img.put(rng.integers(-128, 128, (Hkv, max_seq, D)).astype(np.int8).tobytes(), 64)
        vc = img.put(rng.integers(-128, 128, (Hkv, max_seq, D)).astype(np.int8).tobytes(), 64)
        code.append(ins("DMA_LOAD", GAM, g, 1, dim * 2, dim * 2, dim * 2))
        code.append(ins("RMSNORM", X, GAM, H16, 1, dim, 1000, 1 << 30, 22))
        code.append(ins("QUANT", H16, HQ, dim, 1 << 28, 22))
        linear(*wq, Hq * D, dim, HQ, Q16)
        linear(*wk, Hkv * D, dim, HQ, K16)
        linear(*wv, Hkv * D, dim, HQ, VQ, out_i8=True)
        # the table row of POS sits at ROPE_T; the ISA indexes it with POS, so the base moves back
        rbase = ROPE_T - pos * 2 * D
        code.append(ins("ROPE", Q16, Q16, 1, Hq, D, rbase, 2 * D))
        code.append(ins("ROPE", K16, K16, 1, Hkv, D, rbase, 2 * D))
        code.append(ins("QUANT", Q16, QQ, Hq * D, 1 << 28, 22))
        code.append(ins("QUANT", K16, KQ, Hkv * D, 1 << 28, 22))
        code.append(ins("KV_WRITE", KQ, kc, 1, Hkv, D, kvs))
        code.append(ins("KV_WRITE", VQ, vc, 1, Hkv, D, kvs))
        code.append(ins("ATTN", QQ, ATT, kc, vc, 1, Hq, Hkv, D, kvs, 1 << 29, 30, 1 << 29, 36, flags=2))
        linear(*wo, dim, Hq * D, ATT, X, ep=1, aux=X)
        code.append(ins("RMSNORM", X, GAM, H16, 1, dim, 1000, 1 << 30, 22))
        code.append(ins("QUANT", H16, HQ, dim, 1 << 28, 22))
        linear(*wg, ffn, dim, HQ, G16, ep=2, silu=(1 << 30, 30 | (16 << 8)))
        linear(*wu, ffn, dim, HQ, F16, ep=3, aux=G16)
        code.append(ins("QUANT", F16, FQ, ffn, 1 << 28, 22))
        linear(*wd, dim, ffn, FQ, X, ep=1, aux=X)
    gf = img.put(rng.integers(8000, 24000, dim).astype("<i2").tobytes())
    wl = weights(vocab, dim)
    code.append(ins("DMA_LOAD", GAM, gf, 1, dim * 2, dim * 2, dim * 2))
    code.append(ins("RMSNORM", X, GAM, H16, 1, dim, 1000, 1 << 30, 22))
    code.append(ins("QUANT", H16, HQ, dim, 1 << 28, 22))
    # lm_head chunks: GEMM into SRAM, then each chunk's logits stored to DRAM
    rows = (WMAX // dim) // 16 * 16
    for n0 in range(0, vocab, rows):
        n = min(rows, vocab - n0)
        code.append(ins("DMA_LOAD", WBUF, wl[0] + n0 * dim, 1, n * dim, n * dim, n * dim))
        code.append(ins("DMA_LOAD", RQB, wl[1] + n0 * 8, 1, n * 8, n * 8, n * 8))
        code.append(ins("GEMM", HQ, WBUF, ATT, RQB, 0, 0, 1, n, dim, 0, 0, 0))
        code.append(ins("DMA_STORE", ATT, logits + n0 * 2, 1, n * 2, n * 2, n * 2))
    code.append(ins("HALT"))
    prog = b"".join(code)
    assert len(prog) <= img.base, "program exceeds its region"
    meta = {"instructions": len(code), "logits": logits, "vocab": vocab}
    return prog + bytes(img.base - len(prog)) + bytes(img.data), 0, pos, meta
