"""The instruction-set oracle (oracle/isa_np.py) against the reference's own functional simulator
(runtime/src/funcsim.cpp compiled from the reference sources into oracle/_ref): the same DRAM,
SRAM and 27 performance counters after every seeded program, the same error messages; and the
`.llbin` container reader (llaccel_amd.device.Llbin, llbin.cpp) on containers built here."""
from __future__ import annotations

import ctypes
import json
import struct
from pathlib import Path

import numpy as np
import pytest

from oracle.isa_np import FuncSimNp
from tests import isa_cases as C

REF = Path(__file__).resolve().parents[1] / "oracle" / "_ref" / "libfuncsim_ref.so"


class RefSim:
    """ctypes front of oracle/funcsim_shim.cpp."""

    def __init__(self, fusion: bool, seed: int = 0):
        self.L = L = ctypes.CDLL(str(REF))
        p, u64, u32 = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint32
        L.fs_create.restype = p
        L.fs_create.argtypes = [u64, ctypes.c_int]
        L.fs_create_interleaved.restype = p
        L.fs_create_interleaved.argtypes = [u64, ctypes.c_int, u32]
        for n, a in dict(fs_destroy=[p], fs_write=[p, u64, p, u64], fs_read=[p, u64, p, u64], fs_size=[p],
                         fs_run=[p, u32, u32, p], fs_sram=[p, p]).items():
            getattr(L, n).argtypes = a
        L.fs_size.restype = u64
        L.fs_error.restype = ctypes.c_char_p
        self.h = L.fs_create_interleaved(0, int(fusion), seed) if seed else L.fs_create(0, int(fusion))

    def _ok(self, rc):
        if rc:
            raise RuntimeError(self.L.fs_error().decode())

    def dram_write(self, addr, b):
        self._ok(self.L.fs_write(self.h, addr, ctypes.create_string_buffer(bytes(b), len(b)), len(b)))

    def dram_read(self, addr, n):
        buf = ctypes.create_string_buffer(n)
        self._ok(self.L.fs_read(self.h, addr, buf, n))
        return buf.raw

    def dram_size(self):
        return self.L.fs_size(self.h)

    def run(self, pc, pos):
        perf = (ctypes.c_uint64 * 27)()
        self._ok(self.L.fs_run(self.h, pc, pos, perf))
        return list(perf)

    def sram_snapshot(self):
        buf = ctypes.create_string_buffer(1 << 20)
        self._ok(self.L.fs_sram(self.h, buf))
        return buf.raw

    def __del__(self):
        self.L.fs_destroy(self.h)


needs_ref = pytest.mark.skipif(not REF.exists(), reason="oracle/_ref/libfuncsim_ref.so not built (reference absent)")
CASES = C.cases()


def _run(dev, img, pos):
    dev.dram_write(0, img)
    perf = dev.run(0, pos)
    return perf, dev.sram_snapshot(), dev.dram_read(0, dev.dram_size())


@needs_ref
@pytest.mark.parametrize("cid,img,pos,fusion", CASES, ids=[c[0] for c in CASES])
def test_oracle_equals_reference_simulator(cid, img, pos, fusion):
    ref = RefSim(fusion)
    o = FuncSimNp(0, fusion)
    p1, s1, d1 = _run(ref, img, pos)
    p2, s2, d2 = _run(o, img, pos)
    assert p1 == p2, [(i, a, b) for i, (a, b) in enumerate(zip(p1, p2)) if a != b]
    assert s1 == s2
    assert len(d1) == len(d2) and d1 == d2


@needs_ref
@pytest.mark.parametrize("cid,img,pos,fusion,msg", C.error_cases(), ids=[c[0] for c in C.error_cases()])
def test_oracle_errors_equal_reference_simulator(cid, img, pos, fusion, msg):
    for dev in (RefSim(fusion), FuncSimNp(0, fusion)):
        dev.dram_write(0, img)
        with pytest.raises(RuntimeError, match=msg.replace("[", r"\[").replace("]", r"\]")):
            dev.run(0, pos)


@pytest.mark.parametrize("cid,img,pos,fusion,msg,sram_exact", C.partial_error_cases(),
                         ids=[c[0] for c in C.partial_error_cases()])
def test_oracle_state_after_error_equals_reference_simulator(cid, img, pos, fusion, msg, sram_exact):
    """The rows a failing DMA or KV_WRITE writes before its failing row, and the DRAM an invalid
    requant entry leaves, are the reference simulator's (the GPU device is held to the same state)."""
    devs = (RefSim(fusion), FuncSimNp(0, fusion))
    for dev in devs:
        dev.dram_write(0, img)
        with pytest.raises(RuntimeError, match=msg):
            dev.run(0, pos)
    assert devs[0].dram_size() == devs[1].dram_size()
    assert devs[0].dram_read(0, devs[0].dram_size()) == devs[1].dram_read(0, devs[1].dram_size())
    if sram_exact:
        assert devs[0].sram_snapshot() == devs[1].sram_snapshot()


def test_oracle_plants_are_caught():
    """A mistake planted in the oracle's GEMM (weights untiled transposed) changes its result on a
    non-square case -- the parity test above would see it."""
    img = C.gemm_case(np.random.default_rng(1), 2, 32, 64, 0)
    good = _run(FuncSimNp(0, True), img, 0)[1]
    import oracle.isa_np as I
    orig = I.FuncSimNp._gemm

    def planted(self, w):
        w = list(w)
        w[3] = w[3]  # same operands; transpose the tile bytes in SRAM first
        wa, N, K = w[3], w[9], w[10]
        t = np.frombuffer(bytes(self.sram[wa:wa + N * K]), np.int8).reshape(-1, 16, 16).transpose(0, 2, 1)
        self.sram[wa:wa + N * K] = t.tobytes()
        return orig(self, w)
    I.FuncSimNp._gemm = planted
    try:
        bad = _run(FuncSimNp(0, True), img, 0)[1]
    finally:
        I.FuncSimNp._gemm = orig
    assert bad != good


# ---- .llbin container (llbin.cpp) ----
def _container(sections):
    hdr = struct.pack("<III", 0x4E424C4C, 2, len(sections))
    off = 12 + 24 * len(sections)
    table, body = b"", b""
    for kind, flags, data in sections:
        table += struct.pack("<IIQQ", kind, flags, off + len(body), len(data))
        body += data
    return hdr + table + body


def _image():
    prog = C.ins("NOP") + C.ins("HALT")
    dram = prog + bytes(4096)
    meta = {"programs": [{"M": 1, "pc": 0}], "model": {"head_dim": 64, "n_heads": 14, "n_kv_heads": 2,
                                                       "max_seq": 512, "dim": 896},
            "dram": {"kv_cache": [{"addr": 1024, "bytes": 2048}], "kv_cache_bytes": 2048}}
    return dram, prog, meta


def test_llbin_reader_accepts_a_valid_container():
    from llaccel_amd.device import Llbin
    dram, prog, meta = _image()
    lb = Llbin.parse(_container([(1, 0, dram), (2, 1, prog), (3, 0, json.dumps(meta).encode())]))
    p = lb.program_for_m(1)
    assert p.pc == 0 and len(p.instrs) == 2 and lb.dram_image == dram and lb.meta["model"]["dim"] == 896
    with pytest.raises(RuntimeError, match="no program compiled for M=4"):
        lb.program_for_m(4)


@pytest.mark.parametrize("mutate,msg", [
    (lambda s: [(1, 0, s[0][2][:0])] + s[1:], "llbin has no DRAM image"),
    (lambda s: s + [(2, 1, s[1][2])], "invalid or duplicate program shape"),
    (lambda s: [s[0], (2, 1, s[1][2][:60]), s[2]], "program size not a multiple of 64"),
    (lambda s: [s[0], s[1], (3, 0, json.dumps({"programs": []}).encode())], "program metadata count mismatch"),
    (lambda s: [(1, 0, bytes(64) + s[0][2][64:]), s[1], s[2]], "program section differs from executable DRAM image"),
    (lambda s: s + [(9, 0, b"")], "unknown section kind 9"),
])
def test_llbin_reader_rejects_like_the_reference(mutate, msg):
    from llaccel_amd.device import Llbin
    dram, prog, meta = _image()
    secs = [(1, 0, dram), (2, 1, prog), (3, 0, json.dumps(meta).encode())]
    with pytest.raises(RuntimeError, match=msg):
        Llbin.parse(_container(mutate(secs)))
    with pytest.raises(RuntimeError, match="bad llbin magic"):
        Llbin.parse(b"XXXX" + _container(secs)[4:])


# ---- the host loop (host.cpp) over the oracle and the reference simulator ----
def test_host_loop_on_oracle_equals_reference_simulator(tmp_path):
    """llaccel_amd.host.Host (host.cpp) runs a toy .llbin -- two prefill chunks of M = 4, then greedy
    M = 1 decode launches -- on the numpy oracle and on the reference simulator: identical records
    (argmax, logits rows, per-launch counters); a second generation clears the KV cache first."""
    if not REF.exists():
        pytest.skip("oracle/_ref/libfuncsim_ref.so not built (reference absent)")
    from llaccel_amd.device import Llbin
    from llaccel_amd.host import Host, verify_against_golden
    lb = Llbin.parse(C.toy_llbin())
    prompt = [3, 17, 40, 9, 22, 5]
    recs = []
    for dev in (RefSim(False), FuncSimNp(0, False)):
        dev.name = lambda: "sim"
        dev.max_attention_head_dim = lambda: 256
        h = Host(lb, dev)
        r1 = h.generate_tokens(prompt, 7).to_json()
        r2 = h.generate_tokens(prompt, 7).to_json()
        assert r1 == r2
        recs.append(r1)
    assert recs[0] == recs[1]
    assert [s["M"] for s in recs[0]["steps"]] == [4, 4] + [1] * 7 and len(recs[0]["generated"]) == 7
    g = tmp_path / "golden.json"
    g.write_text(json.dumps(recs[0]))
    lines = []
    r = h.generate_tokens(prompt, 7)
    assert verify_against_golden(r, g, verbose=True, out=lines.append) and lines[-1].startswith("VERIFY: MATCH")
    r.steps[3].logits[5] += 1
    lines.clear()
    assert not verify_against_golden(r, g, out=lines.append)
    assert lines[0].startswith("VERIFY: step 3 logits differ at index 5") and "MISMATCH" in lines[-1]


def test_synthetic_decoder_program_oracle_equals_reference_simulator():
    """llaccel_amd.isa_synth's compiled-style decode step (two layers of small shape): the oracle
    and the reference simulator agree on counters, SRAM and DRAM."""
    if not REF.exists():
        pytest.skip("oracle/_ref/libfuncsim_ref.so not built (reference absent)")
    from llaccel_amd import isa_synth
    img, pc, pos, meta = isa_synth.decoder_program(dim=64, heads=4, kv_heads=2, head_dim=16, ffn=192, vocab=1008,
                                                   layers=2, max_seq=64, pos=20, seed=1)
    r, o = RefSim(True), FuncSimNp(0, True)
    assert _run(r, img, pos) == _run(o, img, pos)


@needs_ref
def test_interleaving_changes_results_of_programs_without_waits():
    """The programs the GPU interleave test uses have no semaphore waits between dependent
    instructions, so the reference simulator's random legal orders change their results: the GPU's
    equality with it under a seed is a check of the order, not of a moot one."""
    rng = np.random.default_rng(1)
    img = C.chain_case(rng)
    base = _run(RefSim(True), img, 0)[1]
    assert any(_run(RefSim(True, s), img, 0)[1] != base for s in (1, 7, 1234))
