"""The GPU instruction-set device (llaccel_amd.device.GpuDevice -> csrc/device.hip) against the
CPU oracle of the reference's functional simulator (oracle/isa_np.py, itself pinned to the
reference simulator in test_isa_oracle.py): after every seeded program the same SRAM, DRAM (size
included) and 27 performance counters, bit for bit; the same errors; state kept across launches."""
from __future__ import annotations

import numpy as np
import pytest

from llaccel_amd.device import GpuDevice
from oracle.isa_np import FuncSimNp
from tests import isa_cases as C

pytestmark = pytest.mark.gpu
CASES = C.cases()


def _run(dev, img, pos):
    dev.dram_write(0, img)
    perf = dev.run(0, pos)
    return perf, dev.sram_snapshot(), dev.dram_read(0, dev.dram_size())


@pytest.mark.parametrize("cid,img,pos,fusion", CASES, ids=[c[0] for c in CASES])
def test_device_equals_oracle(cid, img, pos, fusion):
    print("case", cid, flush=True)
    g = GpuDevice(0, fusion)
    p1, s1, d1 = _run(g, img, pos)
    p2, s2, d2 = _run(FuncSimNp(0, fusion), img, pos)
    assert p1 == p2, [(i, a, b) for i, (a, b) in enumerate(zip(p1, p2)) if a != b]
    assert s1 == s2, np.flatnonzero(np.frombuffer(s1, np.uint8) != np.frombuffer(s2, np.uint8))[:10]
    assert len(d1) == len(d2) and d1 == d2


@pytest.mark.parametrize("cid,img,pos,fusion,msg", C.error_cases(), ids=[c[0] for c in C.error_cases()])
def test_device_errors_equal_oracle(cid, img, pos, fusion, msg):
    g = GpuDevice(0, fusion)
    g.dram_write(0, img)
    with pytest.raises(RuntimeError, match=msg.replace("[", r"\[").replace("]", r"\]")):
        g.run(0, pos)
    # the device stays usable after an error (the next program's stored result and counters are
    # compared; its DRAM after the error is the simulator's, test_device_state_after_error)
    ok = C.vec_case(np.random.default_rng(3), "ADD", 64)
    p1, _, d1 = _run(g, ok, 0)
    p2, _, d2 = _run(FuncSimNp(0, fusion), ok, 0)
    assert p1 == p2 and d1[:len(ok)] == d2[:len(ok)]


@pytest.mark.parametrize("cid,img,pos,fusion,msg,sram_exact", C.partial_error_cases(),
                         ids=[c[0] for c in C.partial_error_cases()])
def test_device_state_after_error(cid, img, pos, fusion, msg, sram_exact):
    """A program that fails part-way leaves DRAM (and, for a DMA or KV_WRITE that fails at a later
    row, SRAM) as the simulator leaves it, with the simulator's message."""
    print("case", cid, flush=True)
    g, o = GpuDevice(0, fusion), FuncSimNp(0, fusion)
    for d in (g, o):
        d.dram_write(0, img)
        with pytest.raises(RuntimeError, match=msg):
            d.run(0, pos)
    assert g.dram_size() == o.dram_size() == 1 << 20
    assert g.dram_read(0, g.dram_size()) == o.dram_read(0, o.dram_size())
    if sram_exact:
        assert g.sram_snapshot() == o.sram_snapshot()


def test_state_persists_across_launches():
    """One device, three launches of one KV_WRITE + ATTN program at positions 9, 10, 11 (the DRAM
    K/V cache keeps every earlier launch's rows), against the oracle doing the same."""
    img, _ = C.attn_case(np.random.default_rng(11), 1, 4, 2, 64, 9, True, max_seq=64)
    g, o = GpuDevice(0, False), FuncSimNp(0, False)
    g.dram_write(0, img)
    o.dram_write(0, img)
    for pos in (9, 10, 11):
        assert g.run(0, pos) == o.run(0, pos)
        assert g.sram_snapshot() == o.sram_snapshot()
    assert g.dram_read(0, g.dram_size()) == o.dram_read(0, o.dram_size())


def test_device_rejects_what_it_cannot_run_like_the_simulator():
    """Operand layouts whose simulator result depends on its element order (an output partly
    overlapping an input) or that the device does not map (a K/V head stride that is not a whole
    number of rows) raise instead of computing something else."""
    b = C.Builder()
    b.emit("SILU", 0x0, 0x20, 64, 1 << 30, 30, 16)
    g = GpuDevice(0, False)
    g.dram_write(0, b.image())
    with pytest.raises(RuntimeError, match="overlapping operands in VEC_SILU"):
        g.run(0, 0)
    b = C.Builder()
    b.emit("ATTN", 0x0, 0x1000, C.DATA, C.DATA + 4096, 1, 1, 1, 64, 1040, 1, 0, 1, 0)
    g.dram_write(0, b.image() + bytes(8192))
    with pytest.raises(RuntimeError, match="kv_stride not a multiple of D"):
        g.run(0, 0)
    assert g.name() == "mi355x" and g.max_attention_head_dim() == 256


def test_host_loop_on_gpu_equals_oracle(tmp_path):
    """The reference's host loop (llaccel_amd.host.Host, host.cpp) on the GPU device: a toy .llbin
    read from disk, two M = 4 prefill chunks and greedy M = 1 decode launches, twice (the KV cache
    is cleared per generation) -- the same record as on the oracle, which verifies as MATCH."""
    from llaccel_amd.device import Llbin
    from llaccel_amd.host import Host, verify_against_golden
    import json
    path = tmp_path / "toy.llbin"
    path.write_bytes(C.toy_llbin())
    lb = Llbin.load(path)
    prompt = [3, 17, 40, 9, 22, 5]
    o = FuncSimNp(0, False)
    o.name = lambda: "sim"
    o.max_attention_head_dim = lambda: 256
    want = Host(lb, o).generate_tokens(prompt, 9).to_json()
    h = Host(lb, GpuDevice(0, False))
    for _ in range(2):
        r = h.generate_tokens(prompt, 9)
        assert r.to_json() == want
    g = tmp_path / "golden.json"
    g.write_text(json.dumps(want))
    assert verify_against_golden(r, g, out=lambda s: None)


@pytest.mark.parametrize("shape", [dict(dim=64, heads=4, kv_heads=2, head_dim=16, ffn=192, vocab=1008, layers=2,
                                        max_seq=64, pos=20),
                                   dict(dim=256, heads=4, kv_heads=1, head_dim=64, ffn=1024, vocab=4096, layers=1,
                                        max_seq=256, pos=200)])
def test_synthetic_decoder_program_equals_oracle(shape):
    """A compiled-style decode step (llaccel_amd.isa_synth: chunked weight streaming, every op of a
    decoder layer, chunked lm_head) on the GPU device and on the oracle: same counters, SRAM, DRAM."""
    from llaccel_amd import isa_synth
    img, pc, pos, meta = isa_synth.decoder_program(**shape, seed=2)
    print("program", shape, meta["instructions"], flush=True)
    assert _run(GpuDevice(0, True), img, pos) == _run(FuncSimNp(0, True), img, pos)


def test_runtime_cli_runs_and_verifies_on_gpu(tmp_path, capsys):
    """`python -m llaccel_amd.host model.llbin --prompt-ids ... --tokens N --verify golden.json --out
    r.json` (the reference runtime's command line, runtime/src/main.cpp): MATCH against the oracle's
    record with exit 0, the record written; a perturbed golden gives MISMATCH and exit 1."""
    import json
    from llaccel_amd import host as Hm
    from llaccel_amd.device import Llbin
    (tmp_path / "toy.llbin").write_bytes(C.toy_llbin())
    (tmp_path / "ids.json").write_text(json.dumps([3, 17, 40, 9, 22, 5]))
    o = FuncSimNp(0, False)
    o.name = lambda: "sim"
    o.max_attention_head_dim = lambda: 256
    want = Hm.Host(Llbin.load(tmp_path / "toy.llbin"), o).generate_tokens([3, 17, 40, 9, 22, 5], 5).to_json()
    (tmp_path / "golden.json").write_text(json.dumps(want))
    args = [str(tmp_path / "toy.llbin"), "--prompt-ids", str(tmp_path / "ids.json"), "--tokens", "5", "--verify",
            str(tmp_path / "golden.json"), "--out", str(tmp_path / "r.json")]
    assert Hm.main(args) == 0
    assert "PyTorch/golden reference:  MATCH" in capsys.readouterr().out
    assert json.loads((tmp_path / "r.json").read_text()) == want
    want["argmax_per_step"][2] += 1
    (tmp_path / "golden.json").write_text(json.dumps(want))
    assert Hm.main(args + ["--quiet"]) == 1
    assert "MISMATCH" in capsys.readouterr().out
    assert Hm.main([str(tmp_path / "toy.llbin"), "--bogus"]) == 2


@pytest.mark.parametrize("seed", [1, 7, 1234])
def test_interleaved_policy_equals_reference_simulator(seed):
    """With an interleave seed the device executes the engine queues in the reference simulator's
    random legal order for that seed (funcsim.cpp:47-90): on programs whose instructions do not wait
    on each other (so the order changes the result) the SRAM, DRAM and counters equal the
    reference simulator's run with the same seed.  Needs oracle/_ref (built with the reference)."""
    from tests.test_isa_oracle import REF, RefSim
    if not REF.exists():
        pytest.skip("oracle/_ref/libfuncsim_ref.so not built (reference absent)")
    rng = np.random.default_rng(seed)
    progs = [(C.chain_case(rng), 0, True), (C.gemm_case(rng, 3, 48, 64, 1), 0, True), (C.sem_case(True), 0, False),
             (C.dma_chain_case(rng), 0, False)]
    for img, pos, fusion in progs:
        g = GpuDevice(0, fusion, seed)
        assert g.name() == "mi355x (interleaved)"
        assert _run(g, img, pos) == _run(RefSim(fusion, seed), img, pos)
