#!/usr/bin/env python
"""Benchmark of the integer decoder datapath on one MI355X.

Headline (BASELINE.json metric): greedy INT8 decode tok/s at the Qwen2.5-0.5B shape
(config 4: 24 layers, dim 896, 14/2 heads, head_dim 64, FFN 4864, vocab 151936, QKV bias),
batch 1, over the 256 positions after a 512-token prefill.  One step = one replay of the captured
decode graph: the one-launch decode step (all 24 layers), the last layer's finish, the lm_head with
the record row, and the greedy step (argmax, embedding gather of the next row), with weights, KV
cache and activations resident in HBM.

The JSON line also carries
  roofline     : the decode kernel family that moves the most bytes per step (dec_step: the
                 one-launch decode step, every layer's weights and K/V rows, 363 MB): algorithmic
                 bytes per launch / average launch duration (HIP events around a graph of that
                 family's launch, whose weights exceed the 256 MB memory-side cache), against 8 TB/s;
                 `traffic` is the HBM bytes per launch measured with rocprofv3 counters
                 (profiles/decode_traffic.json, copy-kernel calibrated); extra.decode_hbm_frac_of_step
                 is the whole step's bytes over its time;
  cpu_baseline : the fastest of three CPU baselines, each timed on a bounded sample of the same
                 decode launches on this host and checked equal to the GPU's (extra.cpu_baselines:
                 cpu-golden-np, the numpy restatement with golden.py's structure, one core;
                 cpu-golden-np-blas, its fast_matmul path through exact FP64 BLAS, all BLAS
                 threads; cpu-ref-c, oracle/numerics.c with OpenMP; plus the host's CPU model, core
                 counts and BLAS configuration);
  extra        : prefill tok/s (the one-launch 512-row prefill as the HIP graph prefill() replays
                 from the second prompt of a shape on; prefill_eager_ms: its ~300 launches
                 enqueued one by one, as the first prompt of a shape runs; prefill_api_ms adds the
                 host side of prefill(): the device copy of the L logits rows it returns, each row
                 downloaded when read -- here the last),
                 per-family decode timings, config 4 at batch 16, config 5 (Qwen3 shape, T = 4096)
                 decode launch time, config-2 GEMM TOPS and GB/s (weights rotated through copies
                 larger than the memory-side cache), the qgraph producer's weight conversion
                 (llhip_quant_rows_i8, lm_head-shaped f32) against HBM and its numpy baseline,
                 the instruction-set device running a compiled-style Qwen2.5-0.5B-shaped
                 decode step beside the reference's functional simulator on one host core, and
                 the float side's calibration and SmoothQuant of a Qwen2.5-0.5B-shaped fp32 model
                 beside its float64 restatement.

    python bench.py [--gpus 1] [--steps 64] [--warmup 8]
    python bench.py --profile decode   # prefill + decode launches only (for rocprofv3)
    python bench.py --profile prefill  # prefill() once, eager, captured and replayed 512-row prefills
    python bench.py --profile gemm     # config 2's M=2048 x K=896 x N=151936 GEMM, 7 launches
    python bench.py --profile copy     # 256 MiB device copies (counter calibration)
    python bench.py --profile quant    # llhip_quant_rows_i8 on a 151936 x 896 f32 matrix, 7 launches
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
METRIC = "INT8 decode tok/s (Qwen2.5-0.5B shape); GEMM int8 TOPS + HBM GB/s % peak"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def build_workload(cfg_name: str, seed: int) -> Path:
    from llaccel_amd import synth

    root = Path(os.environ.get("LLACCEL_BENCH_DIR", Path(tempfile.gettempdir()) / "llaccel_bench"))
    qdir = root / f"{cfg_name}_s{seed}"
    if not (qdir / "qgraph.json").exists():
        t0 = time.time()
        synth.build_qgraph(qdir, cfg_name, seed=seed, fusion=True)
        log(f"built {cfg_name} qgraph in {time.time() - t0:.1f}s -> {qdir}")
    return qdir


def batch_decode(qdir: Path, args, single_tokens) -> dict:
    """Config 4 at batch B: sequence b has the seeded prompt of seed + b and its own KV slot; after
    the batch prefill (one launch of B x 512 rows, timed warm), every decode launch runs the B
    sequences as B rows.  Sequence 0 has the batch-1
    run's prompt, so its tokens must equal the batch-1 warmup tokens."""
    import torch

    from llaccel_amd import golden as G
    from llaccel_amd import synth

    B = args.batch
    g = G.GoldenModel(qdir)
    prompts = [synth.seeded_prompt("qwen25", args.prompt, args.seed + b) for b in range(B)]
    L = len(prompts[0])
    t_pre = []
    for _ in range(2):  # the first call also allocates the B x 512-row activations
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        rows = g.prefill_batch(prompts)
        torch.cuda.synchronize()
        t_pre.append(time.perf_counter() - t0)
    nxt = [G.GoldenModel.argmax(r[-1], g.vocab) for r in rows]
    toks_w, _ = g.decode_batch_loop(nxt, [L] * B, args.warmup)
    same = None if single_tokens is None else bool(np.array_equal(toks_w[:, 0], np.asarray(single_tokens)))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    g.decode_batch_loop([int(t) for t in toks_w[-1]], [L + args.warmup] * B, args.steps, sync=False)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    return {"batch": B, "tok_s": round(B * args.steps / dt, 1), "ms_per_step": round(dt / args.steps * 1e3, 4),
            "steps": args.steps, "prefill_ms_all": round(t_pre[1] * 1e3, 2),
            "prefill_ms_all_first_call": round(t_pre[0] * 1e3, 1),
            "prefill_note": "the B prompts as one launch of B x 512 rows (prefill_batch), logits of every row kept",
            "sequence0_tokens_equal_batch1": same}


def config5_decode(args) -> dict:
    """Config 5: Qwen3-0.6B shape (28 layers, dim 1024, 16/8 heads, head_dim 128, Q/K norm, vocab
    151936), every layer's KV filled with seeded int8 at positions 0..4094, then the 28 layers +
    lm_head of one decode launch at position 4095 (T = 4096 keys per head) captured as one graph
    and replayed; then whole decode steps as decode_loop replays them (embedding gather, layers,
    head and greedy step) at positions 4076 .. 4095 (T = 4077 .. 4096)."""
    import torch

    from llaccel_amd import golden as G

    qdir = build_workload("qwen3", args.seed)
    g = G.GoldenModel(qdir)
    gen = torch.Generator(device="cuda").manual_seed(4095 + args.seed)
    for kc, vc in g._kv.values():
        for t in (kc, vc):
            t.copy_(torch.randint(-128, 128, tuple(t.shape), dtype=torch.int8, device="cuda", generator=gen))
            t[:, :, 4095:] = 0
    T = 4096
    graph = g._chain.capture_family(None, T - 1)
    dt = time_graph(graph, 20)
    kv_bytes = sum(2 * kc[0].numel() for kc, _ in g._kv.values())
    step_bytes = sum(g._chain.step_bytes(T).values())
    # the attention family alone: the T = 4096 key scans and the output projection
    ga = g._chain.capture_family("dec_attention", T - 1)
    ta = time_graph(ga, 20) / g.n_layers
    att_bytes = g._chain.step_bytes(T)["dec_attention"] / g.n_layers
    g.decode_loop(1, T - 20, 2)  # captures the decode graph
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    g.decode_loop(1, T - 20, 20, sync=False)
    torch.cuda.synchronize()
    dl = (time.perf_counter() - t0) / 20
    return {"T": T, "layers": g.n_layers, "ms_per_step": round(dl * 1e3, 4), "tok_s": round(1 / dl, 1),
            "whole_step_positions": [T - 20, T - 1], "layers_head_ms_at_T4096": round(dt * 1e3, 4),
            "kv_bytes_read": kv_bytes, "step_bytes": step_bytes,
            "hbm_frac_of_step": round(step_bytes / dt / 1e9 / HBM_PEAK_GBS, 4),
            "attention_us_per_layer": round(ta * 1e6, 2), "attention_bytes_per_layer": round(att_bytes),
            "attention_hbm_frac": round(att_bytes / ta / 1e9 / HBM_PEAK_GBS, 4),
            "note": "layers + lm_head of one M=1 decode launch at position 4095 (the decode chain's launches, "
                    "replayed at that position); attention: the layer's attention launches with the output "
                    "projection's partial sums"}


def measured_traffic(family: str):
    """HBM bytes (fetched + written) per launch of a decode kernel family, from the committed
    rocprofv3 counter summary (profiles/decode_traffic.json), or None when not measured."""
    f = REPO / "profiles" / "decode_traffic.json"
    if not f.exists():
        return None
    k = json.loads(f.read_text()).get("families", {}).get(family)
    return None if k is None else int(k["fetch_bytes_per_launch"] + k["write_bytes_per_launch"])


def time_graph(graph, reps: int) -> float:
    """Average seconds per replay, HIP events on the current stream."""
    import torch

    graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        graph.replay()
    end.record()
    end.synchronize()
    return start.elapsed_time(end) / 1000.0 / reps


def host_info() -> dict:
    """The CPU the baselines ran on: core counts, model name, the OpenMP and BLAS settings."""
    import os

    model = "?"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    info = {"nproc": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0)), "cpu_model": model,
            "OMP_NUM_THREADS": os.environ.get("OMP_NUM_THREADS")}
    try:
        import threadpoolctl

        info["blas"] = [{k: d.get(k) for k in ("internal_api", "version", "num_threads", "threading_layer")}
                        for d in threadpoolctl.threadpool_info() if d.get("user_api") == "blas"]
    except ImportError:
        info["blas"] = None
    return info


def cpu_baseline(qdir: Path, backend: str, kv0: dict, first_token: int, pos0: int, gpu_rows, gpu_toks,
                 budget_s: float):
    """Time the oracle (`backend`: "np" the reference structure, "blas" the reference's FP64-BLAS
    fast_matmul path, "c" the OpenMP restatement) on decode launches from the GPU's post-prefill KV
    state, checking each launch's logits and argmax equal the GPU's."""
    from oracle import golden_np as O

    o = O.OracleModel(qdir, backend=backend)
    for layer, (k, v) in kv0.items():
        o.kv[layer][0][...] = k
        o.kv[layer][1][...] = v
    tok = first_token
    n = 0
    t0 = time.perf_counter()
    exact = True
    while n < len(gpu_toks):
        row = o.decode(tok, pos0 + n)
        exact &= bool(np.array_equal(row[:gpu_rows.shape[1]], gpu_rows[n]))
        tok = o.argmax(row, o.vocab)
        exact &= tok == int(gpu_toks[n])
        n += 1
        if time.perf_counter() - t0 > budget_s:
            break
    dt = time.perf_counter() - t0
    return n / dt, n, dt, exact


def cpu_baselines(qdir: Path, kv0: dict, first_token: int, pos0: int, gpu_rows, gpu_toks, budget_s: float) -> dict:
    """The three CPU baselines of the measurement plan, each on a bounded sample of the same decode
    launches: cpu-golden-np (1 core), cpu-golden-np-blas (all BLAS threads), cpu-ref-c (OpenMP)."""
    from oracle import golden_np as O

    out = {}
    for label, backend in (("cpu-golden-np", "np"), ("cpu-golden-np-blas", "blas"), ("cpu-ref-c", "c")):
        v, n, dt, exact = cpu_baseline(qdir, backend, kv0, first_token, pos0, gpu_rows, gpu_toks, budget_s)
        if not exact:
            raise SystemExit(f"CPU baseline {label} and the GPU decode launches differ")
        host = host_info()
        if backend == "np":
            cores, how = 1, "numpy int64 a @ w.T (single-threaded) + a Python loop per (row, head) for attention"
        elif backend == "blas":
            cores = max((b["num_threads"] or 1 for b in host["blas"] or []), default=1)
            how = ("GEMMs through exact FP64 BLAS (golden.py:217-240, fast_matmul=True) with all BLAS threads, "
                   "attention as the Python loop per (row, head)")
        else:
            cores = int(O.c_oracle().orc_set_threads(0))
            how = "oracle/numerics.c (int8 GEMV and attention), OpenMP over all host threads"
        out[label] = {"value": round(v, 4), "unit": "tok/s", "cores": cores, "kind": "port",
                      "sample": f"{n} greedy decode launches at positions {pos0}..{pos0 + n - 1} from the GPU's "
                                f"post-prefill KV state ({dt:.1f}s): {how}; logits and argmax bit-identical to the "
                                "GPU: True"}
        log("cpu baseline", label, out[label])
    out["host"] = host_info()
    return out


def gemm_sweep(min_reps: int = 8):
    """Config-2 shapes, i8 out: TOPS and algorithmic GB/s per shape (HIP events over a graph).

    Every launch of the timed graph reads its own copy of W, and the copies together exceed
    twice the 256 MiB memory-side cache, so no launch finds its weights cached by an earlier one."""
    import ctypes

    import torch

    from llaccel_amd import _lib
    from llaccel_amd.golden import capture_graph

    ws = torch.zeros(int(_lib.lib().llhip_workspace_bytes()), dtype=torch.uint8, device="cuda")
    out = []
    shapes = [(M, K, N) for M in (2048, 128, 16, 1) for K, N in ((896, 151936), (896, 4864), (4864, 896), (896, 896))]
    for M, K, N in shapes:  # config 2: the 16 shapes
        copies = max(4, -(-(512 << 20) // (N * K)))
        reps = max(min_reps, copies)
        g = torch.Generator(device="cuda").manual_seed(M + K + N)
        a = torch.randint(-127, 128, (M, K), dtype=torch.int8, device="cuda", generator=g)
        w0 = torch.randint(-127, 128, (N, K), dtype=torch.int8, device="cuda", generator=g)
        ws_w = [w0] + [torch.roll(w0, c, 0) for c in range(1, copies)]
        rq = torch.stack([torch.full((N,), 1 << 30, dtype=torch.int32, device="cuda"),
                          torch.full((N,), 42, dtype=torch.int32, device="cuda")], 1).contiguous()
        o = torch.empty((M, N), dtype=torch.int8, device="cuda")
        p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731

        def launch(w):
            s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)  # the capture stream inside the graph
            _lib.call("llhip_linear", p(a), M, K, K, p(w), N, p(rq), None, 0, None, N, 0, 0, 0, 0, 1, p(o), N, p(ws), s)

        graph = torch.cuda.CUDAGraph()
        with capture_graph(graph):
            for r in range(reps):
                launch(ws_w[r % copies])
        dt = time_graph(graph, 3) / reps
        nbytes = N * K + M * K + 8 * N + M * N
        out.append({"M": M, "K": K, "N": N, "us": round(dt * 1e6, 2), "TOPS": round(2 * M * N * K / dt / 1e12, 1),
                    "GBs": round(nbytes / dt / 1e9, 1), "weight_copies": copies})
        log("gemm", out[-1])
        del a, w0, ws_w, o, graph
    return out


def quantizer_bench(cpu_rows: int = 2048) -> dict:
    """The qgraph producer's weight conversion (llhip_quant_rows_i8) on an lm_head-shaped f32
    matrix (151936 x 896, 544 MB, larger than the memory-side cache): HIP events over a graph of
    launches; algorithmic bytes 4NK read + NK + 8N written.  CPU baseline: the float64 numpy
    restatement (oracle/quant_np.py) on the first `cpu_rows` rows, checked equal to the GPU's."""
    import ctypes

    import torch

    from llaccel_amd import _lib
    from llaccel_amd.golden import capture_graph
    from oracle import quant_np as QN

    N, K, reps = 151936, 896, 10
    g = torch.Generator(device="cuda").manual_seed(17)
    w = torch.randn((N, K), dtype=torch.float32, device="cuda", generator=g) * 0.02
    q = torch.empty((N, K), dtype=torch.int8, device="cuda")
    sc = torch.empty(N, dtype=torch.float64, device="cuda")
    st = torch.zeros(1, dtype=torch.int32, device="cuda")
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731

    def launch():
        s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        _lib.call("llhip_quant_rows_i8", p(w), N, K, K, p(q), K, p(sc), p(st), s)

    graph = torch.cuda.CUDAGraph()
    with capture_graph(graph):
        for _ in range(reps):
            launch()
    dt = time_graph(graph, 3) / reps
    nbytes = 5 * N * K + 8 * N
    wh = w[:cpu_rows].cpu().numpy().astype(np.float64)
    t0 = time.perf_counter()
    cq, cs = QN.quant_rows_i8(wh)
    cdt = time.perf_counter() - t0
    same = bool(np.array_equal(cq, q[:cpu_rows].cpu().numpy()) and np.array_equal(cs, sc[:cpu_rows].cpu().numpy())
                and int(st.item()) == 0)
    out = {"shape": [N, K], "us": round(dt * 1e6, 2), "GBs": round(nbytes / dt / 1e9, 1),
           "frac_hbm": round(nbytes / dt / 1e9 / HBM_PEAK_GBS, 4), "bytes_per_launch": nbytes,
           "cpu_baseline": {"rows_per_s": round(cpu_rows / cdt, 1), "GBs": round(5 * cpu_rows * K / cdt / 1e9, 3),
                            "cores": 1, "kind": "port",
                            "sample": f"first {cpu_rows} rows, float64 numpy restatement; equal to the GPU: {same}"},
           "gpu_rows_per_s": round(N / dt, 1)}
    del graph, w, q
    return out


def blas_threads() -> int:
    """Threads of the host BLAS numpy uses (threadpoolctl), else the host's CPU count."""
    try:
        from threadpoolctl import threadpool_info

        return int(max(i["num_threads"] for i in threadpool_info() if i.get("user_api") == "blas"))
    except (ImportError, ValueError, KeyError):
        return os.cpu_count() or 1


def floatside_bench(cpu_tokens: int = 16) -> dict:
    """The float side on the GPU (llaccel_amd.floatside) over a Qwen2.5-0.5B-shaped fp32 model
    (seeded N(0, 0.02) weights, unit norms, small QKV biases; 494M parameters): calibrate_tokens over
    4 seeded sequences of 256 tokens and smooth_model (alpha 0.5) over the same sequences, wall clock
    around each call (the records are downloaded once, at the end of a call).  CPU baseline: the
    float64 numpy restatement (oracle/float_np.py) calibrating the first `cpu_tokens` tokens of the
    first sequence, whose records the GPU's equal to rtol 1e-4."""
    import torch

    from llaccel_amd.floatside import FloatConfig, FloatModel, _expected_shapes, calibrate_tokens, smooth_model
    from oracle import float_np as FO

    cfg = FloatConfig(dim=896, n_layers=24, n_heads=14, n_kv_heads=2, head_dim=64, ffn=4864, vocab=151936,
                      max_seq=1024, qkv_bias=True, rope_base=1e6, rms_eps=1e-6)
    g = torch.Generator(device="cuda").manual_seed(23)
    params = {}
    for name, shape in _expected_shapes(cfg).items():
        role = name.split("_", 1)[-1]
        if "norm" in role:
            params[name] = torch.ones(shape, dtype=torch.float32, device="cuda")
        elif role in ("bq", "bk", "bv"):
            params[name] = (torch.rand(shape, generator=g, device="cuda") - 0.5) * 0.06
        else:
            params[name] = torch.randn(shape, generator=g, device="cuda") * 0.02
    model = FloatModel(cfg, params)
    rng = np.random.default_rng(5)
    seqs = [rng.integers(0, cfg.vocab, 256).tolist() for _ in range(4)]
    sample = [seqs[0][:cpu_tokens]]
    gpu_sample = calibrate_tokens(model, sample)  # also the warm-up (library heuristics, first launches)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    calibrate_tokens(model, seqs)
    t_cal = time.perf_counter() - t0
    t0 = time.perf_counter()
    meta = smooth_model(model, seqs, 0.5)
    t_sm = time.perf_counter() - t0
    del model
    p64 = {k: v.double().cpu().numpy() for k, v in params.items()}
    del params
    t0 = time.perf_counter()
    want = FO.calibrate_tokens(cfg, p64, sample)
    t_cpu = time.perf_counter() - t0
    worst = max(abs(gpu_sample[k] - v) / max(abs(v), 1e-30) for k, v in want.items())
    ntok = sum(map(len, seqs))
    return {"model": "Qwen2.5-0.5B shape, fp32, seeded weights", "calibration_tokens": ntok,
            "calibrate_ms": round(t_cal * 1e3, 2), "calibrate_tok_s": round(ntok / t_cal, 1),
            "smooth_ms": round(t_sm * 1e3, 2), "smooth_groups": len(meta["groups"]),
            "cpu_baseline": {"tok_s": round(cpu_tokens / t_cpu, 2), "cores": blas_threads(), "kind": "port",
                             "sample": f"calibration of the first {cpu_tokens} tokens, float64 numpy restatement; "
                                       f"GPU records equal to rtol 1e-4: {worst < 1e-4} (worst {worst:.1e})"}}


def isa_device_bench() -> dict:
    """The instruction-set device (llaccel_amd.device.GpuDevice) on a compiled-style M = 1 decode
    step of the Qwen2.5-0.5B shape (llaccel_amd.isa_synth.decoder_program: 24 layers, weights
    streamed into the 1 MiB SRAM in N-chunks, chunked lm_head; ~3200 instructions): wall time per
    run() after one warm-up run.  CPU baseline: the reference's own functional simulator
    (runtime/src/funcsim.cpp compiled into oracle/_ref) on the same program, one run, checked equal
    to the GPU's logits and counters; without it, oracle/isa_np.py on a one-layer program."""
    import ctypes

    from llaccel_amd import isa_synth
    from llaccel_amd.device import GpuDevice

    img, pc, pos, meta = isa_synth.decoder_program(seed=3)
    dev = GpuDevice(0, True)
    dev.dram_write(0, img)
    perf = dev.run(pc, pos)
    t = []
    for _ in range(3):
        t0 = time.perf_counter()
        dev.run(pc, pos)
        t.append(time.perf_counter() - t0)
    gpu_s = min(t)
    logits = dev.dram_read(meta["logits"], meta["vocab"] * 2)
    out = {"program": "compiled-style decode step, Qwen2.5-0.5B shape (synthetic weights)",
           "instructions": meta["instructions"], "dram_bytes": len(img), "gpu_ms_per_run": round(gpu_s * 1e3, 2),
           "gpu_instr_per_s": round(meta["instructions"] / gpu_s, 1),
           "gemm_macs_per_run": perf[6] * 256}
    del dev
    ref = Path(__file__).resolve().parent / "oracle" / "_ref" / "libfuncsim_ref.so"
    if ref.exists():
        L = ctypes.CDLL(str(ref))
        L.fs_create.restype = ctypes.c_void_p
        L.fs_create.argtypes = [ctypes.c_uint64, ctypes.c_int]
        L.fs_write.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_char_p, ctypes.c_uint64]
        L.fs_read.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_uint64]
        L.fs_run.argtypes = [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p]
        L.fs_destroy.argtypes = [ctypes.c_void_p]
        h = L.fs_create(0, 1)
        L.fs_write(h, 0, img, len(img))
        cperf = (ctypes.c_uint64 * 27)()
        t0 = time.perf_counter()
        rc = L.fs_run(h, pc, pos, cperf)
        cdt = time.perf_counter() - t0
        buf = ctypes.create_string_buffer(meta["vocab"] * 2)
        L.fs_read(h, meta["logits"], buf, meta["vocab"] * 2)
        L.fs_destroy(h)
        same = rc == 0 and buf.raw == logits and list(cperf) == perf
        out["cpu_baseline"] = {"ms_per_run": round(cdt * 1e3, 1), "cores": 1, "kind": "reference",
                               "sample": f"the same program, one run on the reference functional simulator; logits "
                                         f"and counters equal to the GPU's: {same}"}
    else:
        from oracle.isa_np import FuncSimNp
        img1, pc1, pos1, meta1 = isa_synth.decoder_program(layers=1, seed=3)
        o = FuncSimNp(0, True)
        o.dram_write(0, img1)
        t0 = time.perf_counter()
        o.run(pc1, pos1)
        out["cpu_baseline"] = {"ms_per_run": round((time.perf_counter() - t0) * 1e3, 1), "cores": 1, "kind": "port",
                               "sample": f"one-layer program ({meta1['instructions']} instructions), numpy restatement"}
    out["speedup_vs_cpu"] = round(out["cpu_baseline"]["ms_per_run"] / out["gpu_ms_per_run"], 1)
    return out


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256, help="timed decode steps (config 4 decodes 256 positions)")
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-budget", type=float, default=6.0, help="seconds of work per CPU baseline (three of them)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-gemm", action="store_true")
    ap.add_argument("--no-config5", action="store_true", help="skip the Qwen3 T=4096 decode timing")
    ap.add_argument("--no-quant", action="store_true", help="skip the weight-quantization kernel timing")
    ap.add_argument("--no-isa", action="store_true", help="skip the instruction-set device timing")
    ap.add_argument("--no-float", action="store_true", help="skip the float-side calibration timing")
    ap.add_argument("--batch", type=int, default=16, help="also time config 4's batch decode (1 = skip)")
    ap.add_argument("--profile", choices=("decode", "copy", "prefill", "gemm", "quant", "config5", "batch"),
                    help="workload-only runs for rocprofv3")
    ap.add_argument("--gemm-shape", default="2048,896,151936", help="M,K,N of --profile gemm")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (this build runs the datapath on a "
              "single MI355X; multi-GPU sharding is design-only)", file=sys.stderr)
        sys.exit(2)

    import torch

    if args.profile == "copy":
        # counter calibration: device-to-device copies of a known size
        n = 256 << 20
        src = torch.randint(0, 255, (n,), dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copied {n} bytes x 10")
        return

    if args.profile == "gemm":
        # a config-2 shape (default the largest), i8 output: 7 launches, each on its own weight copy
        # (every launch reads cold weights)
        import ctypes

        from llaccel_amd import _lib

        M, K, N = (int(v) for v in args.gemm_shape.split(","))
        g = torch.Generator(device="cuda").manual_seed(0)
        a = torch.randint(-127, 128, (M, K), dtype=torch.int8, device="cuda", generator=g)
        ws_w = [torch.randint(-127, 128, (N, K), dtype=torch.int8, device="cuda", generator=g) for _ in range(7)]
        rq = torch.stack([torch.full((N,), 1 << 30, dtype=torch.int32, device="cuda"),
                          torch.full((N,), 42, dtype=torch.int32, device="cuda")], 1).contiguous()
        o = torch.empty((M, N), dtype=torch.int8, device="cuda")
        ws = torch.zeros(int(_lib.lib().llhip_workspace_bytes()), dtype=torch.uint8, device="cuda")
        p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
        s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        for r in range(7):
            _lib.call("llhip_linear", p(a), M, K, K, p(ws_w[r]), N, p(rq), None, 0, None, N, 0, 0, 0, 0, 1, p(o), N,
                      p(ws), s)
        torch.cuda.synchronize()
        log(f"gemm {M}x{K}x{N}: 7 launches")
        return

    if args.profile == "quant":
        # the weight conversion of the qgraph producer on an lm_head-shaped f32 matrix, 7 launches
        import ctypes

        from llaccel_amd import _lib

        N, K = 151936, 896
        g = torch.Generator(device="cuda").manual_seed(17)
        w = torch.randn((N, K), dtype=torch.float32, device="cuda", generator=g) * 0.02
        q = torch.empty((N, K), dtype=torch.int8, device="cuda")
        sc = torch.empty(N, dtype=torch.float64, device="cuda")
        st = torch.zeros(1, dtype=torch.int32, device="cuda")
        p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
        s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        for _ in range(7):
            _lib.call("llhip_quant_rows_i8", p(w), N, K, K, p(q), K, p(sc), p(st), s)
        torch.cuda.synchronize()
        log(f"quant_rows_i8 {N}x{K}: 7 launches")
        return

    if args.profile == "config5":
        log("config 5 decode", config5_decode(args))
        return

    from llaccel_amd import golden as G

    cfg = "qwen25"
    qdir = build_workload(cfg, args.seed)
    if args.profile == "batch":
        log("batch decode", batch_decode(qdir, args, None))
        return
    from llaccel_amd import synth

    prompt = synth.seeded_prompt(cfg, args.prompt, args.seed)
    L = len(prompt)
    g = G.GoldenModel(qdir)
    need = L + max(args.warmup, args.steps) + 1
    if need > g.max_seq:
        raise SystemExit(f"prompt + steps = {need} exceeds max_seq {g.max_seq}")

    # ---- prefill (one launch of the whole prompt) ----
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    rows = g.prefill(prompt)
    torch.cuda.synchronize()
    t_prefill = time.perf_counter() - t0
    nxt = G.GoldenModel.argmax(rows[-1], g.vocab)
    kv0 = g.kv
    # the same launches without the host side of the API (the logits rows of all L positions,
    # downloaded and widened to int64 numpy rows): eagerly enqueued, and as the replayed graph that
    # prefill() captures on the second prompt of a shape
    padded = -(-L // g.prefill_m) * g.prefill_m

    def timed(fn):
        t = []
        for _ in range(3):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            t.append(time.perf_counter() - t0)
        return min(t)

    t_prefill_eager = timed(lambda: g._launch_tokens(prompt, 0, padded))
    g._prefill_launch(prompt, padded)  # the second prefill of this shape: captured
    t_prefill_dev = timed(lambda: g._prefill_launch(prompt, padded))
    # prefill() itself once warm (its graph captured): the launches plus the API's host side -- the
    # device copy of the L logits rows it returns and the one row read here
    t_prefill_api = timed(lambda: G.GoldenModel.argmax(g.prefill(prompt)[-1], g.vocab))
    log(f"prefill {L} tokens: {t_prefill_api * 1e3:.2f} ms through prefill() ({t_prefill * 1e3:.1f} ms the first "
        f"time), {t_prefill_dev * 1e3:.2f} ms on the GPU "
        f"(graph replay; {t_prefill_eager * 1e3:.2f} ms eagerly enqueued)")
    if args.profile == "prefill":
        return

    # ---- decode: warmup steps at positions L.. (the first captures the graph), then the timed steps
    # decode again from position L: config 4's positions L .. L + steps - 1.  Greedy decode is
    # deterministic, so the timed run rewrites the warmup's KV rows with equal values. ----
    toks_w, rows_w = g.decode_loop(nxt, L, args.warmup)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    g.decode_loop(nxt, L, args.steps, sync=False)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    g._chain.check_step()
    tok_s = args.steps / dt
    log(f"decode: {args.steps} steps (positions {L}..{L + args.steps - 1}) in {dt * 1e3:.1f} ms -> {tok_s:.1f} tok/s")
    if args.profile == "decode":
        return

    # ---- per-kernel families of one decode step (graphs of the step's launches of one kind) ----
    # Each family's launches of one step replayed alone at the last timed position, HIP events around
    # 20 replays.  The dominant family by bytes (dec_step: every layer's weights, 363 MB) exceeds the
    # 256 MB memory-side cache, so its replays stream from HBM.
    import ctypes

    T = L + args.steps
    fam = {}
    ch = g._chain
    fbytes = ch.step_bytes(T)
    for kind in ch.families(ctypes.c_void_p(g._st.data_ptr() + 4)):
        n = ch.launches(kind)
        graph = ch.capture_family(kind, T - 1)
        t = time_graph(graph, 20)
        nbytes = fbytes[kind]
        fam[kind] = {"launches": n, "us_per_step": round(t * 1e6, 2), "us_per_launch": round(t / n * 1e6, 3),
                     "bytes_per_launch": round(nbytes / n), "GBs": round(nbytes / t / 1e9, 1)}
        log(f"  {kind:14s} {n:3d} launches {t * 1e6:8.1f} us/step {t / n * 1e6:7.2f} us/launch "
            f"{nbytes / 1e6:8.2f} MB -> {nbytes / t / 1e9:7.1f} GB/s")
        del graph
    # the family that moves the most HBM bytes per step (the share of the step the HBM roofline bounds)
    dom = max(fam, key=lambda k: fam[k]["bytes_per_launch"] * fam[k]["launches"])
    d = fam[dom]
    achieved = d["bytes_per_launch"] / (d["us_per_launch"] * 1e-6) / 1e9
    roofline = {"bound": "hbm", "kernel": f"{dom} (decode, M=1; {d['launches']} launches per step)",
                "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(dom),
                "bytes_per_launch": d["bytes_per_launch"], "avg_launch_us": d["us_per_launch"]}
    step_bytes = sum(fam[k]["bytes_per_launch"] * fam[k]["launches"] for k in fam)

    # the three-launch chain (24 x 3 layer launches, then the head) on the first 64 of the same positions
    chain = None
    if ch._step is not None:
        ch.use_step = False
        g.decode_loop(nxt, L, 2)  # captures the chain's graph
        n_ch = min(64, args.steps)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        g.decode_loop(nxt, L, n_ch, sync=False)
        torch.cuda.synchronize()
        t_ch = time.perf_counter() - t0
        ch.use_step = True
        chain = {"tok_s": round(n_ch / t_ch, 1), "ms_per_step": round(t_ch / n_ch * 1e3, 4), "steps": n_ch,
                 "note": "the same decode as the headline through the three-launch-per-layer chain"}
        log("decode chain", chain)

    # ---- CPU baselines (bounded samples of the same decode launches) ----
    cpu = cpus = None
    if not args.no_cpu:
        # the GPU's record of 32 launches from the post-prefill state, which the CPU runs must equal
        toks_r, rows_r = g.decode_loop(nxt, L, 32)
        cpus = cpu_baselines(qdir, kv0, nxt, L, rows_r, toks_r, args.cpu_budget)
        cpu = dict(cpus["cpu-ref-c"], baseline="cpu-ref-c")  # the fastest of the three is the headline

    batch = None
    if args.batch > 1:
        batch = batch_decode(qdir, args, toks_w)
        log("batch decode", batch)

    extra = {"prefill_tok_s": round(L / t_prefill_dev, 1), "prefill_ms": round(t_prefill_dev * 1e3, 3),
             "prefill_eager_ms": round(t_prefill_eager * 1e3, 3),
             "prefill_api_ms": round(t_prefill_api * 1e3, 3), "prefill_first_call_ms": round(t_prefill * 1e3, 2),
             "decode_step_bytes": step_bytes, "decode_hbm_frac_of_step": round(step_bytes / (dt / args.steps) / 1e9
                                                                                / HBM_PEAK_GBS, 4),
             "decode_roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / step_bytes, 1), "decode_kernel_families": fam,
             "decode_chain": chain}
    if batch is not None:
        extra[f"decode_batch{args.batch}"] = batch
    if cpus is not None:
        extra["cpu_baselines"] = cpus
    if not args.no_config5:
        extra["config5_decode_T4096"] = config5_decode(args)
        log("config 5 decode", extra["config5_decode_T4096"])
    if not args.no_gemm:
        extra["gemm_sweep"] = gemm_sweep()
    if not args.no_quant:
        extra["quantize_rows_i8"] = quantizer_bench()
        log("quantize", extra["quantize_rows_i8"])
    if not args.no_isa:
        extra["isa_device"] = isa_device_bench()
        log("isa device", extra["isa_device"])
    if not args.no_float:
        extra["float_side"] = floatside_bench()
        log("float side", extra["float_side"])

    line = {"metric": METRIC, "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(dt / args.steps * 1e3, 4), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "int8",
            "data": "synthetic: seeded random-init Qwen2.5-0.5B-shaped int8 weights (N(0,0.02) quantized per channel),"
                    " seeded 512-token prompt",
            "config": {"workload": "config 4: Qwen2.5-0.5B-shaped integer decoder (24L, dim 896, 14/2 heads, "
                                   "head_dim 64, FFN 4864, vocab 151936, QKV bias), greedy decode batch 1 after a "
                                   f"{L}-token prefill", "batch": 1, "prompt_tokens": L,
                       "decode_positions": [L, L + args.steps - 1]},
            "roofline": roofline, "cpu_baseline": cpu, "extra": extra}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
