"""Host-side model execution over an instruction-set device: the reference's runtime host loop
(runtime/include/llaccel/host.h, runtime/src/host.cpp) -- character tokenizer, embedding lookup
into the input buffer, chunked prefill with the largest compiled M, greedy decode with the M = 1
program, the golden.json-shaped record with per-launch performance counters, and the check of a
run against a golden trace.  `dev` is any object with the `llaccel::Device` methods
(`llaccel_amd.device.GpuDevice` on MI355X).
"""
from __future__ import annotations

import json
from dataclasses import dataclass, field

from .device import ATTN_TMAX, NUM_PERF, PERF_NAMES, Llbin

_OP_ATTN, _OP_KV_WRITE, _OP_ROPE = 0x40, 0x41, 0x31


@dataclass
class Tokenizer:
    """host.cpp:15-41: character-level, UTF-8 code points looked up in `itos`."""
    itos: list

    @staticmethod
    def load(path) -> "Tokenizer":
        try:
            with open(path, encoding="utf-8") as f:
                j = json.load(f)
        except OSError:
            raise RuntimeError(f"cannot open tokenizer {path}") from None
        return Tokenizer([str(s) for s in j["itos"]])

    def encode(self, text: str) -> list[int]:
        ids = []
        for ch in text:
            try:
                ids.append(self.itos.index(ch))
            except ValueError:
                raise RuntimeError(f"character not in vocabulary: '{ch}'") from None
        return ids

    def decode(self, ids) -> str:
        return "".join(self.itos[i] if i < len(self.itos) else "?" for i in ids)


@dataclass
class StepResult:
    """host.h:22-28."""
    pos: int
    M: int
    argmax: int
    logits: list
    perf: list


@dataclass
class GenerationResult:
    """host.h:30-35 and its JSON form (host.cpp:207-229)."""
    prompt_tokens: list = field(default_factory=list)
    generated: list = field(default_factory=list)
    steps: list = field(default_factory=list)
    total: list = field(default_factory=lambda: [0] * NUM_PERF)

    def to_json(self) -> dict:
        return {"prompt_tokens": list(self.prompt_tokens), "generated": list(self.generated),
                "argmax_per_step": [s.argmax for s in self.steps],
                "logits_last_rows": [list(s.logits) for s in self.steps],
                "steps": [{"pos": s.pos, "M": s.M, "argmax": s.argmax, "perf": dict(zip(PERF_NAMES, s.perf))}
                          for s in self.steps],
                "perf_total": dict(zip(PERF_NAMES, self.total))}


class Host:
    """host.cpp:44-101 (construction and checks), 102-205 (launches and generation)."""

    def __init__(self, bin: Llbin, dev, tok: Tokenizer | None = None):
        self.bin, self.dev, self.tok = bin, dev, None
        m = bin.meta["model"]
        need = 0
        if "head_dim" in m:
            v = m["head_dim"]
            if not isinstance(v, int) or isinstance(v, bool) or v <= 0:
                raise RuntimeError("invalid model head_dim")
            need = v
        for prog in bin.programs:  # instructions checked before upload (host.cpp:58-64)
            for w in prog.instrs:
                op = w[0] & 0xFF
                D = w[9] if op == _OP_ATTN else w[6] if op in (_OP_KV_WRITE, _OP_ROPE) else 0
                need = max(need, D)
        if need > dev.max_attention_head_dim():
            raise RuntimeError(f"model requires attention head dimension {need}; backend {dev.name()} supports at "
                               f"most {dev.max_attention_head_dim()}. Rebuild or select a backend implementing the "
                               f"required head width.")
        self.vocab, self.dim, self.max_seq = int(m["vocab"]), int(m["dim"]), int(m["max_seq"])
        d = bin.meta["dram"]
        self.emb_addr, self.emb_row = int(d["embedding"]["addr"]), int(d["embedding"]["row_bytes"])
        self.in_addr, self.in_row = int(d["input"]["addr"]), int(d["input"]["row_bytes"])
        self.lg_addr, self.lg_row = int(d["logits"]["addr"]), int(d["logits"]["row_bytes"])
        if not bin.programs:
            raise RuntimeError("no programs in llbin")
        if not self.vocab or not self.dim or not self.max_seq:
            raise RuntimeError("invalid zero model dimension")
        self.prefill_m = max(p.M for p in bin.programs)
        if self.lg_row < self.vocab * 2:
            raise RuntimeError("logits row too small for vocab")
        if self.emb_row < self.dim * 2 or self.in_row < self.dim * 2:
            raise RuntimeError("embedding/input row too small for dim")
        size = len(bin.dram_image)

        def region(base, stride, rows):
            if base > size or not stride or rows > (size - base) // stride:
                raise RuntimeError("model buffer metadata exceeds DRAM image")
        if self.max_seq > ATTN_TMAX or self.max_seq % self.prefill_m:
            raise RuntimeError("invalid context/prefill dimensions")
        region(self.emb_addr, self.emb_row, self.vocab)
        region(self.in_addr, self.in_row, self.prefill_m)
        region(self.lg_addr, self.lg_row, self.prefill_m)
        for c in d.get("kv_cache", []):
            region(int(c["addr"]), int(c["bytes"]), 1)
        dev.dram_write(0, bin.dram_image)
        if tok is not None:
            if len(tok.itos) != self.vocab:
                raise RuntimeError("tokenizer size != model vocab")
            self.tok = tok

    def _write_input_row(self, row: int, token: int | None) -> None:
        if token is not None and token >= self.vocab:
            raise RuntimeError("token ID exceeds model vocabulary")
        buf = bytearray(self.in_row)
        if token is not None:
            buf[:self.dim * 2] = self.dev.dram_read(self.emb_addr + token * self.emb_row, self.dim * 2)
        self.dev.dram_write(self.in_addr + row * self.in_row, bytes(buf))

    def _read_logits_row(self, row: int) -> list[int]:
        import numpy as np
        b = self.dev.dram_read(self.lg_addr + row * self.lg_row, self.vocab * 2)
        return np.frombuffer(b, "<i2").astype(int).tolist()

    def launch(self, row_tokens, M: int, pos: int, logits_row: int) -> StepResult:
        if M > self.max_seq or pos > self.max_seq - M:
            raise RuntimeError("sequence exceeds max_seq")
        for r in range(M):
            self._write_input_row(r, row_tokens[r] if r < len(row_tokens) else None)
        prog = self.bin.program_for_m(M)
        perf = self.dev.run(prog.pc, pos)
        logits = self._read_logits_row(logits_row)
        am = max(range(len(logits)), key=lambda i: (logits[i], -i))  # first index of the maximum
        return StepResult(pos, M, am, logits, perf)

    def generate(self, prompt: str, n_tokens: int) -> GenerationResult:
        if self.tok is None:
            raise RuntimeError("text generation requires a character tokenizer; use generateTokens")
        return self.generate_tokens(self.tok.encode(prompt), n_tokens)

    def generate_tokens(self, prompt, n_tokens: int) -> GenerationResult:
        r = GenerationResult(prompt_tokens=list(prompt))
        if not r.prompt_tokens:
            raise RuntimeError("empty prompt")
        L = len(r.prompt_tokens)
        if L > self.max_seq or n_tokens > self.max_seq - L:
            raise RuntimeError("prompt + tokens exceeds max_seq")
        if any(t >= self.vocab for t in r.prompt_tokens):
            raise RuntimeError("prompt token ID exceeds model vocabulary")
        # each generation starts a session: the KV regions are cleared, weights and programs kept
        for c in self.bin.meta["dram"].get("kv_cache", []):
            self.dev.dram_write(int(c["addr"]), bytes(int(c["bytes"])))
        P = self.prefill_m
        n_chunks = (L + P - 1) // P
        nxt = 0
        for c in range(n_chunks):
            rows = r.prompt_tokens[c * P:min(L, (c + 1) * P)]
            last = (L - 1) % P if c == n_chunks - 1 else P - 1
            s = self.launch(rows, P, c * P, last)
            nxt = s.argmax
            r.steps.append(s)
        for i in range(n_tokens):
            r.generated.append(nxt)
            if L + i + 1 >= self.max_seq:
                break
            s = self.launch([nxt], 1, L + i, 0)
            nxt = s.argmax
            r.steps.append(s)
        for s in r.steps:
            r.total = [a + b for a, b in zip(r.total, s.perf)]
        return r


def _int_array(v, name, lo, hi):
    if not isinstance(v, list) or any(not isinstance(x, int) or isinstance(x, bool) or x < lo or x > hi for x in v):
        raise RuntimeError(f"golden {name} must be an array of integers in range")
    return list(v)


def load_prompt_ids(path) -> list[int]:
    """host.h:65: externally tokenized prompt IDs (a JSON array of u32)."""
    with open(path) as f:
        return _int_array(json.load(f), "prompt IDs", 0, 0xFFFFFFFF)


def verify_against_golden(r: GenerationResult, golden_path, verbose: bool = False, out=print) -> bool:
    """host.cpp:243-287: prompt tokens, per-launch argmax and launch count, generated count, then
    every launch's logits row and the generated tokens; the same VERIFY lines."""
    try:
        with open(golden_path) as f:
            g = json.load(f)
    except OSError:
        raise RuntimeError(f"cannot open golden {golden_path}") from None
    gp = _int_array(g["prompt_tokens"], "prompt_tokens", 0, 0xFFFFFFFF)
    gg = _int_array(g["generated"], "generated", 0, 0xFFFFFFFF)
    ga = _int_array(g["argmax_per_step"], "argmax_per_step", 0, 0xFFFFFFFF)
    if "logits_last_rows" not in g:
        raise RuntimeError("golden trace has no logits")
    rows = g["logits_last_rows"]
    if not isinstance(rows, list):
        raise RuntimeError("golden logits_last_rows must be an array")
    gl = [_int_array(row, "logits_last_rows", -32768, 32767) for row in rows]
    ok = True
    if gp != r.prompt_tokens:
        out("VERIFY: prompt tokens differ from golden")
        ok = False
    n = min(len(ga), len(r.steps))
    for i in range(n):
        if ga[i] != r.steps[i].argmax:
            s = r.steps[i]
            out(f"VERIFY: step {i} argmax {s.argmax} != golden {ga[i]} (pos={s.pos} M={s.M})")
            ok = False
            break
    if len(ga) != len(r.steps):
        out(f"VERIFY: launch count {len(r.steps)} != golden {len(ga)}")
        ok = False
    if len(gg) != len(r.generated):
        out(f"VERIFY: generated count {len(r.generated)} != golden {len(gg)}")
        ok = False
    if ok:
        if len(gl) != len(r.steps):
            out(f"VERIFY: logits row count {len(gl)} != launches {len(r.steps)}")
            ok = False
        for i in range(min(len(gl), len(r.steps))):
            a, b = gl[i], list(r.steps[i].logits)
            if a != b:
                k = next((j for j in range(min(len(a), len(b))) if a[j] != b[j]), min(len(a), len(b)))
                out(f"VERIFY: step {i} logits differ at index {k}: {b[k] if k < len(b) else 0} vs golden "
                    f"{a[k] if k < len(a) else 0}")
                ok = False
                break
    ng = min(len(gg), len(r.generated))
    for i in range(ng):
        if not ok:
            break
        if gg[i] != r.generated[i]:
            out(f"VERIFY: generated token {i} differs")
            ok = False
    if verbose or not ok:
        out(f"VERIFY: {'MATCH' if ok else 'MISMATCH'} ({n} launches, {ng} generated tokens compared)")
    return ok


def print_perf(p, launches: int, out=print) -> None:
    """host.cpp:288-299."""
    out(f"Performance ({launches} launches)\n-------------------------")
    for name, v in zip(PERF_NAMES, p):
        out(f"  {name:<22} {v:>14}")
    if p[0]:
        pct = lambda v: 100.0 * v / p[0]  # noqa: E731
        out(f"  GEMM utilization       {pct(p[6]):6.2f} %")
        out(f"  ATTN MAC utilization   {pct(p[13]):6.2f} %")
        out(f"  CP wait stalls         {pct(p[2]):6.2f} %")
        out(f"  DMA busy               {pct(p[14]):6.2f} %")


USAGE = """usage: python -m llaccel_amd.host <model.llbin> [options]
  --backend gpu             (the MI355X instruction-set device; the only backend)
  --prompt TEXT             (default "ROMEO:")
  --prompt-ids PATH         JSON token-ID array; skips character tokenizer
  --tokens N                greedy tokens to generate (default 32)
  --tokenizer PATH          (default: <llbin dir>/tokenizer.json)
  --verify golden.json      compare tokens+logits with python -m llaccel.golden output
  --out result.json         write tokens, logits and per-launch perf counters
  --interleave SEED         random legal engine interleaving (hazard check)
  --quiet                   less output
"""


def main(argv=None) -> int:
    """The reference runtime's command line (runtime/src/main.cpp) on the GPU device: load a .llbin,
    generate, print the output and counters, --verify against a golden trace (exit 1 on MISMATCH),
    --out the record."""
    import sys
    from pathlib import Path

    from .device import GpuDevice
    argv = list(sys.argv[1:] if argv is None else argv)
    if not argv or argv[0] in ("--help", "-h"):
        print(USAGE, end="")
        return 2 if not argv else 0
    a = dict(bin=argv[0], backend="gpu", prompt="ROMEO:", tokenizer="", verify="", out="", prompt_ids="", tokens=32,
             quiet=False, explicit=False, interleave=0)
    try:
        i = 1
        while i < len(argv):
            f = argv[i]
            if f in ("--backend", "--prompt", "--prompt-ids", "--tokens", "--tokenizer", "--verify", "--out",
                     "--interleave"):
                if i + 1 >= len(argv):
                    print(f"{f} needs a value", file=sys.stderr)
                    return 2
                v = argv[i + 1]
                i += 2
                if f in ("--tokens", "--interleave"):
                    if not v.isdigit() or int(v) > 0xFFFFFFFF:
                        raise RuntimeError(f"{f} requires an unsigned 32-bit integer")
                    a[f[2:]] = int(v)
                else:
                    a[f[2:].replace("-", "_")] = v
                    if f == "--prompt":
                        a["explicit"] = True
            elif f == "--quiet":
                a["quiet"] = True
                i += 1
            elif f in ("--help", "-h"):
                print(USAGE, end="")
                return 0
            else:
                print(f"unknown option {f}\n{USAGE}", file=sys.stderr, end="")
                return 2
        if a["prompt_ids"] and (a["explicit"] or a["tokenizer"]):
            raise RuntimeError("--prompt-ids cannot be combined with --prompt or --tokenizer")
        if a["backend"] != "gpu":
            raise RuntimeError("backend must be gpu")
        lb = Llbin.load(a["bin"])
        tok = None
        if not a["prompt_ids"]:
            tok = Tokenizer.load(a["tokenizer"] or str(Path(a["bin"]).parent / "tokenizer.json"))
            ids = None
        else:
            ids = load_prompt_ids(a["prompt_ids"])
        fusion = bool(lb.meta.get("fusion", False)) or lb.meta.get("target", "") == "llaccel-v2"
        dev = GpuDevice(len(lb.dram_image) + (1 << 20), fusion, a["interleave"])
        quiet = a["quiet"]
        if not quiet:
            print("Loading program...")
            for p in lb.programs:
                print(f"  program M={p.M:<2}  instructions: {len(p.instrs)}")
            print(f"  target: {lb.meta.get('target', '?')}  fusion: {'on' if lb.meta.get('fusion') else 'off'}  "
                  f"schedule: {lb.meta.get('schedule', '?')}")
            print(f"\nExecuting on {dev.name()}...")
        host = Host(lb, dev, tok)
        r = host.generate(a["prompt"], a["tokens"]) if tok else host.generate_tokens(ids, a["tokens"])
        if tok:
            print(f"\nprompt:  {a['prompt']}\noutput:  {tok.decode(r.generated)}")
        else:
            print(f"\nprompt IDs: {json.dumps(r.prompt_tokens)}\noutput IDs: {json.dumps(r.generated)}")
        if not quiet:
            print("")
            print_perf(r.total, len(r.steps))
        rc = 0
        if a["verify"]:
            ok = verify_against_golden(r, a["verify"], True)
            print(f"PyTorch/golden reference:  {'MATCH' if ok else 'MISMATCH'}")
            rc = 0 if ok else 1
        if a["out"]:
            try:
                Path(a["out"]).write_text(json.dumps(r.to_json(), indent=1) + "\n")
            except OSError:
                raise RuntimeError(f"cannot write result {a['out']}") from None
        return rc
    except (RuntimeError, ValueError, OSError, KeyError) as e:
        print(f"error: {e}", file=sys.stderr)
        return 1


if __name__ == "__main__":
    raise SystemExit(main())
