"""Host-side model execution over an instruction-set device: the reference runtime's host contract
(runtime/include/llaccel/host.h, runtime/src/host.cpp) -- character tokenizer, embedding rows into
the input buffer, chunked prefill with the largest compiled M, greedy decode with the M = 1 program,
the golden.json-shaped record with per-launch performance counters, and the check of a run against
a golden trace (the VERIFY lines).  `dev` is any object with the `llaccel::Device` methods
(`llaccel_amd.device.GpuDevice` on MI355X).

The record layout, the checks' order and messages, the counters' names and the command-line
options are the reference's interface; the code here is organised around a launch schedule
(`Host.schedule`: prefill chunks, then decode launches that each take the previous argmax), one
staged input block per launch, and a table of golden-trace checks.
"""
from __future__ import annotations

import argparse
import json
import sys
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

from .device import ATTN_TMAX, NUM_PERF, PERF_NAMES, Llbin

_OP_ATTN, _OP_KV_WRITE, _OP_ROPE = 0x40, 0x41, 0x31
U32_MAX = 0xFFFFFFFF


@dataclass
class Tokenizer:
    """Character-level tokenizer (host.cpp:15-41): each code point is its index in `itos`."""
    itos: list

    def __post_init__(self) -> None:
        self._ids = {}
        for i, s in enumerate(self.itos):
            self._ids.setdefault(s, i)  # the first entry of a repeated string wins

    @staticmethod
    def load(path) -> "Tokenizer":
        try:
            table = json.loads(Path(path).read_text(encoding="utf-8"))
        except OSError:
            raise RuntimeError(f"cannot open tokenizer {path}") from None
        return Tokenizer([str(s) for s in table["itos"]])

    def encode(self, text: str) -> list[int]:
        unknown = next((ch for ch in text if ch not in self._ids), None)
        if unknown is not None:
            raise RuntimeError(f"character not in vocabulary: '{unknown}'")
        return [self._ids[ch] for ch in text]

    def decode(self, ids) -> str:
        n = len(self.itos)
        return "".join(self.itos[i] if i < n else "?" for i in ids)


@dataclass
class StepResult:
    """One launch of the record (host.h:22-28)."""
    pos: int
    M: int
    argmax: int
    logits: list
    perf: list


@dataclass
class GenerationResult:
    """A generation's record (host.h:30-35) and its JSON form (host.cpp:207-229)."""
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


def _first_argmax(row: np.ndarray) -> int:
    """Index of the first maximum (numpy's argmax keeps the first)."""
    return int(np.argmax(row))


@dataclass(frozen=True)
class _Region:
    base: int
    stride: int


class Host:
    """A loaded model on a device (host.cpp:44-205): checks the image, then runs generations."""

    def __init__(self, bin: Llbin, dev, tok: Tokenizer | None = None):
        self.bin, self.dev = bin, dev
        model, dram = bin.meta["model"], bin.meta["dram"]
        need = self._head_dim_needed(bin, model)
        if need > dev.max_attention_head_dim():
            raise RuntimeError(f"model requires attention head dimension {need}; backend {dev.name()} supports at "
                               f"most {dev.max_attention_head_dim()}. Rebuild or select a backend implementing the "
                               f"required head width.")
        self.vocab, self.dim, self.max_seq = (int(model[k]) for k in ("vocab", "dim", "max_seq"))
        self.emb, self.inp, self.out = (_Region(int(dram[k]["addr"]), int(dram[k]["row_bytes"]))
                                        for k in ("embedding", "input", "logits"))
        if not bin.programs:
            raise RuntimeError("no programs in llbin")
        if 0 in (self.vocab, self.dim, self.max_seq):
            raise RuntimeError("invalid zero model dimension")
        self.prefill_m = max(p.M for p in bin.programs)
        if self.out.stride < 2 * self.vocab:
            raise RuntimeError("logits row too small for vocab")
        if min(self.emb.stride, self.inp.stride) < 2 * self.dim:
            raise RuntimeError("embedding/input row too small for dim")
        if self.max_seq > ATTN_TMAX or self.max_seq % self.prefill_m:
            raise RuntimeError("invalid context/prefill dimensions")
        size = len(bin.dram_image)
        regions = [(self.emb.base, self.emb.stride, self.vocab), (self.inp.base, self.inp.stride, self.prefill_m),
                   (self.out.base, self.out.stride, self.prefill_m)]
        regions += [(int(c["addr"]), int(c["bytes"]), 1) for c in dram.get("kv_cache", [])]
        for base, stride, rows in regions:
            if base > size or stride == 0 or rows > (size - base) // stride:
                raise RuntimeError("model buffer metadata exceeds DRAM image")
        self.kv_regions = [(int(c["addr"]), int(c["bytes"])) for c in dram.get("kv_cache", [])]
        dev.dram_write(0, bin.dram_image)
        if tok is not None and len(tok.itos) != self.vocab:
            raise RuntimeError("tokenizer size != model vocab")
        self.tok = tok

    @staticmethod
    def _head_dim_needed(bin: Llbin, model: dict) -> int:
        """The widest attention head the image uses: the model's head_dim and every ATTN / ROPE /
        KV_WRITE instruction's D (host.cpp:58-64)."""
        need = 0
        if "head_dim" in model:
            v = model["head_dim"]
            if not isinstance(v, int) or isinstance(v, bool) or v <= 0:
                raise RuntimeError("invalid model head_dim")
            need = v
        field_of = {_OP_ATTN: 9, _OP_KV_WRITE: 6, _OP_ROPE: 6}
        widths = (w[field_of[w[0] & 0xFF]] for p in bin.programs for w in p.instrs if (w[0] & 0xFF) in field_of)
        return max(need, max(widths, default=0))

    # ---- one launch --------------------------------------------------------------------------
    def _stage_input(self, tokens, M: int) -> None:
        """The M input rows as one block: embedding rows of `tokens`, zero rows after them."""
        if any(t >= self.vocab for t in tokens):
            raise RuntimeError("token ID exceeds model vocabulary")
        block = bytearray(M * self.inp.stride)
        for r, t in enumerate(tokens):
            block[r * self.inp.stride:r * self.inp.stride + 2 * self.dim] = \
                self.dev.dram_read(self.emb.base + t * self.emb.stride, 2 * self.dim)
        self.dev.dram_write(self.inp.base, bytes(block))

    def launch(self, row_tokens, M: int, pos: int, logits_row: int) -> StepResult:
        if M > self.max_seq or pos > self.max_seq - M:
            raise RuntimeError("sequence exceeds max_seq")
        self._stage_input(list(row_tokens)[:M], M)
        perf = self.dev.run(self.bin.program_for_m(M).pc, pos)
        row = np.frombuffer(self.dev.dram_read(self.out.base + logits_row * self.out.stride, 2 * self.vocab), "<i2")
        return StepResult(pos, M, _first_argmax(row), row.astype(int).tolist(), perf)

    # ---- a generation ------------------------------------------------------------------------
    def schedule(self, prompt: list, n_tokens: int):
        """The launches of a generation as (tokens, M, pos, logits_row) tuples: prefill chunks of
        prefill_m rows (the last chunk's logits row is the prompt's last token), then one M = 1
        launch per generated token until max_seq.  A decode launch's token is sent in by the caller
        (generator .send), so the schedule stays independent of the device."""
        P, L = self.prefill_m, len(prompt)
        chunks = [prompt[c:c + P] for c in range(0, L, P)]
        for c, rows in enumerate(chunks):
            yield rows, P, c * P, len(rows) - 1 if c == len(chunks) - 1 else P - 1
        for pos in range(L, min(L + n_tokens, self.max_seq - 1)):
            token = yield None  # the caller sends the previous launch's argmax
            yield [token], 1, pos, 0

    def generate(self, prompt: str, n_tokens: int) -> GenerationResult:
        if self.tok is None:
            raise RuntimeError("text generation requires a character tokenizer; use generateTokens")
        return self.generate_tokens(self.tok.encode(prompt), n_tokens)

    def generate_tokens(self, prompt, n_tokens: int) -> GenerationResult:
        prompt = list(prompt)
        if not prompt:
            raise RuntimeError("empty prompt")
        L = len(prompt)
        if L > self.max_seq or n_tokens > self.max_seq - L:
            raise RuntimeError("prompt + tokens exceeds max_seq")
        if max(prompt) >= self.vocab:
            raise RuntimeError("prompt token ID exceeds model vocabulary")
        for addr, nbytes in self.kv_regions:  # a new session: KV cleared, weights and programs kept
            self.dev.dram_write(addr, bytes(nbytes))
        steps, last = [], 0
        plan = self.schedule(prompt, n_tokens)
        for item in plan:
            if item is None:  # a decode launch waits for the previous argmax
                item = plan.send(last)
            steps.append(self.launch(*item))
            last = steps[-1].argmax
        # every generated token was the argmax of the launch before it; a run that stops at
        # max_seq records the token without launching it
        n_pre = -(-L // self.prefill_m)
        generated = [s.argmax for s in steps[n_pre - 1:]][:n_tokens]
        total = [sum(col) for col in zip(*(s.perf for s in steps))]
        return GenerationResult(prompt_tokens=prompt, generated=generated, steps=steps, total=total)


# ---- golden-trace check (host.cpp:243-287) ----------------------------------------------------
def _int_array(v, name, lo, hi):
    if not isinstance(v, list) or any(not isinstance(x, int) or isinstance(x, bool) or not lo <= x <= hi for x in v):
        raise RuntimeError(f"golden {name} must be an array of integers in range")
    return list(v)


def load_prompt_ids(path) -> list[int]:
    """Externally tokenized prompt IDs (host.h:65): a JSON array of u32."""
    with open(path) as f:
        return _int_array(json.load(f), "prompt IDs", 0, U32_MAX)


@dataclass
class _Golden:
    prompt: list
    generated: list
    argmax: list
    rows: list

    @staticmethod
    def load(path) -> "_Golden":
        try:
            g = json.loads(Path(path).read_text())
        except OSError:
            raise RuntimeError(f"cannot open golden {path}") from None
        ints = {k: _int_array(g[k], k, 0, U32_MAX) for k in ("prompt_tokens", "generated", "argmax_per_step")}
        if "logits_last_rows" not in g:
            raise RuntimeError("golden trace has no logits")
        if not isinstance(g["logits_last_rows"], list):
            raise RuntimeError("golden logits_last_rows must be an array")
        rows = [_int_array(r, "logits_last_rows", -32768, 32767) for r in g["logits_last_rows"]]
        return _Golden(ints["prompt_tokens"], ints["generated"], ints["argmax_per_step"], rows)


def _first_diff(a: list, b: list) -> int | None:
    """First index where two lists differ (the shorter length if one is a prefix), or None."""
    k = next((i for i, (x, y) in enumerate(zip(a, b)) if x != y), min(len(a), len(b)))
    return None if k == len(a) == len(b) else k


# Each check returns the VERIFY line of its first finding, or None.  The counts and prompt are
# always checked; the logits rows only when those agree; the generated tokens only when
# everything before them agrees.
def _check_prompt(r, g):
    return "VERIFY: prompt tokens differ from golden" if g.prompt != r.prompt_tokens else None


def _check_argmax(r, g):
    i = _first_diff(g.argmax[:len(r.steps)], [s.argmax for s in r.steps][:len(g.argmax)])
    if i is None or i >= min(len(g.argmax), len(r.steps)):
        return None
    s = r.steps[i]
    return f"VERIFY: step {i} argmax {s.argmax} != golden {g.argmax[i]} (pos={s.pos} M={s.M})"


def _check_launches(r, g):
    return f"VERIFY: launch count {len(r.steps)} != golden {len(g.argmax)}" if len(g.argmax) != len(r.steps) else None


def _check_generated_count(r, g):
    n, ng = len(r.generated), len(g.generated)
    return f"VERIFY: generated count {n} != golden {ng}" if n != ng else None


def _check_row_count(r, g):
    return f"VERIFY: logits row count {len(g.rows)} != launches {len(r.steps)}" if len(g.rows) != len(r.steps) else None


def _check_rows(r, g):
    for i, (want, step) in enumerate(zip(g.rows, r.steps)):
        got = list(step.logits)
        k = _first_diff(want, got)
        if k is not None:
            return (f"VERIFY: step {i} logits differ at index {k}: {got[k] if k < len(got) else 0} vs golden "
                    f"{want[k] if k < len(want) else 0}")
    return None


def _check_tokens(r, g):
    i = _first_diff(g.generated[:len(r.generated)], r.generated[:len(g.generated)])
    return f"VERIFY: generated token {i} differs" if i is not None else None


CHECKS = ((_check_prompt, _check_argmax, _check_launches, _check_generated_count),  # always
          (_check_row_count, _check_rows),                                          # when the above agree
          (_check_tokens,))                                                         # when all above agree


def verify_against_golden(r: GenerationResult, golden_path, verbose: bool = False, out=print) -> bool:
    """Compares a run with a golden trace: prompt tokens, per-launch argmax and launch count,
    generated count, then every launch's logits row, then the generated tokens; prints the VERIFY
    line of each finding (host.cpp:243-287)."""
    g = _Golden.load(golden_path)
    ok = True
    for group in CHECKS:
        if not ok:
            break
        for check in group:
            line = check(r, g)
            if line is not None:
                out(line)
                ok = False
    if verbose or not ok:
        n, ng = min(len(g.argmax), len(r.steps)), min(len(g.generated), len(r.generated))
        out(f"VERIFY: {'MATCH' if ok else 'MISMATCH'} ({n} launches, {ng} generated tokens compared)")
    return ok


# counter indices of the utilisation lines of the performance report (host.cpp:288-299)
_UTILISATION = (("GEMM utilization", 6), ("ATTN MAC utilization", 13), ("CP wait stalls", 2), ("DMA busy", 14))


def print_perf(p, launches: int, out=print) -> None:
    """The performance report: every counter, then utilisations as shares of the cycle count."""
    lines = [f"Performance ({launches} launches)", "-" * 25]
    lines += [f"  {name:<22} {v:>14}" for name, v in zip(PERF_NAMES, p)]
    if p[0]:
        lines += [f"  {label:<22} {100.0 * p[i] / p[0]:6.2f} %" for label, i in _UTILISATION]
    out(lines[0] + "\n" + lines[1])
    for line in lines[2:]:
        out(line)


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


class _UsageError(Exception):
    pass


class _Parser(argparse.ArgumentParser):
    def error(self, message):
        raise _UsageError(message)


def _parser() -> _Parser:
    ap = _Parser(add_help=False, allow_abbrev=False)
    ap.add_argument("bin")
    ap.add_argument("--backend", default="gpu")
    ap.add_argument("--prompt", default=None)
    ap.add_argument("--prompt-ids", default="")
    ap.add_argument("--tokens", default="32")
    ap.add_argument("--tokenizer", default="")
    ap.add_argument("--verify", default="")
    ap.add_argument("--out", default="")
    ap.add_argument("--interleave", default="0")
    ap.add_argument("--quiet", action="store_true")
    return ap


def _u32(flag: str, text: str) -> int:
    if not text.isdigit() or int(text) > U32_MAX:
        raise RuntimeError(f"{flag} requires an unsigned 32-bit integer")
    return int(text)


def main(argv=None) -> int:
    """The reference runtime's command line (runtime/src/main.cpp) on the GPU device: load a .llbin,
    generate, print the output and counters, --verify against a golden trace (exit 1 on MISMATCH),
    --out the record.  Usage errors exit 2."""
    from .device import GpuDevice

    argv = list(sys.argv[1:] if argv is None else argv)
    if not argv or argv[0] in ("--help", "-h") or "--help" in argv or "-h" in argv:
        print(USAGE, end="")
        return 0 if argv else 2
    try:
        a = _parser().parse_args(argv)
    except _UsageError as e:
        print(f"{e}\n{USAGE}", file=sys.stderr, end="")
        return 2
    try:
        tokens, seed = _u32("--tokens", a.tokens), _u32("--interleave", a.interleave)
        if a.prompt_ids and (a.prompt is not None or a.tokenizer):
            raise RuntimeError("--prompt-ids cannot be combined with --prompt or --tokenizer")
        if a.backend != "gpu":
            raise RuntimeError("backend must be gpu")
        lb = Llbin.load(a.bin)
        tok = None if a.prompt_ids else Tokenizer.load(a.tokenizer or Path(a.bin).parent / "tokenizer.json")
        prompt = a.prompt if a.prompt is not None else "ROMEO:"
        fusion = bool(lb.meta.get("fusion", False)) or lb.meta.get("target", "") == "llaccel-v2"
        dev = GpuDevice(len(lb.dram_image) + (1 << 20), fusion, seed)
        say = (lambda *s: None) if a.quiet else print
        say("Loading program...")
        for p in lb.programs:
            say(f"  program M={p.M:<2}  instructions: {len(p.instrs)}")
        say(f"  target: {lb.meta.get('target', '?')}  fusion: {'on' if lb.meta.get('fusion') else 'off'}  "
            f"schedule: {lb.meta.get('schedule', '?')}")
        say(f"\nExecuting on {dev.name()}...")
        host = Host(lb, dev, tok)
        r = host.generate(prompt, tokens) if tok else host.generate_tokens(load_prompt_ids(a.prompt_ids), tokens)
        if tok:
            print(f"\nprompt:  {prompt}\noutput:  {tok.decode(r.generated)}")
        else:
            print(f"\nprompt IDs: {json.dumps(r.prompt_tokens)}\noutput IDs: {json.dumps(r.generated)}")
        if not a.quiet:
            print("")
            print_perf(r.total, len(r.steps))
        ok = True
        if a.verify:
            ok = verify_against_golden(r, a.verify, True)
            print(f"PyTorch/golden reference:  {'MATCH' if ok else 'MISMATCH'}")
        if a.out:
            try:
                Path(a.out).write_text(json.dumps(r.to_json(), indent=1) + "\n")
            except OSError:
                raise RuntimeError(f"cannot write result {a.out}") from None
        return 0 if ok else 1
    except (RuntimeError, ValueError, OSError, KeyError) as e:
        print(f"error: {e}", file=sys.stderr)
        return 1


if __name__ == "__main__":
    raise SystemExit(main())
