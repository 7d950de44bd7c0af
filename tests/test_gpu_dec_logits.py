"""llhip_dec_logits (one decode row's finish, final rmsnorm + quant, lm_head and greedy step as ONE
launch of one workgroup per CU), with the lm_head row-major and in tile order (llhip_dec_logits_panel),
against llhip_dec_finish + llhip_dec_head + llhip_dec_greedy and the C oracle, bit-exact, over
consecutive launches that share one key buffer (its arrival counter must return to zero after each
launch), with the record ring filling up and one launch whose row is read from memory (no partial
sums)."""
from __future__ import annotations

import ctypes
import math

import numpy as np
import pytest

from llaccel_amd import _lib
from oracle import golden_np as O
from tests.gpu_helpers import down, ptr, stream, torch, up

pytestmark = pytest.mark.gpu

R = 4  # accumulator rows of the finished projection


def _state(t, K, N, vocab, cap):
    z = lambda n, dt: t.zeros(n, dtype=dt, device="cuda")  # noqa: E731
    return {"tok": z(1, t.int32), "pos": t.full((1,), 100, dtype=t.int32, device="cuda"), "step": z(1, t.int32),
            "ring": t.full((max(cap, 1), vocab), 7, dtype=t.int16, device="cuda"),
            "ring_tok": t.full((max(cap, 1),), -1, dtype=t.int32, device="cuda"),
            "row": z(K, t.int16), "x": z(K, t.int16), "h": z(K, t.int16), "hq": z(K, t.int8),
            "out": t.full((N,), 3, dtype=t.int16, device="cuda")}


def _descs(op, st, xin, accd, auxd):
    d = _lib.NormLinearDesc()
    p = d.pre
    p.x, p.gamma, p.h_out, p.hq_out, p.ldx, p.K = ptr(xin), ptr(op["g"]), ptr(st["h"]), ptr(st["hq"]), op["K"], op["K"]
    p.eps_t, p.C, p.sh_post, p.Mq, p.Sq, p.prequant = op["eps_t"], op["C"], op["sh"], op["qM"], op["qS"], 0
    d.W, d.rq, d.bias, d.aux, d.out = ptr(op["W"]), ptr(op["rq"]), ptr(op["bias"]), None, ptr(st["out"])
    d.epilogue, d.out_i8, d.M, d.N = 0, 0, 1, op["N"]
    r = _lib.ResidDesc()
    r.acc, r.R, r.rq, r.bias, r.aux, r.x_out = ptr(accd), R, ptr(op["rq_p"]), ptr(op["b_p"]), ptr(auxd), ptr(st["x"])
    return d, r


@pytest.mark.parametrize("K,N,vocab,bias", [(896, 151936, 151936, False), (576, 4112, 4100, True),
                                            (1024, 1008, 1000, True), (64, 16, 9, False)])
def test_dec_logits_equals_three_launches_and_oracle(K, N, vocab, bias):
    t = torch()
    rng = np.random.default_rng(K + N)
    W = rng.integers(-128, 128, (N, K))
    rq = np.stack([rng.integers(1 << 30, 1 << 31, N), rng.integers(36, 41, N)], 1)
    b = rng.integers(-(1 << 18), 1 << 18, N) if bias else None
    rq_p = np.stack([rng.integers(1 << 30, 1 << 31, K), rng.integers(34, 38, K)], 1)
    b_p = rng.integers(-(1 << 20), 1 << 20, K)
    g = rng.integers(-32768, 32768, K)
    embed = rng.integers(-32768, 32768, (vocab, K))
    op = {"K": K, "N": N, "eps_t": 12345, "C": int(2**24 * math.sqrt(K)), "sh": 27, "qM": 1234567891, "qS": 38,
          "W": up(W, np.int8), "rq": up(rq, np.int32), "bias": None if b is None else up(b, np.int32),
          "rq_p": up(rq_p, np.int32), "b_p": up(b_p, np.int32), "g": up(g, np.int16)}
    embd = up(embed, np.int16)
    cap = 2
    new, rows, old = (_state(t, K, N, vocab, cap) for _ in range(3))
    nk = int(_lib.lib().llhip_dec_logits_keys())
    keys_new, keys_rows = (t.zeros(nk, dtype=t.int64, device="cuda") for _ in range(2))
    keys_old = t.zeros(int(_lib.lib().llhip_dec_head_keys(N)), dtype=t.int64, device="cuda")
    s = stream()
    panel = t.full((-(-N // 16) * 16 * K,), 99, dtype=t.int8, device="cuda")
    _lib.call("llhip_dec_logits_panel", ptr(op["W"]), N, K, ptr(panel), s)
    Wp = np.zeros((-(-N // 16) * 16, K), np.int64)
    Wp[:N] = W
    want = Wp.reshape(-1, 16, K // 64, 4, 16).transpose(0, 2, 3, 1, 4).reshape(-1)  # [t][s][kg][col][16]
    assert np.array_equal(down(panel), want)
    for i in range(4):
        print(f"dec_logits K={K} N={N} vocab={vocab} launch {i}", flush=True)
        acc = rng.integers(-(1 << 27), 1 << 27, (R, K))
        aux = rng.integers(-20000, 20000, K)
        from_memory = i == 2  # the row itself, no partial sums to finish
        accd, auxd = up(acc, np.int32), up(aux, np.int16)
        xin = up(aux, np.int16)
        for st, keys in ((new, keys_new), (rows, keys_rows), (old, keys_old)):
            d, r = _descs(op, st, xin, None if from_memory else accd, auxd)
            rr = None if from_memory else ctypes.byref(r)
            if st is not old:
                _lib.call("llhip_dec_logits", ctypes.byref(d), ptr(panel) if st is new else None, rr, vocab, ptr(keys),
                          ptr(st["tok"]), ptr(st["pos"]), ptr(st["step"]), ptr(st["ring"]), vocab, ptr(st["ring_tok"]),
                          cap, ptr(embd), K, ptr(st["row"]), s)
            else:
                _lib.call("llhip_dec_finish", ctypes.byref(d.pre), rr, s)
                d.pre.prequant = 1
                _lib.call("llhip_dec_head", ctypes.byref(d), vocab, ptr(keys), ptr(st["step"]), ptr(st["ring"]),
                          vocab, cap, s)
                _lib.call("llhip_dec_greedy", ptr(keys), keys.numel(), ptr(st["tok"]), ptr(st["pos"]), ptr(st["step"]),
                          ptr(st["ring_tok"]), cap, ptr(embd), K, ptr(st["row"]), s)
        for name in new:
            if from_memory and name == "x":
                continue  # no finished row to write
            assert np.array_equal(down(new[name]), down(old[name])), (i, name)
            assert np.array_equal(down(rows[name]), down(old[name])), (i, name)
        assert int(keys_new[-1].item()) == 0 and int(keys_rows[-1].item()) == 0  # the arrival counters are back at zero
        # the oracle: finish, rmsnorm, quant, lm_head, first argmax below vocab, embedding row
        x = aux if from_memory else O.vadd(O.requant16(acc.sum(0) + b_p, rq_p[:, 0], rq_p[:, 1]), aux, 0)
        if not from_memory:
            assert np.array_equal(down(new["x"]), x)
        h = O.rmsnorm_row(x, g, op["eps_t"], op["C"], op["sh"])
        hq = O.vquant(h, op["qM"], op["qS"])
        assert np.array_equal(down(new["h"]), h) and np.array_equal(down(new["hq"]), hq)
        logits = O.linear_c(hq[None, :], W, rq, b, False, "none", None, 0, None)[0]
        assert np.array_equal(down(new["out"]), logits)
        tok = int(np.argmax(logits[:vocab]))
        assert int(new["tok"].item()) == tok and int(new["pos"].item()) == 101 + i and int(new["step"].item()) == i + 1
        assert np.array_equal(down(new["row"]), embed[tok])
        if i < cap:
            assert np.array_equal(down(new["ring"][i]), logits[:vocab]) and int(new["ring_tok"][i].item()) == tok
    assert np.array_equal(down(new["ring_tok"]), down(old["ring_tok"]))


def test_dec_logits_refuses_what_it_does_not_cover():
    t = torch()
    K, N = 896, 1024
    op = {"K": K, "N": N, "eps_t": 1, "C": 1 << 24, "sh": 24, "qM": 1 << 30, "qS": 38,
          "W": t.zeros((N, K), dtype=t.int8, device="cuda"), "rq": t.zeros((N, 2), dtype=t.int32, device="cuda"),
          "bias": None, "rq_p": t.zeros((K, 2), dtype=t.int32, device="cuda"), "b_p": None,
          "g": t.zeros(K, dtype=t.int16, device="cuda")}
    st = _state(t, K, N, N, 1)
    keys = t.zeros(int(_lib.lib().llhip_dec_logits_keys()), dtype=t.int64, device="cuda")
    embd = t.zeros((N, K), dtype=t.int16, device="cuda")

    def call(d, vocab=N):
        _lib.call("llhip_dec_logits", ctypes.byref(d), None, None, vocab, ptr(keys), ptr(st["tok"]), ptr(st["pos"]),
                  ptr(st["step"]), ptr(st["ring"]), N, ptr(st["ring_tok"]), 1, ptr(embd), K, ptr(st["row"]), stream())

    d, _ = _descs(op, st, st["x"], None, None)
    d.pre.prequant = 1
    with pytest.raises(ValueError):
        call(d)  # the row must be normalised here, not read quantised
    d, _ = _descs(op, st, st["x"], None, None)
    d.M = 2
    with pytest.raises(ValueError):
        call(d)
    d, _ = _descs(op, st, st["x"], None, None)
    with pytest.raises(ValueError):
        call(d, vocab=N + 1)
    d.pre.K = d.pre.ldx = 880  # not a multiple of 64
    with pytest.raises(ValueError):
        call(d)
    with pytest.raises(ValueError):
        _lib.call("llhip_dec_logits_panel", ptr(op["W"]), N, 880, ptr(t.empty(N * 880, dtype=t.int8, device="cuda")),
                  stream())
    d, _ = _descs(op, st, st["x"], None, None)
    call(d)
    t.cuda.synchronize()
    assert int(keys[-1].item()) == 0
