"""Op-list fusion for GoldenModel: replaces runs of consecutive qgraph ops with one fused
launch (include/llhip.h: llhip_attn_in, llhip_mlp_in, llhip_norm_linear).

A fused step writes every activation its ops name, with the values the separate ops give
(the kernels compute the same integer formulas), so `acts`, later consumers and the launch
record are unaffected.  It keeps the per-op steps it replaces and runs those instead when
its shape limits do not hold (more than 16 rows per launch, an LDS staging overflow, a
normalised width above 1024), so every graph runs; graphs that do not match a pattern simply
keep their per-op steps.

Recognised runs (the op order the reference's quantizer and compiler emit, refquant.py:426-467):
  attn_in : rmsnorm, quant, linear q, linear k, linear v, [rmsnorm heads q, rmsnorm heads k],
            rope q, rope k, quant q, quant k, kv_write
  mlp_in  : rmsnorm, quant, linear(silu), linear(mul aux=silu out), quant          (fused graph)
            rmsnorm, quant, linear g, linear u, silu(g), mul(sg, u), quant         (unfused graph)
  norm_linear: rmsnorm, quant, linear (any epilogue)                               (e.g. lm_head)
"""
from __future__ import annotations

import ctypes

from . import _lib

LDS_LIMIT = 48 * 1024
NORM_MAX_K = 1024  # the fused RMSNorm prologue holds a row in two 8-element chunks per lane


def _vp(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


class FusedStep:
    """`kind` names the fused kernel; `fallback` are the per-op steps it replaces, `wide` the
    launches that run instead when the fused kernel does not take the rows (see wide_steps)."""

    def __init__(self, model, kind, fallback, fill, entry, desc_cls, K, bytes_fn, name, ops):
        self.model, self.kind, self.fallback, self.fill = model, kind, fallback, fill
        self.entry, self.desc = entry, desc_cls()
        self.K, self.bytes_fn, self.name, self.ops = K, bytes_fn, name, ops
        self.wide = wide_steps(model, ops, fallback)
        self.lead = None  # a _LinearNormStep for the preceding resadd linear (see _pair_linear_norm)

    def takes_wide(self, M):
        return M > 16 or M * (self.K + 16) > LDS_LIMIT or self.K > NORM_MAX_K

    def __call__(self, M, pos, pd=None):
        if self.takes_wide(M):
            if self.lead is not None:
                # the preceding linear deferred itself: it runs here with this run's leading rmsnorm + quant
                self.lead(M, pos, pd)
                rest = self.wide[1:]
            else:
                rest = self.wide
            for st in rest:
                st(M, pos, pd)
            return
        self.fill(self.desc, M, pos, pd)
        m = self.model
        # several rows: normalise them once (one launch) instead of in every workgroup's prologue
        self.desc.pre.prequant = int(M > 1)
        if M > 1:
            _lib.call("llhip_rmsnorm_quant", ctypes.byref(self.desc.pre), M, m._stream_handle())
        _lib.call(self.entry, ctypes.byref(self.desc), m._stream_handle())


class _NormQuantStep:
    """rmsnorm -> quant of its output for any number of rows: one llhip_rmsnorm_quant launch (one
    workgroup per row) writing both activations."""

    def __init__(self, model, rn, qu):
        self.model, self.rn, self.qu = model, rn, qu
        self.desc = _lib.NormQuantDesc()

    def __call__(self, M, pos, pd=None):
        _pre(self.model, self.desc, self.rn, self.qu)
        self.desc.prequant = 0
        _lib.call("llhip_rmsnorm_quant", ctypes.byref(self.desc), M, self.model._stream_handle())


class _RopeQuantStep:
    """rope -> quant of the query rows, and rope -> quant of the key rows with the layer's kv_write
    (quantised keys and the v rows into the caches), in one llhip_rope_quant2 launch."""

    def __init__(self, model, rope_q, quant_q, rope_k, quant_k, kvw):
        self.model, self.parts = model, ((rope_q, quant_q, None), (rope_k, quant_k, kvw))
        self.desc = (_lib.RopeQuantDesc(), _lib.RopeQuantDesc())

    def _fill(self, d, ro, qu, kvw, M, pos, pd):
        m = self.model
        H, D = int(ro["H"]), int(ro["D"])
        cos_t, sin_t = m._dt["rope_cos"], m._dt["rope_sin"]
        if kvw is None:
            from .golden import _pos_args

            pdev, rpos, stride = _pos_args(pd)
            kc = vc = v = None
            ldv = 0
        else:
            kc, vc, pdev, rpos, stride = m._kv_args(int(kvw["layer"]), pd)
            vbuf = m._buf(kvw["v"])
            v, ldv = _vp(vbuf), vbuf.shape[1]
        d.x, d.M, d.H, d.D, d.ldx = _vp(m._buf(ro["in"])), M, H, D, H * D
        d.cos_tab, d.sin_tab, d.table_rows, d.pos = _vp(cos_t), _vp(sin_t), int(cos_t.shape[0]), pos
        d.pos_dev, d.row_pos = pdev, rpos
        d.y, d.yq, d.qM, d.qS = _vp(m._buf(ro["out"])), _vp(m._buf(qu["out"])), int(qu["M"]), int(qu["S"])
        d.kc, d.v, d.ldv, d.vc, d.max_seq, d.slot_stride = kc, v, ldv, vc, m.max_seq, stride
        from .golden import _seq_rows

        d.seq_rows = _seq_rows(pd)

    def __call__(self, M, pos, pd=None):
        for d, (ro, qu, kvw) in zip(self.desc, self.parts):
            self._fill(d, ro, qu, kvw, M, pos, pd)
        _lib.call("llhip_rope_quant2", ctypes.byref(self.desc[0]), ctypes.byref(self.desc[1]),
                  self.model._stream_handle())


class _LinearNormStep:
    """A resadd linear (i16 out) and the rmsnorm -> quant of its output rows in one
    llhip_linear_norm call (one finishing launch for both when the linear is split along K)."""

    def __init__(self, model, lin, rn, qu):
        self.model, self.lin = model, lin
        self.norm = _NormQuantStep(model, rn, qu)

    def __call__(self, M, pos, pd=None):
        m, o = self.model, self.lin
        _pre(m, self.norm.desc, self.norm.rn, self.norm.qu)
        self.norm.desc.prequant = 0
        N, K = int(o["N"]), int(o["K"])
        out, aux = m._buf(o["out"]), m._buf(o["aux"])
        _lib.call("llhip_linear_norm", _vp(m._buf(o["in"])), M, K, K, _vp(m._dt[o["w"]]), N, _vp(m._dt[o["rq"]]),
                  _vp(m._dt[o["bias"]]) if o.get("bias") else None, _vp(aux), aux.shape[1], _vp(out), out.shape[1],
                  ctypes.byref(self.norm.desc), _vp(m._ws), m._stream_handle())


class _DeferredLinear:
    """The plan's step for a resadd linear whose output the next fused run normalises first: for the
    rows that run takes on its wide path, the run makes the linear's call itself (its `lead`,
    one llhip_linear_norm call), so this step does nothing; otherwise it is the linear's own step."""

    def __init__(self, step, fused):
        self.step, self.fused = step, fused
        self.kind, self.bytes_fn, self.name = step.kind, step.bytes_fn, step.name

    def __call__(self, M, pos, pd=None):
        if not self.fused.takes_wide(M):
            self.step(M, pos, pd)


class _GroupLinearStep:
    """Linears of one input with epilogue none (the q, k, v projections) in one
    llhip_linear_group launch."""

    def __init__(self, model, lins):
        self.model, self.lins = model, lins
        self.probs = (_lib.LinearProblem * len(lins))()

    def fill(self):
        m = self.model
        for pr, o in zip(self.probs, self.lins):
            out = m._buf(o["out"])
            pr.W, pr.N, pr.rq = _vp(m._dt[o["w"]]), int(o["N"]), _vp(m._dt[o["rq"]])
            pr.bias = _vp(m._dt[o["bias"]]) if o.get("bias") else None
            pr.out, pr.ldo, pr.out_i8 = _vp(out), out.shape[1], int(o.get("out_dtype", "i16") == "i8")

    def __call__(self, M, pos, pd=None):
        m = self.model
        self.fill()
        a = self.lins[0]
        _lib.call("llhip_linear_group", _vp(m._buf(a["in"])), M, int(a["K"]), int(a["K"]), len(self.lins), self.probs,
                  _vp(m._ws), m._stream_handle())


class _GroupRopeStep:
    """The q, k, v linears and the rope -> quant of the q and k rows with the layer's kv_write in ONE
    llhip_linear_group_rope launch (head_dim 64: a 64-column GEMM tile is one head, the rotation
    is the GEMM's epilogue); shapes or alignments it refuses run the two launches instead."""

    def __init__(self, model, group, rope):
        self.model, self.group, self.rope = model, group, rope
        self.fused = True   # cleared once the fused entry refuses this graph's operands
        self.launched = 0   # fused launches made (a test hook)

    def __call__(self, M, pos, pd=None):
        if self.fused:
            g, r, m = self.group, self.rope, self.model
            g.fill()
            for d, (ro, qu, kvw) in zip(r.desc, r.parts):
                r._fill(d, ro, qu, kvw, M, pos, pd)
            a = g.lins[0]
            try:
                _lib.call("llhip_linear_group_rope", _vp(m._buf(a["in"])), M, int(a["K"]), int(a["K"]), g.probs,
                          ctypes.byref(r.desc[0]), ctypes.byref(r.desc[1]), _vp(m._ws), m._stream_handle())
                self.launched += 1
                return
            except ValueError:
                # refused before any launch.  The two launches run instead; only when they take these
                # operands was the refusal a property of the graph (then the fused entry is not tried
                # again) -- an error of this call (positions past the table, say) propagates from them
                # and leaves the fused entry on for later calls
                self.group(M, pos, pd)
                self.rope(M, pos, pd)
                self.fused = False
                return
        self.group(M, pos, pd)
        self.rope(M, pos, pd)


class _GateUpStep:
    """The gate (silu epilogue) and up (mul epilogue on the gate's output) linears of one input
    and the quant of the product in one llhip_gate_up launch."""

    def __init__(self, model, g, u, q):
        self.model, self.g, self.u, self.q = model, g, u, q
        self.desc = _lib.GateUpDesc()
        # the gate output is read only by the up linear (its aux) and the up output only by the
        # quant: in a launch that collects no activations (model._lean) neither is written
        # (llhip_gate_up takes NULL for them on its one-launch path: K % 64 == 0 and 16-byte aligned
        # weights; weights are views into the qgraph's blob at its offsets, which need not be aligned)
        self.lean_ok = (int(g["K"]) % 64 == 0 and _reads(model, g["out"]) == 1 and _reads(model, u["out"]) == 1
                        and model.q.output_name not in (g["out"], u["out"])
                        and model._dt[g["w"]].data_ptr() % 16 == 0 and model._dt[u["w"]].data_ptr() % 16 == 0)

    def __call__(self, M, pos, pd=None):
        m, g, u, q, d = self.model, self.g, self.u, self.q, self.desc
        dt, s = m._dt, g["silu"]
        sg = m._buf(g["out"])
        d.A, d.M, d.K, d.lda = _vp(m._buf(g["in"])), M, int(g["K"]), int(g["K"])
        d.Wg, d.rqg = _vp(dt[g["w"]]), _vp(dt[g["rq"]])
        d.bg = _vp(dt[g["bias"]]) if g.get("bias") else None
        d.Wu, d.rqu = _vp(dt[u["w"]]), _vp(dt[u["rq"]])
        d.bu = _vp(dt[u["bias"]]) if u.get("bias") else None
        d.N, d.ld = int(g["N"]), sg.shape[1]
        d.silu_Mi, d.silu_Si, d.silu_sh = int(s["Mi"]), int(s["Si"]), int(s["sh_out"])
        d.mul_sh, d.fq_M, d.fq_S = int(u["aux_shift"]), int(q["M"]), int(q["S"])
        d.sg_out, d.f_out, d.fq_out = _vp(sg), _vp(m._buf(u["out"])), _vp(m._buf(q["out"]))
        if self.lean_ok and getattr(m, "_lean", False):
            d.sg_out = d.f_out = None
        _lib.call("llhip_gate_up", ctypes.byref(d), m._stream_handle())


def _reads(model, name: str) -> int:
    """How many ops of the model's op list read activation `name`."""
    return sum(1 for o in model.q.ops for k, v in o.items() if k not in ("op", "out") and isinstance(v, str) and v == name)


def _gate_up(model, ops, i):
    """ops[i:i+3] = linear g (silu) -> linear u (mul by g's output) -> quant of u's output, one input."""
    if i + 2 >= len(ops):
        return None
    g, u, q = ops[i:i + 3]
    if not (_is(g, "linear") and _is(u, "linear") and _is(q, "quant")):
        return None
    if (g.get("epilogue") != "silu" or u.get("epilogue") != "mul" or u.get("aux") != g["out"] or g["in"] != u["in"]
            or q["in"] != u["out"] or int(g["N"]) != int(u["N"]) or int(g["K"]) != int(u["K"])):
        return None
    if g.get("out_dtype", "i16") != "i16" or u.get("out_dtype", "i16") != "i16":
        return None
    return _GateUpStep(model, g, u, q)


def wide_steps(model, ops, steps):
    """Launches of a fused run for more rows than its fused kernel takes (prompt chunks): the run's
    per-op steps, with each rmsnorm + quant as one launch, three linears of one input
    (q, k, v) as one grouped launch, the gate and up linears and the quant of their product as
    one launch, and attn_in's group rope q, rope k, quant q, quant k, kv_write as one.  The
    arithmetic of every op is unchanged."""
    out, i = [], 0
    while i < len(ops):
        a = ops[i]
        if (i + 1 < len(ops) and _is(a, "rmsnorm") and int(a.get("heads", 1)) == 1 and _is(ops[i + 1], "quant")
                and ops[i + 1]["in"] == a["out"]):
            K = int(model._dt[a["gamma"]].shape[0])
            if K % 16 == 0 and K <= NORM_MAX_K:
                out.append(_NormQuantStep(model, a, ops[i + 1]))
                i += 2
                continue
        gu = _gate_up(model, ops, i)
        if gu is not None:
            out.append(gu)
            i += 3
            continue
        if i + 2 < len(ops):
            lins = ops[i:i + 3]
            if (all(_plain_linear(o) for o in lins) and len({o["in"] for o in lins}) == 1
                    and len({int(o["K"]) for o in lins}) == 1):
                out.append(_GroupLinearStep(model, lins))
                i += 3
                continue
        if i + 4 < len(ops):
            rq_, rk_, qq_, kq_, kvw = ops[i:i + 5]
            if (_is(rq_, "rope") and _is(rk_, "rope") and _is(qq_, "quant") and _is(kq_, "quant")
                    and _is(kvw, "kv_write") and qq_["in"] == rq_["out"] and kq_["in"] == rk_["out"]
                    and kvw["k"] == kq_["out"] and int(kvw["Hkv"]) == int(rk_["H"]) and int(kvw["D"]) == int(rk_["D"])
                    and model._act_spec[kvw["v"]][1] >= int(rk_["H"]) * int(rk_["D"])):
                rope = _RopeQuantStep(model, rq_, qq_, rk_, kq_, kvw)
                prev = out[-1] if out else None
                if (isinstance(prev, _GroupLinearStep) and int(rq_["D"]) == 64
                        and [o["out"] for o in prev.lins] == [rq_["in"], rk_["in"], kvw["v"]]):
                    out[-1] = _GroupRopeStep(model, prev, rope)  # q, k, v, rope, quant, kv_write: one launch
                else:
                    out.append(rope)
                i += 5
                continue
        out.append(steps[i])
        i += 1
    return out


def _pre(model, d, op_norm, op_quant):
    """Fill a NormQuantDesc for rmsnorm(op_norm) -> quant(op_quant)."""
    x = model._buf(op_norm["in"])
    d.x = _vp(x)
    d.gamma = _vp(model._dt[op_norm["gamma"]])
    d.h_out = _vp(model._buf(op_norm["out"]))
    d.hq_out = _vp(model._buf(op_quant["out"]))
    d.ldx = x.shape[1]
    d.K = int(model._dt[op_norm["gamma"]].shape[0])
    d.eps_t, d.C, d.sh_post = int(op_norm["eps_t"]), int(op_norm["C"]), int(op_norm["sh_post"])
    d.Mq, d.Sq = int(op_quant["M"]), int(op_quant["S"])


def _is(op, kind, **kw):
    if op.get("op") != kind:
        return False
    return all(op.get(k, None) == v for k, v in kw.items())


def _plain_linear(op):
    return op.get("op") == "linear" and (op.get("epilogue", "none") or "none") == "none"


def _norm_quant_head(ops, i, spec):
    """ops[i], ops[i+1] = rmsnorm (one head) -> quant of its output, with K % 8 == 0."""
    if i + 1 >= len(ops):
        return None
    a, b = ops[i], ops[i + 1]
    if not _is(a, "rmsnorm") or int(a.get("heads", 1)) != 1 or not _is(b, "quant") or b["in"] != a["out"]:
        return None
    if a["in"] not in spec or spec[a["in"]][0] != "i16" or spec[a["in"]][1] % 8:
        return None
    return a, b


def match_attn_in(model, ops, i, steps):
    spec = model._act_spec
    head = _norm_quant_head(ops, i, spec)
    if head is None:
        return None
    rn, qu = head
    j = i + 2
    lin = ops[j:j + 3]
    if len(lin) < 3 or not all(_plain_linear(o) and o["in"] == qu["out"] for o in lin):
        return None
    q_op, k_op, v_op = lin
    if q_op.get("out_dtype", "i16") != "i16" or k_op.get("out_dtype", "i16") != "i16" or v_op.get("out_dtype") != "i8":
        return None
    j += 3
    has_norm = False
    nq = nk = None
    if j + 1 < len(ops) and _is(ops[j], "rmsnorm") and _is(ops[j + 1], "rmsnorm"):
        nq, nk = ops[j], ops[j + 1]
        if nq["in"] != q_op["out"] or nk["in"] != k_op["out"]:
            return None
        has_norm = True
        j += 2
    qs = nq["out"] if has_norm else q_op["out"]
    ks = nk["out"] if has_norm else k_op["out"]
    if j + 4 >= len(ops):
        return None
    rq_, rk_, qq_, kq_, kvw = ops[j:j + 5]
    if not (_is(rq_, "rope") and _is(rk_, "rope") and _is(qq_, "quant") and _is(kq_, "quant") and _is(kvw, "kv_write")):
        return None
    if rq_["in"] != qs or rk_["in"] != ks or qq_["in"] != rq_["out"] or kq_["in"] != rk_["out"]:
        return None
    if kvw["k"] != kq_["out"] or kvw["v"] != v_op["out"]:
        return None
    H, D = int(rq_["H"]), int(rq_["D"])
    Hkv = int(rk_["H"])
    if int(rk_["D"]) != D or int(kvw["Hkv"]) != Hkv or int(kvw["D"]) != D or Hkv < 1 or H % Hkv:
        return None
    K = int(model._dt[rn["gamma"]].shape[0])
    if D % 16 or D > 256 or int(q_op["N"]) != H * D or int(k_op["N"]) != Hkv * D or int(v_op["N"]) != Hkv * D:
        return None
    if any(int(o["K"]) != K for o in lin):
        return None
    if has_norm and (int(nq.get("heads", 1)) != H or int(nk.get("heads", 1)) != Hkv
                     or int(model._dt[nq["gamma"]].shape[0]) != D or int(model._dt[nk["gamma"]].shape[0]) != D):
        return None
    if model.rope_cos.shape[0] < model.max_seq or model.rope_cos.shape[1] != D // 2:
        return None
    n_ops = j + 5 - i
    layer = int(kvw["layer"])
    dt = model._dt

    def fill(d, M, pos, pd):
        _pre(model, d.pre, rn, qu)
        for r, o in enumerate(lin):
            d.W[r] = _vp(dt[o["w"]])
            d.rq[r] = _vp(dt[o["rq"]])
            d.bias[r] = _vp(dt[o["bias"]]) if o.get("bias") else None
            d.lin_out[r] = _vp(model._buf(o["out"]))
        if has_norm:
            for r, o in enumerate((nq, nk)):
                d.nrm_gamma[r] = _vp(dt[o["gamma"]])
                d.nrm_out[r] = _vp(model._buf(o["out"]))
                d.nrm_eps[r], d.nrm_C[r], d.nrm_sh[r] = int(o["eps_t"]), int(o["C"]), int(o["sh_post"])
        d.cos_tab, d.sin_tab = _vp(dt["rope_cos"]), _vp(dt["rope_sin"])
        kcp, vcp, d.pos_dev, d.row_pos, d.slot_stride = model._kv_args(layer, pd)
        for r, (ro, qo) in enumerate(((rq_, qq_), (rk_, kq_))):
            d.rope_out[r] = _vp(model._buf(ro["out"]))
            d.quant_out[r] = _vp(model._buf(qo["out"]))
            d.quant_M[r], d.quant_S[r] = int(qo["M"]), int(qo["S"])
        d.kc, d.vc = kcp, vcp
        d.max_seq, d.M, d.H, d.Hkv, d.D, d.pos, d.has_norm = model.max_seq, M, H, Hkv, D, pos, int(has_norm)

    n_all = (H + 2 * Hkv) * D
    n_bias = sum(int(o["N"]) for o in lin if o.get("bias"))

    def nbytes(M):
        # q/k/v weights + rq + bias, the x rows in, q/k (i16, before and after RoPE), v and
        # the quantised q/k rows out, the K/V cache rows written
        return (n_all * K + 8 * n_all + 4 * n_bias + 2 * M * K + M * (H + Hkv) * D * (2 + 2 + 1) + M * Hkv * D
                + 2 * M * Hkv * D)

    return n_ops, FusedStep(model, "attn_in", steps[i:i + n_ops], fill, "llhip_attn_in", _lib.AttnInDesc, K, nbytes,
                            q_op["out"], ops[i:i + n_ops])


def match_mlp_in(model, ops, i, steps):
    spec = model._act_spec
    head = _norm_quant_head(ops, i, spec)
    if head is None:
        return None
    rn, qu = head
    K = int(model._dt[rn["gamma"]].shape[0])
    j = i + 2
    if j + 2 >= len(ops):
        return None
    a, b = ops[j], ops[j + 1]
    if not (a.get("op") == "linear" and b.get("op") == "linear" and a["in"] == qu["out"] and b["in"] == qu["out"]):
        return None
    if a.get("out_dtype", "i16") != "i16" or b.get("out_dtype", "i16") != "i16":
        return None
    N = int(a["N"])
    if int(b["N"]) != N or int(a["K"]) != K or int(b["K"]) != K:
        return None
    ea, eb = a.get("epilogue", "none") or "none", b.get("epilogue", "none") or "none"
    fused_graph = ea == "silu" and eb == "mul" and b.get("aux") == a["out"]
    unfused_graph = ea == "none" and eb == "none"
    if fused_graph:
        silu, sh_mul = a["silu"], int(b["aux_shift"])
        sg_name, f_name, g_name, u_name = a["out"], b["out"], None, None
        j += 2
    elif unfused_graph:
        if j + 3 >= len(ops):
            return None
        si, mu = ops[j + 2], ops[j + 3]
        if not (_is(si, "silu") and _is(mu, "mul") and si["in"] == a["out"]):
            return None
        if {mu["a"], mu["b"]} != {si["out"], b["out"]}:
            return None
        silu, sh_mul = {"Mi": si["Mi"], "Si": si["Si"], "sh_out": si["sh_out"]}, int(mu["sh"])
        sg_name, f_name, g_name, u_name = si["out"], mu["out"], a["out"], b["out"]
        j += 4
    else:
        return None
    if j >= len(ops) or not _is(ops[j], "quant") or ops[j]["in"] != f_name:
        return None
    fq = ops[j]
    n_ops = j + 1 - i
    dt = model._dt

    def fill(d, M, pos, pd):
        _pre(model, d.pre, rn, qu)
        d.Wg, d.Wu = _vp(dt[a["w"]]), _vp(dt[b["w"]])
        d.rqg, d.rqu = _vp(dt[a["rq"]]), _vp(dt[b["rq"]])
        d.bg = _vp(dt[a["bias"]]) if a.get("bias") else None
        d.bu = _vp(dt[b["bias"]]) if b.get("bias") else None
        d.g_out = _vp(model._buf(g_name)) if g_name else None
        d.u_out = _vp(model._buf(u_name)) if u_name else None
        d.sg_out, d.f_out, d.fq_out = _vp(model._buf(sg_name)), _vp(model._buf(f_name)), _vp(model._buf(fq["out"]))
        d.silu_Mi, d.silu_Si, d.silu_sh = int(silu["Mi"]), int(silu["Si"]), int(silu["sh_out"])
        d.mul_sh, d.fq_M, d.fq_S, d.M, d.N = sh_mul, int(fq["M"]), int(fq["S"]), M, N

    n_bias = (N if a.get("bias") else 0) + (N if b.get("bias") else 0)
    n_out = 5 + (4 if g_name else 0)  # sg, f (i16) and f.q (i8) per element, g and u for unfused graphs

    def nbytes(M):
        # gate + up weights, rq, bias, the x rows in, the outputs
        return 2 * N * K + 16 * N + 4 * n_bias + 2 * M * K + M * N * n_out

    return n_ops, FusedStep(model, "mlp_in", steps[i:i + n_ops], fill, "llhip_mlp_in", _lib.MlpInDesc, K, nbytes,
                            f_name, ops[i:i + n_ops])


_EPI = {"none": 0, "resadd": 1, "silu": 2, "mul": 3}


def match_norm_linear(model, ops, i, steps):
    spec = model._act_spec
    head = _norm_quant_head(ops, i, spec)
    if head is None or i + 2 >= len(ops):
        return None
    rn, qu = head
    lo = ops[i + 2]
    if lo.get("op") != "linear" or lo["in"] != qu["out"]:
        return None
    K = int(model._dt[rn["gamma"]].shape[0])
    if int(lo["K"]) != K:
        return None
    ep = lo.get("epilogue", "none") or "none"
    out_i8 = lo.get("out_dtype", "i16") == "i8"
    N = int(lo["N"])
    dt = model._dt
    s = lo.get("silu") or {}

    def fill(d, M, pos, pd):
        _pre(model, d.pre, rn, qu)
        d.W, d.rq = _vp(dt[lo["w"]]), _vp(dt[lo["rq"]])
        d.bias = _vp(dt[lo["bias"]]) if lo.get("bias") else None
        d.aux = _vp(model._buf(lo["aux"])) if ep in ("resadd", "mul") else None
        d.out = _vp(model._buf(lo["out"]))
        d.epilogue, d.aux_shift = _EPI[ep], int(lo.get("aux_shift", 0) or 0)
        d.silu_Mi, d.silu_Si, d.silu_sh = int(s.get("Mi", 0)), int(s.get("Si", 0)), int(s.get("sh_out", 0))
        d.out_i8, d.M, d.N = int(out_i8), M, N

    has_aux = ep in ("resadd", "mul")

    def nbytes(M):
        # weights, rq, bias, the x rows in (i16), outputs (+ aux rows)
        return (N * K + 8 * N + (4 * N if lo.get("bias") else 0) + 2 * M * K + M * N * (1 if out_i8 else 2)
                + (2 * M * N if has_aux else 0))

    return 3, FusedStep(model, "norm_linear", steps[i:i + 3], fill, "llhip_norm_linear", _lib.NormLinearDesc, K,
                        nbytes, lo["out"], ops[i:i + 3])


MATCHERS = (match_attn_in, match_mlp_in, match_norm_linear)


def fuse(model, ops, steps):
    """New plan: matched runs of `ops` (steps[i] is op i's per-op step) become FusedSteps."""
    out, src = [], []  # src[j]: the op index of a per-op step, None for a fused run
    i = 0
    while i < len(ops):
        if i >= len(steps):
            break
        got = None
        for m in MATCHERS:
            got = m(model, ops, i, steps)
            if got is not None:
                n = got[0]
                # never swallow a deferred graph error: the reference raises it at that op
                if i + n > len(steps) or any(getattr(s, "kind", "") == "error" for s in steps[i:i + n]):
                    got = None
                break
        if got is None:
            out.append(steps[i])
            src.append(i)
            i += 1
        else:
            n, st = got
            out.append(st)
            src.append(None)
            i += n
    _pair_linear_norm(model, ops, out, src)
    out.extend(steps[len(ops):])
    return out


def _pair_linear_norm(model, ops, out, src):
    """A resadd linear (i16 out) followed by a fused run that starts with rmsnorm -> quant of the
    linear's output (o_proj before the MLP run, down before the next layer's attention run or the
    head): on the run's wide path the two become one llhip_linear_norm call, which finishes a
    split-K linear and normalises its rows in one launch."""
    for j in range(len(out) - 1):
        f = out[j + 1]
        if src[j] is None or getattr(out[j], "kind", "") != "linear" or not isinstance(f, FusedStep):
            continue
        if not f.wide or not isinstance(f.wide[0], _NormQuantStep):
            continue
        a, nq = ops[src[j]], f.wide[0]
        if not (_is(a, "linear") and (a.get("epilogue") or "none") == "resadd" and a.get("out_dtype", "i16") == "i16"
                and nq.rn is f.ops[0] and nq.rn["in"] == a["out"] and int(a["K"]) % 16 == 0):
            continue
        K = int(model._dt[nq.rn["gamma"]].shape[0])
        if K != int(a["N"]) or K % 16 or K > NORM_MAX_K:
            continue
        f.lead = _LinearNormStep(model, a, nq.rn, nq.qu)
        out[j] = _DeferredLinear(out[j], f)
