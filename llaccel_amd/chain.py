"""Decode chain: a one-row launch of a fused qgraph as three kernel launches per layer.

The fused plan (llaccel_amd.fusion) runs a layer of the reference's fused graph (the op order of
refquant.py:426-467 with --fusion) as five launches: attn_in, attention, linear wo (resadd),
mlp_in, linear wd (resadd).  For one row (a decode launch, golden.py:392-397) the two resadd
projections move into their producers: each attention head adds its exact int32 partial sums of
wo (the head's K range) into an accumulator row, each mlp_in workgroup adds the partial sums of wd
over its 16 FFN columns into one of R accumulator rows, and the next launch finishes the
projection -- bias, requant16 and the residual add of golden.py:316-342 -- in its prologue
(include/llhip.h, llhip_dec_*).  Integer sums do not depend on their order, so every activation
is the one the separate launches write.

    layer l:  llhip_dec_attn_in  [finish wd(l-1)] rmsnorm quant q k v [q/k norm] rope quant kv_write
              llhip_dec_attention attention + wo partial sums          (clears the wd accumulators)
              llhip_dec_mlp      finish wo, rmsnorm quant gate/up quant + wd partial sums
    final:    llhip_dec_finish   finish wd(L-1), rmsnorm, quant (one workgroup)
              llhip_dec_head     lm_head [greedy keys + record row]
              llhip_dec_greedy   (decode loop) argmax, record, position, next input row

The chain exists only for graphs whose every layer has that shape; other graphs keep the fused
plan.  The kernels read the output projections in panel layouts made once on the device:
wo as [H][dim][D] (a head's K range contiguous) and wd as [FFN/16][dim][16].

Decode step: for a launch at a device position (the decode loop) whose layers have no Q/K norm and
head_dim 64, all layers run as one persistent launch instead (llhip_dec_step: the same three stages
per layer, handed between workgroups inside the launch), followed by the one-launch greedy head
(llhip_dec_logits) where it applies, else the same finish, head and greedy launches.  It writes the KV caches and the last layer's residual row and partial sums,
not the other activations, so launches that collect activations keep the three launches per layer.
"""
from __future__ import annotations

import ctypes

from . import _lib
from . import fusion

WD_ROWS = 8  # accumulator rows of the down projection (workgroup b adds into row b % 8)


def _vp(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _resadd_linear(op, src, aux, N, K):
    """op is `linear src -> out` with the resadd epilogue on `aux`, i16 output, N x K weights."""
    return (op.get("op") == "linear" and op["in"] == src and (op.get("epilogue") or "none") == "resadd"
            and op.get("aux") == aux and op.get("out_dtype", "i16") == "i16" and int(op["N"]) == N
            and int(op["K"]) == K)


class _Layer:
    def __init__(self, attn_in, att_op, wo, mlp, wd, resid_in):
        self.attn_in, self.att, self.wo, self.mlp, self.wd = attn_in, att_op, wo, mlp, wd
        self.resid_in = resid_in


class Chain:
    """The decode-chain steps of a model (build with `build`); `run(pos, pd)` launches one row,
    `run(pos, pd, greedy=...)` the decode loop's launch with the greedy step."""

    def __init__(self, model, layers, head, head_ops):
        torch = _torch()
        self.model, self.layers, self.head, self.head_ops = model, layers, head, head_ops
        dev = model.device
        self.dim = model.dim
        self.acc_wo = torch.zeros(self.dim, dtype=torch.int32, device=dev)
        self.acc_wd = torch.zeros((WD_ROWS, self.dim), dtype=torch.int32, device=dev)
        vp = int(head.desc_N)
        self.keys = torch.zeros(int(_lib.lib().llhip_dec_head_keys(vp)), dtype=torch.int64, device=dev)
        # the one-launch head's keys and arrival counter (zero-filled once; each launch leaves the
        # counter at zero)
        self.logit_keys = torch.zeros(int(_lib.lib().llhip_dec_logits_keys()), dtype=torch.int64, device=dev)
        self.use_logits = True  # the greedy head as one launch (llhip_dec_logits) where it applies
        self._panel = None  # the lm_head in llhip_dec_logits' tile order, made on first use
        self.wo_panel, self.wd_panel = [], []
        for ly in layers:
            H, D = int(ly.att["H"]), int(ly.att["D"])
            w = model._dt[ly.wo["w"]]  # [dim][H*D]
            self.wo_panel.append(w.view(self.dim, H, D).permute(1, 0, 2).contiguous())
            wd = model._dt[ly.wd["w"]]  # [dim][F]
            F = wd.shape[1]
            Fp = -(-F // 16) * 16
            pad = torch.zeros((self.dim, Fp), dtype=torch.int8, device=dev)
            pad[:, :F] = wd
            self.wd_panel.append(pad.view(self.dim, Fp // 16, 16).permute(1, 0, 2).contiguous())
        self._resid = _lib.ResidDesc()
        self._att = _lib.DecAttnDesc()
        # state of the one-launch long-context attention (zero-filled once, shared by the layers,
        # which run one after another)
        nb = max(int(_lib.lib().llhip_dec_attn_state_bytes(int(ly.att["H"]), int(ly.att["D"]))) for ly in layers)
        self.att_state = torch.zeros(nb, dtype=torch.uint8, device=dev)
        self.use_step = True  # one-launch decode step where the graph allows it (llhip_dec_step)
        self._step = None
        self._step_key = None
        self.step_unsupported = None  # the reason llhip_dec_step_create gave, once it refused

    def __del__(self):
        st = getattr(self, "_step", None)
        if st:
            try:
                _lib.lib().llhip_dec_step_destroy(st)
            except Exception:
                pass

    # ---- the one-launch decode step ---------------------------------------------------------
    def _step_layer(self, i, ly, pd):
        m = self.model
        dt = m._dt
        t = _lib.StepLayer()
        fa, fm = ly.attn_in, ly.mlp
        fa.fill(fa.desc, 1, 0, pd)
        fm.fill(fm.desc, 1, 0, pd)
        if fa.desc.has_norm:
            return None
        a, f = fa.desc, fm.desc
        t.g1, t.eps1, t.C1, t.sh1, t.Mq1, t.Sq1 = a.pre.gamma, a.pre.eps_t, a.pre.C, a.pre.sh_post, a.pre.Mq, a.pre.Sq
        for r in range(3):
            t.W[r], t.rq[r], t.bias[r] = a.W[r], a.rq[r], a.bias[r]
        for r in range(2):
            t.quant_M[r], t.quant_S[r] = a.quant_M[r], a.quant_S[r]
        t.kc, t.vc = a.kc, a.vc
        att = ly.att
        t.Ms, t.Ss, t.Mo, t.So = int(att["Ms"]), int(att["Ss"]), int(att["Mo"]), int(att["So"])
        t.prob_bits = int(att.get("prob_bits", 8))
        t.wo_panel = _vp(self.wo_panel[i])
        t.rq_o = _vp(dt[ly.wo["rq"]])
        t.bias_o = _vp(dt[ly.wo["bias"]]) if ly.wo.get("bias") else None
        t.g2, t.eps2, t.C2, t.sh2, t.Mq2, t.Sq2 = f.pre.gamma, f.pre.eps_t, f.pre.C, f.pre.sh_post, f.pre.Mq, f.pre.Sq
        t.Wg, t.Wu, t.rqg, t.rqu, t.bg, t.bu = f.Wg, f.Wu, f.rqg, f.rqu, f.bg, f.bu
        t.silu_Mi, t.silu_Si, t.silu_sh, t.mul_sh, t.fq_M, t.fq_S = (f.silu_Mi, f.silu_Si, f.silu_sh, f.mul_sh,
                                                                     f.fq_M, f.fq_S)
        t.wd_panel = _vp(self.wd_panel[i])
        t.rq_d = _vp(dt[ly.wd["rq"]])
        t.bias_d = _vp(dt[ly.wd["bias"]]) if ly.wd.get("bias") else None
        return t

    def step(self, pd):
        """The llhip_dec_step handle for launches at the device position pd (created on first use),
        or None when the graph's shape is outside it (the reason is kept in step_unsupported)."""
        if not self.use_step or not isinstance(pd, ctypes.c_void_p) or not pd.value or self.step_unsupported:
            return None
        m = self.model
        # the handle holds the cache, input-row and position addresses of its creation
        key = (pd.value, getattr(m, "_kv_gen", 0), m._slot, m._act[m.q.input_name].data_ptr())
        if self._step is not None and self._step_key == key:
            return self._step
        if _torch().cuda.is_current_stream_capturing():
            return None  # creating one allocates: never inside a graph capture
        L = len(self.layers)
        arr = (_lib.StepLayer * L)()
        for i, ly in enumerate(self.layers):
            t = self._step_layer(i, ly, pd)
            if t is None:
                self.step_unsupported = "Q/K norm"
                return None
            arr[i] = t
        a0, f0 = self.layers[0].att, self.layers[0].mlp.desc
        d = _lib.DecStepDesc()
        d.layers, d.L, d.dim = arr, L, self.dim
        d.H, d.Hkv, d.D, d.F, d.max_seq = int(a0["H"]), int(a0["Hkv"]), int(a0["D"]), int(f0.N), m.max_seq
        d.x_in = _vp(m._act[m.q.input_name])
        d.cos_tab, d.sin_tab, d.pos_dev = _vp(m._dt["rope_cos"]), _vp(m._dt["rope_sin"]), pd
        lib = _lib.lib()
        h = lib.llhip_dec_step_create(ctypes.byref(d))
        if not h:
            self.step_unsupported = (lib.llhip_last_error() or b"").decode() or "unsupported"
            return None
        if self._step:
            lib.llhip_dec_step_destroy(self._step)
        self._step, self._step_key = h, key
        acc, res = ctypes.c_void_p(), ctypes.c_void_p()
        _lib.call("llhip_dec_step_outputs", h, ctypes.byref(acc), ctypes.byref(res))
        self._step_acc, self._step_res = acc, res
        return h

    def check_step(self):
        """Raise if a decode-step launch or a one-launch attention hit its bounded-wait timeout
        (synchronises the device)."""
        n, err = ctypes.c_int64(), ctypes.c_int64()
        _lib.call("llhip_dec_attn_status", _vp(self.att_state), ctypes.byref(n), ctypes.byref(err))
        if err.value:
            raise RuntimeError(f"decode attention: a hand-off wait timed out (error word {err.value})")
        if not self._step:
            return
        n, err = ctypes.c_int64(), ctypes.c_int64()
        _lib.call("llhip_dec_step_status", self._step, ctypes.byref(n), ctypes.byref(err))
        if err.value:
            self.use_step = False
            self.model._graph = None  # a captured decode graph holds the step's launch
            raise RuntimeError(f"decode step: a hand-off wait timed out (error word {err.value}); "
                               "the step is disabled for this model")

    # ---- descriptors ------------------------------------------------------------------------
    def _fill_resid(self, op, acc, R, aux=None):
        """Finishing `op` (linear, resadd) from `acc` [R][dim] (a tensor or a device pointer), adding
        the residual `aux` (default: the op's aux activation)."""
        m, r = self.model, self._resid
        r.acc, r.R = (acc if isinstance(acc, ctypes.c_void_p) else _vp(acc)), R
        r.rq = _vp(m._dt[op["rq"]])
        r.bias = _vp(m._dt[op["bias"]]) if op.get("bias") else None
        r.aux = aux if aux is not None else _vp(m._buf(op["aux"]))
        r.x_out = _vp(m._buf(op["out"]))
        return ctypes.byref(r)

    def _launch_layer(self, i, ly, pos, pd, only=None):
        """Layer i's three launches (or, with `only`, the launch of that family alone)."""
        s = self.model._stream_handle()
        if only is None or only == "dec_attn_in":
            self._attn_in(i, ly, pos, pd, s)
        if only is None or only == "dec_attention":
            self._attention(i, ly, pos, pd, s)
        if only is None or only == "dec_mlp":
            self._mlp(i, ly, pos, pd, s)

    def _attn_in(self, i, ly, pos, pd, s):
        fs = ly.attn_in
        fs.fill(fs.desc, 1, pos, pd)
        fs.desc.pre.prequant = 0
        resid = self._fill_resid(self.layers[i - 1].wd, self.acc_wd, WD_ROWS) if i else None
        _lib.call("llhip_dec_attn_in", ctypes.byref(fs.desc), resid, _vp(self.acc_wo), self.dim, s)

    def _attention(self, i, ly, pos, pd, s):
        m = self.model
        a, d = ly.att, self._att
        kcp, vcp, pdev, _, _ = m._kv_args(int(a["layer"]), pd)
        d.q, d.kc, d.vc, d.out = _vp(m._buf(a["q"])), kcp, vcp, _vp(m._buf(a["out"]))
        d.pos_dev, d.pos = pdev, pos
        d.H, d.Hkv, d.D, d.max_seq = int(a["H"]), int(a["Hkv"]), int(a["D"]), m.max_seq
        d.Ms, d.Ss, d.Mo, d.So = int(a["Ms"]), int(a["Ss"]), int(a["Mo"]), int(a["So"])
        d.prob_bits = int(a.get("prob_bits", 8))
        d.wo_panel, d.N, d.acc = _vp(self.wo_panel[i]), self.dim, _vp(self.acc_wo)
        d.zero, d.zero_n = _vp(self.acc_wd), WD_ROWS * self.dim
        d.state, d.state_bytes = _vp(self.att_state), self.att_state.numel()
        _lib.call("llhip_dec_attention", ctypes.byref(d), _vp(m._ws), s)

    def _mlp(self, i, ly, pos, pd, s):
        fm = ly.mlp
        fm.fill(fm.desc, 1, pos, pd)
        fm.desc.pre.prequant = 0
        _lib.call("llhip_dec_mlp", ctypes.byref(fm.desc), self._fill_resid(ly.wo, self.acc_wo, 1),
                  _vp(self.wd_panel[i]), _vp(self.acc_wd), WD_ROWS, self.dim, s)

    def run(self, pos, pd=None, greedy=None, only=None):
        """One row at position pos (or *pd).  greedy = (token, pos, step) device int32 pointers plus
        (ring_rows, ring_ld, ring_tokens, ring_cap): the decode loop's greedy step and record.
        `only` names one family (dec_attn_in, dec_attention, dec_mlp, dec_head) whose launches alone
        run -- a measurement aid: the values they compute are then meaningless."""
        m = self.model
        st = self.step(pd) if only in (None, "dec_step", "dec_head") else None
        if only == "dec_step":
            if st is None:
                raise ValueError(f"no decode step for this graph: {self.step_unsupported}")
            _lib.call("llhip_dec_step_run", st, m._stream_handle())
            return
        if st is not None and only is None:
            _lib.call("llhip_dec_step_run", st, m._stream_handle())
        elif st is None or only != "dec_head":
            for i, ly in enumerate(self.layers):
                self._launch_layer(i, ly, pos, pd, only)
        if only not in (None, "dec_head"):
            return
        fh = self.head
        fh.fill(fh.desc, 1, pos, pd)
        s = m._stream_handle()
        fh.desc.pre.prequant = 0
        if st is not None:
            resid = self._fill_resid(self.layers[-1].wd, self._step_acc, WD_ROWS, aux=self._step_res)
        else:
            resid = self._fill_resid(self.layers[-1].wd, self.acc_wd, WD_ROWS)
        if greedy is not None and self.use_logits and self._logits_fit(fh.desc):
            # finish, norm, quant, lm_head and the greedy step in one launch
            tok, posp, step, ring_rows, ring_ld, ring_tok, ring_cap = greedy
            _lib.call("llhip_dec_logits", ctypes.byref(fh.desc), _vp(self._head_panel(fh.desc)), resid, m.vocab,
                      _vp(self.logit_keys), tok, posp, step, ring_rows, ring_ld, ring_tok, ring_cap,
                      _vp(m._dt["embed"]), self.dim, _vp(m._act[m.q.input_name]), s)
            return
        # the last down projection finished, normalised and quantised once; the lm_head workgroups
        # read the quantised row
        _lib.call("llhip_dec_finish", ctypes.byref(fh.desc.pre), resid, s)
        fh.desc.pre.prequant = 1
        if greedy is None:
            _lib.call("llhip_dec_head", ctypes.byref(fh.desc), m.vocab, None, None, None, 0, 0, s)
            return
        tok, posp, step, ring_rows, ring_ld, ring_tok, ring_cap = greedy
        _lib.call("llhip_dec_head", ctypes.byref(fh.desc), m.vocab, _vp(self.keys), step, ring_rows, ring_ld,
                  ring_cap, s)
        _lib.call("llhip_dec_greedy", _vp(self.keys), self.keys.numel(), tok, posp, step, ring_tok, ring_cap,
                  _vp(m._dt["embed"]), self.dim, _vp(m._act[m.q.input_name]), s)

    def prepare_head(self):
        """What the greedy head needs made before a capture: the tile-order lm_head."""
        fh = self.head
        fh.fill(fh.desc, 1, 0, None)
        if self.use_logits and self._logits_fit(fh.desc):
            self._head_panel(fh.desc)

    def _head_panel(self, d):
        """The lm_head weights in llhip_dec_logits' tile order (built once, on the model's stream)."""
        if self._panel is None:
            torch = _torch()
            N, K = int(d.N), int(d.pre.K)
            panel = torch.empty(-(-N // 16) * 16 * K, dtype=torch.int8, device=self.model.device)
            _lib.call("llhip_dec_logits_panel", d.W, N, K, _vp(panel), self.model._stream_handle())
            self._panel = panel
        return self._panel

    @staticmethod
    def _logits_fit(d):
        """llhip_dec_logits' shape: one row, plain epilogue, K a multiple of 64 up to 1024, 16-byte
        aligned weights."""
        K = int(d.pre.K)
        return (d.M == 1 and d.epilogue == 0 and not d.out_i8 and K % 64 == 0 and K <= 1024
                and int(d.W or 0) % 16 == 0 and d.N >= 16)

    # ---- measurement ------------------------------------------------------------------------
    FAMILIES = ("dec_attn_in", "dec_attention", "dec_mlp", "dec_head")  # the three-launch chain
    STEP_FAMILIES = ("dec_step", "dec_head")  # the one-launch step: every layer, then the head

    def families(self, pd=None):
        """The kernel families of a decode step as run(): the one-launch step's when it serves this
        graph (pd: the device position pointer the step is created for), else the chain's."""
        return self.STEP_FAMILIES if self.step(pd) is not None else self.FAMILIES

    def launches(self, family: str) -> int:
        if family == "dec_head":  # with the greedy step: one launch, or the finish, lm_head and greedy
            return 1 if self._one_launch_head() else 3
        return 1 if family == "dec_step" else len(self.layers)

    def _one_launch_head(self) -> bool:
        fh = self.head
        fh.fill(fh.desc, 1, 0, None)
        return self.use_logits and self._logits_fit(fh.desc)

    def capture_family(self, family: str | None, pos: int):
        """A HIP graph of one decode step's launches of `family` at the device position `pos` (for
        timing them in isolation: the values are then meaningless; dec_head with the decode loop's
        greedy step), or with family None the whole step's layers and head (without the greedy
        step), which can be replayed at one position."""
        m = self.model
        torch = _torch()
        m._decode_state(1)
        m._st.copy_(torch.tensor([0, pos, 0], dtype=torch.int32))
        base = m._st.data_ptr()
        pd = ctypes.c_void_p(base + 4)
        greedy = None
        if family == "dec_head":
            greedy = (ctypes.c_void_p(base), pd, ctypes.c_void_p(base + 8), _vp(m._ring_rows), m.vocab,
                      _vp(m._ring_tok), m._ring_cap)
        self.prepare_head()
        from .golden import capture_graph

        g = torch.cuda.CUDAGraph()
        with capture_graph(g):
            self.run(0, pd, greedy=greedy, only=family)
        return g

    def step_bytes(self, T: int):
        """Algorithmic HBM bytes of one row's launch at context T, per chain kernel family: the bytes
        of the ops each family computes (the linear(M,N,K) and attention formulas of the measurement
        plan), so the families add up to the fused plan's step."""
        fam = {"dec_attn_in": 0, "dec_attention": 0, "dec_mlp": 0, "dec_head": 0}  # dec_finish: in dec_head
        for ly in self.layers:
            fam["dec_attn_in"] += ly.attn_in.bytes_fn(1)
            fam["dec_attention"] += ly.att_bytes(1, T) + ly.wo_bytes(1)
            fam["dec_mlp"] += ly.mlp.bytes_fn(1) + ly.wd_bytes(1)
        fam["dec_head"] = self.head.bytes_fn(1)
        fam["dec_step"] = fam["dec_attn_in"] + fam["dec_attention"] + fam["dec_mlp"]  # the same ops, one launch
        return fam


def _torch():
    import torch

    return torch


def build(model):
    """The decode chain of `model`'s op list, or None when a layer does not have the chain's shape."""
    ops, steps = model.q.ops, model._plan_unfused
    if any(getattr(s, "kind", "") == "error" for s in steps) or len(steps) != len(ops):
        return None
    spec = model._act_spec
    resid = model.q.input_name
    dim = model.dim
    i, layers = 0, []
    while i < len(ops):
        got = fusion.match_attn_in(model, ops, i, steps)
        if got is None:
            break
        n, fa = got
        rn = fa.ops[0]
        if rn["in"] != resid or fa.K != dim:
            return None
        j = i + n
        if j + 1 >= len(ops):
            return None
        att, wo = ops[j], ops[j + 1]
        qq = fa.ops[-3]  # quant q (rope q, rope k, quant q, quant k, kv_write end the run)
        kvw = fa.ops[-1]
        if att.get("op") != "attention" or att["q"] != qq["out"] or int(att["layer"]) != int(kvw["layer"]):
            return None
        H, D = int(att["H"]), int(att["D"])
        if not _resadd_linear(wo, att["out"], resid, dim, H * D) or D % 16 or D > 256:
            return None
        j += 2
        got = fusion.match_mlp_in(model, ops, j, steps)
        if got is None:
            return None
        n, fm = got
        if fm.ops[0]["in"] != wo["out"] or fm.K != dim:
            return None
        fq = fm.ops[-1]
        j += n
        if j >= len(ops):
            return None
        wd = ops[j]
        F = spec[fq["out"]][1]
        if not _resadd_linear(wd, fq["out"], wo["out"], dim, F):
            return None
        ly = _Layer(fa, att, wo, fm, wd, resid)
        a_at = i + len(fa.ops)  # op index of the attention; wo follows it
        ly.att_bytes, ly.wo_bytes, ly.wd_bytes = steps[a_at].bytes_fn, steps[a_at + 1].bytes_fn, steps[j].bytes_fn
        layers.append(ly)
        resid = wd["out"]
        i = j + 1
    if not layers:
        return None
    got = fusion.match_norm_linear(model, ops, i, steps)
    if got is None:
        return None
    n, fh = got
    lo = fh.ops[-1]
    if (fh.ops[0]["in"] != resid or i + n != len(ops) or lo["out"] != model.q.output_name or fh.K != dim
            or lo.get("out_dtype", "i16") != "i16" or int(lo["N"]) < model.vocab):
        return None
    fh.desc_N = int(lo["N"])
    for ly in layers:  # the finished projections' operands must be 16-byte addressable
        for op in (ly.wo, ly.wd):
            if op.get("bias") and model._dt[op["bias"]].data_ptr() % 16:
                return None
            if model._dt[op["rq"]].data_ptr() % 16:
                return None
    return Chain(model, layers, fh, fh.ops)
