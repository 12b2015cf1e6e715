"""Turn a plan into the device task table and run it (the reference's fleet/build_graph.py:478-593).

The reference attaches every tensor to a mirage PersistentKernel, issues one mpk.<op>_layer per
call and JIT-compiles the worker switch. Here the tensors are device buffers the host owns
(fleet.runtime.DeviceBuffer), each call becomes one fx_stage (include/fleet_mi355x.h), and the table
is validated and uploaded by fx_load_plan -- no code generation. Three calls are folded into a
neighbour (no stage of their own):
  prologue.embed     -> L0.qkva reads W_embed[tokens[step]] (or, once past the prompt, the previous
                        head's argmax); L0.o_proj takes the same row as its residual;
  L{l}.router        -> L{l}.w13 (FX_F_ROUTER): worker e computes router row e inside the gate|up
                        stage, whose shared-expert weights stream meanwhile;
  L{l}.combine       -> L{l}.w2: each worker computes its 8 output rows for every slot and combines
                        them with the residual;
  head.argmax_reduce -> the next iteration's embed; the last iteration's runs as the epilogue.
Every packet input of a stage names the stage that produces it (fx_stage.src): the last writer
before it in the table, or, for the head's argmax read by the next iteration's embed, a stage of
the previous iteration (a negative index).
"""
import numpy as np

from fleet import graph_plan as G
from fleet import runtime as R
from fleet.pack_weights import Dims, REAL_DIMS, XCDS, rope_tables


def make_tensors(rt, plan, packed, capture, meta):
    """name -> DeviceBuffer: `new` tensors allocated and zeroed (packet tensors start at tag 0),
    inputs taken from packed weights, the captured cache/tables and the meta tensors (shapes checked)."""
    host = {}
    for name, t in plan.tensors.items():
        if t.kind == "new":
            host[name] = rt.alloc(t.shape, t.dtype).zero()
            continue
        kind, _, key = t.source.partition(":") if ":" in t.source else ("weight", "", t.source)
        src = {"weight": packed, "capture": capture, "meta": meta}[kind][key]
        assert tuple(src.shape) == tuple(t.shape), (name, src.shape, t.shape)
        host[name] = src
    return host


def _stage(**kw):
    return R.FxStage().set(**kw)


def compile_stages(plan, host):
    """(stages, epilogue): the fx_stage table of one iteration and the post-loop stages. Each stage's
    packet inputs are resolved to their producing stage (src)."""
    d = plan.dims
    stages, epi, labels = [], [], []
    reads = []          # per stage: [(src slot, tensor name)]
    pend_embed = None
    pend_router = None
    pend_attend = None   # the attention call whose work the next merge stage takes (attn "xcd")
    B = lambda n: host[n].ptr if n else 0

    def add(st, label, ins):
        stages.append(st)
        labels.append(label)
        reads.append(ins)

    for c in plan.calls:
        a = c.args
        m = c.method
        if m == "embed_layer":
            pend_embed = c
            continue
        if m == "moe_mul_sum_add_layer":
            assert stages and stages[-1].op == R.FX_OP_MOE_W2, "combine must follow its w2"
            continue
        if m == "moe_router_layer":
            pend_router = c
            continue
        if pend_router is not None and m != "gang_moe_w13_gemv_layer":
            raise ValueError("the router must be followed by its w13")
        if m == "argmax_reduce_layer":
            epi.append((_stage(op=R.FX_OP_ARGMAX, aux={3: B(a["input"]), 4: B("tokens")}), [(0, a["input"])]))
            continue
        layer = int(c.label.split(".")[0][1:]) if c.label.startswith("L") else -1
        common = dict(layer=layer, eps=plan.eps)
        if m == "linear_gemv_layer":
            W = host[a["weight"]]
            fp8 = plan.fp8_head and a.get("amax") is not None
            rows_k = (d.V, d.H) if fp8 else (W.shape[0], W.shape[1])
            st = _stage(op=R.FX_OP_GEMV, n_rows=rows_k[0], k=rows_k[1], w=W.ptr, out=B(a["output"]),
                        in_kind=R.FX_IN_VEC, **common)
            ins = []
            flags = R.FX_F_FP8 if fp8 else 0
            if host[a["output"]].dtype == "pk16":
                flags |= R.FX_F_OUT_LL
            if a.get("norm"):
                flags |= R.FX_F_NORM
                st.w_norm = B(a["w_norm"])
            if a.get("amax"):
                flags |= R.FX_F_ARGMAX | R.FX_F_HEAD
                st.aux[3] = B(a["amax"])
            lab = c.label
            if pend_embed is not None and a["input"] == pend_embed.args["output"]:
                lab = c.label + "+embed"
                st.in_kind = R.FX_IN_EMBED
                st.aux[0] = B("W_embed")
                st.aux[3] = B("amax")
                st.aux[4] = B("tokens")
                ins.append((1, "amax"))
                embed_out = pend_embed.args["output"]
                pend_embed = None
            else:
                st.x = B(a["input"])
                ins.append((0, a["input"]))
            if a.get("residual"):
                if layer == 0 and a["residual"] == "x_res" and plan.calls[0].method == "embed_layer":
                    # layer 0's residual stream is the embedding row itself
                    flags |= R.FX_F_RES_EMBED
                    st.aux[0] = B("W_embed")
                    st.aux[4] = B("tokens")
                else:
                    flags |= R.FX_F_RESIDUAL
                    st.res = B(a["residual"])
                    ins.append((2, a["residual"]))
            if plan.attn == "xcd" and a["input"] == "attn":
                # o_proj right after the single-XCD attention: XCD 7's workers take no rows
                flags |= R.FX_F_SKIP_XCD
            st.flags = flags
            add(st, lab, ins)
            continue
        assert pend_embed is None, "prologue.embed must be followed by L0.qkva"
        if m == "mla_prep_layer":
            st = _stage(op=R.FX_OP_MLA_PREP, n_rows=d.NH, d_c=d.D_C, d_r=d.D_R, d_n=d.D_N, s_max=plan.s_max,
                        x=B(a["qkva"]), w=B(a["w_uk"]), w_norm=B(a["w_kv_norm"]), out=B(a["ql_nope"]),
                        aux={0: B(a["c_kv"]), 1: B(a["k_pe"]), 2: B(a["q_pe"]), 3: B(a["cos"]), 4: B(a["sin"]),
                             5: B(a["crow"])}, **common)
            if plan.attn == "valu":
                # the VALU attention reads the XCD's own heads: prep's packets stay in the XCD
                st.flags |= R.FX_F_XLOCAL
            ins = [(0, a["qkva"])]
        elif m == "mla_attend_layer":
            st = _stage(op=R.FX_OP_MLA_ATTEND, n_rows=d.NH, d_c=d.D_C, d_r=d.D_R, d_n=d.D_N, split=a["split"],
                        n_splits=a["n_splits"], prow=G.partials_row(d.D_C), s_max=plan.s_max,
                        scale=a["softmax_scale"], x=B(a["ql_nope"]), out=B(a["partials"]),
                        aux={0: B(a["c_kv"]), 1: B(a["k_pe"]), 2: B(a["q_pe"]), 5: B(a["crow"]), 6: B(a["done"])},
                        **common)
            if plan.attn == "mfma":
                st.flags |= R.FX_F_MFMA
            if plan.attn == "xcd":
                # the attention runs inside the merge stage; this stage stays as a (no-op) marker
                st.flags |= R.FX_F_XCD
                pend_attend = a
            ins = [(0, a["ql_nope"])]
        elif m == "mla_merge_uv_layer":
            st = _stage(op=R.FX_OP_MLA_MERGE_UV, n_rows=d.NH, d_c=d.D_C, d_r=d.D_R, d_n=d.D_V, split=a["split"],
                        n_splits=a["n_splits"], prow=G.partials_row(d.D_C), x=B(a["input"]), w=B(a["w_uv"]),
                        out=B(a["output"]), aux={4: B(a.get("o_merged")), 6: B(a["done"])}, **common)
            ins = [(0, a["done"])]
            if plan.attn == "mfma":
                st.flags |= R.FX_F_MFMA
                # long caches: each of a head's 8 merge workers merges 64 columns and they exchange
                # them through these packets
                st.aux[7] = B(a.get("slices"))
            if plan.attn == "xcd":
                # the attention and the merge on one XCD: the attention's operands in the spare fields
                att = pend_attend
                assert att is not None and att["partials"] == a["input"] and att["done"] == a["done"], \
                    "the merge must follow its attention"
                st.flags |= R.FX_F_XCD
                st.s_max = plan.s_max
                st.scale = att["softmax_scale"]
                for k, name in ((0, "c_kv"), (1, "k_pe"), (2, "q_pe"), (3, "ql_nope"), (5, "crow")):
                    st.aux[k] = B(att[name])
                pend_attend = None
                ins = [(0, att["ql_nope"])]
        elif m == "gang_linear_silu_layer":
            st = _stage(op=R.FX_OP_DENSE_GU, n_rows=d.I_DENSE, k=d.H, x=B(a["input"]), w_norm=B(a["w_norm"]),
                        w=B(a["weight"]), out=B(a["output"]), aux={6: B(a.get("h"))}, **common)
            ins = [(0, a["input"])]
        elif m == "gang_moe_w13_gemv_layer":
            rl = host[a["route_log"]]
            st = _stage(op=R.FX_OP_MOE_W13, n_rows=d.I_MOE, k=d.H, n_slots=d.N_SLOTS, topk=d.TOPK,
                        n_forced=d.N_SHARED, scaling=G.ROUTED_SCALING, aux_i0=d.E, aux_i1=rl.shape[1],
                        prow=rl.shape[0], x=B(a["input"]), w_norm=B(a["w_norm"]), w=B(a["weight"]), out=B(a["output"]),
                        aux={0: B(a["logits_x"]), 1: B(a["topk_w"]), 2: B(a["routing"]), 3: B(a["mask"]),
                             4: B(a["logits"]), 5: rl.ptr, 6: B(a["h"]), 7: B(a["sel"])}, **common)
            ins = [(1, a["input"])]
            lab = c.label
            if plan.fp8_experts:
                st.flags |= R.FX_F_FP8
            if pend_router is not None:
                assert pend_router.args["w_norm"] == a["w_norm"] and pend_router.args["logits_x"] == a["logits_x"]
                st.flags |= R.FX_F_ROUTER
                st.res = B(pend_router.args["w_gate"])
                lab = c.label + "+router"
                pend_router = None
            else:
                ins.append((0, a["logits_x"]))
            add(st, lab, ins)
            continue
        elif m == "gang_moe_w2_linear_layer":
            comb = next(cc for cc in plan.calls if cc.label == c.label.replace(".w2", ".combine"))
            st = _stage(op=R.FX_OP_MOE_W2, n_rows=d.H, k=d.I_MOE, n_slots=d.N_SLOTS, topk=d.TOPK, n_forced=d.N_SHARED,
                        scaling=G.ROUTED_SCALING, aux_i0=d.E, x=B(a["input"]), w=B(a["weight"]),
                        res=B(comb.args["residual"]), out=B(comb.args["output"]),
                        aux={0: B(a["logits_x"]), 1: B(a["output"])}, **common)
            if plan.fp8_experts:
                st.flags |= R.FX_F_FP8
            ins = [(0, a["input"]), (1, a["logits_x"]), (2, comb.args["residual"])]
        else:
            raise ValueError(f"unknown plan method {m}")
        add(st, c.label, ins)
    assert pend_embed is None, "a plan cannot end on prologue.embed"
    if pend_router is not None:     # a plan truncated after L{l}.router: the router alone
        a = pend_router.args
        add(_stage(op=R.FX_OP_MOE_ROUTER, n_rows=d.E, k=d.H, topk=d.TOPK, x=B(a["input"]), w_norm=B(a["w_norm"]),
                   w=B(a["w_gate"]), out=B(a["logits_x"]), layer=int(pend_router.label.split(".")[0][1:]), eps=plan.eps),
            pend_router.label, [(0, a["input"])])
    # resolve packet sources: the last writer before the stage, else the last writer of the table
    # (previous iteration, negative index); a tensor with no writer gets -1 (never awaited: only the
    # embed's amax when the plan has no head)
    n = len(stages)
    writer = {}
    outputs = []
    for i, st in enumerate(stages):
        outs = {st.out}
        if st.op == R.FX_OP_MLA_PREP:
            outs |= {st.aux[2], st.aux[5]}
        if st.op == R.FX_OP_MLA_ATTEND:
            outs = {st.aux[6]}
        if st.op == R.FX_OP_GEMV and st.flags & R.FX_F_ARGMAX:
            outs.add(st.aux[3])
        if st.op == R.FX_OP_MOE_W13 and st.flags & R.FX_F_ROUTER:
            outs.add(st.aux[0])
        outputs.append(outs)
    for i in range(n):
        for k, name in reads[i]:
            ptr = host[name].ptr
            before = [j for j in range(i) if ptr in outputs[j]]
            after = [j for j in range(i, n) if ptr in outputs[j]]
            if before:
                stages[i].src[k] = before[-1]
            elif after:
                stages[i].src[k] = after[-1] - n
            else:
                assert name == "amax", f"{labels[i]}: no stage writes {name}"
                stages[i].src[k] = -1
    if getattr(plan, "pair", False):
        # o_proj + the MoE gate|up stage after it: one operator of the persistent kernel (FX_F_PAIR)
        no = R.FX_F_ARGMAX | R.FX_F_HEAD | R.FX_F_SKIP_XCD | R.FX_F_FP8
        for i in range(n - 1):
            if (stages[i].op == R.FX_OP_GEMV and not (stages[i].flags & no)
                    and stages[i + 1].op == R.FX_OP_MOE_W13 and not (stages[i + 1].flags & R.FX_F_HEAD)):
                stages[i].flags |= R.FX_F_PAIR
                if plan.attn == "mfma" and i > 0 and stages[i - 1].op == R.FX_OP_MLA_MERGE_UV:
                    # the merge's workers (ranks 16..31) take no o_proj rows: they go straight on to
                    # the expert stage's first loads
                    stages[i].flags |= R.FX_F_LOW16
    epi_st = []
    for st, ins in epi:
        for k, name in ins:
            ptr = host[name].ptr
            w = [j for j in range(n) if ptr in outputs[j]]
            st.src[k] = (w[-1] - n) if w else -1
        epi_st.append(st)
    compile_stages.labels = labels
    return stages, epi_st


class Runner:
    """The built graph: rt + plan + host tensors + task table (what the reference's build() returns
    as (mpk, host, plan))."""

    def __init__(self, rt, plan, host, stages, epi):
        self.rt, self.plan, self.host = rt, plan, host
        self.stages, self.epi = stages, epi
        rt.load_plan(stages, epi)

    def run(self, iters, step0, n_prompt):
        """`iters` decode iterations at positions step0.. (fx_run); tokens must hold the prompt."""
        assert step0 + iters <= self.plan.s_max, (step0, iters, self.plan.s_max)
        self.rt.run(iters, step0, n_prompt, self.host["tokens"])
        self.last_iters = iters

    def launch(self, iters, step0, n_prompt):
        """Enqueue `iters` iterations as one launch without waiting (fx_launch); finish() waits."""
        assert step0 + iters <= self.plan.s_max, (step0, iters, self.plan.s_max)
        self.rt.launch(iters, step0, n_prompt, self.host["tokens"])
        self.last_iters = iters

    def finish(self):
        self.rt.finish()

    def profile(self, iters, step0, n_prompt, iteration=0):
        """Run with per-stage stamps recorded for `iteration`; returns a list of per-stage dicts:
        label, start (us from the iteration's first stamp), wait (slowest worker's arrival-to-inputs),
        busy (slowest worker's inputs-to-outputs), end (last worker done, from the iteration start),
        span (first start to last end)."""
        self.rt.set_profile(iteration)
        try:
            self.run(iters, step0, n_prompt)
        finally:
            self.rt.set_profile(-1)
        st = self.rt.read_profile(len(self.stages)).astype(np.float64) / 100.0   # us
        t0 = st[0, :, 0][st[0, :, 0] > 0].min()
        rows = []
        for i, lab in enumerate(self.labels):
            s0, s1, s2, s3 = (st[i, :, k] for k in range(4))
            ok = s0 > 0
            if not ok.any():
                rows.append({"label": lab, "start": 0.0, "wait": 0.0, "busy": 0.0, "end": 0.0, "span": 0.0, "marks": []})
                continue
            has_in = ok & (s1 > 0) & (s2 > 0)
            wait = (s1[has_in] - s0[has_in]).max() if has_in.any() else 0.0
            busy = (s2[has_in] - s1[has_in]).max() if has_in.any() else 0.0
            # op-specific marks 4..7: the median over workers that stamped them, from their input stamp
            marks = []
            for k in range(4, 8):
                m = has_in & (st[i, :, k] > 0)
                marks.append(float(np.median(st[i, m, k] - s1[m])) if m.any() else None)
            rows.append({"label": lab, "start": s0[ok].min() - t0, "wait": wait, "busy": busy,
                         "end": s3[ok].max() - t0, "span": s3[ok].max() - s0[ok].min(), "marks": marks})
        return rows

    def timing_us(self):
        t = self.rt.timing(self.last_iters)
        return np.diff(t.astype(np.float64)) / 100.0    # s_memrealtime ticks are 100 MHz

    def x_res(self):
        """The residual stream after the last layer (bf16 bits)."""
        return self.host["x_res"].download()


def make_meta(rt, s_max, prompt):
    tokens = rt.alloc((s_max + 1,), "i64").zero()
    t = np.zeros(s_max + 1, np.int64)
    t[:len(prompt)] = prompt
    tokens.upload(t)
    return {"tokens": tokens}


def make_capture(rt, plan, cache=None, tables=None):
    """cos/sin tables and the per-layer latent caches (zeroed, or uploaded from host arrays
    cache['c_kv'][l], cache['k_pe'][l] for rows [0, len)). tables: (cos, sin) bf16 bits [s_max, D_R]
    of the model (checkpoint.ModelConfig.tables), default plain RoPE with theta 10000."""
    d = plan.dims
    cos, sin = tables if tables is not None else rope_tables(plan.s_max, d.D_R)
    assert cos.shape == (plan.s_max, d.D_R) and sin.shape == cos.shape, (cos.shape, plan.s_max)
    cap = {"cos": rt.alloc(cos.shape, "bf16").upload(cos), "sin": rt.alloc(sin.shape, "bf16").upload(sin)}
    for l in range(plan.layers):
        cap[f"c_kv_{l}"] = rt.alloc((plan.s_max, d.D_C), "bf16").zero()
        cap[f"k_pe_{l}"] = rt.alloc((plan.s_max, d.D_R), "bf16").zero()
        if cache is not None:
            ck, kp = cache["c_kv"][l], cache["k_pe"][l]
            cap[f"c_kv_{l}"].upload_at(ck, 0)
            cap[f"k_pe_{l}"].upload_at(kp, 0)
    return cap


def build(rt, packed, capture, meta, dims: Dims = REAL_DIMS, s_max=1056, layers=27, head=True, stop_after=None,
          **plan_kw):
    plan = G.build_plan(dims, s_max, layers, head, **plan_kw)
    if stop_after:
        plan.truncate(stop_after)
    host = make_tensors(rt, plan, packed, capture, meta)
    stages, epi = compile_stages(plan, host)
    runner = Runner(rt, plan, host, stages, epi)
    runner.labels = list(compile_stages.labels)
    return runner


def plan_json(plan):
    return {"dims": plan.dims.__dict__, "s_max": plan.s_max, "layers": plan.layers, "head": plan.head,
            "split": plan.split, "n_splits": plan.n_splits, "attn": plan.attn, "fp8_experts": plan.fp8_experts,
            "fp8_head": plan.fp8_head,
            "calls": [{"method": c.method, "label": c.label, "tasks": c.tasks,
                       "args": {k: v for k, v in c.args.items() if isinstance(v, (str, int, float, bool)) or v is None}}
                      for c in plan.calls]}
