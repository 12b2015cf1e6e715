"""Turn a plan into the device task table and run it (the reference's fleet/build_graph.py:478-593).

The reference attaches every tensor to a mirage PersistentKernel, issues one mpk.<op>_layer per
call and JIT-compiles the worker switch. Here the tensors are device buffers the host owns
(fleet.runtime.DeviceBuffer), each call becomes one fx_stage (include/fleet_mi355x.h), and the table
is validated and uploaded by fx_load_plan -- no code generation. Three calls are folded into the input
prologue of the GEMV that follows them (no sync of their own):
  prologue.embed     -> L0.qkva reads W_embed[tokens[step]] (or, once past the prompt, the previous
                        head's argmax) and worker 0 writes x_res;
  L{l}.combine       -> the next GEMV (L{l+1}.qkva or head.lm_head) computes x_res + sum w_s out8[s]
                        itself and worker 0 writes it to the other x_res buffer (two physical x_res
                        buffers alternate, so no stage reads and writes the same one);
  head.argmax_reduce -> the next iteration's embed prologue; the last iteration's runs as the epilogue.
A truncated plan (--stop-after) that ends on a combine runs it as a standalone stage.
"""
import numpy as np

from fleet import graph_plan as G
from fleet import runtime as R
from fleet.pack_weights import Dims, REAL_DIMS, XCDS, rope_tables


def make_tensors(rt, plan, packed, capture, meta):
    """name -> DeviceBuffer: `new` tensors allocated and zeroed, inputs taken from packed weights,
    the captured cache/tables and the meta tensors (shapes checked)."""
    host = {}
    for name, t in plan.tensors.items():
        if t.kind == "new":
            host[name] = rt.alloc(t.shape, t.dtype).zero()
            continue
        kind, _, key = t.source.partition(":") if ":" in t.source else ("weight", "", t.source)
        src = {"weight": packed, "capture": capture, "meta": meta}[kind][key]
        assert tuple(src.shape) == tuple(t.shape), (name, src.shape, t.shape)
        host[name] = src
    host["x_res_b"] = rt.alloc((plan.dims.H,), "bf16").zero()
    return host


def _stage(**kw):
    return R.FxStage().set(**kw)


def compile_stages(plan, host):
    """(stages, epilogue, x_final): the fx_stage table of one iteration, the post-loop stages, and the
    name of the physical buffer that holds x_res after the last call."""
    d = plan.dims
    cur, other = "x_res", "x_res_b"
    stages, epi = [], []
    labels = []
    pend_embed = pend_combine = None
    sync_of = {G.GLOBAL: R.FX_SYNC_GLOBAL, G.XCD: R.FX_SYNC_XCD, G.NONE: R.FX_SYNC_NONE}
    B = lambda n: host[n].ptr if n else 0

    def xr(name):
        return cur if name == "x_res" else name

    def standalone_combine(c):
        stages.append(_stage(op=R.FX_OP_MOE_COMBINE, sync=R.FX_SYNC_GLOBAL, n_rows=d.H, n_slots=d.N_SLOTS,
                             x=B(cur), out=B(cur), aux={0: B(c.args["input"]), 1: B(c.args["weight"])},
                             layer=int(c.label.split(".")[0][1:])))
        labels.append(c.label)

    for c in plan.calls:
        a = c.args
        m = c.method
        if m == "embed_layer":
            pend_embed = c
            continue
        if m == "moe_mul_sum_add_layer":
            pend_combine = c
            continue
        if m == "argmax_reduce_layer":
            epi.append(_stage(op=R.FX_OP_ARGMAX, sync=R.FX_SYNC_NONE, aux={3: B(a["input"]), 4: B("tokens")}))
            continue
        layer = int(c.label.split(".")[0][1:]) if c.label.startswith("L") else -1
        sync = sync_of[c.sync]
        if m == "linear_gemv_layer":
            W = host[a["weight"]]
            st = _stage(op=R.FX_OP_GEMV, sync=sync, layer=layer, n_rows=W.shape[0], k=W.shape[1], eps=plan.eps,
                        w=W.ptr, out=B(xr(a["output"])), in_kind=R.FX_IN_VEC)
            flags = 0
            if a.get("norm"):
                flags |= R.FX_F_NORM
                st.w_norm = B(a["w_norm"])
            if a.get("residual"):
                flags |= R.FX_F_RESIDUAL
                st.res = B(xr(a["residual"]))
            if a.get("amax"):
                flags |= R.FX_F_ARGMAX | R.FX_F_HEAD
                st.aux[3] = B(a["amax"])
            lab = c.label
            if pend_embed is not None and a["input"] == "x_res":
                lab = c.label + "+embed"
                st.in_kind = R.FX_IN_EMBED
                st.aux[0] = B("W_embed")
                st.aux[3] = B("amax")
                st.aux[4] = B("tokens")
                st.aux[2] = B(cur)
                flags |= R.FX_F_WRITE_X
                pend_embed = None
            elif pend_combine is not None and a["input"] == "x_res":
                lab = c.label + "+combine"
                st.in_kind = R.FX_IN_COMBINE
                st.x = B(cur)
                st.aux[0] = B(pend_combine.args["input"])
                st.aux[1] = B(pend_combine.args["weight"])
                st.n_slots = d.N_SLOTS
                st.aux[2] = B(other)
                flags |= R.FX_F_WRITE_X
                cur, other = other, cur
                pend_combine = None
            else:
                if pend_combine is not None:
                    standalone_combine(pend_combine)
                    pend_combine = None
                st.x = B(xr(a["input"]))
            if st.out == B("x_res") or st.out == B("x_res_b"):
                st.out = B(cur)
            if st.res:
                st.res = B(cur)
            st.flags = flags
            stages.append(st)
            labels.append(lab)
            continue
        assert pend_embed is None, "prologue.embed must be followed by L0.qkva"
        if pend_combine is not None:
            standalone_combine(pend_combine)
            pend_combine = None
        common = dict(sync=sync, layer=layer, eps=plan.eps)
        if m == "mla_prep_layer":
            st = _stage(op=R.FX_OP_MLA_PREP, n_rows=d.NH, d_c=d.D_C, d_r=d.D_R, d_n=d.D_N, s_max=plan.s_max,
                        x=B(a["qkva"]), w=B(a["w_uk"]), w_norm=B(a["w_kv_norm"]), out=B(a["ql_nope"]),
                        aux={0: B(a["c_kv"]), 1: B(a["k_pe"]), 2: B(a["q_pe"]), 3: B(a["cos"]), 4: B(a["sin"])},
                        **common)
        elif m == "mla_attend_layer":
            st = _stage(op=R.FX_OP_MLA_ATTEND, n_rows=d.NH, d_c=d.D_C, d_r=d.D_R, d_n=d.D_N, split=a["split"],
                        n_splits=a["n_splits"], prow=G.partials_row(d.D_C), s_max=plan.s_max, s_scores=plan.s_max,
                        scale=a["softmax_scale"], x=B(a["ql_nope"]), out=B(a["partials"]),
                        aux={0: B(a["c_kv"]), 1: B(a["k_pe"]), 2: B(a["q_pe"]), 3: B(a.get("scores")),
                             4: B(a["o_merged"])}, **common)
        elif m == "mla_merge_uv_layer":
            st = _stage(op=R.FX_OP_MLA_MERGE_UV, n_rows=d.NH, d_c=d.D_C, d_r=d.D_R, d_n=d.D_V, x=B(a["input"]),
                        w=B(a["w_uv"]), out=B(a["output"]), **common)
        elif m == "gang_linear_silu_layer":
            st = _stage(op=R.FX_OP_DENSE_GU, n_rows=d.I_DENSE, k=d.H, x=B(cur), w_norm=B(a["w_norm"]),
                        w=B(a["weight"]), out=B(a["output"]), aux={6: B(a.get("h"))}, **common)
        elif m == "moe_router_layer":
            st = _stage(op=R.FX_OP_MOE_ROUTER, n_rows=d.E, k=d.H, topk=d.TOPK, x=B(cur), w_norm=B(a["w_norm"]),
                        w=B(a["w_gate"]), out=B(a["logits_x"]), **common)
        elif m == "gang_moe_w13_gemv_layer":
            rl = host[a["route_log"]]
            st = _stage(op=R.FX_OP_MOE_W13, n_rows=d.I_MOE, k=d.H, n_slots=d.N_SLOTS, topk=d.TOPK,
                        n_forced=d.N_SHARED, scaling=G.ROUTED_SCALING, aux_i0=d.E, aux_i1=rl.shape[1],
                        prow=rl.shape[0], x=B(cur), w_norm=B(a["w_norm"]), w=B(a["weight"]), out=B(a["output"]),
                        aux={0: B(a["logits_x"]), 1: B(a["topk_w"]), 2: B(a["routing"]), 3: B(a["mask"]),
                             4: B(a["logits"]), 5: rl.ptr, 6: B(a["h"]), 7: B(a["sel"])}, **common)
        elif m == "gang_moe_w2_linear_layer":
            st = _stage(op=R.FX_OP_MOE_W2, n_rows=d.H, k=d.I_MOE, x=B(a["input"]), w=B(a["weight"]),
                        out=B(a["output"]), aux={7: B(a["sel"])}, **common)
        else:
            raise ValueError(f"unknown plan method {m}")
        stages.append(st)
        labels.append(c.label)
    assert pend_embed is None, "a plan cannot end on prologue.embed"
    if pend_combine is not None:
        standalone_combine(pend_combine)
    compile_stages.labels = labels
    return stages, epi, cur


class Runner:
    """The built graph: rt + plan + host tensors + task table (what the reference's build() returns
    as (mpk, host, plan))."""

    def __init__(self, rt, plan, host, stages, epi, x_final):
        self.rt, self.plan, self.host = rt, plan, host
        self.stages, self.epi, self.x_final = stages, epi, x_final
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
        label, sync, start (us from the iteration's first stamp), busy (slowest worker's share),
        spread (last minus first worker to finish), gap (until the next stage starts)."""
        self.rt.set_profile(iteration)
        try:
            self.run(iters, step0, n_prompt)
        finally:
            self.rt.set_profile(-1)
        st = self.rt.read_profile(len(self.stages))[:, 8:, :].astype(np.float64) / 100.0   # workers only, us
        t0 = st[0, :, 0].min()
        rows = []
        for i, lab in enumerate(self.labels):
            start, end = st[i, :, 0].min() - t0, st[i, :, 1].max() - t0
            nxt = st[i + 1, :, 0].min() - t0 if i + 1 < len(self.labels) else end
            busy = (st[i, :, 1] - st[i, :, 0]).max()
            rows.append({"label": lab, "sync": int(self.stages[i].sync), "start": start, "busy": busy,
                         "spread": st[i, :, 1].max() - st[i, :, 1].min(), "span": end - start, "gap": nxt - end})
        return rows

    def timing_us(self):
        t = self.rt.timing(self.last_iters)
        return np.diff(t.astype(np.float64)) / 100.0    # s_memrealtime ticks are 100 MHz

    def x_res(self):
        return self.host[self.x_final].download()


def make_meta(rt, s_max, prompt):
    tokens = rt.alloc((s_max + 1,), "i64").zero()
    t = np.zeros(s_max + 1, np.int64)
    t[:len(prompt)] = prompt
    tokens.upload(t)
    return {"tokens": tokens}


def make_capture(rt, plan, cache=None):
    """cos/sin tables and the per-layer latent caches (zeroed, or uploaded from host arrays
    cache['c_kv'][l], cache['k_pe'][l] for rows [0, len))."""
    d = plan.dims
    cos, sin = rope_tables(plan.s_max, d.D_R)
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
    stages, epi, x_final = compile_stages(plan, host)
    runner = Runner(rt, plan, host, stages, epi, x_final)
    runner.labels = list(compile_stages.labels)
    return runner


def plan_json(plan):
    return {"dims": plan.dims.__dict__, "s_max": plan.s_max, "layers": plan.layers, "head": plan.head,
            "split": plan.split, "n_splits": plan.n_splits,
            "calls": [{"method": c.method, "label": c.label, "sync": c.sync, "tasks": c.tasks,
                       "args": {k: v for k, v in c.args.items() if isinstance(v, (str, int, float, bool)) or v is None}}
                      for c in plan.calls]}
