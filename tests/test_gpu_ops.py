"""Per-operator parity on the GPU: every stage of the task table, launched alone through the C ABI
(fx_run_stage: the kernel-suite entry, the counterpart of fleet/tasks/kernel_tests_mi300.cu), against
the CPU oracle on the same inputs at the real shapes. The bar is bit-exact: both sides follow the
same FP32 spec (fixed summation orders, own exp/log), so any differing element is a failure.
Outputs are prefilled with a sentinel (0xFFFF / NaN) to catch stray or missing writes, as the
reference suite does (fleet/tasks/kernel_tests.py:54-59)."""
import numpy as np
import pytest

from oracle import oracle as O
from fleet import runtime as R
from fleet import pack_weights as P
from fleet.graph_plan import partials_row
from fxtest import SEED, rng_bf16, mismatch

pytestmark = pytest.mark.gpu

H, NH, DC, DR, DN = 2048, 16, 512, 64, 128
Q_OUT = NH * (DN + DR)
SENT16 = 0xFFFF


_KEEP = []   # every device buffer of the current test stays alive until the test ends


@pytest.fixture(autouse=True)
def _keepalive():
    yield
    _KEEP.clear()


def dev(rt, arr, dtype):
    b = rt.alloc(arr.shape, dtype)
    b.upload(arr)
    _KEEP.append(b)
    return b


def sentinel(rt, shape, dtype):
    b = rt.alloc(shape, dtype)
    _KEEP.append(b)
    if dtype == "f32":
        b.upload(np.full(shape, np.nan, np.float32))
    elif dtype in ("bf16", "u16"):
        b.upload(np.full(shape, SENT16, np.uint16))
    elif dtype == "i32":
        b.upload(np.full(shape, -7, np.int32))
    else:
        b.zero()
    return b


def gemv_stage(W, x, out, K, N, norm=None, res=None, eps=1e-6, **kw):
    st = R.FxStage().set(op=R.FX_OP_GEMV, n_rows=N, k=K, w=W.ptr, x=x.ptr if x is not None else 0, out=out.ptr,
                         eps=eps)
    flags = 0
    if norm is not None:
        flags |= R.FX_F_NORM
        st.w_norm = norm.ptr
    if res is not None:
        flags |= R.FX_F_RESIDUAL
        st.res = res.ptr
    st.flags = flags
    for k, v in kw.items():
        setattr(st, k, v)
    return st


@pytest.mark.parametrize("N,K,norm,res", [(3648, 2048, True, False), (2048, 2048, False, True),
                                          (2048, 10944, False, True), (256, 512, False, False),
                                          (1000, 1408, True, False)])
def test_gemv_forms(rt, N, K, norm, res):
    print(f"[gemv] N={N} K={K} norm={norm} res={res}", flush=True)
    rng = np.random.default_rng(N + K)
    W = rng_bf16(rng, (N, K), 0.02)
    x = rng_bf16(rng, K)
    nw = rng_bf16(rng, K, 0.5) if norm else None
    r = rng_bf16(rng, N) if res else None
    dW, dx = dev(rt, W, "bf16"), dev(rt, x, "bf16")
    dn = dev(rt, nw, "bf16") if norm else None
    dr = dev(rt, r, "bf16") if res else None
    out = sentinel(rt, (N,), "bf16")
    rt.run_stage(gemv_stage(dW, dx, out, K, N, norm=dn, res=dr))
    exp, _ = O.linear(W, x, norm_w=nw, res=r)
    assert mismatch(out.download(), exp) == 0


def test_gemv_embed_prologue_and_head_argmax(rt):
    """L0.qkva's embedding prologue (token from tokens[step], x_res written by worker 0) and the LM
    head's per-worker argmax reduced by the ARGMAX stage into tokens[step + 1]."""
    rng = np.random.default_rng(3)
    V = 102400
    Wemb = rt.alloc((V, H), "bf16")
    _KEEP.append(Wemb)
    rt.gen_normal_bf16(Wemb, V * H, SEED, P.fnv1a32("model.embed_tokens.weight"), 0.02)
    Wq = dev(rt, rng_bf16(rng, (Q_OUT + DC + DR, H), 0.02), "bf16")
    nw = rng_bf16(rng, H)
    dnw = dev(rt, nw, "bf16")
    tokens = np.zeros(64, np.int64)
    tokens[17] = 77777
    dtok = dev(rt, tokens, "i64")
    amax = sentinel(rt, (2 * R.WORKERS,), "f32")
    xres = sentinel(rt, (H,), "bf16")
    qkva = sentinel(rt, (Q_OUT + DC + DR,), "bf16")
    st = gemv_stage(Wq, None, qkva, H, Q_OUT + DC + DR, norm=dnw, in_kind=R.FX_IN_EMBED,
                    flags=R.FX_F_NORM | R.FX_F_WRITE_X)
    st.aux[0], st.aux[2], st.aux[3], st.aux[4] = Wemb.ptr, xres.ptr, amax.ptr, dtok.ptr
    rt.run_stage(st, step=17)
    row = Wemb.download_range(77777 * H, H)
    assert np.array_equal(xres.download(), row)
    exp, _ = O.linear(Wq.download(), row, norm_w=nw)
    assert mismatch(qkva.download(), exp) == 0
    # head: logits over a 102400-row vocabulary + argmax into tokens[step + 1]
    Wlm = rt.alloc((V, H), "bf16")
    _KEEP.append(Wlm)
    rt.gen_normal_bf16(Wlm, V * H, SEED, P.fnv1a32("lm_head.weight"), 0.02)
    logits = sentinel(rt, (V,), "bf16")
    xh = rng_bf16(rng, H)
    st = gemv_stage(Wlm, dev(rt, xh, "bf16"), logits, H, V, norm=dnw, flags=R.FX_F_NORM | R.FX_F_ARGMAX)
    st.aux[3] = amax.ptr
    rt.run_stage(st, step=17)
    exp, _ = O.linear(Wlm.download(), xh, norm_w=nw)
    got = logits.download()
    assert mismatch(got, exp) == 0
    am = R.FxStage().set(op=R.FX_OP_ARGMAX, aux={3: amax.ptr, 4: dtok.ptr})
    rt.run_stage(am, step=17)
    assert int(dtok.download()[18]) == O.argmax_bf16(exp)


def test_gemv_combine_prologue_and_standalone_combine(rt):
    rng = np.random.default_rng(4)
    x = rng_bf16(rng, H)
    out8 = rng_bf16(rng, (8, H), 0.3)
    w = np.concatenate([rng.random(6).astype(np.float32) * 0.3, np.ones(2, np.float32)])
    dx, d8, dw = dev(rt, x, "bf16"), dev(rt, out8, "bf16"), dev(rt, w, "f32")
    xo = sentinel(rt, (H,), "bf16")
    W = rng_bf16(rng, (512, H), 0.02)
    dW = dev(rt, W, "bf16")
    nw = rng_bf16(rng, H)
    out = sentinel(rt, (512,), "bf16")
    st = gemv_stage(dW, dx, out, H, 512, norm=dev(rt, nw, "bf16"), in_kind=R.FX_IN_COMBINE, n_slots=8,
                    flags=R.FX_F_NORM | R.FX_F_WRITE_X)
    st.aux[0], st.aux[1], st.aux[2] = d8.ptr, dw.ptr, xo.ptr
    rt.run_stage(st)
    comb = O.moe_combine(out8, w, x)
    assert mismatch(xo.download(), comb) == 0
    exp, _ = O.linear(W, comb, norm_w=nw)
    assert mismatch(out.download(), exp) == 0
    # the standalone form (a plan truncated after L{l}.combine), in place
    st = R.FxStage().set(op=R.FX_OP_MOE_COMBINE, n_rows=H, n_slots=8, x=dx.ptr, out=dx.ptr, aux={0: d8.ptr, 1: dw.ptr})
    rt.run_stage(st)
    assert mismatch(dx.download(), comb) == 0


def test_mla_prep(rt):
    rng = np.random.default_rng(5)
    s_max, step = 1056, 1029
    qkva = rng_bf16(rng, Q_OUT + DC + DR)
    w_kv = rng_bf16(rng, DC, 0.5)
    W_uk = rng_bf16(rng, (NH, DN, DC), 0.05)
    cos, sin = P.rope_tables(s_max)
    ckv = sentinel(rt, (s_max, DC), "bf16")
    kpe = sentinel(rt, (s_max, DR), "bf16")
    ql = sentinel(rt, (NH, DC), "bf16")
    qp = sentinel(rt, (NH, DR), "bf16")
    st = R.FxStage().set(op=R.FX_OP_MLA_PREP, n_rows=NH, d_c=DC, d_r=DR, d_n=DN, s_max=s_max, eps=1e-6,
                         x=dev(rt, qkva, "bf16").ptr, w=dev(rt, W_uk, "bf16").ptr, w_norm=dev(rt, w_kv, "bf16").ptr,
                         out=ql.ptr, aux={0: ckv.ptr, 1: kpe.ptr, 2: qp.ptr, 3: dev(rt, cos, "bf16").ptr,
                                          4: dev(rt, sin, "bf16").ptr})
    rt.run_stage(st, step=step)
    c_row, k_row, e_ql, e_qp = O.mla_prep(qkva, w_kv, W_uk, cos[step], sin[step])
    gck, gkp = ckv.download(), kpe.download()
    assert mismatch(gck[step], c_row) == 0 and mismatch(gkp[step], k_row) == 0
    assert (np.delete(gck, step, 0) == SENT16).all() and (np.delete(gkp, step, 0) == SENT16).all()
    assert mismatch(ql.download(), e_ql) == 0
    assert mismatch(qp.download(), e_qp) == 0


@pytest.mark.parametrize("s_max,step,split", [(1056, 1023, 32), (1056, 1040, 32), (4096, 4095, 128), (300, 40, 32),
                                              (32768, 32767, 1024)])
def test_mla_attend_merge_uv(rt, s_max, step, split):
    print(f"[attend] s_max={s_max} step={step} split={split}", flush=True)
    rng = np.random.default_rng(s_max + step)
    n_splits = -(-s_max // split)
    prow = partials_row(DC)
    ql, qp = rng_bf16(rng, (NH, DC)), rng_bf16(rng, (NH, DR))
    ck, kp = rng_bf16(rng, (s_max, DC)), rng_bf16(rng, (s_max, DR))
    scale = float(np.float32(1 / np.sqrt(192)))
    part = sentinel(rt, (n_splits, NH, prow), "f32")
    om = sentinel(rt, (NH, DC), "bf16")
    st = R.FxStage().set(op=R.FX_OP_MLA_ATTEND, n_rows=NH, d_c=DC, d_r=DR, d_n=DN, split=split, n_splits=n_splits,
                         prow=prow, s_max=s_max, scale=scale, x=dev(rt, ql, "bf16").ptr, out=part.ptr,
                         aux={0: dev(rt, ck, "bf16").ptr, 1: dev(rt, kp, "bf16").ptr, 2: dev(rt, qp, "bf16").ptr,
                              4: om.ptr})
    rt.run_stage(st, step=step)
    exp = O.mla_attend(ql, qp, ck, kp, step, scale, split=split, n_splits=n_splits)
    got = part.download()
    assert mismatch(got[:, :, :DC + 1], exp[:, :, :DC + 1]) == 0
    W_uv = rng_bf16(rng, (NH, DN, DC), 0.05)
    e_attn, e_obf = O.mla_merge_uv(exp, W_uv, step, split=split)
    assert mismatch(om.download(), e_obf) == 0
    attn = sentinel(rt, (NH * DN,), "bf16")
    st = R.FxStage().set(op=R.FX_OP_MLA_MERGE_UV, n_rows=NH, d_c=DC, d_r=DR, d_n=DN, x=om.ptr,
                         w=dev(rt, W_uv, "bf16").ptr, out=attn.ptr)
    rt.run_stage(st, step=step)
    assert mismatch(attn.download(), e_attn) == 0


def test_router_experts(rt):
    """router (per XCD) -> w13 + SiLU (expert of slot = XCD) -> w2, against the oracle's moe_router,
    moe_w13_silu and moe_w2 on the selected experts' slabs (66 experts generated on the device)."""
    rng = np.random.default_rng(6)
    d = P.REAL_DIMS
    I, E = d.I_MOE, d.E
    lay = P.seeded_layout(d, layers=2, head=False)
    bufs = P.fill_seeded(rt, d, SEED, layers=2, head=False, keys={"W_gate_1", "W13_1", "W2_1"})
    _KEEP.extend(bufs.values())
    x = rng_bf16(rng, H)
    nw = rng_bf16(rng, H, 0.5)
    dx, dn = dev(rt, x, "bf16"), dev(rt, nw, "bf16")
    lx = sentinel(rt, (8, E), "f32")
    rt.run_stage(R.FxStage().set(op=R.FX_OP_MOE_ROUTER, n_rows=E, k=H, topk=d.TOPK, eps=1e-6, x=dx.ptr, w_norm=dn.ptr,
                                 w=bufs["W_gate_1"].ptr, out=lx.ptr))
    Wg = bufs["W_gate_1"].download()
    h, logits, topk_w, routing, mask = O.moe_router(x, Wg, norm_w=nw)
    glx = lx.download()
    for xc in range(d.TOPK):
        assert mismatch(glx[xc], logits) == 0
    outs = {n: sentinel(rt, s, t) for n, s, t in [("act8", (8, I), "bf16"), ("topk_w", (8,), "f32"),
                                                  ("routing", (E + 2,), "i32"), ("mask", (E + 3,), "i32"),
                                                  ("logits", (E,), "f32"), ("h", (H,), "bf16"), ("sel", (8,), "i32"),
                                                  ("route_log", (4, 26, 8), "i32")]}
    st = R.FxStage().set(op=R.FX_OP_MOE_W13, n_rows=I, k=H, n_slots=8, topk=d.TOPK, n_forced=2, scaling=1.0,
                         aux_i0=E, aux_i1=26, prow=4, layer=1, eps=1e-6, x=dx.ptr, w_norm=dn.ptr,
                         w=bufs["W13_1"].ptr, out=outs["act8"].ptr,
                         aux={0: lx.ptr, 1: outs["topk_w"].ptr, 2: outs["routing"].ptr, 3: outs["mask"].ptr,
                              4: outs["logits"].ptr, 5: outs["route_log"].ptr, 6: outs["h"].ptr, 7: outs["sel"].ptr})
    rt.run_stage(st)
    assert mismatch(outs["h"].download(), h) == 0
    assert mismatch(outs["logits"].download(), logits) == 0
    assert mismatch(outs["topk_w"].download(), topk_w) == 0
    assert np.array_equal(outs["routing"].download(), routing)
    assert np.array_equal(outs["mask"].download(), mask)
    assert np.array_equal(outs["sel"].download(), mask[:8])
    ids = [int(e) for e in mask[:8]]
    W13 = np.stack([bufs["W13_1"].download_range(e * 2 * I * H, 2 * I * H).reshape(2 * I, H) for e in ids])
    W2 = np.stack([bufs["W2_1"].download_range(e * H * I, H * I).reshape(H, I) for e in ids])
    local = np.arange(9, dtype=np.int32)
    e_act = O.moe_w13_silu(h, W13, local, 8)
    assert mismatch(outs["act8"].download(), e_act) == 0
    out8 = sentinel(rt, (8, H), "bf16")
    rt.run_stage(R.FxStage().set(op=R.FX_OP_MOE_W2, n_rows=H, k=I, x=outs["act8"].ptr, w=bufs["W2_1"].ptr,
                                 out=out8.ptr, aux={7: outs["sel"].ptr}))
    assert mismatch(out8.download(), O.moe_w2(e_act, W2, local, 8)) == 0
    # the generator that filled W13 / W2 on the device equals the CPU generator on these slabs
    from fxtest import cpu_gen
    pt = lay["W13_1"]
    for e in (ids[0], 64, 65):
        segs = P.expert_segments(pt, e, 2 * I * H)
        cpu = P.materialize(pt, SEED, cpu_gen, segs, (2 * I, H))
        assert np.array_equal(cpu, bufs["W13_1"].download_range(e * 2 * I * H, 2 * I * H).reshape(2 * I, H))
    pt = lay["W2_1"]
    for e in (65,):
        segs = P.expert_segments(pt, e, H * I)
        cpu = P.materialize(pt, SEED, cpu_gen, segs, (H, I))
        assert np.array_equal(cpu, bufs["W2_1"].download_range(e * H * I, H * I).reshape(H, I))


def test_dense_gate_up(rt):
    rng = np.random.default_rng(7)
    d = P.REAL_DIMS
    Id = d.I_DENSE
    x = rng_bf16(rng, H)
    nw = rng_bf16(rng, H, 0.5)
    bufs = P.fill_seeded(rt, d, SEED, layers=1, head=False, keys={"W_gu_0", "W_down_0"})
    _KEEP.extend(bufs.values())
    act = sentinel(rt, (Id,), "bf16")
    hb = sentinel(rt, (H,), "bf16")
    rt.run_stage(R.FxStage().set(op=R.FX_OP_DENSE_GU, n_rows=Id, k=H, eps=1e-6, x=dev(rt, x, "bf16").ptr,
                                 w_norm=dev(rt, nw, "bf16").ptr, w=bufs["W_gu_0"].ptr, out=act.ptr, aux={6: hb.ptr}))
    Wgu, Wd = bufs["W_gu_0"].download(), bufs["W_down_0"].download()
    h, e_act, e_out = O.dense_mlp(x, nw, Wgu, Wd)
    assert mismatch(hb.download(), h) == 0
    assert mismatch(act.download(), e_act) == 0


def test_generator_matches_cpu(rt):
    """fx_gen_normal_bf16 (contiguous and strided forms) equals the oracle's generator bit for bit."""
    b = rt.alloc((100003,), "bf16")
    _KEEP.append(b)
    rt.gen_normal_bf16(b, 100003, 7, 12345, 0.02, src_offset=5)
    assert np.array_equal(b.download(), O.gen_normal_bf16(7, 12345, 100003, 0.02, offset=5))
    s = rt.alloc((64, 1408), "bf16")
    _KEEP.append(s)
    rt.gen_normal_bf16(s, 64 * 1408, 7, 999, 1.0, src_offset=1408, rows=64, row_len=1408, dst_stride=1408,
                       src_stride=2816)
    exp = np.stack([O.gen_normal_bf16(7, 999, 1408, 1.0, offset=1408 + r * 2816) for r in range(64)])
    assert np.array_equal(s.download(), exp)
