"""Per-operator parity on the GPU: every stage of the task table, launched alone through the C ABI
(fx_run_stage: the kernel-suite entry, the counterpart of fleet/tasks/kernel_tests_mi300.cu), against
the CPU oracle on the same inputs at the real shapes. The bar is bit-exact: both sides follow the
same FP32 spec (fixed summation orders, own exp/log), so any differing element is a failure.

Packet inputs are written with the tag the stage expects (tbase + src + 1) and every packet output
must come back with the stage's own tag (tbase + sidx + 1), which also catches a packet the stage
failed to write. Plain outputs are prefilled with a sentinel (0xFFFF / NaN) to catch stray or
missing writes, as the reference suite does (fleet/tasks/kernel_tests.py:54-59)."""
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
TB, SIDX, SRC = 1000, 5, 4          # inputs tagged TB + SRC + 1 = TIN, outputs TB + SIDX + 1 = TOUT
TIN, TOUT = TB + SRC + 1, TB + SIDX + 1


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


def pk(rt, values, dtype="pk16", tag=TIN):
    """A packet tensor holding `values` with `tag`."""
    b = rt.alloc(values.shape, dtype)
    b.upload_packets(values, tag)
    _KEEP.append(b)
    return b


def pk_out(rt, shape, dtype="pk16"):
    b = rt.alloc(shape, dtype).zero()
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


def gemv_stage(W, x, out, K, N, norm=None, res=None, eps=1e-6, flags=0, **kw):
    st = R.FxStage().set(op=R.FX_OP_GEMV, n_rows=N, k=K, w=W.ptr, x=x.ptr if x is not None else 0, out=out.ptr,
                         eps=eps, src=[SRC, SRC, SRC, SRC])
    if norm is not None:
        flags |= R.FX_F_NORM
        st.w_norm = norm.ptr
    if res is not None:
        flags |= R.FX_F_RESIDUAL
        st.res = res.ptr
    if out.dtype == "pk16":
        flags |= R.FX_F_OUT_LL
    st.flags = flags
    for k, v in kw.items():
        setattr(st, k, v)
    return st


@pytest.mark.parametrize("N,K,norm,res,ll", [(3648, 2048, True, False, True), (2048, 2048, False, True, True),
                                             (2048, 10944, False, True, True), (256, 512, False, False, True),
                                             (1000, 1408, True, False, False)])
def test_gemv_forms(rt, N, K, norm, res, ll):
    print(f"[gemv] N={N} K={K} norm={norm} res={res} packets={ll}", flush=True)
    rng = np.random.default_rng(N + K)
    W = rng_bf16(rng, (N, K), 0.02)
    x = rng_bf16(rng, K)
    nw = rng_bf16(rng, K, 0.5) if norm else None
    r = rng_bf16(rng, N) if res else None
    dW, dx = dev(rt, W, "bf16"), pk(rt, x)
    dn = dev(rt, nw, "bf16") if norm else None
    dr = pk(rt, r) if res else None
    out = pk_out(rt, (N,)) if ll else sentinel(rt, (N,), "bf16")
    rt.run_stage(gemv_stage(dW, dx, out, K, N, norm=dn, res=dr), tbase=TB, sidx=SIDX)
    exp, _ = O.linear(W, x, norm_w=nw, res=r)
    got = out.download(tag=TOUT) if ll else out.download()
    assert mismatch(got, exp) == 0


def test_gemv_embed_residual_and_head_argmax(rt):
    """L0.qkva's embedding prologue (token from tokens[step]), L0.o_proj's embedding-row residual,
    and the LM head's per-worker argmax reduced by the ARGMAX stage into tokens[step + 1]."""
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
    amax = pk_out(rt, (2 * R.WORKERS,), "pk32")
    qkva = pk_out(rt, (Q_OUT + DC + DR,))
    st = gemv_stage(Wq, None, qkva, H, Q_OUT + DC + DR, norm=dnw, in_kind=R.FX_IN_EMBED)
    st.aux[0], st.aux[3], st.aux[4] = Wemb.ptr, amax.ptr, dtok.ptr
    rt.run_stage(st, step=17, tbase=TB, sidx=SIDX)
    row = Wemb.download_range(77777 * H, H)
    exp, _ = O.linear(Wq.download(), row, norm_w=nw)
    assert mismatch(qkva.download(tag=TOUT), exp) == 0
    # o_proj of layer 0: residual = the embedding row of the token
    Wo = rng_bf16(rng, (H, H), 0.02)
    attn = rng_bf16(rng, H)
    xo = pk_out(rt, (H,))
    st = gemv_stage(dev(rt, Wo, "bf16"), pk(rt, attn), xo, H, H, flags=R.FX_F_RES_EMBED)
    st.aux[0], st.aux[4] = Wemb.ptr, dtok.ptr
    rt.run_stage(st, step=17, tbase=TB, sidx=SIDX)
    exp, _ = O.linear(Wo, attn, res=row)
    assert mismatch(xo.download(tag=TOUT), exp) == 0
    # head: logits over a 102400-row vocabulary + argmax into tokens[step + 1]
    Wlm = rt.alloc((V, H), "bf16")
    _KEEP.append(Wlm)
    rt.gen_normal_bf16(Wlm, V * H, SEED, P.fnv1a32("lm_head.weight"), 0.02)
    logits = sentinel(rt, (V,), "bf16")
    xh = rng_bf16(rng, H)
    st = gemv_stage(Wlm, pk(rt, xh), logits, H, V, norm=dnw, flags=R.FX_F_ARGMAX)
    st.aux[3] = amax.ptr
    rt.run_stage(st, step=17, tbase=TB, sidx=SIDX)
    exp, _ = O.linear(Wlm.download(), xh, norm_w=nw)
    assert mismatch(logits.download(), exp) == 0
    am = amax.download(tag=TOUT).reshape(R.WORKERS, 2)
    assert float(am[:, 0].max()) == float(O.bf16_to_f32(exp).max())
    st = R.FxStage().set(op=R.FX_OP_ARGMAX, aux={3: amax.ptr, 4: dtok.ptr}, src=[SIDX, 0, 0, 0])
    rt.run_stage(st, step=17, tbase=TB, sidx=SIDX + 1)
    assert int(dtok.download()[18]) == O.argmax_bf16(exp)


def test_mla_prep(rt):
    rng = np.random.default_rng(5)
    s_max, step = 1056, 1029
    qkva = rng_bf16(rng, Q_OUT + DC + DR)
    w_kv = rng_bf16(rng, DC, 0.5)
    W_uk = rng_bf16(rng, (NH, DN, DC), 0.05)
    cos, sin = P.rope_tables(s_max)
    ckv = sentinel(rt, (s_max, DC), "bf16")
    kpe = sentinel(rt, (s_max, DR), "bf16")
    ql = pk_out(rt, (NH, DC))
    qp = pk_out(rt, (NH, DR))
    crow = pk_out(rt, (8, DC + DR))
    st = R.FxStage().set(op=R.FX_OP_MLA_PREP, n_rows=NH, d_c=DC, d_r=DR, d_n=DN, s_max=s_max, eps=1e-6,
                         x=pk(rt, qkva).ptr, w=dev(rt, W_uk, "bf16").ptr, w_norm=dev(rt, w_kv, "bf16").ptr,
                         out=ql.ptr, aux={0: ckv.ptr, 1: kpe.ptr, 2: qp.ptr, 3: dev(rt, cos, "bf16").ptr,
                                          4: dev(rt, sin, "bf16").ptr, 5: crow.ptr}, src=[SRC, 0, 0, 0])
    rt.run_stage(st, step=step, tbase=TB, sidx=SIDX)
    c_row, k_row, e_ql, e_qp = O.mla_prep(qkva, w_kv, W_uk, cos[step], sin[step])
    gck, gkp = ckv.download(), kpe.download()
    assert mismatch(gck[step], c_row) == 0 and mismatch(gkp[step], k_row) == 0
    assert (np.delete(gck, step, 0) == SENT16).all() and (np.delete(gkp, step, 0) == SENT16).all()
    assert mismatch(ql.download(tag=TOUT), e_ql) == 0
    assert mismatch(qp.download(tag=TOUT), e_qp) == 0
    row = np.concatenate([c_row, k_row])
    assert mismatch(crow.download(tag=TOUT), np.tile(row, (8, 1))) == 0


ATTEND_POINTS = [(1056, 1023, 32), (1056, 1040, 32), (1056, 1024, 64), (4096, 4095, 128), (300, 40, 32), (64, 0, 32),
                 (32768, 32767, 1024), (16416, 16383, 160),
                 (8192, 4127, 32)]                  # 129 live splits: the merge's lse beyond 128 splits
MFMA_POINTS = [(16416, 16383, 96),                  # 171 live splits, the sliced merge's most
               (16416, 16383, 128),                 # exactly 128 live splits
               (16416, 16384, 128),                 # its next token: 129
               (8192, 8191, 32),                    # 256 live splits, one per worker
               (8448, 8447, 32)]                    # 264: workers 0..7 run two splits


@pytest.mark.parametrize("attn,s_max,step,split", [("valu",) + p for p in ATTEND_POINTS] +
                         [("mfma",) + p for p in ATTEND_POINTS + MFMA_POINTS])
def test_mla_attend_merge_uv(rt, attn, s_max, step, split):
    print(f"[attend] attn={attn} s_max={s_max} step={step} split={split}", flush=True)
    mfma = attn == "mfma"
    rng = np.random.default_rng(s_max + step)
    n_splits = -(-s_max // split)
    live = -(-(step + 1) // split)
    prow = partials_row(DC)
    ql, qp = rng_bf16(rng, (NH, DC)), rng_bf16(rng, (NH, DR))
    ck, kp = rng_bf16(rng, (s_max, DC)), rng_bf16(rng, (s_max, DR))
    scale = float(np.float32(1 / np.sqrt(192)))
    # the caches hold garbage at `step`: the kernel must take that row from the crow packets
    ckd, kpd = ck.copy(), kp.copy()
    ckd[step] = SENT16
    kpd[step] = SENT16
    crow = pk(rt, np.tile(np.concatenate([ck[step], kp[step]]), (8, 1)))
    part = sentinel(rt, (n_splits, NH, prow), "f32")
    done = pk_out(rt, (8, 32), "pk32")
    flags = R.FX_F_MFMA if mfma else 0
    st = R.FxStage().set(op=R.FX_OP_MLA_ATTEND, flags=flags, n_rows=NH, d_c=DC, d_r=DR, d_n=DN, split=split,
                         n_splits=n_splits, prow=prow, s_max=s_max, scale=scale, x=pk(rt, ql).ptr, out=part.ptr,
                         aux={0: dev(rt, ckd, "bf16").ptr, 1: dev(rt, kpd, "bf16").ptr, 2: pk(rt, qp).ptr,
                              5: crow.ptr, 6: done.ptr}, src=[SRC, 0, 0, 0])
    rt.run_stage(st, step=step, tbase=TB, sidx=SIDX)
    attend = O.mla_attend_mfma if mfma else O.mla_attend
    exp = attend(ql, qp, ck, kp, step, scale, split=split, n_splits=n_splits)
    got = part.download()
    bad = mismatch(got[:live, :, :DC + 1], exp[:live, :, :DC + 1])
    if bad:
        d = np.argwhere(got[:live, :, :DC + 1].view(np.uint32) != exp[:live, :, :DC + 1].view(np.uint32))
        print(f"[attend] {bad} partials differ, first (split, head, col) {d[:6].tolist()}", flush=True)
    assert bad == 0
    if mfma:
        # one done packet per worker that owned a live split (split j on worker j % 256)
        nown = min(live, 256)
        words = done.download_raw()
        vals, tags = R.unpack_packets(words, "pk32")
        assert (tags[:nown] == TOUT).all() and (tags[nown:] == 0).all()
        assert int(vals[:nown].view(np.uint32).sum()) == live
    else:
        counts = done.download(tag=TOUT).view(np.uint32).reshape(8, 32)
        assert (counts.sum(axis=1) == live).all()
    # merge + W_uv: inputs tagged TOUT (src = SIDX with the same tbase), outputs TB + SIDX + 2
    W_uv = rng_bf16(rng, (NH, DN, DC), 0.05)
    e_attn, e_obf = O.mla_merge_uv(exp, W_uv, step, split=split)
    attn = pk_out(rt, (NH * DN,))
    om = sentinel(rt, (NH, DC), "bf16")
    # the matrix-core merge takes the slice-exchange packets (used from 9 to 176 live splits: each of
    # a head's 8 workers merges 64 columns)
    slices = pk_out(rt, (NH, DC)) if mfma else None
    aux = {4: om.ptr, 6: done.ptr}
    if mfma:
        aux[7] = slices.ptr
    st = R.FxStage().set(op=R.FX_OP_MLA_MERGE_UV, flags=flags, n_rows=NH, d_c=DC, d_r=DR, d_n=DN, split=split,
                         n_splits=n_splits,
                         prow=prow, x=part.ptr, w=dev(rt, W_uv, "bf16").ptr, out=attn.ptr,
                         aux=aux, src=[SIDX, 0, 0, 0])
    rt.run_stage(st, step=step, tbase=TB, sidx=SIDX + 1)
    assert mismatch(om.download(), e_obf) == 0
    assert mismatch(attn.download(tag=TOUT + 1), e_attn) == 0
    if mfma and 8 < live <= 176:
        # the exchanged slices are the merged o of every head, tagged by the merge stage
        assert mismatch(slices.download(tag=TOUT + 1).reshape(NH, DC), e_obf) == 0


XCD_POINTS = [(1056, 1023, 32),                     # 32 live splits: one per rank of the XCD
              (1056, 1040, 32),                     # 33: rank 0 runs two
              (8192, 4127, 32)]                     # 129: four or five per rank, lse beyond 128 splits


@pytest.mark.parametrize("s_max,step,split", ATTEND_POINTS + XCD_POINTS)
def test_mla_attend_merge_xcd(rt, s_max, step, split):
    """The single-XCD matrix-core attention and its merge in one stage (FX_F_XCD on the merge): the
    partials, the done packets of XCD 7's ranks, o_merged and attn, against the oracle's matrix-core
    attention and merge + W_uv."""
    print(f"[attend-xcd] s_max={s_max} step={step} split={split}", flush=True)
    rng = np.random.default_rng(s_max + step + 7)
    n_splits = -(-s_max // split)
    live = -(-(step + 1) // split)
    prow = partials_row(DC)
    ql, qp = rng_bf16(rng, (NH, DC)), rng_bf16(rng, (NH, DR))
    ck, kp = rng_bf16(rng, (s_max, DC)), rng_bf16(rng, (s_max, DR))
    scale = float(np.float32(1 / np.sqrt(192)))
    ckd, kpd = ck.copy(), kp.copy()
    ckd[step] = SENT16
    kpd[step] = SENT16
    crow = pk(rt, np.tile(np.concatenate([ck[step], kp[step]]), (8, 1)))
    part = sentinel(rt, (n_splits, NH, prow), "f32")
    done = pk_out(rt, (8, 32), "pk32")
    W_uv = rng_bf16(rng, (NH, DN, DC), 0.05)
    attn = pk_out(rt, (NH * DN,))
    om = sentinel(rt, (NH, DC), "bf16")
    st = R.FxStage().set(op=R.FX_OP_MLA_MERGE_UV, flags=R.FX_F_XCD, n_rows=NH, d_c=DC, d_r=DR, d_n=DN, split=split,
                         n_splits=n_splits, prow=prow, s_max=s_max, scale=scale, x=part.ptr,
                         w=dev(rt, W_uv, "bf16").ptr, out=attn.ptr,
                         aux={0: dev(rt, ckd, "bf16").ptr, 1: dev(rt, kpd, "bf16").ptr, 2: pk(rt, qp).ptr,
                              3: pk(rt, ql).ptr, 4: om.ptr, 5: crow.ptr, 6: done.ptr}, src=[SRC, 0, 0, 0])
    rt.run_stage(st, step=step, tbase=TB, sidx=SIDX)
    exp = O.mla_attend_mfma(ql, qp, ck, kp, step, scale, split=split, n_splits=n_splits)
    got = part.download()
    bad = mismatch(got[:live, :, :DC + 1], exp[:live, :, :DC + 1])
    if bad:
        d = np.argwhere(got[:live, :, :DC + 1].view(np.uint32) != exp[:live, :, :DC + 1].view(np.uint32))
        print(f"[attend-xcd] {bad} partials differ, first (split, head, col) {d[:6].tolist()}", flush=True)
    assert bad == 0
    # one done packet per rank that owned a live split (split j on rank j % 32), split counts summing to live
    nown = min(live, 32)
    vals, tags = R.unpack_packets(done.download_raw(), "pk32")
    assert (tags[:nown] == TOUT).all() and (tags[nown:] == 0).all()
    assert int(vals[:nown].view(np.uint32).sum()) == live
    e_attn, e_obf = O.mla_merge_uv(exp, W_uv, step, split=split)
    assert mismatch(om.download(), e_obf) == 0
    assert mismatch(attn.download(tag=TOUT), e_attn) == 0


def test_router_experts_combine(rt):
    """router (row e on worker e) -> w13 + SiLU (slot = XCD) -> w2 + combine (8 rows per worker, all
    slots), against the oracle's moe_router, moe_w13_silu, moe_w2 and moe_combine on the selected
    experts' slabs (66 experts generated on the device)."""
    rng = np.random.default_rng(6)
    d = P.REAL_DIMS
    I, E = d.I_MOE, d.E
    lay = P.seeded_layout(d, layers=2, head=False)
    bufs = P.fill_seeded(rt, d, SEED, layers=2, head=False, keys={"W_gate_1", "W13_1", "W2_1"})
    _KEEP.extend(bufs.values())
    x = rng_bf16(rng, H)
    nw = rng_bf16(rng, H, 0.5)
    dx, dn = pk(rt, x), dev(rt, nw, "bf16")
    lx = pk_out(rt, (E,), "pk32")
    rt.run_stage(R.FxStage().set(op=R.FX_OP_MOE_ROUTER, n_rows=E, k=H, topk=d.TOPK, eps=1e-6, x=dx.ptr, w_norm=dn.ptr,
                                 w=bufs["W_gate_1"].ptr, out=lx.ptr, src=[SRC, 0, 0, 0]), tbase=TB, sidx=SIDX)
    Wg = bufs["W_gate_1"].download()
    h, logits, topk_w, routing, mask = O.moe_router(x, Wg, norm_w=nw)
    assert mismatch(lx.download(tag=TOUT), logits) == 0
    outs = {n: sentinel(rt, s, t) for n, s, t in [("topk_w", (8,), "f32"), ("routing", (E + 2,), "i32"),
                                                  ("mask", (E + 3,), "i32"), ("logits", (E,), "f32"),
                                                  ("h", (H,), "bf16"), ("sel", (8,), "i32"),
                                                  ("route_log", (4, 26, 8), "i32")]}
    act8 = pk_out(rt, (8, I))
    # w13: logits tagged TOUT (src SIDX), x tagged TIN (src SRC); outputs TB + SIDX + 2
    st = R.FxStage().set(op=R.FX_OP_MOE_W13, n_rows=I, k=H, n_slots=8, topk=d.TOPK, n_forced=2, scaling=1.0,
                         aux_i0=E, aux_i1=26, prow=4, layer=1, eps=1e-6, x=dx.ptr, w_norm=dn.ptr,
                         w=bufs["W13_1"].ptr, out=act8.ptr, src=[SIDX, SRC, 0, 0],
                         aux={0: lx.ptr, 1: outs["topk_w"].ptr, 2: outs["routing"].ptr, 3: outs["mask"].ptr,
                              4: outs["logits"].ptr, 5: outs["route_log"].ptr, 6: outs["h"].ptr, 7: outs["sel"].ptr})
    rt.run_stage(st, tbase=TB, sidx=SIDX + 1)
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
    assert mismatch(act8.download(tag=TOUT + 1), e_act) == 0
    # the same stage with the router folded in (FX_F_ROUTER): logits computed and read back in-stage
    lxb, act8b = pk_out(rt, (E,), "pk32"), pk_out(rt, (8, I))
    st.flags = R.FX_F_ROUTER
    st.res = bufs["W_gate_1"].ptr
    st.aux[0], st.out = lxb.ptr, act8b.ptr
    st.src[0] = 0
    rt.run_stage(st, tbase=TB, sidx=SIDX + 1)
    assert mismatch(lxb.download(tag=TOUT + 1), logits) == 0
    assert mismatch(act8b.download(tag=TOUT + 1), e_act) == 0
    assert np.array_equal(outs["sel"].download(), mask[:8])
    # w2 + combine: act8 (src SIDX + 1), logits (src SIDX), residual x (src SRC); outputs TB + SIDX + 3
    out8 = sentinel(rt, (8, H), "bf16")
    xn = pk_out(rt, (H,))
    rt.run_stage(R.FxStage().set(op=R.FX_OP_MOE_W2, n_rows=H, k=I, n_slots=8, topk=d.TOPK, n_forced=2, scaling=1.0,
                                 aux_i0=E, x=act8.ptr, w=bufs["W2_1"].ptr, res=dx.ptr, out=xn.ptr,
                                 aux={0: lx.ptr, 1: out8.ptr}, src=[SIDX + 1, SIDX, SRC, 0]), tbase=TB, sidx=SIDX + 2)
    e_out8 = O.moe_w2(e_act, W2, local, 8)
    assert mismatch(out8.download(), e_out8) == 0
    assert mismatch(xn.download(tag=TOUT + 2), O.moe_combine(e_out8, topk_w, x)) == 0
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


@pytest.mark.parametrize("I", [512, 1024, 1400])
def test_expert_gate_up_walk_lengths(rt, I):
    """The expert gate|up stage at other intermediate sizes, over the same seeded expert buffer cut
    into experts of 2 I rows: the routed walk of a worker then has 6 (I = 512: three pair tiles per
    wave, the walk's tail only), 12 (I = 1,024: one rolling round and the tail) or 16-17 (I = 1,400:
    the rolling loop, and the leftover group split by rows) groups instead of the real 16-17 at I =
    1,408, and the shared walk 2, 4 or 5-6. Bit-exact against the oracle's moe_w13_silu on the same
    slabs and routing."""
    rng = np.random.default_rng(16)
    d = P.REAL_DIMS
    E = d.E
    print(f"[w13 walk] I={I}", flush=True)
    bufs = P.fill_seeded(rt, d, SEED, layers=2, head=False, keys={"W_gate_1", "W13_1"})
    _KEEP.extend(bufs.values())
    x = rng_bf16(rng, H)
    nw = rng_bf16(rng, H, 0.5)
    dx, dn = pk(rt, x), dev(rt, nw, "bf16")
    h, logits, topk_w, routing, mask = O.moe_router(x, bufs["W_gate_1"].download(), norm_w=nw)
    lx = pk(rt, logits, "pk32", tag=TOUT)
    outs = {n: sentinel(rt, sh, t) for n, sh, t in [("topk_w", (8,), "f32"), ("routing", (E + 2,), "i32"),
                                                   ("mask", (E + 3,), "i32"), ("logits", (E,), "f32")]}
    act8 = pk_out(rt, (8, I))
    st = R.FxStage().set(op=R.FX_OP_MOE_W13, n_rows=I, k=H, n_slots=8, topk=d.TOPK, n_forced=2, scaling=1.0,
                         aux_i0=E, aux_i1=26, prow=4, layer=1, eps=1e-6, x=dx.ptr, w_norm=dn.ptr,
                         w=bufs["W13_1"].ptr, out=act8.ptr, src=[SIDX, SRC, 0, 0],
                         aux={0: lx.ptr, 1: outs["topk_w"].ptr, 2: outs["routing"].ptr, 3: outs["mask"].ptr,
                              4: outs["logits"].ptr})
    rt.run_stage(st, tbase=TB, sidx=SIDX + 1)
    assert np.array_equal(outs["mask"].download(), mask)
    ids = [int(e) for e in mask[:8]]
    W13 = np.stack([bufs["W13_1"].download_range(e * 2 * I * H, 2 * I * H).reshape(2 * I, H) for e in ids])
    e_act = O.moe_w13_silu(h, W13, np.arange(9, dtype=np.int32), 8)
    assert mismatch(act8.download(tag=TOUT + 1), e_act) == 0


def test_dense_gate_up(rt):
    rng = np.random.default_rng(7)
    d = P.REAL_DIMS
    Id = d.I_DENSE
    x = rng_bf16(rng, H)
    nw = rng_bf16(rng, H, 0.5)
    bufs = P.fill_seeded(rt, d, SEED, layers=1, head=False, keys={"W_gu_0", "W_down_0"})
    _KEEP.extend(bufs.values())
    act = pk_out(rt, (Id,))
    hb = sentinel(rt, (H,), "bf16")
    rt.run_stage(R.FxStage().set(op=R.FX_OP_DENSE_GU, n_rows=Id, k=H, eps=1e-6, x=pk(rt, x).ptr,
                                 w_norm=dev(rt, nw, "bf16").ptr, w=bufs["W_gu_0"].ptr, out=act.ptr, aux={6: hb.ptr},
                                 src=[SRC, 0, 0, 0]), tbase=TB, sidx=SIDX)
    Wgu, Wd = bufs["W_gu_0"].download(), bufs["W_down_0"].download()
    h, e_act, e_out = O.dense_mlp(x, nw, Wgu, Wd)
    assert mismatch(hb.download(), h) == 0
    assert mismatch(act.download(tag=TOUT), e_act) == 0


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
