"""The allocation-free attention entry (fx_mla_attend_merge_noalloc) against the kernel-suite path it
varies (fx_run_stage of the attend stage, then of the merge stage, with caller-owned partials and
done buffers): the merged o and the W_uv output bit for bit, on two calls in a row -- the second
with a smaller input, so stale partials and done packets of the first call would show -- for both
attention kernels. Also: a plan with more splits than the scratch holds is refused."""
import numpy as np
import pytest

from fleet import runtime as R
from fleet.graph_plan import partials_row
from fxtest import rng_bf16, mismatch

pytestmark = pytest.mark.gpu

NH, DC, DR, DN = 16, 512, 64, 128
TB, SIDX, SRC = 2000, 5, 4
TIN, TOUT = TB + SRC + 1, TB + SIDX + 1


def _inputs(rt, keep, s_max, step, split, seed):
    rng = np.random.default_rng(seed)
    n_splits = -(-s_max // split)
    ql, qp = rng_bf16(rng, (NH, DC)), rng_bf16(rng, (NH, DR))
    ck, kp = rng_bf16(rng, (s_max, DC)), rng_bf16(rng, (s_max, DR))
    W_uv = rng_bf16(rng, (NH, DN, DC), 0.05)

    def dev(a, dt):
        b = rt.alloc(a.shape, dt)
        b.upload(a)
        keep.append(b)
        return b

    def pkt(v):
        b = rt.alloc(v.shape, "pk16")
        b.upload_packets(v, TIN)
        keep.append(b)
        return b

    crow = pkt(np.tile(np.concatenate([ck[step], kp[step]]), (8, 1)))
    return dict(n_splits=n_splits, q=pkt(ql), qp=pkt(qp), ck=dev(ck, "bf16"), kp=dev(kp, "bf16"), crow=crow,
                W=dev(W_uv, "bf16"))


def _stages(inp, s_max, split, flags, part, done, attn, om):
    prow = partials_row(DC)
    a = R.FxStage().set(op=R.FX_OP_MLA_ATTEND, flags=flags, n_rows=NH, d_c=DC, d_r=DR, d_n=DN, split=split,
                        n_splits=inp["n_splits"], prow=prow, s_max=s_max, scale=float(np.float32(1 / np.sqrt(192))),
                        x=inp["q"].ptr, out=part, aux={0: inp["ck"].ptr, 1: inp["kp"].ptr, 2: inp["qp"].ptr,
                                                       5: inp["crow"].ptr, 6: done}, src=[SRC, 0, 0, 0])
    m = R.FxStage().set(op=R.FX_OP_MLA_MERGE_UV, flags=flags, n_rows=NH, d_c=DC, d_r=DR, d_n=DN, split=split,
                        n_splits=inp["n_splits"], prow=prow, x=part, w=inp["W"].ptr, out=attn.ptr,
                        aux={4: om.ptr, 6: done}, src=[SIDX, 0, 0, 0])
    if flags & R.FX_F_XCD:
        # the single-XCD merge runs the attention itself: its operands, and the prep as its source
        m.set(s_max=s_max, scale=a.scale, aux={0: inp["ck"].ptr, 1: inp["kp"].ptr, 2: inp["qp"].ptr, 3: inp["q"].ptr,
                                               4: om.ptr, 5: inp["crow"].ptr, 6: done}, src=[SRC, 0, 0, 0])
    return a, m


@pytest.mark.parametrize("attn", ["mfma", "xcd", "valu"])
def test_noalloc_attention_matches_the_kernel_suite_path(rt, attn):
    flags = {"mfma": R.FX_F_MFMA, "xcd": R.FX_F_XCD, "valu": 0}[attn]
    keep = []
    # two calls in a row on the same GPU: a large one, then a smaller one
    for s_max, step, split, seed in ((1056, 1023, 32, 1), (300, 40, 32, 2)):
        print(f"[noalloc] attn={attn} s_max={s_max} step={step} split={split}", flush=True)
        inp = _inputs(rt, keep, s_max, step, split, seed)
        # the existing path: caller-owned partials and done packets
        part = rt.alloc((inp["n_splits"], NH, partials_row(DC)), "f32").zero()
        done = rt.alloc((256,), "pk32").zero()
        attn_ref = rt.alloc((NH * DN,), "pk16").zero()
        om_ref = rt.alloc((NH, DC), "bf16").zero()
        keep += [part, done, attn_ref, om_ref]
        a, m = _stages(inp, s_max, split, flags, part.ptr, done.ptr, attn_ref, om_ref)
        rt.run_stage(a, step=step, tbase=TB, sidx=SIDX)
        rt.run_stage(m, step=step, tbase=TB, sidx=SIDX + 1)
        # the allocation-free entry: partials / done pointers of the stages are ignored (null here)
        attn_na = rt.alloc((NH * DN,), "pk16").zero()
        om_na = rt.alloc((NH, DC), "bf16").zero()
        keep += [attn_na, om_na]
        a2, m2 = _stages(inp, s_max, split, flags, 0, 0, attn_na, om_na)
        rt.attend_merge_noalloc(a2, m2, step=step, tbase=TB, sidx=SIDX)
        assert mismatch(om_na.download(), om_ref.download()) == 0
        assert mismatch(attn_na.download(tag=TOUT + 1), attn_ref.download(tag=TOUT + 1)) == 0


def test_noalloc_refuses_plans_beyond_its_scratch(rt):
    keep = []
    s_max, split = 6144, 32                       # 192 splits > FX_NOALLOC_MAX_SPLITS (160)
    inp = _inputs(rt, keep, s_max, 100, split, 3)
    attn_na = rt.alloc((NH * DN,), "pk16").zero()
    om_na = rt.alloc((NH, DC), "bf16").zero()
    keep += [attn_na, om_na]
    a, m = _stages(inp, s_max, split, R.FX_F_MFMA, 0, 0, attn_na, om_na)
    with pytest.raises(R.FxError, match="n_splits"):
        rt.attend_merge_noalloc(a, m, step=100, tbase=TB, sidx=SIDX)
