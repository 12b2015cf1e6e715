"""Pins of the CPU oracle (oracle/) against what fixes it independently of its own code.

Each check is chosen so that a plausible mistake (a dropped term, a wrong sign or index, a
transposed operand, a wrong rounding point) fails it:
  * known-answer vectors the reference's own tests hold (harness/tests/test_numpy_ref.py:84-90,
    340-349) and Random123's published Philox4x32-10 vectors;
  * independent implementations: torch's bf16 conversion and bf16 arithmetic (RoPE as HF writes
    it, modeling_deepseek.py:339-371), libm exp/log, torch silu;
  * float64 brute force of every reduction (GEMV, RMSNorm, attention, router, experts), whose
    error bound the FP32 spec order must respect;
  * invariants: one split equals many splits, empty splits, the decompressed attention form
    (numpy_ref.py:187-198), mask permutation, special cases that reduce to a permutation.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from oracle import model as M

F32 = np.float32


def bf(x):
    return O.f32_to_bf16(np.asarray(x, F32))


def fb(u):
    return O.bf16_to_f32(u)


def rng_bf16(rng, shape, scale=1.0):
    return bf(rng.standard_normal(shape).astype(F32) * F32(scale))


# ---- bf16 rounding (numpy_ref.py:36-42; test_numpy_ref.py:84-90) -------------------------------

def test_bf16_known_answers_vs_torch():
    x = np.array([1.0, 1.00390625, 1.001, 3.14159, -2.5e-3, 65504.0], F32)
    got = fb(bf(x))
    exp = torch.tensor(x).bfloat16().float().numpy()
    assert np.array_equal(got, exp)
    xs = np.random.default_rng(0).standard_normal(10000).astype(F32) * 100
    assert np.array_equal(fb(bf(xs)), torch.tensor(xs).bfloat16().float().numpy())


def test_bf16_ties_to_even():
    # 1 + 2^-8 is exactly half a bf16 ulp above 1: ties to the even neighbour 1.0;
    # 1 + 3*2^-8 ties between 1+2^-7 (odd) and 1+2^-6 (even).
    assert fb(bf([1.0 + 2 ** -8]))[0] == 1.0
    assert fb(bf([1.0 + 3 * 2 ** -8]))[0] == 1.0 + 2 ** -6


# ---- Philox4x32-10 (Salmon et al. 2011; Random123 kat_vectors) ---------------------------------

@pytest.mark.parametrize("ctr,key,exp", [
    ([0, 0, 0, 0], [0, 0], [0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8]),
    ([0xffffffff] * 4, [0xffffffff] * 2, [0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd]),
    ([0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344], [0xa4093822, 0x299f31d0],
     [0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1]),
])
def test_philox_known_answers(ctr, key, exp):
    assert O.philox4x32_raw(ctr, key).tolist() == exp


def test_normal_generator_statistics_and_slicing():
    from scipy import stats
    z = O.gen_normal_bf16(1234, 7, 200000, 1.0).astype(np.uint16)
    v = fb(z).astype(np.float64)
    assert abs(v.mean()) < 0.01 and abs(v.std() - 1.0) < 0.01
    assert stats.kstest(v, "norm").pvalue > 1e-3
    w = fb(O.gen_normal_bf16(1234, 7, 200000, 0.02)).astype(np.float64)
    assert abs(w.std() - 0.02) < 0.0003
    # any slice regenerates the same values (counter-based)
    part = O.gen_normal_bf16(1234, 7, 1001, 1.0, offset=5003)
    assert np.array_equal(part, z[5003:6004])
    # streams and seeds are independent
    assert not np.array_equal(O.gen_normal_bf16(1234, 8, 1000, 1.0), z[:1000])
    assert not np.array_equal(O.gen_normal_bf16(1235, 7, 1000, 1.0), z[:1000])


def test_tokens_uniform_in_vocab():
    t = O.gen_tokens(5, 3, 100000, 102400)
    assert t.min() >= 0 and t.max() < 102400
    counts = np.bincount(t // 10240, minlength=10)
    assert counts.min() > 9000 and counts.max() < 11000


# ---- exp / log / silu of the spec --------------------------------------------------------------

def test_exp_log_against_libm():
    xs = np.linspace(-87, 0, 100001, dtype=F32)
    e = O.exp_s(xs).astype(np.float64)
    ref = np.exp(xs.astype(np.float64))
    assert np.max(np.abs(e - ref) / np.spacing(ref.astype(F32))) < 4
    assert O.exp_s(np.array([0.0], F32))[0] == 1.0
    assert O.exp_s(np.array([-np.inf, -88.0], F32)).tolist() == [0.0, 0.0]
    assert np.all(np.diff(O.exp_s(xs)) >= 0)            # monotone: softmax order is preserved
    xl = np.exp(np.linspace(-16, 20, 100001)).astype(F32)
    lg = O.log_s(xl).astype(np.float64)
    ref = np.log(xl.astype(np.float64))
    assert np.max(np.abs(lg - ref)) < 4e-6 * np.maximum(1.0, np.abs(ref)).max()
    assert O.log_s(np.array([1.0], F32))[0] == 0.0


def test_silu_against_torch():
    # test_numpy_ref.py:330-335 uses rtol 1e-6 against torch's silu
    x = np.linspace(-8, 8, 257, dtype=F32)
    got = O.silu_s(x)
    exp = torch.nn.functional.silu(torch.tensor(x)).numpy()
    assert np.allclose(got, exp, rtol=1e-6, atol=1e-7)


# ---- the lane-order dot product ----------------------------------------------------------------

def test_dot_lanes_bound_and_order():
    rng = np.random.default_rng(1)
    for K in (64, 128, 512, 1408, 2048, 10944):
        a, b = rng_bf16(rng, K), rng_bf16(rng, K)
        got = float(O.dot_lanes(a, b))
        p = fb(a).astype(np.float64) * fb(b).astype(np.float64)
        assert abs(got - p.sum()) <= 2 * K * 2 ** -24 * np.abs(p).sum()
    # order known answer: K = 16 is two chunks on lanes 0 and 1. Lane 0 sums 1 + 2^-24 (a tie:
    # stays 1.0), lane 1 holds 2^-24, the butterfly adds 1 + 2^-24 = 1.0. Any order that adds
    # the two small terms first gets 1 + 2^-23 instead.
    a = np.zeros(16, F32)
    a[0], a[1], a[8] = 1.0, 2.0 ** -24, 2.0 ** -24
    assert float(O.dot_lanes(bf(a), bf(np.ones(16)))) == 1.0
    a2 = a.copy()
    a2[1], a2[8], a2[9] = 0.0, 2.0 ** -24, 2.0 ** -24      # both small terms on lane 1: exact sum first
    assert float(O.dot_lanes(bf(a2), bf(np.ones(16)))) == 1.0 + 2.0 ** -23


# ---- RMSNorm (numpy_ref.py:54-60) --------------------------------------------------------------

def test_rmsnorm_closed_form():
    rng = np.random.default_rng(2)
    for D in (512, 2048):
        x = rng_bf16(rng, D)
        w = rng_bf16(rng, D, 0.5)
        got = fb(O.rmsnorm(x, w))
        xf = fb(x).astype(np.float64)
        ref = fb(w).astype(np.float64) * xf / np.sqrt((xf ** 2).mean() + 1e-6)
        assert np.all(np.abs(got - ref) <= 2 * 2 ** -7 * np.abs(ref) + 1e-30)
    # constant row: var = c^2, xn rounds to sign(c), y = w exactly
    x = bf(np.full(2048, 3.0))
    w = rng_bf16(rng, 2048)
    assert np.array_equal(O.rmsnorm(x, w), w)
    # a planted mistake in the reference formula (no eps, mean over D-1) is distinguishable
    x = rng_bf16(rng, 64)
    ref_bad = fb(x) / np.sqrt((fb(x).astype(np.float64) ** 2).sum() / 63)
    assert not np.array_equal(fb(O.rmsnorm(x, bf(np.ones(64)))), fb(bf(ref_bad)))


# ---- RoPE (numpy_ref.py:63-71, HF modeling_deepseek.py:339-371) --------------------------------

def _hf_rope_torch(x, cos, sin):
    """HF apply_rotary_pos_emb in torch bf16 arithmetic: de-interleave, q*cos + rotate_half(q)*sin."""
    t = torch.from_numpy(fb(x)).bfloat16()
    d = t.shape[-1]
    t = t.view(*t.shape[:-1], d // 2, 2).transpose(-1, -2).reshape(*t.shape[:-1], d)
    rot = torch.cat([-t[..., d // 2:], t[..., :d // 2]], dim=-1)
    c = torch.from_numpy(fb(cos)).bfloat16()
    s = torch.from_numpy(fb(sin)).bfloat16()
    return bf((t * c + rot * s).float().numpy())


def test_rope_bit_exact_vs_torch_bf16():
    rng = np.random.default_rng(3)
    cos, sin = M.rope_tables(1100)
    for pos in (0, 1, 517, 1023, 1099):
        x = rng_bf16(rng, (16, 64))
        assert np.array_equal(O.rope(x, cos[pos], sin[pos]), _hf_rope_torch(x, cos[pos], sin[pos]))
    # position 0: cos = 1, sin = 0, so RoPE is the de-interleave permutation exactly
    x = rng_bf16(rng, 64)
    perm = np.concatenate([np.arange(0, 64, 2), np.arange(1, 64, 2)])
    assert np.array_equal(O.rope(x, cos[0], sin[0]), x[perm])


def test_rope_tables_layout():
    cos, sin = M.rope_tables(64)
    inv = 1.0 / 10000 ** (np.arange(0, 64, 2) / 64)
    assert np.array_equal(cos[5, :32], cos[5, 32:])
    assert np.allclose(fb(sin[5, :32]), np.sin(5 * inv), atol=2 ** -8)


# ---- linears (numpy_ref.py:295-313) ------------------------------------------------------------

def _close_bf16(got, ref64, ulps=1):
    ref = np.asarray(ref64, np.float64)
    return np.all(np.abs(fb(got) - ref) <= ulps * 2 ** -7 * np.abs(ref) + 1e-6 * np.abs(ref).max())


def test_linear_forms_vs_float64():
    rng = np.random.default_rng(4)
    W = rng_bf16(rng, (300, 2048), 0.02)
    x = rng_bf16(rng, 2048)
    res = rng_bf16(rng, 300)
    Wf, xf = fb(W).astype(np.float64), fb(x).astype(np.float64)
    out, _ = O.linear(W, x)
    assert _close_bf16(out, Wf @ xf)
    out, _ = O.linear(W, x, res=res)
    assert _close_bf16(out, Wf @ xf + fb(res))
    nw = rng_bf16(rng, 2048)
    out, h = O.linear(W, x, norm_w=nw)
    assert np.array_equal(h, O.rmsnorm(x, nw))
    assert _close_bf16(out, Wf @ fb(h).astype(np.float64))
    # planted: a transposed-operand product is far off
    Wsq = rng_bf16(rng, (64, 64))
    xs = rng_bf16(rng, 64)
    o, _ = O.linear(Wsq, xs)
    assert not _close_bf16(o, fb(Wsq).astype(np.float64).T @ fb(xs))


# ---- MLA prep / attend / merge (numpy_ref.py:85-198) -------------------------------------------

def _prep_inputs(rng, nh=16, d_n=128, d_r=64, d_c=512):
    qkva = rng_bf16(rng, nh * (d_n + d_r) + d_c + d_r)
    w_kv = rng_bf16(rng, d_c, 0.5)
    W_uk = rng_bf16(rng, (nh, d_n, d_c), 0.05)
    return qkva, w_kv, W_uk


def test_mla_prep_vs_closed_form():
    rng = np.random.default_rng(5)
    qkva, w_kv, W_uk = _prep_inputs(rng)
    cos, sin = M.rope_tables(2000)
    step = 1500
    c_row, k_pe_row, ql, qp = O.mla_prep(qkva, w_kv, W_uk, cos[step], sin[step])
    q = qkva[:16 * 192].reshape(16, 192)
    assert np.array_equal(c_row, O.rmsnorm(qkva[3072:3584], w_kv))
    assert np.array_equal(k_pe_row, O.rope(qkva[3584:], cos[step], sin[step]))
    assert np.array_equal(qp, _hf_rope_torch(q[:, 128:], cos[step], sin[step]))
    ref = np.einsum("hn,hnc->hc", fb(q[:, :128]).astype(np.float64), fb(W_uk).astype(np.float64))
    assert _close_bf16(ql, ref)


def _attn_inputs(rng, S, nh=16, d_c=512, d_r=64):
    return rng_bf16(rng, (nh, d_c)), rng_bf16(rng, (nh, d_r)), rng_bf16(rng, (S, d_c)), rng_bf16(rng, (S, d_r))


def _attention64(ql, qp, ck, kp, step, scale):
    s = (fb(ql).astype(np.float64) @ fb(ck[:step + 1]).astype(np.float64).T
         + fb(qp).astype(np.float64) @ fb(kp[:step + 1]).astype(np.float64).T) * scale
    p = np.exp(s - s.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    return p @ fb(ck[:step + 1]).astype(np.float64)


@pytest.mark.parametrize("attn", ["valu", "mfma"])
@pytest.mark.parametrize("S,step,split", [(64, 40, 32), (1056, 1023, 32), (300, 299, 96), (4096, 4095, 128)])
def test_mla_attend_merge_vs_brute_force(S, step, split, attn):
    """Both attention orders (the vector-ALU chains, mla_attend; the matrix-core instruction's,
    mla_attend_mfma) against float64 softmax attention."""
    rng = np.random.default_rng(6 + S)
    ql, qp, ck, kp = _attn_inputs(rng, S)
    scale = float(F32(1 / np.sqrt(192)))
    attend = O.mla_attend if attn == "valu" else O.mla_attend_mfma
    part = attend(ql, qp, ck, kp, step, scale, split=split)
    n_splits = -(-S // split)
    live = -(-(step + 1) // split)
    assert part.shape == (n_splits, 16, 516)
    assert np.isneginf(part[live:, :, 512]).all() and (part[live:, :, :512] == 0).all()
    W_uv = rng_bf16(rng, (16, 128, 512), 0.05)
    attn, obf = O.mla_merge_uv(part, W_uv, step, split=split)
    o64 = _attention64(ql, qp, ck, kp, step, scale)
    assert np.max(np.abs(fb(obf) - o64)) <= 2 ** -7 * np.abs(o64).max() + 1e-3 * np.abs(o64).max()
    ref_attn = np.einsum("hc,hvc->hv", fb(obf).astype(np.float64), fb(W_uv).astype(np.float64)).reshape(-1)
    assert _close_bf16(attn, ref_attn)
    # one split over everything equals many splits up to FP32 / bf16(p) rounding (test_numpy_ref.py:145-148)
    S1 = -(-S // 32) * 32
    one = attend(ql, qp, ck, kp, step, scale, split=S1)
    attn1, _ = O.mla_merge_uv(one, W_uv, step, split=S1)
    assert np.linalg.norm(fb(attn1) - fb(attn)) / np.linalg.norm(fb(attn)) < 1e-2


def test_mla_attend_mfma_exact_case():
    """With q = 0 every score is 0 and every probability 1, so each split's partial is the plain
    mean of its value rows and its lse is log(rows): with small dyadic cache values every sum is
    exact in any order, and the matrix-core attention's partials equal the vector-ALU chains' bit
    for bit (a wrong position or column in the value products would move an element)."""
    rng = np.random.default_rng(11)
    S, step = 96, 80
    ql, qp = bf(np.zeros((16, 512))), bf(np.zeros((16, 64)))
    ck = bf(rng.integers(-8, 9, (S, 512)) * 2.0 ** -6)
    kp = bf(rng.integers(-8, 9, (S, 64)) * 2.0 ** -6)
    pm = O.mla_attend_mfma(ql, qp, ck, kp, step, 0.125, split=32)
    pv = O.mla_attend(ql, qp, ck, kp, step, 0.125, split=32)
    assert np.array_equal(pm.view(np.uint32), pv.view(np.uint32))
    for j in range((step + 1) // 32):   # the full splits: the mean of 32 rows is exact
        rows = fb(ck[32 * j:32 * j + 32]).astype(np.float64)
        assert np.array_equal(pm[j, 3, :512].astype(np.float64), rows.mean(axis=0))


def test_mla_scores_and_lse():
    rng = np.random.default_rng(7)
    S, step = 96, 70
    ql, qp, ck, kp = _attn_inputs(rng, S)
    scale = float(F32(1 / np.sqrt(192)))
    part, scores = O.mla_attend(ql, qp, ck, kp, step, scale, split=32, with_scores=True)
    s64 = (fb(ql).astype(np.float64) @ fb(ck).astype(np.float64).T
           + fb(qp).astype(np.float64) @ fb(kp).astype(np.float64).T) * scale
    assert np.allclose(scores[:, :step + 1], s64[:, :step + 1], rtol=1e-5, atol=1e-5)
    for j in range(3):
        lo, hi = 32 * j, min(32 * j + 32, step + 1)
        lse64 = np.log(np.exp(s64[:, lo:hi]).sum(axis=1))
        assert np.allclose(part[j, :, 512], lse64, atol=1e-4)


def test_decompressed_attention_equivalence():
    """numpy_ref.py:187-198: the absorbed form equals keys/values decompressed by W_uk/W_uv."""
    rng = np.random.default_rng(8)
    S, step, nh = 200, 150, 16
    q = rng_bf16(rng, (nh, 192))
    W_uk = rng_bf16(rng, (nh, 128, 512), 0.05)
    W_uv = rng_bf16(rng, (nh, 128, 512), 0.05)
    ck, kp = rng_bf16(rng, (S, 512)), rng_bf16(rng, (S, 64))
    ql = bf(np.einsum("hn,hnc->hc", fb(q[:, :128]), fb(W_uk)))
    scale = float(F32(1 / np.sqrt(192)))
    part = O.mla_attend(ql, q[:, 128:], ck, kp, step, scale, split=32)
    attn, _ = O.mla_merge_uv(part, W_uv, step, split=32)
    c = fb(ck[:step + 1]).astype(np.float64)
    k_nope = np.einsum("hnc,sc->hsn", fb(W_uk).astype(np.float64), c)
    v = np.einsum("hvc,sc->hsv", fb(W_uv).astype(np.float64), c)
    s = (np.einsum("hn,hsn->hs", fb(q[:, :128]).astype(np.float64), k_nope)
         + fb(q[:, 128:]).astype(np.float64) @ fb(kp[:step + 1]).astype(np.float64).T) * scale
    p = np.exp(s - s.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    ref = np.einsum("hs,hsv->hv", p, v).reshape(-1)
    assert np.linalg.norm(fb(attn) - ref) / np.linalg.norm(ref) < 3e-2


# ---- router, experts, combine (numpy_ref.py:205-321) --------------------------------------------

def test_router_tie_break_and_combine_known_answers():
    """test_numpy_ref.py:340-349: experts 1 and 3 tie; the lower index wins; combine known answer."""
    h = bf(np.ones(8))
    W = np.zeros((4, 8), F32)
    W[1] = W[3] = 1.0
    _, logits, topk_w, routing, mask = O.moe_router(h, bf(W), topk=2, n_forced=2)
    assert mask[:2].tolist() == [1, 3] and routing.tolist() == [0, 1, 0, 2, 3, 4]
    assert mask.tolist() == [1, 3, 4, 5, -1, -1, 4]
    assert topk_w[2:].tolist() == [1.0, 1.0]
    out8 = bf(np.arange(4 * 6, dtype=F32).reshape(4, 6))
    got = O.moe_combine(out8, np.array([0.5, 0.25, 1.0, 1.0], F32), bf(np.zeros(6)))
    exp = bf(0.5 * fb(out8[0]) + 0.25 * fb(out8[1]) + fb(out8[2]) + fb(out8[3]))
    assert np.array_equal(got, exp)


def test_router_vs_float64():
    rng = np.random.default_rng(9)
    x = rng_bf16(rng, 2048)
    nw = bf(np.ones(2048))
    Wg = rng_bf16(rng, (64, 2048), 0.02)
    h, logits, topk_w, routing, mask = O.moe_router(x, Wg, norm_w=nw)
    assert np.array_equal(h, O.rmsnorm(x, nw))
    l64 = fb(Wg).astype(np.float64) @ fb(h).astype(np.float64)
    assert np.allclose(logits, l64, rtol=1e-5, atol=1e-5)
    p64 = np.exp(l64 - l64.max())
    p64 /= p64.sum()
    order = np.argsort(-p64, kind="stable")
    gaps = -np.diff(p64[order][:7])
    if gaps.min() > 1e-5:
        assert mask[:6].tolist() == order[:6].tolist()
    assert np.allclose(topk_w[:6], p64[mask[:6]], rtol=1e-5)
    assert mask[6:8].tolist() == [64, 65] and mask[66] == 8 and (mask[8:66] == -1).all()
    for k, e in enumerate(mask[:8]):
        assert routing[e] == k + 1
    assert (routing > 0).sum() == 8


def test_experts_vs_float64_and_mask_permutation():
    rng = np.random.default_rng(10)
    H, I = 2048, 1408
    h = rng_bf16(rng, H)
    W13 = rng_bf16(rng, (4, 2 * I, H), 0.02)
    W2 = rng_bf16(rng, (4, H, I), 0.02)
    mask = np.array([2, 0, 3, 1, 4], np.int32)
    act = O.moe_w13_silu(h, W13, mask, 4)
    out8 = O.moe_w2(act, W2, mask, 4)
    for s, e in enumerate(mask[:4]):
        gu = fb(W13[e]).astype(np.float64) @ fb(h).astype(np.float64)
        g, u = fb(bf(gu[:I])).astype(np.float64), fb(bf(gu[I:])).astype(np.float64)
        a64 = g / (1 + np.exp(-g)) * u
        assert _close_bf16(act[s], a64, ulps=2)
        o64 = fb(W2[e]).astype(np.float64) @ fb(act[s]).astype(np.float64)
        assert _close_bf16(out8[s], o64)
    perm = np.array([1, 3, 0, 2, 4], np.int32)
    pmask = mask.copy()
    pmask[:4] = mask[perm[:4]]
    assert np.array_equal(O.moe_w13_silu(h, W13, pmask, 4), act[perm[:4]])


def test_dense_mlp_vs_float64():
    rng = np.random.default_rng(11)
    H, I = 2048, 10944
    x = rng_bf16(rng, H)
    nw = bf(np.ones(H))
    W_gu = rng_bf16(rng, (2 * I, H), 0.02)
    W_d = rng_bf16(rng, (H, I), 0.02)
    h, act, out = O.dense_mlp(x, nw, W_gu, W_d)
    assert np.array_equal(h, O.rmsnorm(x, nw))
    gu = fb(W_gu).astype(np.float64) @ fb(h).astype(np.float64)
    g, u = fb(bf(gu[:I])).astype(np.float64), fb(bf(gu[I:])).astype(np.float64)
    assert _close_bf16(act, g / (1 + np.exp(-g)) * u, ulps=2)
    ref = fb(W_d).astype(np.float64) @ fb(act).astype(np.float64) + fb(x)
    assert _close_bf16(out, ref)


def test_argmax_lowest_index_on_ties():
    l = bf(np.array([0.5, 2.0, -1.0, 2.0, 1.0], F32))
    assert O.argmax_bf16(l) == 1
