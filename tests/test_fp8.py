"""FP8 expert weights on the CPU: the oracle's e4m3fn decode and weight-only quantizer against torch's
float8_e4m3fn (the OCP format: round to nearest even, 448 the largest finite value), the FP8 dot
and expert GEMVs against float64 on the dequantized weights, and the byte count of an FP8 token.
The reference only projects this path (README.md:130, docs/acceleration/04-technique-ledger.md:12:
weight-only FP8 of the experts, 1.83x by its arithmetic); the format pins are torch's."""
import numpy as np
import pytest

from oracle import oracle as O
from fleet import pack_weights as P


def test_e4m3_decode_matches_torch():
    torch = pytest.importorskip("torch")
    ours = O.e4m3_decode()
    ref = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    same = (ours == ref) | (np.isnan(ours) & np.isnan(ref))
    assert same.all(), np.flatnonzero(~same)
    assert ours[0x7E] == 448.0 and ours[0x01] == 2.0 ** -9 and ours[0x38] == 1.0 and np.isnan(ours[0xFF])


def test_quantizer_matches_torch_rounding():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(5)
    rows = [rng.standard_normal(256) * 0.02, rng.standard_normal(256) * 300, np.zeros(256),
            np.concatenate([np.full(8, 1e-30), rng.standard_normal(248) * 1e-3]), np.linspace(-5, 7, 256)]
    w = P.f32_to_bf16(np.stack(rows).astype(np.float32))
    q, s = O.quantize_fp8(w)
    wf = P.bf16_to_f32(w)
    amax = np.abs(wf).max(axis=1)
    np.testing.assert_array_equal(s, np.where(amax > 0, (amax / np.float32(448)).astype(np.float32), 1.0))
    ref = torch.from_numpy((wf / s[:, None]).astype(np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(q, ref), np.argwhere(q != ref)[:5]
    # the row maximum maps to 448 (code 0x7E), the zero row to codes 0 with scale 1
    assert all(np.abs(O.e4m3_decode()[q[r]]).max() == 448.0 for r in (0, 1, 3, 4))
    assert (q[2] == 0).all() and s[2] == 1.0


def test_fp8_expert_gemvs_against_float64():
    rng = np.random.default_rng(9)
    H, I, slots = 256, 64, 3
    W13 = P.f32_to_bf16(rng.standard_normal((slots, 2 * I, H)).astype(np.float32) * 0.05)
    W2 = P.f32_to_bf16(rng.standard_normal((slots, H, I)).astype(np.float32) * 0.05)
    h = P.f32_to_bf16(rng.standard_normal(H).astype(np.float32))
    q13, s13 = O.quantize_fp8(W13.reshape(-1, H))
    q2, s2 = O.quantize_fp8(W2.reshape(-1, I))
    q13, s13, q2, s2 = q13.reshape(slots, 2 * I, H), s13.reshape(slots, 2 * I), q2.reshape(slots, H, I), s2.reshape(slots, H)
    mask = np.arange(slots + 1, dtype=np.int32)
    act = O.moe_w13_silu_fp8(h, q13, s13, mask, slots)
    out8 = O.moe_w2_fp8(act, q2, s2, mask, slots)
    tab = O.e4m3_decode().astype(np.float64)
    hf = P.bf16_to_f32(h).astype(np.float64)
    gu = np.einsum("sik,k->si", tab[q13], hf) * s13
    g, u = P.bf16_to_f32(P.f32_to_bf16(gu[:, :I])), P.bf16_to_f32(P.f32_to_bf16(gu[:, I:]))
    want_act = g / (1 + np.exp(-g.astype(np.float64))) * u
    got_act = P.bf16_to_f32(act).astype(np.float64)
    assert np.allclose(got_act, want_act, rtol=2 ** -7, atol=1e-4)
    want_out = np.einsum("snk,sk->sn", tab[q2], got_act) * s2
    assert np.allclose(P.bf16_to_f32(out8), want_out, rtol=2 ** -7, atol=1e-4)
    # and the dequantized weights stay within FP8 rounding of the bf16 ones (3 mantissa bits)
    deq = tab[q13] * s13[..., None]
    w = P.bf16_to_f32(W13).astype(np.float64)
    assert np.all(np.abs(deq - w) <= np.abs(w) * 2 ** -4 + s13[..., None] * 2.0 ** -9)


def test_fp8_bytes_per_token():
    d = P.REAL_DIMS
    b16, b8 = P.bytes_per_token(d, 1024), P.bytes_per_token(d, 1024, fp8_experts=True)
    experts = (d.L - 1) * d.N_SLOTS * 3 * d.I_MOE * d.H          # bf16 elements of the 8 slots' experts
    scales = (d.L - 1) * d.N_SLOTS * (2 * d.I_MOE + d.H) * 4
    assert b16 - b8 == experts - scales
    assert P.fp8_nbytes(d, "W13_1") == d.E_TOTAL * 2 * d.I_MOE * (d.H + 4)


def test_fp8_linear_against_float64():
    """The FP8 LM head's linear (rmsnorm prologue, dot over codes x row, the row's scale, bf16): float64
    on the dequantized codes within the FP32 summation bound; exact on small integers; the normalised
    row equals the bf16 linear's."""
    rng = np.random.default_rng(11)
    N, K = 96, 2048
    w = P.f32_to_bf16((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    x = P.f32_to_bf16(rng.standard_normal(K).astype(np.float32))
    nw = P.f32_to_bf16((1 + 0.1 * rng.standard_normal(K)).astype(np.float32))
    q, s = O.quantize_fp8(w)
    out, h = O.linear_fp8(q, s, x, norm_w=nw, eps=1e-6)
    _, h_bf = O.linear(w, x, norm_w=nw, eps=1e-6)
    assert np.array_equal(h, h_bf)
    tab = O.e4m3_decode().astype(np.float64)
    hv = P.bf16_to_f32(h).astype(np.float64)
    ref = (tab[q] @ hv) * s.astype(np.float64)
    got = P.bf16_to_f32(out).astype(np.float64)
    bound = 2.0 ** -8 * np.abs(ref) + 2.0 ** -22 * (np.abs(tab[q]) @ np.abs(hv)) * s + 1e-30
    assert (np.abs(got - ref) <= bound).all(), np.max(np.abs(got - ref) / bound)
    # a wrong scale row would be caught: rows differ in scale by construction
    assert len(np.unique(s)) >= 16
    # exact case: codes 1.0 (0x38) and 2.0 (0x40), integer inputs, scale 1 -> the exact integer sum
    qe = np.where(rng.random((4, 64)) < 0.5, 0x38, 0x40).astype(np.uint8)
    xe = P.f32_to_bf16(rng.integers(-8, 9, 64).astype(np.float32))
    oe, _ = O.linear_fp8(qe, np.ones(4, np.float32), xe)
    want = tab[qe] @ P.bf16_to_f32(xe).astype(np.float64)
    assert np.array_equal(P.bf16_to_f32(oe).astype(np.float64), want)
