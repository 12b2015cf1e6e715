"""Batched GPU prefill: the prompt's forward pass over positions 0 .. n_prompt - 2 at once, writing
every layer's latent-cache rows; the decode (fx_run) then starts at position n_prompt - 1.

The reference has no prefill of its own: it captures the caches from the HF model's prefill
(harness/run_reference.py:367-376, 414-425) and uploads them before the decode
(harness/run_fleet.py:533-537). Here the same rows come from this library: the plain GEMMs through
fx_gemm (rocBLAS, bf16 in, FP32 accumulate) and the row work in between through the fx_pf_*
kernels, which round at the decode spec's points (numpy_ref.py). Per layer, M = n_prompt - 1 rows:

  h1 = rmsnorm(x)                                   fx_pf_rmsnorm
  qkva = bf16(h1 W_qkva^T)                          fx_gemm
  c_kv / k_pe rows at positions 0..M-1, q_pe        fx_pf_prep
  ql[h] = bf16(q_nope[h] W_uk[h])                   fx_gemm, batched over heads
  S[h] = ql[h] c_kv^T + q_pe[h] k_pe^T (FP32)       fx_gemm x 2, heads in chunks (memory bound)
  P[h] = bf16(exp(S * scale - max)), l[h]           fx_pf_softmax (causal: keys 0..i)
  o[h] = bf16((P[h] c_kv) / l[h])                   fx_gemm (FP32) + fx_pf_attn_out
  attn[:, h] = bf16(o[h] W_uv[h]^T)                 fx_gemm, batched over heads
  x_mid = bf16(attn W_o^T + x)                      fx_gemm (beta = 1)
  layer 0: x = bf16(silu-gated(rmsnorm(x_mid) W_gu^T) W_down^T + x_mid)
  MoE:     logits = rmsnorm(x_mid) W_gate^T (FP32); ids, w = route (fx_pf_route); rows grouped
           by expert (host), gathered; per expert bf16(h W13[e]^T) -> silu -> bf16(. W2[e]^T);
           x = bf16(x_mid + sum_s out_s w_s) in slot order (fx_pf_combine)

With FP8 experts (W13q_l / W2q_l) each layer's experts are expanded back to bf16 (code x row scale,
fx_dequantize_fp8) for the GEMMs. Attention is one softmax over the whole causal row (the decode splits it into 32-position tiles
with an online softmax), and the GEMMs reduce in rocBLAS's order, so the cache rows agree with the
decode path's within bf16 rounding, not bit for bit; a route may differ where two router
probabilities are within rounding of each other.
"""
import numpy as np

from fleet import runtime as R
from fleet.pack_weights import Dims

SCORE_BUDGET = 4 << 30      # bytes of FP32 scores + bf16 probabilities per head chunk


class Prefill:
    """Scratch for a prompt of n_prompt tokens; run() fills the caches of `layers` layers."""

    def __init__(self, rt, packed, capture, dims: Dims, n_prompt, layers, eps, scale, scaling=1.0):
        self.rt, self.W, self.cap, self.d = rt, packed, capture, dims
        self.M = n_prompt - 1
        self.layers, self.eps, self.scale, self.scaling = layers, float(eps), float(scale), float(scaling)
        d, M = dims, self.M
        self.s_max = capture["c_kv_0"].shape[0]
        assert n_prompt <= self.s_max, (n_prompt, self.s_max)
        if M <= 0:
            return
        self.hc = int(max(1, min(d.NH, SCORE_BUDGET // (6 * M * M))))
        a = rt.alloc
        self.x = a((M, d.H), "bf16")
        self.x_mid = a((M, d.H), "bf16")
        self.h = a((M, d.H), "bf16")
        self.qkva = a((M, d.Q_OUT + d.KVA_OUT), "bf16")
        self.q_pe = a((M, d.NH, d.D_R), "bf16")
        self.ql = a((d.NH, M, d.D_C), "bf16")
        self.S = a((self.hc, M, M), "f32")
        self.P = a((self.hc, M, M), "bf16")
        self.l = a((self.hc, M), "f32")
        self.O = a((self.hc, M, d.D_C), "f32")
        self.obf = a((d.NH, M, d.D_C), "bf16")
        self.attn = a((M, d.NH * d.D_V), "bf16")
        if layers >= 1:
            self.gu = a((M, 2 * d.I_DENSE), "bf16")
            self.act = a((M, d.I_DENSE), "bf16")
        if layers >= 2:
            S = d.N_SLOTS
            self.logits = a((M, d.E), "f32")
            self.ids = a((M, S), "i32")
            self.wts = a((M, S), "f32")
            self.perm = a((M * S,), "i32")
            self.inv = a((M * S,), "i32")
            self.hg = a((M * S, d.H), "bf16")
            self.mid = a((M * S, 2 * d.I_MOE), "bf16")
            self.act8 = a((M * S, d.I_MOE), "bf16")
            self.og = a((M * S, d.H), "bf16")
            if "W13q_1" in packed:   # FP8 experts: each layer's experts back to bf16 for the GEMMs
                self.w13 = a((d.E_TOTAL, 2 * d.I_MOE, d.H), "bf16")
                self.w2 = a((d.E_TOTAL, d.H, d.I_MOE), "bf16")

    # ---- thin wrappers (pointers as ints, byte offsets added by the caller) ----------------------
    def gemm(self, ta, tb, M, N, K, A, lda, B, ldb, D, ldd, d_f32=False, beta=0.0, C=None, ldc=0, batch=1,
             sa=0, sb=0, sc=0, sd=0, alpha=1.0):
        rt = self.rt
        rt.check(rt.L.fx_gemm(rt.h, int(ta), int(tb), M, N, K, alpha, A, lda, sa, B, ldb, sb, beta, C, ldc, sc, D, ldd,
                              sd, int(d_f32), batch, None), "fx_gemm")

    def run(self, tokens):
        """Fill the caches at positions 0 .. M-1 from tokens[0 .. M-1] (the meta tokens buffer)."""
        if self.M <= 0:
            return
        rt, d, M, L = self.rt, self.d, self.M, self.rt.L
        h_ = rt.h
        rt.check(L.fx_pf_embed(h_, tokens.ptr, self.W["W_embed"].ptr, self.x.ptr, M, d.H, None), "fx_pf_embed")
        for l in range(self.layers):
            self._attention(l)
            if l == 0:
                self._dense(l)
            else:
                self._moe(l)
        rt.synchronize()

    def _attention(self, l):
        rt, d, M, L, W = self.rt, self.d, self.M, self.rt.L, self.W
        h_ = rt.h
        QKV = d.Q_OUT + d.KVA_OUT
        ckv, kpe = self.cap[f"c_kv_{l}"], self.cap[f"k_pe_{l}"]
        rt.check(L.fx_pf_rmsnorm(h_, self.x.ptr, d.H, W[f"w_norm1_{l}"].ptr, self.h.ptr, d.H, M, d.H, self.eps, None),
                 "fx_pf_rmsnorm")
        self.gemm(0, 1, M, QKV, d.H, self.h.ptr, d.H, W[f"W_qkva_{l}"].ptr, d.H, self.qkva.ptr, QKV)
        rt.check(L.fx_pf_prep(h_, self.qkva.ptr, QKV, W[f"w_kv_norm_{l}"].ptr, self.cap["cos"].ptr, self.cap["sin"].ptr,
                              ckv.ptr, kpe.ptr, self.q_pe.ptr, 0, M, self.s_max, d.NH, d.D_N, d.D_C, self.eps, None),
                 "fx_pf_prep")
        # ql[h] = q_nope[h] W_uk[h]: A = the head's nope columns of qkva
        self.gemm(0, 0, M, d.D_C, d.D_N, self.qkva.ptr, QKV, W[f"W_uk_{l}"].ptr, d.D_C, self.ql.ptr, d.D_C,
                  batch=d.NH, sa=d.D_N + d.D_R, sb=d.D_N * d.D_C, sd=M * d.D_C)
        for h0 in range(0, d.NH, self.hc):
            hc = min(self.hc, d.NH - h0)
            # S = ql c_kv^T + q_pe k_pe^T over keys 0..M-1 (FP32)
            self.gemm(0, 1, M, M, d.D_C, self.ql.ptr + 2 * h0 * M * d.D_C, d.D_C, ckv.ptr, d.D_C, self.S.ptr, M,
                      d_f32=True, batch=hc, sa=M * d.D_C, sb=0, sd=M * M)
            self.gemm(0, 1, M, M, d.D_R, self.q_pe.ptr + 2 * h0 * d.D_R, d.NH * d.D_R, kpe.ptr, d.D_R, self.S.ptr, M,
                      d_f32=True, beta=1.0, C=self.S.ptr, ldc=M, batch=hc, sa=d.D_R, sb=0, sc=M * M, sd=M * M)
            rt.check(L.fx_pf_softmax(h_, self.S.ptr, M, M * M, self.P.ptr, M, M * M, self.l.ptr, M, M, hc, M, 0,
                                     self.scale, None), "fx_pf_softmax")
            # O = P c_kv (FP32), o = bf16(O / l)
            self.gemm(0, 0, M, d.D_C, M, self.P.ptr, M, ckv.ptr, d.D_C, self.O.ptr, d.D_C, d_f32=True, batch=hc,
                      sa=M * M, sb=0, sd=M * d.D_C)
            rt.check(L.fx_pf_attn_out(h_, self.O.ptr, self.l.ptr, self.obf.ptr + 2 * h0 * M * d.D_C, M, hc, d.D_C,
                                      None), "fx_pf_attn_out")
        # attn[:, h] = o[h] W_uv[h]^T
        self.gemm(0, 1, M, d.D_V, d.D_C, self.obf.ptr, d.D_C, W[f"W_uv_{l}"].ptr, d.D_C, self.attn.ptr, d.NH * d.D_V,
                  batch=d.NH, sa=M * d.D_C, sb=d.D_V * d.D_C, sd=d.D_V)
        # x_mid = attn W_o^T + x
        self.gemm(0, 1, M, d.H, d.NH * d.D_V, self.attn.ptr, d.NH * d.D_V, W[f"W_o_{l}"].ptr, d.NH * d.D_V,
                  self.x_mid.ptr, d.H, beta=1.0, C=self.x.ptr, ldc=d.H)

    def _dense(self, l):
        rt, d, M, L, W = self.rt, self.d, self.M, self.rt.L, self.W
        I = d.I_DENSE
        rt.check(L.fx_pf_rmsnorm(rt.h, self.x_mid.ptr, d.H, W[f"w_norm2_{l}"].ptr, self.h.ptr, d.H, M, d.H, self.eps,
                                 None), "fx_pf_rmsnorm")
        self.gemm(0, 1, M, 2 * I, d.H, self.h.ptr, d.H, W[f"W_gu_{l}"].ptr, d.H, self.gu.ptr, 2 * I)
        rt.check(L.fx_pf_silu(rt.h, self.gu.ptr, self.act.ptr, M, I, None), "fx_pf_silu")
        self.gemm(0, 1, M, d.H, I, self.act.ptr, I, W[f"W_down_{l}"].ptr, I, self.x.ptr, d.H, beta=1.0,
                  C=self.x_mid.ptr, ldc=d.H)

    def _moe(self, l):
        rt, d, M, L, W = self.rt, self.d, self.M, self.rt.L, self.W
        S, I, H = d.N_SLOTS, d.I_MOE, d.H
        rt.check(L.fx_pf_rmsnorm(rt.h, self.x_mid.ptr, H, W[f"w_norm2_{l}"].ptr, self.h.ptr, H, M, H, self.eps, None),
                 "fx_pf_rmsnorm")
        self.gemm(0, 1, M, d.E, H, self.h.ptr, H, W[f"W_gate_{l}"].ptr, H, self.logits.ptr, d.E, d_f32=True)
        rt.check(L.fx_pf_route(rt.h, self.logits.ptr, self.ids.ptr, self.wts.ptr, M, d.E, d.TOPK, d.N_SHARED,
                               self.scaling, None), "fx_pf_route")
        ids = self.ids.download().reshape(M, S)
        if ids.min() < 0 or ids.max() >= d.E_TOTAL:
            raise R.FxError(f"prefill layer {l}: expert id out of range")
        flat = ids.reshape(-1)
        order = np.argsort(flat, kind="stable").astype(np.int32)       # (m, s) pairs grouped by expert
        perm = (order // S).astype(np.int32)                           # the token row of each pair
        inv = np.empty(M * S, np.int32)
        inv[order] = np.arange(M * S, dtype=np.int32)
        counts = np.bincount(flat, minlength=d.E_TOTAL)
        self.perm.upload(perm)
        self.inv.upload(inv)
        rt.check(L.fx_pf_gather(rt.h, self.h.ptr, self.perm.ptr, self.hg.ptr, M * S, H, None), "fx_pf_gather")
        if f"W13q_{l}" in W:
            for key, dst, rows, K in ((f"W13q_{l}", self.w13, d.E_TOTAL * 2 * I, H), (f"W2q_{l}", self.w2, d.E_TOTAL * H, I)):
                rt.check(L.fx_dequantize_fp8(rt.h, W[key].ptr, dst.ptr, rows, K, None), "fx_dequantize_fp8")
            W13, W2 = self.w13, self.w2
        else:
            W13, W2 = W[f"W13_{l}"], W[f"W2_{l}"]
        off = 0
        for e in range(d.E_TOTAL):
            n = int(counts[e])
            if n:
                self.gemm(0, 1, n, 2 * I, H, self.hg.ptr + 2 * off * H, H, W13.ptr + 2 * e * 2 * I * H, H,
                          self.mid.ptr + 2 * off * 2 * I, 2 * I)
            off += n
        rt.check(L.fx_pf_silu(rt.h, self.mid.ptr, self.act8.ptr, M * S, I, None), "fx_pf_silu")
        off = 0
        for e in range(d.E_TOTAL):
            n = int(counts[e])
            if n:
                self.gemm(0, 1, n, H, I, self.act8.ptr + 2 * off * I, I, W2.ptr + 2 * e * H * I, I,
                          self.og.ptr + 2 * off * H, H)
            off += n
        rt.check(L.fx_pf_combine(rt.h, self.x_mid.ptr, self.og.ptr, self.inv.ptr, self.wts.ptr, self.x.ptr, M, H, S,
                                 None), "fx_pf_combine")

    def free(self):
        for v in list(vars(self).values()):
            if isinstance(v, R.DeviceBuffer):
                v.free()
