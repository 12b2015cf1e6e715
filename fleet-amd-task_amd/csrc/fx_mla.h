// MLA absorbed decode attention (harness/numpy_ref.py:85-174; the reference's mla_prep_mi300.cuh,
// mla_attend_mfma_mi300.cuh, mla_merge_uv_mi300.cuh). Heads are split over XCDs: XCD x owns heads
// 2x and 2x + 1, so prep -> attend -> merge of a head only ever syncs inside its XCD. The kernels
// assume nh = 16, d_c = 512, d_r = 64, d_n = d_v = 128 (checked by fx_load_plan).
#pragma once
#include "fx_gemv.h"

__device__ __forceinline__ void rope64_store(const float* xin, const uint16_t* cosr, const uint16_t* sinr, void* dst,
                                             uint32_t dst_off, int i) {
  // i in [0, 64): de-interleave (even, odd) pairs, x*cos + rotate_half(x)*sin, bf16 at every op
  // (harness/numpy_ref.py:63-71, HF modeling_deepseek.py:339-371)
  const float xd = i < 32 ? xin[2 * i] : xin[2 * (i - 32) + 1];
  const float rot = i < 32 ? -xin[2 * i + 1] : xin[2 * (i - 32)];
  const float a = bf16r(xd * bf2f(cosr[i]));
  const float b = bf16r(rot * bf2f(sinr[i]));
  stc2(dst, dst_off + (uint32_t)i * 2, f2bf(a + b));
}

// FX_OP_MLA_PREP (harness/numpy_ref.py:85-103): tasks per XCD: hp*4 ql_nope column blocks of 128,
// then one task for the cache row (c_kv norm, k_pe rope) and the XCD's q_pe rows.
__device__ __forceinline__ void op_mla_prep(const fx_stage& s, FxEnv& env) {
  const int nh = s.n_rows, d_c = s.d_c, d_r = s.d_r, d_n = s.d_n;
  const int hp = nh / FX_XCDS;
  const int qstride = d_n + d_r;
  const int q_out = nh * qstride;
  const void* qkva = (const void*)s.x;
  const int nblk = d_c / 128;
  const int n_ql = hp * nblk;
  float* xs = (float*)(env.lds + LDS_XS);
  float* red = (float*)(env.lds + LDS_RED);
  for (int t = env.xrank; t <= n_ql; t += env.xworkers) {
    if (t < n_ql) {
      const int h = env.xcd * hp + t / nblk;
      const int cb = t % nblk;
      const int lane = lane_id();
      const int grp = lane >> 4, k = lane & 15;
      const int c0 = cb * 128 + wave_id() * 32 + grp * 8;
      // q_nope[h][8k .. 8k+8)
      u32x4 qv = ldc16(qkva, (uint32_t)(h * qstride + 8 * k) * 2);
      float q[8] = {bf_lo(qv.x), bf_hi(qv.x), bf_lo(qv.y), bf_hi(qv.y), bf_lo(qv.z), bf_hi(qv.z), bf_lo(qv.w), bf_hi(qv.w)};
      const uint16_t* Wh = (const uint16_t*)s.w + (size_t)h * d_n * d_c;
      u32x4 wr[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) wr[e] = ldw16(Wh + (size_t)(8 * k + e) * d_c + c0);
      float acc[8];
#pragma unroll
      for (int c = 0; c < 8; ++c) acc[c] = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float wv[8] = {bf_lo(wr[e].x), bf_hi(wr[e].x), bf_lo(wr[e].y), bf_hi(wr[e].y),
                       bf_lo(wr[e].z), bf_hi(wr[e].z), bf_lo(wr[e].w), bf_hi(wr[e].w)};
#pragma unroll
        for (int c = 0; c < 8; ++c) acc[c] = __builtin_fmaf(q[e], wv[c], acc[c]);
      }
#pragma unroll
      for (int c = 0; c < 8; ++c) acc[c] = butterfly(acc[c], 16);
      if (k == 0) {
        u32x4 o;
        o.x = pack2(acc[0], acc[1]); o.y = pack2(acc[2], acc[3]);
        o.z = pack2(acc[4], acc[5]); o.w = pack2(acc[6], acc[7]);
        stc16((void*)s.out, (uint32_t)(h * d_c + c0) * 2, o);
      }
    } else {
      // cache row at `step` (every XCD writes the same values) and the XCD's q_pe rows
      const uint16_t* cosr = (const uint16_t*)s.aux[3] + (size_t)env.step * d_r;
      const uint16_t* sinr = (const uint16_t*)s.aux[4] + (size_t)env.step * d_r;
      load_vec_sc1(xs, (const uint8_t*)qkva + (size_t)q_out * 2, d_c);
      float* kp = red + 256;   // k_pe raw [64], q_pe raw [hp][64]
      if (threadIdx.x < d_r) kp[threadIdx.x] = bf2f(ldc2(qkva, (uint32_t)(q_out + d_c + threadIdx.x) * 2));
      for (int i = threadIdx.x; i < hp * d_r; i += FX_THREADS) {
        const int h = env.xcd * hp + i / d_r;
        kp[64 + i] = bf2f(ldc2(qkva, (uint32_t)(h * qstride + d_n + i % d_r) * 2));
      }
      rmsnorm_inplace(xs, (const uint16_t*)s.w_norm, d_c, s.eps, red);
      store_vec_sc1((uint8_t*)s.aux[0] + (size_t)env.step * d_c * 2, xs, d_c);
      if (threadIdx.x < d_r) rope64_store(kp, cosr, sinr, (void*)s.aux[1], (uint32_t)env.step * d_r * 2, threadIdx.x);
      for (int i = threadIdx.x; i < hp * d_r; i += FX_THREADS) {
        const int hh = i / d_r;
        const int h = env.xcd * hp + hh;
        rope64_store(kp + 64 + hh * d_r, cosr, sinr, (void*)s.aux[2], (uint32_t)(h * d_r) * 2, i % d_r);
      }
      __syncthreads();
    }
  }
}


// FX_OP_MLA_ATTEND (harness/numpy_ref.py:110-149) for the XCD's two heads: one split per task, tiles
// of 32 positions, online softmax; partials [split][head][prow] = (o, lse). The last task of the XCD
// to finish merges its heads' live splits (harness/numpy_ref.py:152-165) into o_merged (aux4).
#define ATT_T 32
#define ATT_ROW 584   // bf16 elements per staged row: 576 + 8 pad (1168 bytes: conflict-free b128 reads)
#define ATT_CHUNKS 72 // 16-byte chunks of one position: 64 latent + 8 rope

__device__ __forceinline__ void attend_merge(const fx_stage& s, const FxEnv& env);

__device__ __forceinline__ void op_mla_attend(const fx_stage& s, FxEnv& env) {
  const int nh = s.n_rows, d_c = s.d_c, d_r = s.d_r, prow = s.prow;
  const int hp = 2;
  const int h0 = env.xcd * hp;
  const int step = env.step;
  const int split = s.split, n_splits = s.n_splits;
  const float scale = s.scale;
  float* ql = (float*)(env.lds + LDS_XS);                 // [2][512]
  float* qp = ql + 2 * 512;                               // [2][64]
  float* sp = qp + 2 * 64;                                // [2][32][5] partial scores
  float* pb = sp + 2 * 32 * 5;                            // [2][32] bf16(p)
  float* pp = pb + 64;                                    // [2][32] p
  float* hs = pp + 64;                                    // [2][4] m, l, alpha, m_new
  uint16_t* tile = (uint16_t*)(env.lds + LDS_TILE);       // [32][ATT_ROW]
  const uint16_t* ckv = (const uint16_t*)s.aux[0];
  const uint16_t* kpe = (const uint16_t*)s.aux[1];
  void* part = (void*)s.out;
  bool did_task = false;
  for (int j = env.xrank; j < n_splits; j += env.xworkers) {
    did_task = true;
    const int lo = j * split;
    int hi = lo + split;
    if (hi > step + 1) hi = step + 1;
    __syncthreads();
    // q rows of the XCD's heads (sc1: written by the prep stage of this XCD)
    for (int i = threadIdx.x; i < hp * d_c / 8; i += FX_THREADS) {
      const int hh = i / (d_c / 8), c = (i % (d_c / 8)) * 8;
      unpack8(ldc16((const void*)s.x, (uint32_t)((h0 + hh) * d_c + c) * 2), ql + hh * 512 + c);
    }
    if (threadIdx.x < hp * d_r) {
      const int hh = threadIdx.x / d_r, r = threadIdx.x % d_r;
      qp[hh * 64 + r] = bf2f(ldc2((const void*)s.aux[2], (uint32_t)((h0 + hh) * d_r + r) * 2));
    }
    if (threadIdx.x < hp) { hs[threadIdx.x * 4 + 0] = -__builtin_inff(); hs[threadIdx.x * 4 + 1] = 0.0f; }
    // accumulators: thread -> head ph = tid >> 7, columns pc .. pc + 3
    const int ph = threadIdx.x >> 7, pc = (threadIdx.x & 127) * 4;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int t0 = lo; t0 < hi; t0 += ATT_T) {
      const int nt = (t0 + ATT_T < hi ? t0 + ATT_T : hi) - t0;
      // stage rows t0 .. t0 + nt - 1 (never a row past `step`): 9 independent loads per thread
      u32x4 v[9];
#pragma unroll
      for (int k = 0; k < 9; ++k) {
        const int q = threadIdx.x + k * FX_THREADS;
        const int r = q / ATT_CHUNKS, c = q % ATT_CHUNKS;
        const int rr = r < nt ? r : 0;
        v[k] = c < 64 ? ld16(ckv + (size_t)(t0 + rr) * d_c + c * 8) : ld16(kpe + (size_t)(t0 + rr) * d_r + (c - 64) * 8);
      }
      __syncthreads();
#pragma unroll
      for (int k = 0; k < 9; ++k) {
        const int q = threadIdx.x + k * FX_THREADS;
        const int r = q / ATT_CHUNKS, c = q % ATT_CHUNKS;
        if (r < nt) *(u32x4*)(tile + r * ATT_ROW + c * 8) = v[k];
      }
      __syncthreads();
      // scores: thread (h, t, k): chain k over latent columns [128k, 128k + 128); k == 0 also the
      // rope chain; s = ((((n0 + n1) + n2) + n3) + pe) * scale
      {
        const int h = threadIdx.x >> 7, t = (threadIdx.x >> 2) & 31, k = threadIdx.x & 3;
        float a = 0.0f, b = 0.0f;
        if (t < nt) {
          const uint16_t* kr = tile + t * ATT_ROW;
          const float* qr = ql + h * 512;
#pragma unroll 4
          for (int c = k * 128; c < k * 128 + 128; c += 8) {
            const u32x4 kv = *(const u32x4*)(kr + c);
            const float4 q0 = *(const float4*)(qr + c), q1 = *(const float4*)(qr + c + 4);
            a = __builtin_fmaf(q0.x, bf_lo(kv.x), a);
            a = __builtin_fmaf(q0.y, bf_hi(kv.x), a);
            a = __builtin_fmaf(q0.z, bf_lo(kv.y), a);
            a = __builtin_fmaf(q0.w, bf_hi(kv.y), a);
            a = __builtin_fmaf(q1.x, bf_lo(kv.z), a);
            a = __builtin_fmaf(q1.y, bf_hi(kv.z), a);
            a = __builtin_fmaf(q1.z, bf_lo(kv.w), a);
            a = __builtin_fmaf(q1.w, bf_hi(kv.w), a);
          }
          if (k == 0) {
            const float* qpr = qp + h * 64;
#pragma unroll
            for (int r = 0; r < 64; r += 8) {
              const u32x4 kv = *(const u32x4*)(kr + 512 + r);
              b = __builtin_fmaf(qpr[r + 0], bf_lo(kv.x), b);
              b = __builtin_fmaf(qpr[r + 1], bf_hi(kv.x), b);
              b = __builtin_fmaf(qpr[r + 2], bf_lo(kv.y), b);
              b = __builtin_fmaf(qpr[r + 3], bf_hi(kv.y), b);
              b = __builtin_fmaf(qpr[r + 4], bf_lo(kv.z), b);
              b = __builtin_fmaf(qpr[r + 5], bf_hi(kv.z), b);
              b = __builtin_fmaf(qpr[r + 6], bf_lo(kv.w), b);
              b = __builtin_fmaf(qpr[r + 7], bf_hi(kv.w), b);
            }
          }
        }
        sp[(h * 32 + t) * 5 + k] = a;
        if (k == 0) sp[(h * 32 + t) * 5 + 4] = b;
      }
      __syncthreads();
      // softmax of the tile on wave 0 (lane = h * 32 + t); the sum of p runs sequentially in t
      if (threadIdx.x < 64) {
        const int h = threadIdx.x >> 5, t = threadIdx.x & 31;
        float sc = -__builtin_inff();
        if (t < nt) {
          const float* q = sp + (h * 32 + t) * 5;
          float v2 = q[0] + q[1];
          v2 = v2 + q[2];
          v2 = v2 + q[3];
          v2 = v2 + q[4];
          sc = v2 * scale;
          if (s.aux[3] && t0 + t < s.s_scores) stcf((void*)s.aux[3], (h0 + h) * s.s_scores + t0 + t, sc);
        }
        float mt = sc;
        for (int off = 1; off < 32; off <<= 1) mt = fmaxf(mt, shfl_xor_f(mt, off));
        const float m = hs[h * 4 + 0];
        const float m_new = m > mt ? m : mt;
        const float alpha = exp_s(m - m_new);
        const float p = t < nt ? exp_s(sc - m_new) : 0.0f;
        pp[h * 32 + t] = p;
        pb[h * 32 + t] = bf16r(p);
        if (t == 0) { hs[h * 4 + 2] = alpha; hs[h * 4 + 3] = m_new; }
      }
      __syncthreads();
      if (threadIdx.x < 2) {
        const int h = threadIdx.x;
        float psum = 0.0f;
        for (int t = 0; t < nt; ++t) psum = psum + pp[h * 32 + t];
        float l = hs[h * 4 + 1];
        l = l * hs[h * 4 + 2] + psum;
        hs[h * 4 + 1] = l;
        hs[h * 4 + 0] = hs[h * 4 + 3];
      }
      // value product over the tile, sequential in t: tp[c] = sum_t bf16(p_t) v_t[c];
      // acc = acc * alpha + tp
      {
        const float alpha = hs[ph * 4 + 2];
        float tp[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int t = 0; t < nt; ++t) {
          const float pv = pb[ph * 32 + t];
          const u32x2 kv = *(const u32x2*)(tile + t * ATT_ROW + pc);
          tp[0] = __builtin_fmaf(pv, bf_lo(kv.x), tp[0]);
          tp[1] = __builtin_fmaf(pv, bf_hi(kv.x), tp[1]);
          tp[2] = __builtin_fmaf(pv, bf_lo(kv.y), tp[2]);
          tp[3] = __builtin_fmaf(pv, bf_hi(kv.y), tp[3]);
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float a = acc[c] * alpha;
          acc[c] = a + tp[c];
        }
      }
      __syncthreads();
    }
    // o = acc / l, lse = m + log(l); an empty split stores o = 0, lse = -inf
    {
      const uint32_t base = (uint32_t)((j * nh + h0 + ph) * prow);
      u32x4 o;
      if (lo > step) {
        o.x = o.y = o.z = o.w = 0u;
      } else {
        const float l = hs[ph * 4 + 1];
        o.x = __float_as_uint(acc[0] / l);
        o.y = __float_as_uint(acc[1] / l);
        o.z = __float_as_uint(acc[2] / l);
        o.w = __float_as_uint(acc[3] / l);
      }
      stc16(part, (base + pc) * 4, o);
      if ((threadIdx.x & 127) == 0) {
        float lse = -__builtin_inff();
        if (lo <= step) lse = hs[ph * 4 + 0] + log_s(hs[ph * 4 + 1]);
        stcf(part, base + d_c, lse);
      }
    }
  }
  if (!did_task) return;
  // arrival on the XCD's counter: the last of the n_splits tasks merges
  wait_mem();
  __syncthreads();
  int* misc = (int*)(env.lds + LDS_MISC);
  if (threadIdx.x == 0) {
    int done = 0;
    for (int j = env.xrank; j < n_splits; j += env.xworkers) ++done;
    const uint32_t old = __hip_atomic_fetch_add(&env.sync[FX_CNT_ATTEND(env.xcd)], (uint32_t)done, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
    const bool last = old + done == (uint32_t)n_splits;
    if (last) flag_st(&env.sync[FX_CNT_ATTEND(env.xcd)], 0u);
    misc[0] = last ? 1 : 0;
  }
  __syncthreads();
  if (misc[0]) attend_merge(s, env);
}

// merge the live splits of the XCD's two heads: M = max lse, w_j = exp(lse_j - M),
// o = (sum_j w_j o_j, sequential fma) / (sum_j w_j, sequential) -> bf16.
// The o_j rows are fetched 16 splits at a time with independent loads.
#define MERGE_BATCH 16
__device__ __forceinline__ void attend_merge(const fx_stage& s, const FxEnv& env) {
  const int nh = s.n_rows, d_c = s.d_c, prow = s.prow;
  const int h0 = env.xcd * 2;
  const int live = (env.step + 1 + s.split - 1) / s.split;
  const void* part = (const void*)s.out;
  float* wj = (float*)(env.lds + LDS_TILE);   // [2][live]
  float* red = (float*)(env.lds + LDS_RED);
  if (wave_id() < 2) {
    const int h = wave_id();
    float mx = -__builtin_inff();
    for (int j = lane_id(); j < live; j += 64) mx = fmaxf(mx, ldcf(part, (uint32_t)((j * nh + h0 + h) * prow + d_c)));
    mx = wave_max(mx);
    for (int j = lane_id(); j < live; j += 64)
      wj[h * live + j] = exp_s(ldcf(part, (uint32_t)((j * nh + h0 + h) * prow + d_c)) - mx);
  }
  __syncthreads();
  if (threadIdx.x < 2) {
    float den = 0.0f;
    for (int j = 0; j < live; ++j) den = den + wj[threadIdx.x * live + j];
    red[threadIdx.x] = den;
  }
  __syncthreads();
  const int ph = threadIdx.x >> 7, pc = (threadIdx.x & 127) * 4;
  float num[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int j0 = 0; j0 < live; j0 += MERGE_BATCH) {
    u32x4 o[MERGE_BATCH];
#pragma unroll
    for (int k = 0; k < MERGE_BATCH; ++k) {
      const int j = j0 + k < live ? j0 + k : live - 1;
      o[k] = ldc16(part, (uint32_t)((j * nh + h0 + ph) * prow + pc) * 4);
    }
#pragma unroll
    for (int k = 0; k < MERGE_BATCH; ++k) {
      const float w = j0 + k < live ? wj[ph * live + j0 + k] : 0.0f;
      if (j0 + k >= live) continue;
      num[0] = __builtin_fmaf(w, __uint_as_float(o[k].x), num[0]);
      num[1] = __builtin_fmaf(w, __uint_as_float(o[k].y), num[1]);
      num[2] = __builtin_fmaf(w, __uint_as_float(o[k].z), num[2]);
      num[3] = __builtin_fmaf(w, __uint_as_float(o[k].w), num[3]);
    }
  }
  const float den = red[ph];
  u32x2 r;
  r.x = pack2(num[0] / den, num[1] / den);
  r.y = pack2(num[2] / den, num[3] / den);
  stc8((void*)s.aux[4], (uint32_t)((h0 + ph) * d_c + pc) * 2, r);
}

// FX_OP_MLA_MERGE_UV: attn[h*d_v + v] = bf16(dot(o_merged[h], W_uv[h][v])) for the XCD's heads
// (harness/numpy_ref.py:168-174); the merge itself ran at the end of the attend stage.
__device__ __forceinline__ void op_mla_merge_uv(const fx_stage& s, FxEnv& env) {
  const int d_c = s.d_c, d_v = s.d_n;   // the d_n field carries d_v here
  const int hp = 2;
  const int h0 = env.xcd * hp;
  float* xs = (float*)(env.lds + LDS_XS);
  int r0, r1;
  range_split(hp * d_v, env.xworkers, env.xrank, r0, r1);
  const uint16_t* W = (const uint16_t*)s.w + (size_t)h0 * d_v * d_c;
  // rows r0..r1 of this XCD's 2 * d_v; a group never straddles the two heads
  const int mid = d_v;
  const int na = r0 < mid ? (r1 < mid ? r1 : mid) - r0 : 0;        // rows of head 0
  const int ga = (na + 3) / 4;
  const int nb = (r1 - r0) - na;
  const int gb = (nb + 3) / 4;
  const int rb0 = r0 + na;
  auto rowof = [&](int g, int i) {
    if (g < ga) { const int r = r0 + g * 4 + i; return r < r0 + na ? r : -1; }
    const int r = rb0 + (g - ga) * 4 + i;
    return r < r1 ? r : -1;
  };
  Tile<4, 1> t0;
  gemv_prime(t0, W, d_c, ga + gb, rowof);
  load_vec_sc1(xs, (const uint8_t*)s.x + (size_t)h0 * d_c * 2, hp * d_c);
  __syncthreads();
  void* out = (void*)s.out;
  // the row's head decides which half of xs it multiplies: walk the groups of each head apart
  Tile<4, 1> t1;
  for (int g = wave_id(); g < ga + gb; g += FX_WAVES) {
    if (g != wave_id()) tile_load(t0, W, d_c, g, rowof);
    float acc[4];
    const float* x = xs + (g < ga ? 0 : d_c);
    tile_dot(t0, x, d_c, acc);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (t0.row[i] >= 0 && lane_id() == i) stc2(out, (uint32_t)(h0 * d_v + t0.row[i]) * 2, f2bf(acc[i]));
  }
  (void)t1;
}
