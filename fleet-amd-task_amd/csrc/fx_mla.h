// MLA absorbed decode attention (harness/numpy_ref.py:85-174; the reference's mla_prep_mi300.cuh,
// mla_attend_mfma_mi300.cuh, mla_merge_uv_mi300.cuh). Heads are split over XCDs: XCD x owns heads
// 2x and 2x + 1, so prep -> attend -> merge of a head only ever exchanges data inside its XCD. The
// kernels assume nh = 16, d_c = 512, d_r = 64, d_n = d_v = 128 (checked by fx_load_plan).
#pragma once
#include "fx_gemv.h"

#define MLA_HP 2          // heads per XCD
#define PREP_ROW_RANK 31  // the XCD rank that normalises / ropes the cache row and q_pe

// rope of one 64-vector (i in [0, 64)): de-interleave the (even, odd) pairs, x*cos + rotate_half(x)*sin,
// bf16 at every op (harness/numpy_ref.py:63-71, HF modeling_deepseek.py:339-371)
// element i with its table entries c = cos[i], sn = sin[i] already read
__device__ __forceinline__ float rope64_cs(const float* xin, float c, float sn, int i) {
  const float xd = i < 32 ? xin[2 * i] : xin[2 * (i - 32) + 1];
  const float rot = i < 32 ? -xin[2 * i + 1] : xin[2 * (i - 32)];
  const float a = bf16r(xd * c);
  const float b = bf16r(rot * sn);
  return bf16r(a + b);
}
__device__ __forceinline__ float rope64(const float* xin, const uint16_t* cosr, const uint16_t* sinr, int i) {
  return rope64_cs(xin, bf2f(cosr[i]), bf2f(sinr[i]), i);
}

// FX_OP_MLA_PREP (harness/numpy_ref.py:85-103). Per XCD: 32 wave tasks of ql_nope (head, 32
// columns: dot_lanes over d_n = 128, 16 chunks of 8) -- task t on rank t % 31, wave t / 31 -- and,
// on rank 31, the cache row (kv_a RMSNorm, k_pe RoPE; stored by XCD 0, published to the XCD as
// packets) and the XCD's q_pe rows.
__device__ __forceinline__ void op_mla_prep(const fx_stage& s, FxEnv& env) {
  const int d_c = s.d_c, d_r = s.d_r, d_n = s.d_n, nh = s.n_rows;
  const int qstride = d_n + d_r;
  const int q_out = nh * qstride;
  const int h0 = env.xcd * MLA_HP;
  const void* qkva = (const void*)s.x;
  const uint32_t tin = tag_in(s, env, 0), tout = tag_out(env);
  // FX_F_XLOCAL: the packets are read by the same XCD's attention only (heads 2x, 2x + 1 on XCD x)
  const bool loc = (__builtin_amdgcn_readfirstlane(s.flags) & FX_F_XLOCAL) != 0;
  if (env.xrank != PREP_ROW_RANK) {
    const int t = env.xrank + (PREP_ROW_RANK)*wave_id();
    if (t >= MLA_HP * (d_c / 32)) return;
    const int h = h0 + t / (d_c / 32);
    const int lane = lane_id();
    const int grp = lane >> 4, k = lane & 15;
    const int c0 = (t % (d_c / 32)) * 32 + grp * 8;
    const uint16_t* Wh = (const uint16_t*)s.w + (size_t)h * d_n * d_c;
    u32x4 wr[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) wr[e] = ldw16(Wh + (size_t)(8 * k + e) * d_c + c0);
    fx_issue_here();
    // q_nope[h][8k .. 8k + 8): pairs (h * qstride + 8k) / 4, + 1
    u32x4 qv[2];
    pk_wait_pairs<2>(qkva, (h * qstride + 8 * k) >> 2, 1, q_out >> 2, tin, env.err, qv);
    prof_mark(env, 1);
    const float q[8] = {bf_lo(qv[0].x), bf_hi(qv[0].x), bf_lo(qv[0].z), bf_hi(qv[0].z),
                        bf_lo(qv[1].x), bf_hi(qv[1].x), bf_lo(qv[1].z), bf_hi(qv[1].z)};
    float acc[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[c] = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float wv[8];
      unpack8(wr[e], wv);
#pragma unroll
      for (int c = 0; c < 8; ++c) acc[c] = __builtin_fmaf(q[e], wv[c], acc[c]);
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[c] = butterfly(acc[c], 16);
    if (k == 0) {
      const uint32_t pkt = (uint32_t)(h * d_c + c0) >> 1;
      pk_put2((void*)s.out, pkt, pack2(acc[0], acc[1]), pack2(acc[2], acc[3]), tout, loc);
      pk_put2((void*)s.out, pkt + 2, pack2(acc[4], acc[5]), pack2(acc[6], acc[7]), tout, loc);
    }
    prof_mark(env, 2);
    return;
  }
  // ---- rank 31: cache row and q_pe of the XCD's heads
  float* xs = (float*)(env.lds + LDS_XS);        // latent [d_c]
  float* red = (float*)(env.lds + LDS_RED);
  float* kp = red + 256;                          // k_pe raw [64], q_pe raw [2][64]
  float* rp = red + 512;                          // roped k_pe [64], q_pe [2][64]
  const uint16_t* cosr = (const uint16_t*)s.aux[3] + (size_t)env.step * d_r;
  const uint16_t* sinr = (const uint16_t*)s.aux[4] + (size_t)env.step * d_r;
  const NormW nw = d_c <= 8 * FX_THREADS ? norm_prefetch((const uint16_t*)s.w_norm, d_c) : NormW{};
  // this thread's RoPE table entries (k_pe and the two q_pe rows), also requested ahead of the input
  const bool roper = fx_tid() < d_r * (1 + MLA_HP);
  float rc = 0.0f, rsn = 0.0f;
  if (roper) {
    rc = bf2f(cosr[fx_tid() % d_r]);
    rsn = bf2f(sinr[fx_tid() % d_r]);
  }
  fx_issue_here();
  {
    // pairs: latent (q_out .. q_out + d_c) -> 128, k_pe -> 16, q_pe of the two heads -> 2 x 16
    const int t = fx_tid();
    int q = -1;
    float* dst = nullptr;
    if (t < d_c / 4) { q = (q_out >> 2) + t; dst = xs + 4 * t; }
    else if (t < d_c / 4 + d_r / 4) { q = ((q_out + d_c) >> 2) + (t - d_c / 4); dst = kp + 4 * (t - d_c / 4); }
    else if (t < d_c / 4 + d_r / 4 + MLA_HP * d_r / 4) {
      const int u = t - d_c / 4 - d_r / 4, hh = u / (d_r / 4), j = u % (d_r / 4);
      q = (((h0 + hh) * qstride + d_n) >> 2) + j;
      dst = kp + 64 + hh * 64 + 4 * j;
    }
    if (q >= 0) {
      u32x4 v[1];
      pk_wait_pairs<1>(qkva, q, 0, q + 1, tin, env.err, v);
      dst[0] = bf_lo(v[0].x);
      dst[1] = bf_hi(v[0].x);
      dst[2] = bf_lo(v[0].z);
      dst[3] = bf_hi(v[0].z);
    }
  }
  prof_mark(env, 1);
  rmsnorm_staged(xs, nw, (const uint16_t*)s.w_norm, d_c, s.eps, red);
  if (roper) {
    const int v = fx_tid() / d_r, i = fx_tid() % d_r;
    rp[fx_tid()] = rope64_cs(kp + 64 * v, rc, rsn, i);
  }
  __syncthreads();
  if (env.xcd == 0) {
    // the cache row (plain), complete before any packet of this worker is published
    store_vec_sc1((uint8_t*)s.aux[0] + (size_t)env.step * d_c * 2, xs, d_c);
    if (fx_tid() < d_r / 8) {
      const float* r = rp + 8 * fx_tid();
      u32x4 v;
      v.x = pack2(r[0], r[1]);
      v.y = pack2(r[2], r[3]);
      v.z = pack2(r[4], r[5]);
      v.w = pack2(r[6], r[7]);
      stc16((uint8_t*)s.aux[1] + (size_t)env.step * d_r * 2, fx_tid() * 16, v);
    }
    wait_mem();
  }
  // crow packets of this XCD: latent (d_c / 2) then k_pe (d_r / 2); q_pe packets of its heads
  void* crow = (uint8_t*)s.aux[5] + (size_t)env.xcd * (d_c + d_r) / 2 * 8;
  for (int t = fx_tid(); t < (d_c + d_r) / 4; t += FX_THREADS) {
    const float* r = t < d_c / 4 ? xs + 4 * t : rp + 4 * (t - d_c / 4);
    pk_put2(crow, (uint32_t)(2 * t), pack2(r[0], r[1]), pack2(r[2], r[3]), tout, loc);
  }
  if (fx_tid() < MLA_HP * d_r / 4) {
    const int hh = fx_tid() / (d_r / 4), j = fx_tid() % (d_r / 4);
    const float* r = rp + 64 + hh * 64 + 4 * j;
    pk_put2((void*)s.aux[2], (uint32_t)(((h0 + hh) * d_r) / 2 + 2 * j), pack2(r[0], r[1]), pack2(r[2], r[3]), tout,
            loc);
  }
  prof_mark(env, 2);
}

// FX_OP_MLA_ATTEND (harness/numpy_ref.py:110-149) for the XCD's two heads: split j on rank j % 32,
// tiles of 32 positions, online softmax; partials [split][head][prow] = (o, lse) for the live
// splits. Rows before `step` come from the caches, row `step` from the XCD's crow packets. Each
// worker then publishes a done packet (after its partials are complete).
#define ATT_T 32
#define ATT_ROW 584   // bf16 elements per staged row: 576 + 8 pad (1168 bytes: conflict-free b128 reads)
#define ATT_CHUNKS 72 // 16-byte chunks of one position: 64 latent + 8 rope

// LDS of the attention stage: a pass stages up to two consecutive tiles of one split (64 rows of
// ATT_ROW), then q and the per-pass scratch
#define ATT_PASS (2 * ATT_T)
#define ATT_Q_OFF (ATT_PASS * ATT_ROW * 2)                     // 74752
#define ATT_SP_OFF (ATT_Q_OFF + (MLA_HP * 512 + MLA_HP * 64) * 4)
#define ATT_PB_OFF (ATT_SP_OFF + 2 * MLA_HP * ATT_T * 5 * 4)
#define ATT_HS_OFF (ATT_PB_OFF + 2 * MLA_HP * ATT_T * 4)
static_assert(ATT_HS_OFF + MLA_HP * 5 * 4 <= LDS_STAGE, "attention LDS overlaps the stage descriptor");
#define ATT_LOADS ((ATT_PASS * ATT_CHUNKS + FX_THREADS - 1) / FX_THREADS)   // 18 16-byte loads per thread

// rows t0 .. t0 + nt - 1 (nt <= 64) below `step` into registers (row `step` and later rows are never
// read from the caches: a line loaded before it is written could stay stale in this XCD's caches)
__device__ __forceinline__ void att_issue_rows(u32x4* v, const uint16_t* ckv, const uint16_t* kpe, int t0, int nt,
                                               int step, int d_c, int d_r) {
#pragma unroll
  for (int k = 0; k < ATT_LOADS; ++k) {
    const int q = fx_tid() + k * FX_THREADS;
    const int r = q / ATT_CHUNKS, c = q % ATT_CHUNKS;
    int rr = t0 + (r < nt ? r : 0);
    if (rr >= step) rr = t0 < step ? t0 : -1;
    if (rr < 0) { v[k] = (u32x4){0u, 0u, 0u, 0u}; continue; }   // no cached row yet (step == t0)
    v[k] = c < 64 ? ld16(ckv + (size_t)rr * d_c + c * 8) : ld16(kpe + (size_t)rr * d_r + (c - 64) * 8);
  }
  fx_issue_here();
}

// FX_OP_MLA_ATTEND. A worker walks its splits j = xrank, xrank + 32, .. in passes of up to two
// consecutive 32-position tiles: the scores and value products of the two tiles are computed side by
// side (independent chains), the online softmax still advances tile by tile in position order.
__device__ __forceinline__ void op_mla_attend(const fx_stage& s, FxEnv& env) {
  const int nh = s.n_rows, d_c = s.d_c, d_r = s.d_r, prow = s.prow;
  const int h0 = env.xcd * MLA_HP;
  const int step = env.step;
  const int split = s.split;
  const int n_live = (step + 1 + split - 1) / split;
  const float scale = s.scale;
  const uint32_t tin = tag_in(s, env, 0);
  uint16_t* buf = (uint16_t*)env.lds;                            // [64][ATT_ROW]
  float* ql = (float*)(env.lds + ATT_Q_OFF);                     // [2][512]
  float* qp = ql + MLA_HP * 512;                                 // [2][64]
  float* sp = (float*)(env.lds + ATT_SP_OFF);                    // [2 tiles][2 heads][32][5] partial scores
  float* pb = (float*)(env.lds + ATT_PB_OFF);                    // [2 tiles][2 heads][32] bf16(p)
  float* hs = (float*)(env.lds + ATT_HS_OFF);                    // [2 heads][4]: m, l, alpha A, alpha B
  float* psB = hs + MLA_HP * 4;                                  // [2 heads] tile B's sum of p
  const uint16_t* ckv = (const uint16_t*)s.aux[0];
  const uint16_t* kpe = (const uint16_t*)s.aux[1];
  const void* crow = (const uint8_t*)s.aux[5] + (size_t)env.xcd * (d_c + d_r) / 2 * 8;
  void* part = (void*)s.out;
  int done = 0;
  bool have_q = false;
  auto split_hi = [&](int j) { const int h = j * split + split; return h > step + 1 ? step + 1 : h; };
  auto pass_rows = [&](int t0, int hi) { return (t0 + ATT_PASS < hi ? t0 + ATT_PASS : hi) - t0; };
  // the rows of the next pass are requested as soon as the current pass is staged in LDS
  u32x4 v[ATT_LOADS];
  if (env.xrank < n_live) {
    const int lo = env.xrank * split;
    att_issue_rows(v, ckv, kpe, lo, pass_rows(lo, split_hi(env.xrank)), step, d_c, d_r);
  }
  // online-softmax state of the running split (wave 0, lane (h, t): identical on a head's 32 lanes)
  float m_run = -__builtin_inff(), l_run = 0.0f;
  for (int j = env.xrank; j < n_live; j += env.xworkers) {
    const int lo = j * split;
    const int hi = split_hi(j);
    __syncthreads();
    if (!have_q) {
      // q rows of the XCD's heads: ql 2 x 128 pairs (thread t), qp 2 x 16 pairs (threads 0..31)
      const int t = fx_tid();
      {
        const int hh = t / (d_c / 4), i = t % (d_c / 4);
        const int q = ((h0 + hh) * d_c >> 2) + i;
        u32x4 w[1];
        pk_wait_pairs<1>((const void*)s.x, q, 0, q + 1, tin, env.err, w);
        float* dst = ql + hh * 512 + 4 * i;
        dst[0] = bf_lo(w[0].x);
        dst[1] = bf_hi(w[0].x);
        dst[2] = bf_lo(w[0].z);
        dst[3] = bf_hi(w[0].z);
      }
      if (t < MLA_HP * d_r / 4) {
        const int hh = t / (d_r / 4), i = t % (d_r / 4);
        const int q = ((h0 + hh) * d_r >> 2) + i;
        u32x4 w[1];
        pk_wait_pairs<1>((const void*)s.aux[2], q, 0, q + 1, tin, env.err, w);
        float* dst = qp + hh * 64 + 4 * i;
        dst[0] = bf_lo(w[0].x);
        dst[1] = bf_hi(w[0].x);
        dst[2] = bf_lo(w[0].z);
        dst[3] = bf_hi(w[0].z);
      }
      have_q = true;
      prof_mark(env, 1);
    }
    m_run = -__builtin_inff();
    l_run = 0.0f;
    // accumulators: thread -> head ph = tid >> 7, columns pc .. pc + 3
    const int ph = fx_tid() >> 7, pc = (fx_tid() & 127) * 4;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int t0 = lo; t0 < hi; t0 += ATT_PASS) {
      const int nt = pass_rows(t0, hi);
      const int ntA = nt < ATT_T ? nt : ATT_T, ntB = nt - ntA;
#pragma unroll
      for (int k = 0; k < ATT_LOADS; ++k) {
        const int q = fx_tid() + k * FX_THREADS;
        const int r = q / ATT_CHUNKS, c = q % ATT_CHUNKS;
        if (r < nt && t0 + r != step) *(u32x4*)(buf + r * ATT_ROW + c * 8) = v[k];
      }
      {
        // request the next pass (this split's next 64 positions, or the worker's next split)
        int nj = j, nt0 = t0 + ATT_PASS, nhi = hi;
        if (nt0 >= hi) { nj = j + env.xworkers; nt0 = nj * split; nhi = nj < n_live ? split_hi(nj) : 0; }
        if (nj < n_live) att_issue_rows(v, ckv, kpe, nt0, pass_rows(nt0, nhi), step, d_c, d_r);
      }
      if (step >= t0 && step < t0 + nt && fx_tid() < (d_c + d_r) / 4) {
        // row `step` from the XCD's packet copy of the cache row
        u32x4 w[1];
        pk_wait_pairs<1>(crow, fx_tid(), 0, fx_tid() + 1, tin, env.err, w);
        uint32_t* dst = (uint32_t*)(buf + (step - t0) * ATT_ROW) + 2 * fx_tid();
        dst[0] = w[0].x;
        dst[1] = w[0].z;
      }
      __syncthreads();
      // scores: thread (h, k, t): chain k over latent columns [128k, 128k + 128) of row t of tile A
      // and of tile B side by side; k == 0 also the rope chains; s = ((((n0 + n1) + n2) + n3) + pe)
      // * scale. Consecutive lanes take consecutive rows (row stride 1168 B: conflict-free b128
      // reads) and share q (broadcast). A missing tile-B row is computed on stale data and dropped.
      {
        const int h = fx_tid() >> 7, k = (fx_tid() >> 5) & 3, t = fx_tid() & 31;
        float a = 0.0f, a2 = 0.0f, b = 0.0f, b2 = 0.0f;
        const uint16_t* kr = buf + t * ATT_ROW;
        const uint16_t* kr2 = buf + (ATT_T + t) * ATT_ROW;
        const float* qr = ql + h * 512;
        if (t < ntA && ntB == 0) {
          // tile A alone (one 32-position tile in the pass): the same chains without tile B's
#pragma unroll 8
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
              const float4 q0 = *(const float4*)(qpr + r), q1 = *(const float4*)(qpr + r + 4);
              b = __builtin_fmaf(q0.x, bf_lo(kv.x), b);
              b = __builtin_fmaf(q0.y, bf_hi(kv.x), b);
              b = __builtin_fmaf(q0.z, bf_lo(kv.y), b);
              b = __builtin_fmaf(q0.w, bf_hi(kv.y), b);
              b = __builtin_fmaf(q1.x, bf_lo(kv.z), b);
              b = __builtin_fmaf(q1.y, bf_hi(kv.z), b);
              b = __builtin_fmaf(q1.z, bf_lo(kv.w), b);
              b = __builtin_fmaf(q1.w, bf_hi(kv.w), b);
            }
          }
        } else if (t < ntA) {
#pragma unroll 8
          for (int c = k * 128; c < k * 128 + 128; c += 8) {
            const u32x4 kv = *(const u32x4*)(kr + c);
            const u32x4 kv2 = *(const u32x4*)(kr2 + c);
            const float4 q0 = *(const float4*)(qr + c), q1 = *(const float4*)(qr + c + 4);
            a = __builtin_fmaf(q0.x, bf_lo(kv.x), a);
            a2 = __builtin_fmaf(q0.x, bf_lo(kv2.x), a2);
            a = __builtin_fmaf(q0.y, bf_hi(kv.x), a);
            a2 = __builtin_fmaf(q0.y, bf_hi(kv2.x), a2);
            a = __builtin_fmaf(q0.z, bf_lo(kv.y), a);
            a2 = __builtin_fmaf(q0.z, bf_lo(kv2.y), a2);
            a = __builtin_fmaf(q0.w, bf_hi(kv.y), a);
            a2 = __builtin_fmaf(q0.w, bf_hi(kv2.y), a2);
            a = __builtin_fmaf(q1.x, bf_lo(kv.z), a);
            a2 = __builtin_fmaf(q1.x, bf_lo(kv2.z), a2);
            a = __builtin_fmaf(q1.y, bf_hi(kv.z), a);
            a2 = __builtin_fmaf(q1.y, bf_hi(kv2.z), a2);
            a = __builtin_fmaf(q1.z, bf_lo(kv.w), a);
            a2 = __builtin_fmaf(q1.z, bf_lo(kv2.w), a2);
            a = __builtin_fmaf(q1.w, bf_hi(kv.w), a);
            a2 = __builtin_fmaf(q1.w, bf_hi(kv2.w), a2);
          }
          if (k == 0) {
            const float* qpr = qp + h * 64;
#pragma unroll
            for (int r = 0; r < 64; r += 8) {
              const u32x4 kv = *(const u32x4*)(kr + 512 + r);
              const u32x4 kv2 = *(const u32x4*)(kr2 + 512 + r);
              const float4 q0 = *(const float4*)(qpr + r), q1 = *(const float4*)(qpr + r + 4);
              b = __builtin_fmaf(q0.x, bf_lo(kv.x), b);
              b2 = __builtin_fmaf(q0.x, bf_lo(kv2.x), b2);
              b = __builtin_fmaf(q0.y, bf_hi(kv.x), b);
              b2 = __builtin_fmaf(q0.y, bf_hi(kv2.x), b2);
              b = __builtin_fmaf(q0.z, bf_lo(kv.y), b);
              b2 = __builtin_fmaf(q0.z, bf_lo(kv2.y), b2);
              b = __builtin_fmaf(q0.w, bf_hi(kv.y), b);
              b2 = __builtin_fmaf(q0.w, bf_hi(kv2.y), b2);
              b = __builtin_fmaf(q1.x, bf_lo(kv.z), b);
              b2 = __builtin_fmaf(q1.x, bf_lo(kv2.z), b2);
              b = __builtin_fmaf(q1.y, bf_hi(kv.z), b);
              b2 = __builtin_fmaf(q1.y, bf_hi(kv2.z), b2);
              b = __builtin_fmaf(q1.z, bf_lo(kv.w), b);
              b2 = __builtin_fmaf(q1.z, bf_lo(kv2.w), b2);
              b = __builtin_fmaf(q1.w, bf_hi(kv.w), b);
              b2 = __builtin_fmaf(q1.w, bf_hi(kv2.w), b2);
            }
          }
        }
        float* spA = sp + (h * ATT_T + t) * 5;
        float* spB = sp + ((MLA_HP + h) * ATT_T + t) * 5;
        spA[k] = a;
        spB[k] = a2;
        if (k == 0) { spA[4] = b; spB[4] = b2; }
      }
      __syncthreads();
      if (done == 0 && t0 == lo) prof_mark(env, 4);
      // softmax, tile A on wave 0 and tile B on wave 1 (lane = h * 32 + t): m_A = max(m, max_t s_A),
      // m_B = max(m_A, max_t s_B), alpha = exp(m_prev - m_new), p = exp(s - m_new); each tile's sum
      // of p runs sequentially in t (lane by lane through scalar reads). The running (m, l) stays on
      // wave 0: l = (l * alpha_A + psum_A) * alpha_B + psum_B, the tile order of the spec.
      if (fx_tid() < 64 || (fx_tid() < 128 && ntB > 0)) {
        const int tile = fx_tid() >> 6;
        const int h = (fx_tid() >> 5) & 1, t = fx_tid() & 31;
        auto tile_score = [&](int tl, int ntt) {
          float sc = -__builtin_inff();
          if (t < ntt) {
            const float* q = sp + ((tl * MLA_HP + h) * ATT_T + t) * 5;
            float v2 = q[0] + q[1];
            v2 = v2 + q[2];
            v2 = v2 + q[3];
            v2 = v2 + q[4];
            sc = v2 * scale;
          }
          return sc;
        };
        auto max32 = [&](float x) {
          x = fmaxf(x, xor_lane<1>(x));
          x = fmaxf(x, xor_lane<2>(x));
          x = fmaxf(x, xor_lane<4>(x));
          x = fmaxf(x, xor_lane<8>(x));
          return fmaxf(x, xor_lane<16>(x));
        };
        const float scA = tile_score(0, ntA);
        const float mtA = max32(scA);
        const float mA = m_run > mtA ? m_run : mtA;          // m after tile A
        float mB = mA;                                       // m after tile B
        float scB = -__builtin_inff();
        if (ntB > 0) {
          scB = tile_score(1, ntB);
          const float mtB = max32(scB);
          mB = mA > mtB ? mA : mtB;
        }
        const float sc = tile ? scB : scA;
        const float m_prev = tile ? mA : m_run, m_new = tile ? mB : mA;
        const int ntt = tile ? ntB : ntA;
        const float alpha = exp_s(m_prev - m_new);
        const float p = t < ntt ? exp_s(sc - m_new) : 0.0f;
        pb[(tile * MLA_HP + h) * ATT_T + t] = bf16r(p);
        float ps0 = 0.0f, ps1 = 0.0f;
#pragma unroll
        for (int u = 0; u < 32; ++u) {
          ps0 = ps0 + __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, p), u));
          ps1 = ps1 + __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, p), 32 + u));
        }
        const float ps = h ? ps1 : ps0;
        if (t == 0) {
          hs[h * 4 + 2 + tile] = alpha;
          if (tile) psB[h] = ps;
        }
        if (tile == 0) l_run = l_run * alpha + ps;
        m_run = mB;   // waves 0 and 1 track the same m
      }
      __syncthreads();
      if (done == 0 && t0 == lo) prof_mark(env, 5);
      if (fx_tid() < 64) {
        // wave 0 folds tile B's sum into l and publishes (m, l) for the split's output
        const int h = (fx_tid() >> 5) & 1, t = fx_tid() & 31;
        if (ntB > 0) l_run = l_run * hs[h * 4 + 3] + psB[h];
        if (t == 0) {
          hs[h * 4 + 0] = m_run;
          hs[h * 4 + 1] = l_run;
        }
      }
      // value products, tile A and tile B side by side, each sequential in t:
      // tp[c] = sum_t bf16(p_t) v_t[c]; acc = acc * alpha_A + tp_A, then acc * alpha_B + tp_B
      {
        float tp[4] = {0.0f, 0.0f, 0.0f, 0.0f}, tq[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        const float* pA = pb + ph * ATT_T;
        const float* pB = pb + (MLA_HP + ph) * ATT_T;
        auto rows8 = [&](int t8, u32x2* kv, u32x2* kv2, float* pv, float* pv2) {
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            kv[u] = *(const u32x2*)(buf + (t8 + u) * ATT_ROW + pc);
            kv2[u] = *(const u32x2*)(buf + (ATT_T + t8 + u) * ATT_ROW + pc);
            pv[u] = pA[t8 + u];
            pv2[u] = pB[t8 + u];
          }
        };
        if (ntA == ATT_T && ntB == 0) {
          // one full tile
#pragma unroll
          for (int t8 = 0; t8 < ATT_T; t8 += 8) {
            u32x2 kv[8];
            float pv[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
              kv[u] = *(const u32x2*)(buf + (t8 + u) * ATT_ROW + pc);
              pv[u] = pA[t8 + u];
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
              tp[0] = __builtin_fmaf(pv[u], bf_lo(kv[u].x), tp[0]);
              tp[1] = __builtin_fmaf(pv[u], bf_hi(kv[u].x), tp[1]);
              tp[2] = __builtin_fmaf(pv[u], bf_lo(kv[u].y), tp[2]);
              tp[3] = __builtin_fmaf(pv[u], bf_hi(kv[u].y), tp[3]);
            }
          }
        } else if (ntA == ATT_T && ntB == ATT_T) {
          // two full tiles: no row tests
#pragma unroll
          for (int t8 = 0; t8 < ATT_T; t8 += 8) {
            u32x2 kv[8], kv2[8];
            float pv[8], pv2[8];
            rows8(t8, kv, kv2, pv, pv2);
#pragma unroll
            for (int u = 0; u < 8; ++u) {
              tp[0] = __builtin_fmaf(pv[u], bf_lo(kv[u].x), tp[0]);
              tq[0] = __builtin_fmaf(pv2[u], bf_lo(kv2[u].x), tq[0]);
              tp[1] = __builtin_fmaf(pv[u], bf_hi(kv[u].x), tp[1]);
              tq[1] = __builtin_fmaf(pv2[u], bf_hi(kv2[u].x), tq[1]);
              tp[2] = __builtin_fmaf(pv[u], bf_lo(kv[u].y), tp[2]);
              tq[2] = __builtin_fmaf(pv2[u], bf_lo(kv2[u].y), tq[2]);
              tp[3] = __builtin_fmaf(pv[u], bf_hi(kv[u].y), tp[3]);
              tq[3] = __builtin_fmaf(pv2[u], bf_hi(kv2[u].y), tq[3]);
            }
          }
        } else {
          // 8 rows of each tile loaded at a time, then their fmas in t order (rows past a tile's end
          // carry p = 0 and are skipped: their staged rows are stale)
          for (int t8 = 0; t8 < ntA; t8 += 8) {
            u32x2 kv[8], kv2[8];
            float pv[8], pv2[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
              kv[u] = *(const u32x2*)(buf + (t8 + u) * ATT_ROW + pc);
              kv2[u] = *(const u32x2*)(buf + (ATT_T + t8 + u) * ATT_ROW + pc);
              pv[u] = pA[t8 + u];
              pv2[u] = pB[t8 + u];
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
              if (t8 + u < ntA) {
                tp[0] = __builtin_fmaf(pv[u], bf_lo(kv[u].x), tp[0]);
                tp[1] = __builtin_fmaf(pv[u], bf_hi(kv[u].x), tp[1]);
                tp[2] = __builtin_fmaf(pv[u], bf_lo(kv[u].y), tp[2]);
                tp[3] = __builtin_fmaf(pv[u], bf_hi(kv[u].y), tp[3]);
              }
              if (t8 + u < ntB) {
                tq[0] = __builtin_fmaf(pv2[u], bf_lo(kv2[u].x), tq[0]);
                tq[1] = __builtin_fmaf(pv2[u], bf_hi(kv2[u].x), tq[1]);
                tq[2] = __builtin_fmaf(pv2[u], bf_lo(kv2[u].y), tq[2]);
                tq[3] = __builtin_fmaf(pv2[u], bf_hi(kv2[u].y), tq[3]);
              }
            }
          }
        }
        const float alphaA = hs[ph * 4 + 2];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float a = acc[c] * alphaA;
          acc[c] = a + tp[c];
        }
        if (ntB > 0) {
          const float alphaB = hs[ph * 4 + 3];
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const float a = acc[c] * alphaB;
            acc[c] = a + tq[c];
          }
        }
      }
      __syncthreads();
      if (done == 0 && t0 == lo) prof_mark(env, 6);
    }
    // o = acc / l, lse = m + log(l)
    {
      const uint32_t base = (uint32_t)((j * nh + h0 + ph) * prow);
      const float l = hs[ph * 4 + 1];
      u32x4 o;
      o.x = __float_as_uint(acc[0] / l);
      o.y = __float_as_uint(acc[1] / l);
      o.z = __float_as_uint(acc[2] / l);
      o.w = __float_as_uint(acc[3] / l);
      // read only by this XCD's merge (its heads): XCD-local stores
      stl16(part, (base + pc) * 4, o);
      if ((fx_tid() & 127) == 0) stl4(part, (base + d_c) * 4, __float_as_uint(hs[ph * 4 + 0] + log_s(l)));
    }
    ++done;
  }
  // done packet: this worker's partials are complete
  wait_mem();
  __syncthreads();
  prof_mark(env, 7);
  if (fx_tid() == 0)
    pk_put((void*)s.aux[6], (uint32_t)(env.xcd * FX_XWORKERS + env.xrank), (uint32_t)done, tag_out(env), true);
  prof_mark(env, 2);
}

// The merge of head h (harness/numpy_ref.py:152-165): M = max lse, w_j = exp(lse_j - M), o = (sum_j
// w_j o_j, sequential fma) / (sum_j w_j, sequential) -> bf16, over the first `live` splits' partials
// ([split][head][prow]: o, then lse). xs[0, d_c) receives o (thread t: columns 2t, 2t + 1); wj
// (LDS, live floats) and red[0] are scratch. The caller syncs before reading xs.
#define MERGE_BATCH 40   // splits whose partials are requested at once (every live split up to ctx 1280)
__device__ __forceinline__ void merge_head(const void* part, int nh, int h, int prow, int d_c, int live, float* xs,
                                           float* wj, float* red, const FxEnv& env) {
  // wave 0 requests the lse of splits lane, lane + 64 first: loads complete in issue order, so the
  // weights below need not wait for the wave's partial-o loads
  float l0 = -__builtin_inff(), l1 = -__builtin_inff();
  if (wave_id() == 0) {
    if (lane_id() < live) l0 = ldcf(part, (uint32_t)((lane_id() * nh + h) * prow + d_c));
    if (lane_id() + 64 < live) l1 = ldcf(part, (uint32_t)(((lane_id() + 64) * nh + h) * prow + d_c));
  }
  // every thread: 2 columns of o; the first MERGE_BATCH live splits' values are requested before
  // anything waits (live is uniform: the branches are scalar)
  const int pc = fx_tid() * 2;
  u32x2 o[MERGE_BATCH];
#pragma unroll
  for (int k = 0; k < MERGE_BATCH; ++k)
    if (k < live) o[k] = ldc8(part, (uint32_t)((k * nh + h) * prow + pc) * 4);
  // wave 0: lse_j, M = max lse, w_j = exp(lse_j - M) into LDS, den = sum_j w_j in j order
  if (wave_id() == 0) {
    // the rest of the lse (more than 128 splits) from LDS
    float mx = fmaxf(l0, l1);
    for (int j = lane_id() + 128; j < live; j += 64) {
      const float v = ldcf(part, (uint32_t)((j * nh + h) * prow + d_c));
      wj[j] = v;
      mx = fmaxf(mx, v);
    }
    mx = wave_max(mx);
    float den = 0.0f;
    for (int j0 = 0; j0 < live; j0 += 64) {
      const int j = j0 + lane_id();
      const float lse = j0 == 0 ? l0 : (j0 == 64 ? l1 : (j < live ? wj[j] : -__builtin_inff()));
      const float w = j < live ? exp_s(lse - mx) : 0.0f;
      if (j < live) wj[j] = w;
      const int n = live - j0 < 64 ? live - j0 : 64;
      for (int u = 0; u < n; ++u) den = den + __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), u));
    }
    if (lane_id() == 0) red[0] = den;
    prof_mark(env, 4);
  }
  __syncthreads();
  // num = sum_j w_j o_j[c] in j order (fma)
  float num[2] = {0.0f, 0.0f};
  for (int j0 = 0; j0 < live; j0 += MERGE_BATCH) {
    if (j0 > 0) {
#pragma unroll
      for (int k = 0; k < MERGE_BATCH; ++k)
        if (j0 + k < live) o[k] = ldc8(part, (uint32_t)(((j0 + k) * nh + h) * prow + pc) * 4);
    }
#pragma unroll
    for (int k = 0; k < MERGE_BATCH; ++k) {
      if (j0 + k >= live) continue;
      const float w = wj[j0 + k];
      num[0] = __builtin_fmaf(w, __uint_as_float(o[k].x), num[0]);
      num[1] = __builtin_fmaf(w, __uint_as_float(o[k].y), num[1]);
    }
  }
  prof_mark(env, 6);
  __syncthreads();
  const float den = red[0];
  xs[pc] = bf16r(num[0] / den);
  xs[pc + 1] = bf16r(num[1] / den);
}

// The same merge by the 8 workers of a head on one XCD (matrix-core attention, more than
// MERGE_SLICE_MIN live splits): worker v of the head merges columns [64 v, 64 v + 64) only.
// Its 64-column slices of every live split's partial come into LDS with direct-to-LDS loads, all
// requested at once (one round trip instead of one per MERGE_BATCH splits, and an eighth of the
// bytes per worker); column c is then num = sum_j w_j o_j[c] in j order (fma) / den, the same
// arithmetic as merge_head. The 8 slices are exchanged as XCD-local packets (opk, [nh][d_c] pk16,
// tag `tag`) and xs[0, d_c) receives the whole head; ends with a barrier, as every thread then reads
// columns other threads wrote.
#ifndef MERGE_SLICE_MIN
#define MERGE_SLICE_MIN 8   // the sliced merge takes more live splits than this
#endif
#define MERGE_SLICE_COLS 64
#define MERGE_SLICE_MAX 176                 // live splits whose slices fit (4 per KiB)
#define MERGE_SLICE_LDS (LDS_TILE + 2048)   // the slices' LDS, past the weights wj[live] at LDS_TILE
static_assert(MERGE_SLICE_LDS + MERGE_SLICE_MAX / 4 * 1024 <= LDS_STAGE, "merge slices overlap the stage LDS");
static_assert(MERGE_SLICE_MAX * 4 <= 2048, "the merge weights overlap the slices");
__device__ __forceinline__ void merge_head_sliced(const void* part, int nh, int h, int prow, int d_c, int live, int v,
                                                  float* xs, float* wj, float* red, void* opk, uint32_t tag,
                                                  const FxEnv& env) {
  char* land = env.lds + MERGE_SLICE_LDS;
  // wave 0: the lse of splits lane, lane + 64 first (loads complete in issue order)
  float l0 = -__builtin_inff(), l1 = -__builtin_inff();
  if (wave_id() == 0) {
    if (lane_id() < live) l0 = ldcf(part, (uint32_t)((lane_id() * nh + h) * prow + d_c));
    if (lane_id() + 64 < live) l1 = ldcf(part, (uint32_t)(((lane_id() + 64) * nh + h) * prow + d_c));
  }
  // every wave: instruction k brings splits 4k .. 4k + 3 (16 lanes x 16 B each) to land + 1 KiB k
  const int nins = (live + 3) >> 2;
  const int lane = lane_id();
  for (int k = wave_id(); k < nins; k += FX_WAVES) {
    int j = 4 * k + (lane >> 4);
    j = j < live ? j : live - 1;
    const char* src = (const char*)part + ((size_t)(j * nh + h) * prow + MERGE_SLICE_COLS * v) * 4 + (lane & 15) * 16;
    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                     (__attribute__((address_space(3))) void*)(land + k * 1024), 16, 0, FX_SC1);
  }
  if (wave_id() == 0) {
    float mx = fmaxf(l0, l1);
    for (int j = lane + 128; j < live; j += 64) {
      const float x = ldcf(part, (uint32_t)((j * nh + h) * prow + d_c));
      wj[j] = x;
      mx = fmaxf(mx, x);
    }
    mx = wave_max(mx);
    float den = 0.0f;
    for (int j0 = 0; j0 < live; j0 += 64) {
      const int j = j0 + lane;
      const float lse = j0 == 0 ? l0 : (j0 == 64 ? l1 : (j < live ? wj[j] : -__builtin_inff()));
      const float w = j < live ? exp_s(lse - mx) : 0.0f;
      if (j < live) wj[j] = w;
      const int n = live - j0 < 64 ? live - j0 : 64;
      for (int u = 0; u < n; ++u) den = den + __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), u));
    }
    if (lane == 0) red[0] = den;
    prof_mark(env, 4);
  }
  wait_mem();
  __syncthreads();
  const int c0 = MERGE_SLICE_COLS * v;
  if (fx_tid() < MERGE_SLICE_COLS) {
    const float* P = (const float*)land + fx_tid();
    float num = 0.0f;
    for (int j = 0; j < live; ++j) num = __builtin_fmaf(wj[j], P[j * MERGE_SLICE_COLS], num);
    xs[c0 + fx_tid()] = bf16r(num / red[0]);
  }
  prof_mark(env, 6);
  __syncthreads();
  if (fx_tid() < MERGE_SLICE_COLS / 4) {
    const float* r = xs + c0 + 4 * fx_tid();
    pk_put2(opk, (uint32_t)((h * d_c + c0) / 2 + 2 * fx_tid()), pack2(r[0], r[1]), pack2(r[2], r[3]), tag, true);
  }
  // the head's d_c / 4 pairs of packets from its 8 workers (this one's included)
  if (fx_tid() < (d_c >> 2)) {
    u32x4 w[1];
    const int q = (h * d_c >> 2) + fx_tid();
    pk_wait_pairs<1>(opk, q, 0, q + 1, tag, env.err, w);
    xs[4 * fx_tid() + 0] = bf_lo(w[0].x);
    xs[4 * fx_tid() + 1] = bf_hi(w[0].x);
    xs[4 * fx_tid() + 2] = bf_lo(w[0].z);
    xs[4 * fx_tid() + 3] = bf_hi(w[0].z);
  }
  __syncthreads();
}

// FX_OP_MLA_MERGE_UV: ranks 0..15 / 16..31 of XCD x merge head 2x / 2x + 1 (merge_head), then
// attn[h*d_v + v] = bf16(dot(o, W_uv[h][v])) for 8 rows v each (harness/numpy_ref.py:168-174).
// With FX_F_MFMA the merge runs on ranks 16..31 of every XCD only (workers 128..255), 8 per head
// (16 W_uv rows each): ranks 16..23 / 24..31 of XCD x take head 2x / 2x + 1. Every merge worker
// reads all of its head's partials; the eight readers of a head share one XCD's L2, so HBM sees
// each partial once, and the attention's workers (0 .. live - 1) are not on the merge's critical
// path while live <= 128.
#define MERGE_MFMA_FIRST_RANK 16
#define MERGE_MFMA_PER_HEAD 8
__device__ __forceinline__ void op_mla_merge_uv(const fx_stage& s, FxEnv& env) {
  const int nh = s.n_rows, d_c = s.d_c, d_v = s.d_n, prow = s.prow;
  const bool mfma = (s.flags & FX_F_MFMA) != 0;
  if (mfma && env.xrank < MERGE_MFMA_FIRST_RANK) return;
  const int mr = env.xrank - MERGE_MFMA_FIRST_RANK;
  const int h = env.xcd * MLA_HP + (mfma ? mr / MERGE_MFMA_PER_HEAD : env.xrank >> 4);
  const int nrows = mfma ? d_v / MERGE_MFMA_PER_HEAD : d_v / 16;   // 16 or 8
  const int v0 = mfma ? (mr % MERGE_MFMA_PER_HEAD) * nrows : (env.xrank & 15) * nrows;
  const int live = (env.step + 1 + s.split - 1) / s.split;
  float* xs = (float*)(env.lds + LDS_XS);
  float* red = (float*)(env.lds + LDS_RED);
  const uint16_t* W = (const uint16_t*)s.w + (size_t)h * d_v * d_c;
  auto rowof = [&](int g, int i) { const int r = v0 + g * 4 + i; return r < v0 + nrows ? r : -1; };
  const int ngroups = (nrows + 3) / 4;
  Tile<4, 1> t0;
  gemv_prime(t0, W, d_c, ngroups, rowof);
  if (mfma) {
    // split j ran on worker j % 256: the done packets of workers 0 .. min(live, 256) - 1
    if (wave_id() == 0)
      pk_wait_singles<4>((const void*)s.aux[6], lane_id(), 64, live < FX_WORKERS ? live : FX_WORKERS,
                         tag_in(s, env, 0), env.err);
  } else if (wave_id() == 0) {
    // the XCD's 32 done packets
    u32x4 v[1];
    const int first = env.xcd * FX_XWORKERS / 2;
    pk_wait_pairs<1>((const void*)s.aux[6], first + (lane_id() & 15), 0, first + FX_XWORKERS / 2, tag_in(s, env, 0),
                     env.err, v);
  }
  __syncthreads();
  prof_mark(env, 1);
  const bool sliced = mfma && s.aux[7] && live > MERGE_SLICE_MIN && live <= MERGE_SLICE_MAX;
  if (sliced)
    merge_head_sliced((const void*)s.x, nh, h, prow, d_c, live, mr % MERGE_MFMA_PER_HEAD, xs,
                      (float*)(env.lds + LDS_TILE), red, (void*)s.aux[7], tag_out(env), env);
  else
    merge_head((const void*)s.x, nh, h, prow, d_c, live, xs, (float*)(env.lds + LDS_TILE), red, env);
  const int pc = fx_tid() * 2;
  if (v0 == 0 && s.aux[4]) stc4((void*)s.aux[4], (uint32_t)(h * d_c + pc) * 2, pack2(xs[pc], xs[pc + 1]));
  __syncthreads();
  prof_mark(env, 5);
  float* o8 = red + 16;
  gemv_pipe(t0, W, d_c, xs, ngroups, rowof, [&](int g, const int* row, const float* acc) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (row[i] >= 0 && lane_id() == 0) o8[row[i] - v0] = bf16r(acc[i]);
  });
  __syncthreads();
  if (fx_tid() < nrows / 4) {
    const float* r = o8 + 4 * fx_tid();
    pk_put2((void*)s.out, (uint32_t)((h * d_v + v0) / 2 + 2 * fx_tid()), pack2(r[0], r[1]), pack2(r[2], r[3]),
            tag_out(env));
  }
  prof_mark(env, 2);
}
