// MLA absorbed decode attention on gfx950's matrix cores (harness/numpy_ref.py:110-149; the
// reference's mla_attend_mfma_mi300.cuh:49-282). The latent KV head is shared by all 16 query heads
// (MQA), so the work is split by positions, not heads: split j (positions [j * split, (j + 1) *
// split)) runs on worker j % 256 for all 16 heads at once, and every cache row is read once per
// layer. Per 32-position tile:
//   QK^T  S[16 heads][32 positions] = two 16x16 output tiles (waves 0, 1), each 18 chained
//         v_mfma_f32_16x16x32_bf16 over the 576-wide row (latent columns, then rope columns);
//         A = Q, B = 16 staged cache rows (both bf16 in LDS, ds_read_b128);
//   softmax per head over the tile (four heads per wave): max, exp, the two 16-position
//         butterflies, bf16(p);
//   PV    tile_pv[16 heads][512 columns] = 32 16x16 output tiles (8 per wave), one instruction over
//         the tile's 32 positions each; A = bf16(p), B = the staged value rows read transposed
//         (ds_read_b64_tr_b16), then acc = acc * alpha + tile_pv on the VALU.
// The order of every sum is the instruction's own (four groups of 8 products per instruction, see
// oracle/fleet_oracle.c or_mfma_dot32), restated by the oracle's or_mla_attend_mfma.
#pragma once
#include "fx_mla.h"

typedef __bf16 fx_bf16x8 __attribute__((ext_vector_type(8)));
typedef short fx_i16x4 __attribute__((ext_vector_type(4)));
typedef float fx_f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) char lds_char;

#define AM_T 32                       // positions per tile
#define AM_NH 16                      // heads (the instruction's M)
#define AM_DK 576                     // 512 latent + 64 rope columns per row
#define AM_KS (AM_DK / 32)            // 18 K-steps of the score chain
#define AM_ROW 1168                   // bytes per staged row: 576 bf16 + 16 B pad
#define AM_Q_OFF 0                                    // Q [16][AM_ROW]
#define AM_KV_OFF (AM_NH * AM_ROW)                    // tile rows [32][AM_ROW]
#define AM_S_OFF (AM_KV_OFF + AM_T * AM_ROW)          // scaled scores f32 [16][32]
#define AM_P_ROW 80                                   // bytes per row of bf16(p) (32 + 8 pad)
#define AM_P_OFF (AM_S_OFF + AM_NH * AM_T * 4)        // bf16(p) [16][AM_P_ROW]
#define AM_H_OFF (AM_P_OFF + AM_NH * AM_P_ROW)        // per head: alpha [16], m [16], l [16]
#define AM_LOADS ((AM_T * (AM_DK / 8) + FX_THREADS - 1) / FX_THREADS)   // 9 16-byte loads per thread
static_assert(AM_H_OFF + 3 * AM_NH * 4 <= LDS_STAGE, "MFMA attention LDS overlaps the stage descriptor");
static_assert(AM_T * (AM_DK / 8) == AM_LOADS * FX_THREADS, "a tile is whole 16-byte loads per thread");

__device__ __forceinline__ fx_bf16x8 lds_b128(const char* p) { return *(const fx_bf16x8*)p; }
__device__ __forceinline__ fx_i16x4 lds_tr16(const char* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) fx_i16x4*)(lds_char*)(void*)p);
}

// rows t0 .. t0 + nt - 1 of a tile that lie below `step`, into registers (chunk q = tid + 256 k:
// row q / 72, 16-byte chunk q % 72: latent chunks 0..63, rope chunks 64..71). Row `step` and later
// rows are never read from the caches (they come from the cache-row packets or are zero).
// (buffer loads with 32-bit byte offsets: the row index stays below 2^21 for any cache that fits)
__device__ __forceinline__ void am_issue_rows(u32x4* v, const uint16_t* ckv, const uint16_t* kpe, int t0, int nt,
                                              int step) {
  const __amdgpu_buffer_rsrc_t rc = rsrc(ckv), rk = rsrc(kpe);
#pragma unroll
  for (int k = 0; k < AM_LOADS; ++k) {
    const int q = fx_tid() + k * FX_THREADS;
    const int r = q / 72, c = q % 72;
    const int rr = t0 + r;
    if (r >= nt || rr >= step) { v[k] = (u32x4){0u, 0u, 0u, 0u}; continue; }
    v[k] = c < 64 ? __builtin_amdgcn_raw_buffer_load_b128(rc, (uint32_t)(rr * 1024 + c * 16), 0, 0)
                  : __builtin_amdgcn_raw_buffer_load_b128(rk, (uint32_t)(rr * 128 + (c - 64) * 16), 0, 0);
  }
  fx_issue_here();
}

// The matrix-core attention of splits j = j0, j0 + jstep, .. below the live count, every head per
// split. Inputs: q of every head (ql_nope packets, 2048 pairs, and q_pe packets aux[2], 256 pairs),
// row `step` from the crow packets of this XCD (aux[5]); the cached rows from c_kv (aux[0]) and
// k_pe (aux[1]). Partials ([split][head][prow]: o, then lse) are stored device-coherent, or
// XCD-local (`local`: every reader runs on this XCD). after_q() runs once q is in LDS. Returns the
// number of splits done; the caller waits for the stores and publishes its done packet.
template <class AfterQ>
__device__ __forceinline__ int am_attend(const fx_stage& s, FxEnv& env, const void* qln, void* part, int j0, int jstep,
                                         bool local, uint32_t tin, AfterQ after_q) {
  const int step = env.step, split = s.split, prow = s.prow;
  const int n_live = (step + 1 + split - 1) / split;
  const float scale = s.scale;
  char* lds = env.lds;
  const int lane = lane_id(), wave = wave_id();
  const int li = lane & 15, lg = lane >> 4;
  const uint16_t* ckv = (const uint16_t*)s.aux[0];
  const uint16_t* kpe = (const uint16_t*)s.aux[1];
  const void* crow = (const uint8_t*)s.aux[5] + (size_t)env.xcd * AM_DK / 2 * 8;
  float* S = (float*)(lds + AM_S_OFF);
  float* H = (float*)(lds + AM_H_OFF);
  auto split_hi = [&](int j) { const int h = j * split + split; return h > step + 1 ? step + 1 : h; };
  auto tile_n = [&](int t0, int hi) { return t0 + AM_T < hi ? AM_T : hi - t0; };
  // the first tile's rows are requested before q is awaited
  u32x4 v[AM_LOADS];
  {
    const int lo = j0 * split;
    am_issue_rows(v, ckv, kpe, lo, tile_n(lo, split_hi(j0)), step);
  }
  // ---- q of every head: ql_nope (2048 pairs of packets) and q_pe (256 pairs), bf16 into LDS rows
  {
    u32x4 w[8];
    pk_wait_pairs<8>(qln, fx_tid(), FX_THREADS, 2048, tin, env.err, w);
#pragma unroll
    for (int n = 0; n < 8; ++n) {
      const int p = fx_tid() + n * FX_THREADS;      // pair p: head p / 128, columns 4 (p % 128) ..
      u32x2 b;
      b.x = w[n].x;
      b.y = w[n].z;
      *(u32x2*)(lds + AM_Q_OFF + (p >> 7) * AM_ROW + (p & 127) * 8) = b;
    }
    u32x4 e[1];
    pk_wait_pairs<1>((const void*)s.aux[2], fx_tid(), 0, 256, tin, env.err, e);
    u32x2 b;
    b.x = e[0].x;
    b.y = e[0].z;
    *(u32x2*)(lds + AM_Q_OFF + (fx_tid() >> 4) * AM_ROW + 1024 + (fx_tid() & 15) * 8) = b;
  }
  prof_mark(env, 1);
  after_q();
  int done = 0;
  for (int j = j0; j < n_live; j += jstep) {
    const int lo = j * split, hi = split_hi(j);
    // online-softmax state of head lg + 4 * wave (the same on the 16 lanes li of lane group lg)
    float m_run = -__builtin_inff(), l_run = 0.0f;
    // value accumulators: wave w owns columns 128 w .. 128 w + 127 as 8 16-column tiles; lane (li, lg)
    // holds rows (heads) 4 lg .. 4 lg + 3 of column 16 n + li
    fx_f32x4 acc[8];
#pragma unroll
    for (int n = 0; n < 8; ++n) acc[n] = (fx_f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    for (int t0 = lo; t0 < hi; t0 += AM_T) {
      const int nt = tile_n(t0, hi);
      __syncthreads();
      // ---- stage the tile: cached rows from registers, row `step` from the cache-row packets,
      // rows past the tile's end as zeros (their value products must be exactly zero)
#pragma unroll
      for (int k = 0; k < AM_LOADS; ++k) {
        const int q = fx_tid() + k * FX_THREADS;
        const int r = q / 72, c = q % 72;
        if (t0 + r != step) *(u32x4*)(lds + AM_KV_OFF + r * AM_ROW + c * 16) = v[k];
      }
      if (step >= t0 && step < t0 + nt && fx_tid() < AM_DK / 4) {
        u32x4 w[1];
        pk_wait_pairs<1>(crow, fx_tid(), 0, fx_tid() + 1, tin, env.err, w);
        u32x2 b;
        b.x = w[0].x;
        b.y = w[0].z;
        *(u32x2*)(lds + AM_KV_OFF + (step - t0) * AM_ROW + fx_tid() * 8) = b;
      }
      {
        // request the next tile (this split's, or the worker's next split's first)
        int nt0 = t0 + AM_T, nhi = hi;
        if (nt0 >= hi) {
          const int nj = j + jstep;
          nt0 = nj * split;
          nhi = nj < n_live ? split_hi(nj) : 0;
        }
        if (nt0 < nhi) am_issue_rows(v, ckv, kpe, nt0, tile_n(nt0, nhi), step);
      }
      __syncthreads();
      // ---- scores: wave q < 2 computes positions 16 q .. 16 q + 15 for every head
      if (wave < 2) {
        // A = Q[li][32 ks + 8 lg .. + 8], B = row 16 q + li at the same columns, both from LDS
        fx_f32x4 sc = {0.0f, 0.0f, 0.0f, 0.0f};
        const char* qr = lds + AM_Q_OFF + li * AM_ROW + 16 * lg;
        const char* kr = lds + AM_KV_OFF + (16 * wave + li) * AM_ROW + 16 * lg;
#pragma unroll
        for (int ks = 0; ks < AM_KS; ++ks)
          sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(lds_b128(qr + 64 * ks), lds_b128(kr + 64 * ks), sc, 0, 0, 0);
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) S[(4 * lg + jj) * AM_T + 16 * wave + li] = sc[jj] * scale;
      }
      __syncthreads();
      // ---- softmax: lane (li, lg) of wave w takes head lg + 4 w, positions li and li + 16
      {
        const int h = lg + 4 * wave;
        const float s0 = li < nt ? S[h * AM_T + li] : -__builtin_inff();
        const float s1 = li + 16 < nt ? S[h * AM_T + 16 + li] : -__builtin_inff();
        float mt = fmaxf(s0, s1);
        mt = fmaxf(mt, xor_lane<1>(mt));
        mt = fmaxf(mt, xor_lane<2>(mt));
        mt = fmaxf(mt, xor_lane<4>(mt));
        mt = fmaxf(mt, xor_lane<8>(mt));
        const float m_new = m_run > mt ? m_run : mt;
        const float alpha = exp_s(m_run - m_new);
        const float p0 = li < nt ? exp_s(s0 - m_new) : 0.0f;
        const float p1 = li + 16 < nt ? exp_s(s1 - m_new) : 0.0f;
        const float u0 = butterfly(p0, 16), u1 = butterfly(p1, 16);
        const float psum = u0 + u1;
        l_run = l_run * alpha + psum;
        m_run = m_new;
        uint16_t* prow_l = (uint16_t*)(lds + AM_P_OFF + h * AM_P_ROW);
        prow_l[li] = (uint16_t)f2bf(p0);
        prow_l[16 + li] = (uint16_t)f2bf(p1);
        if (li == 0) H[h] = alpha;
      }
      __syncthreads();
      // ---- value products: wave w, column tiles 128 w + 16 n; B rows read transposed
      {
        const fx_bf16x8 pf = lds_b128(lds + AM_P_OFF + li * AM_P_ROW + 16 * lg);
        float al[4];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) al[jj] = H[4 * lg + jj];
        // lane (li, lg) supplies row 8 lg + li / 4 (+ 4), columns c0 + 4 (li % 4) .. + 4
        const char* vb = lds + AM_KV_OFF + (8 * lg + (li >> 2)) * AM_ROW + 8 * (li & 3);
#pragma unroll
        for (int n = 0; n < 8; ++n) {
          const int c0 = 128 * wave + 16 * n;
          // whole-vector casts: the B operand's elements 0..3 are the first read, 4..7 the second
          const u32x2 lo4 = __builtin_bit_cast(u32x2, lds_tr16(vb + 2 * c0));
          const u32x2 hi4 = __builtin_bit_cast(u32x2, lds_tr16(vb + 4 * AM_ROW + 2 * c0));
          const fx_bf16x8 bf = __builtin_bit_cast(fx_bf16x8, (u32x4){lo4.x, lo4.y, hi4.x, hi4.y});
          const fx_f32x4 tp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pf, bf, (fx_f32x4){0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const float a = acc[n][jj] * al[jj];
            acc[n][jj] = a + tp[jj];
          }
        }
      }
    }
    // ---- o = acc / l, lse = m + log(l)
    __syncthreads();
    if (li == 0) {
      H[16 + lg + 4 * wave] = m_run;
      H[32 + lg + 4 * wave] = l_run;
    }
    __syncthreads();
    {
      float linv[4];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) linv[jj] = H[32 + 4 * lg + jj];
#pragma unroll
      for (int n = 0; n < 8; ++n) {
        const int c = 128 * wave + 16 * n + li;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const uint32_t off = (uint32_t)((j * AM_NH + 4 * lg + jj) * prow + c) * 4;
          const uint32_t val = __float_as_uint(acc[n][jj] / linv[jj]);
          if (local) stl4(part, off, val);
          else stc4(part, off, val);
        }
      }
      if (fx_tid() < AM_NH) {
        const uint32_t off = (uint32_t)((j * AM_NH + fx_tid()) * prow + 512) * 4;
        const uint32_t val = __float_as_uint(H[16 + fx_tid()] + log_s(H[32 + fx_tid()]));
        if (local) stl4(part, off, val);
        else stc4(part, off, val);
      }
    }
    ++done;
  }
  return done;
}

// FX_OP_MLA_ATTEND with FX_F_MFMA: splits over all workers (split j on worker j % 256), every head
// per split. Partials as the VALU form ([split][head][prow]: o, then lse); then one done packet per
// worker that owned a live split, at done[worker] (the merge polls workers 0 .. min(live, 256) - 1).
__device__ __forceinline__ void op_mla_attend_mfma(const fx_stage& s, FxEnv& env) {
  const int n_live = (env.step + 1 + s.split - 1) / s.split;
  if (env.worker >= n_live) return;
  const int done = am_attend(s, env, (const void*)s.x, (void*)s.out, env.worker, FX_WORKERS, false, tag_in(s, env, 0),
                             [] {});
  // done packet of this worker: its partials are complete
  wait_mem();
  __syncthreads();
  prof_mark(env, 7);
  if (fx_tid() == 0) pk_put((void*)s.aux[6], (uint32_t)env.worker, (uint32_t)done, tag_out(env));
  prof_mark(env, 2);
}

// FX_OP_MLA_MERGE_UV with FX_F_XCD: the attention of every head and its merge, both on the 32
// workers of XCD FX_ATT_XCD, so that the partials and the done packets never leave that XCD's L2
// (XCD-local stores, ~0.3 us from store to the reader's load against ~1.4 us device-coherent under
// the weight stream). Split j runs on rank j % 32; rank r then merges head r / 2 and computes its
// W_uv rows 64 (r % 2) .. + 63, whose weights are requested as soon as q has arrived. The stage
// carries the attention's operands in the merge's spare fields: aux[3] = ql_nope packets (the
// attention's x), aux[0] c_kv, aux[1] k_pe, aux[2] q_pe packets, aux[5] crow packets, scale; src[0]
// = their producer (the prep). x = partials, aux[6] = done packets (one per rank), w = W_uv,
// out = attn packets, aux[4] = o_merged dump or null.
#define FX_ATT_XCD 7
#define XCD_MERGE_ROWS 64
__device__ __forceinline__ void op_mla_attend_merge_xcd(const fx_stage& s, FxEnv& env) {
  if (env.xcd != FX_ATT_XCD) return;
  const int d_c = s.d_c, d_v = s.d_n, nh = s.n_rows;
  const int r = env.xrank;
  const int live = (env.step + 1 + s.split - 1) / s.split;
  const uint32_t tin = tag_in(s, env, 0), tout = tag_out(env);
  const int h = r >> 1, v0 = (r & 1) * XCD_MERGE_ROWS;
  const uint16_t* W = (const uint16_t*)s.w + (size_t)h * d_v * d_c;
  // wave w: W_uv rows v0 + 16 w .. + 15 (one 16-row group per wave, K = 512: one chunk per lane)
  auto rowof = [&](int g, int i) { return v0 + 16 * g + i; };
  Tile<16, 1> tw;
  auto prime = [&] { tile_load(tw, W, d_c, wave_id(), rowof); };
  void* part = (void*)s.x;
  int done = 0;
  if (r < live) done = am_attend(s, env, (const void*)s.aux[3], part, r, FX_XWORKERS, true, tin, prime);
  else prime();
  // this rank's partials are complete (the store counter drains in order, the W_uv rows with it:
  // they were requested before the first tile was scored)
  wait_mem();
  __syncthreads();
  prof_mark(env, 4);
  if (fx_tid() == 0 && r < live) pk_put((void*)s.aux[6], (uint32_t)r, (uint32_t)done, tout, true);
  if (wave_id() == 0)
    pk_wait_singles<1>((const void*)s.aux[6], lane_id(), 64, live < FX_XWORKERS ? live : FX_XWORKERS, tout, env.err);
  __syncthreads();
  prof_mark(env, 5);
  float* xs = (float*)(env.lds + LDS_XS);
  merge_head(part, nh, h, s.prow, d_c, live, xs, (float*)(env.lds + LDS_TILE), (float*)(env.lds + LDS_RED), env);
  if (v0 == 0 && s.aux[4])
    stc4((void*)s.aux[4], (uint32_t)(h * d_c + fx_tid() * 2) * 2, pack2(xs[fx_tid() * 2], xs[fx_tid() * 2 + 1]));
  __syncthreads();
  prof_mark(env, 6);
  float* o8 = (float*)(env.lds + LDS_RED) + 16;
  {
    float acc[16];
    tile_dot(tw, xs, d_c, acc);
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (lane_id() == 0) o8[16 * wave_id() + i] = bf16r(acc[i]);
  }
  __syncthreads();
  if (fx_tid() < XCD_MERGE_ROWS / 4) {
    const float* o = o8 + 4 * fx_tid();
    pk_put2((void*)s.out, (uint32_t)((h * d_v + v0) / 2 + 2 * fx_tid()), pack2(o[0], o[1]), pack2(o[2], o[3]), tout);
  }
  prof_mark(env, 2);
}
