// Operators of the decode task table (one fx_stage each), as device functions executed by one
// worker workgroup (256 threads) for its share of the stage. The same code runs inside the
// persistent kernel and in the per-stage launcher of the kernel suite.
//
// Work split (248 workers = 256 CUs minus one scheduler per XCD; worker w sits on XCD w % 8 and is
// rank w / 8 of the 31 workers of its XCD):
//   global stages (GEMVs, dense MLP, combine): contiguous row ranges over all workers;
//   XCD stages (MLA prep/attend/merge for the XCD's nh/8 heads, router, expert slot = XCD):
//   split over the XCD's 31 workers.
// Each function's arithmetic is the spec of fx_device.h; the reference function it restates is
// cited at each operator.
#pragma once
#include "fx_device.h"
#include "../../include/fleet_mi355x.h"

struct FxEnv {
  int worker, nworkers;   // global worker index and count
  int xcd, xrank, xworkers;
  int step, iter;
  int n_prompt;
  int64_t* tokens;
  uint32_t* sync;         // runtime sync area (flags + counters)
  char* lds;
};

// sync area layout (uint32 index, one 128-byte line per flag)
#define FX_FLAG_ARRIVE(b) ((b) * 32)
#define FX_FLAG_GO(b) ((256 + (b)) * 32)
#define FX_FLAG_XCD(x) ((512 + (x)) * 32)
#define FX_CNT_ATTEND(x) ((520 + (x)) * 32)
#define FX_FLAG_ERROR (528 * 32)
#define FX_SYNC_WORDS (529 * 32)

// LDS layout
#define LDS_XS 0                         // f32 [11264]  GEMV input
#define LDS_RED (45056)                  // f32 [1024]   reductions / small tables
#define LDS_MISC (LDS_RED + 4096)        // misc scalars
#define LDS_TILE (LDS_MISC + 1024)       // attention tile / merge tables (<= 37.5 KiB)
#define LDS_STAGE (FX_LDS_BYTES - 256)   // the current fx_stage (persistent kernel)

__device__ __forceinline__ void range_split(int n, int parts, int i, int& lo, int& hi) {
  lo = (int)(((long long)n * i) / parts);
  hi = (int)(((long long)n * (i + 1)) / parts);
}

// ------------------------------------------------------------------------------------------------
// GEMV core: groups of R rows per wave, lane-chunk order, result on every lane of the wave.

template <int R, int NJ, class RowFn, class EmitFn>
__device__ __forceinline__ void gemv_groups(const uint16_t* __restrict__ W, int K, const float* xs, int ngroups,
                                            RowFn rowof, EmitFn emit) {
  const int lane = lane_id();
  const int nchunk = K >> 3;
  const int nl = lanes_for(nchunk);
  for (int g = wave_id(); g < ngroups; g += FX_WAVES) {
    int row[R];
    bool valid[R];
    int any_row = -1;
#pragma unroll
    for (int i = 0; i < R; ++i) {
      row[i] = rowof(g, i);
      valid[i] = row[i] >= 0;
      if (valid[i] && any_row < 0) any_row = row[i];
    }
#pragma unroll
    for (int i = 0; i < R; ++i)
      if (!valid[i]) row[i] = any_row;
    u32x4 wv[R][NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int c = lane + 64 * j;
      const int cc = c < nchunk ? c : nchunk - 1;
#pragma unroll
      for (int i = 0; i < R; ++i) wv[i][j] = ldw16(W + (size_t)row[i] * K + (size_t)cc * 8);
    }
    float acc[R];
#pragma unroll
    for (int i = 0; i < R; ++i) acc[i] = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int c = lane + 64 * j;
      if (c < nchunk) {
        float xv[8];
        const float4* xp = (const float4*)(xs + c * 8);
        float4 a = xp[0], b = xp[1];
        xv[0] = a.x; xv[1] = a.y; xv[2] = a.z; xv[3] = a.w;
        xv[4] = b.x; xv[5] = b.y; xv[6] = b.z; xv[7] = b.w;
#pragma unroll
        for (int i = 0; i < R; ++i) acc[i] = fma8(wv[i][j], xv, acc[i]);
      }
    }
#pragma unroll
    for (int i = 0; i < R; ++i) acc[i] = butterfly(acc[i], nl);
    emit(g, row, valid, acc);
  }
}

// ------------------------------------------------------------------------------------------------
// GEMV input prologues (all threads; ends with the normalised bf16 row as f32 in xs)

__device__ __forceinline__ void load_vec_sc1(float* xs, const void* src, int K) {
  for (int i = threadIdx.x * 8; i < K; i += FX_THREADS * 8) {
    u32x4 v = ldc16(src, (uint32_t)i * 2);
    xs[i + 0] = bf_lo(v.x); xs[i + 1] = bf_hi(v.x);
    xs[i + 2] = bf_lo(v.y); xs[i + 3] = bf_hi(v.y);
    xs[i + 4] = bf_lo(v.z); xs[i + 5] = bf_hi(v.z);
    xs[i + 6] = bf_lo(v.w); xs[i + 7] = bf_hi(v.w);
  }
}

// x_res + sum_s out8[s] * topk_w[s], slot order, mul then add (harness/numpy_ref.py:316-321)
__device__ __forceinline__ void combine_into(float* xs, const void* x, const void* out8, const void* topk_w, int n_slots,
                                             int K, float* w) {
  __syncthreads();
  if (threadIdx.x < (unsigned)n_slots) w[threadIdx.x] = ldcf(topk_w, threadIdx.x);
  __syncthreads();
  for (int i = threadIdx.x * 8; i < K; i += FX_THREADS * 8) {
    u32x4 v = ldc16(x, (uint32_t)i * 2);
    float acc[8] = {bf_lo(v.x), bf_hi(v.x), bf_lo(v.y), bf_hi(v.y), bf_lo(v.z), bf_hi(v.z), bf_lo(v.w), bf_hi(v.w)};
    for (int s = 0; s < n_slots; ++s) {
      u32x4 o = ldc16(out8, (uint32_t)(s * K + i) * 2);
      float ov[8] = {bf_lo(o.x), bf_hi(o.x), bf_lo(o.y), bf_hi(o.y), bf_lo(o.z), bf_hi(o.z), bf_lo(o.w), bf_hi(o.w)};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float t = ov[e] * w[s];
        acc[e] = acc[e] + t;
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) xs[i + e] = bf16r(acc[e]);
  }
}

// greedy id from the per-worker (max, index) pairs: the lowest index among the maxima
__device__ __forceinline__ int64_t argmax_reduce(const void* amax, int nworkers) {
  float best = -__builtin_inff();
  int best_i = 0x7fffffff;
  for (int w = lane_id(); w < nworkers; w += 64) {
    float v = ldcf(amax, 2 * w);
    int i = (int)ldc4(amax, (2 * w + 1) * 4);
    if (v > best || (v == best && i < best_i)) { best = v; best_i = i; }
  }
  for (int off = 1; off < 64; off <<= 1) {
    float ov = shfl_xor_f(best, off);
    int oi = __shfl_xor(best_i, off, 64);
    if (ov > best || (ov == best && oi < best_i)) { best = ov; best_i = oi; }
  }
  return best_i;
}

// rmsnorm in place on xs (harness/numpy_ref.py:54-60): var = dot_lanes(x, x) / K,
// rs = 1 / sqrt(var + eps), y = bf16(w * bf16(x * rs)). Ends with __syncthreads.
__device__ __forceinline__ void rmsnorm_inplace(float* xs, const uint16_t* wn, int K, float eps, float* red) {
  __syncthreads();
  if (wave_id() == 0) {
    float ss = sumsq_wave(xs, K);
    if (lane_id() == 0) {
      float var = ss / (float)K;
      red[0] = 1.0f / sqrtf(var + eps);
    }
  }
  __syncthreads();
  const float rs = red[0];
  for (int i = threadIdx.x * 8; i < K; i += FX_THREADS * 8) {
    u32x4 wv = ld16(wn + i);
    float w8[8] = {bf_lo(wv.x), bf_hi(wv.x), bf_lo(wv.y), bf_hi(wv.y), bf_lo(wv.z), bf_hi(wv.z), bf_lo(wv.w), bf_hi(wv.w)};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float xn = bf16r(xs[i + e] * rs);
      xs[i + e] = bf16r(w8[e] * xn);
    }
  }
  __syncthreads();
}

__device__ __forceinline__ void store_vec_sc1(void* dst, const float* xs, int K) {
  for (int i = threadIdx.x * 8; i < K; i += FX_THREADS * 8) {
    u32x4 v;
    v.x = pack2(xs[i + 0], xs[i + 1]);
    v.y = pack2(xs[i + 2], xs[i + 3]);
    v.z = pack2(xs[i + 4], xs[i + 5]);
    v.w = pack2(xs[i + 6], xs[i + 7]);
    stc16(dst, (uint32_t)i * 2, v);
  }
}

// ------------------------------------------------------------------------------------------------
// FX_OP_GEMV: harness/numpy_ref.py:295-313 (linear, linear_norm, linear_residual); embedding and
// combine prologues for the layer inputs; per-worker argmax for the LM head.

template <int NJ>
__device__ void op_gemv_body(const fx_stage& s, const FxEnv& env, float* xs, int r0, int r1) {
  const uint16_t* W = (const uint16_t*)s.w;
  const int K = s.k;
  void* out = (void*)s.out;
  const void* res = (const void*)s.res;
  const bool residual = (s.flags & FX_F_RESIDUAL) != 0;
  const bool want_max = (s.flags & FX_F_ARGMAX) != 0;
  constexpr int R = NJ <= 4 ? 4 : 1;
  const int nrows = r1 - r0;
  const int ngroups = (nrows + R - 1) / R;
  float best = -__builtin_inff();
  int best_i = 0x7fffffff;
  gemv_groups<R, NJ>(
      W, K, xs, ngroups, [&](int g, int i) { int r = r0 + g * R + i; return r < r1 ? r : -1; },
      [&](int g, const int* row, const bool* valid, const float* acc) {
        const int lane = lane_id();
#pragma unroll
        for (int i = 0; i < R; ++i) {
          if (!valid[i]) continue;
          float v = acc[i];
          if (residual) v = v + bf2f(ldc2(res, (uint32_t)row[i] * 2));
          uint32_t b = f2bf(v);
          if (lane == i) stc2(out, (uint32_t)row[i] * 2, b);
          if (want_max) {
            float fv = bf2f(b);
            if (fv > best || (fv == best && row[i] < best_i)) { best = fv; best_i = row[i]; }
          }
        }
      });
  if (want_max) {
    float* red = (float*)(env.lds + LDS_RED);
    int* redi = (int*)(env.lds + LDS_RED + 64);
    if (lane_id() == 0) { red[wave_id()] = best; redi[wave_id()] = best_i; }
    __syncthreads();
    if (threadIdx.x == 0) {
      float b = red[0];
      int bi = redi[0];
      for (int w = 1; w < FX_WAVES; ++w)
        if (red[w] > b || (red[w] == b && redi[w] < bi)) { b = red[w]; bi = redi[w]; }
      stcf((void*)s.aux[3], 2 * env.worker, b);
      stc4((void*)s.aux[3], (2 * env.worker + 1) * 4, (uint32_t)bi);
    }
  }
}

__device__ void op_gemv(const fx_stage& s, const FxEnv& env) {
  float* xs = (float*)(env.lds + LDS_XS);
  float* red = (float*)(env.lds + LDS_RED);
  const int K = s.k;
  // ---- input row
  if (s.in_kind == FX_IN_EMBED) {
    int64_t* misc = (int64_t*)(env.lds + LDS_MISC);
    if (wave_id() == 0) {
      int64_t tok;
      if (env.step < env.n_prompt) {
        u32x2 t = ldc8(env.tokens, (uint32_t)env.step * 8);
        tok = (int64_t)(((uint64_t)t.y << 32) | t.x);
      } else {
        tok = argmax_reduce((const void*)s.aux[3], env.nworkers);
        if (env.worker == 0 && lane_id() == 0) {
          u32x2 t;
          t.x = (uint32_t)tok;
          t.y = (uint32_t)((uint64_t)tok >> 32);
          stc8(env.tokens, (uint32_t)env.step * 8, t);
        }
      }
      if (lane_id() == 0) misc[0] = tok;
    }
    __syncthreads();
    const int64_t tok = misc[0];
    const uint16_t* row = (const uint16_t*)s.aux[0] + (size_t)tok * K;
    for (int i = threadIdx.x * 8; i < K; i += FX_THREADS * 8) {
      u32x4 v = ld16(row + i);
      xs[i + 0] = bf_lo(v.x); xs[i + 1] = bf_hi(v.x);
      xs[i + 2] = bf_lo(v.y); xs[i + 3] = bf_hi(v.y);
      xs[i + 4] = bf_lo(v.z); xs[i + 5] = bf_hi(v.z);
      xs[i + 6] = bf_lo(v.w); xs[i + 7] = bf_hi(v.w);
    }
  } else if (s.in_kind == FX_IN_COMBINE) {
    combine_into(xs, (const void*)s.x, (const void*)s.aux[0], (const void*)s.aux[1], s.n_slots, K,
                 (float*)(env.lds + LDS_MISC + 512));
  } else {
    load_vec_sc1(xs, (const void*)s.x, K);
  }
  if ((s.flags & FX_F_WRITE_X) && env.worker == 0) {
    __syncthreads();
    store_vec_sc1((void*)s.aux[2], xs, K);
  }
  if (s.flags & FX_F_NORM) rmsnorm_inplace(xs, (const uint16_t*)s.w_norm, K, s.eps, red);
  else __syncthreads();
  // ---- rows
  int r0, r1;
  range_split(s.n_rows, env.nworkers, env.worker, r0, r1);
  const int nchunk = K >> 3;
  const int nj = (nchunk + 63) / 64;
  if (nj <= 1) op_gemv_body<1>(s, env, xs, r0, r1);
  else if (nj <= 3) op_gemv_body<3>(s, env, xs, r0, r1);
  else if (nj <= 4) op_gemv_body<4>(s, env, xs, r0, r1);
  else op_gemv_body<22>(s, env, xs, r0, r1);
}

// ------------------------------------------------------------------------------------------------
// gate|up pairs with SiLU (harness/numpy_ref.py:256-292 fused): act[i] = bf16(silu(g) * u),
// g = bf16(W[i] h), u = bf16(W[I + i] h). Pairs [p0, p1) of the I pairs of W (2I rows).

__device__ __forceinline__ void gate_up_pairs(const uint16_t* W, int I, int K, const float* xs, int p0, int p1, void* act,
                                              uint32_t act_off) {
  const int npairs = p1 - p0;
  const int ngroups = (npairs + 1) / 2;
  gemv_groups<4, 4>(
      W, K, xs, ngroups,
      [&](int g, int i) {
        int p = p0 + g * 2 + (i >> 1);
        if (p >= p1) return -1;
        return (i & 1) ? I + p : p;
      },
      [&](int g, const int* row, const bool* valid, const float* acc) {
        const int lane = lane_id();
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          if (!valid[2 * q]) continue;
          float gv = bf16r(acc[2 * q]);
          float uv = bf16r(acc[2 * q + 1]);
          float a = silu_s(gv) * uv;
          if (lane == q) stc2(act, act_off + (uint32_t)row[2 * q] * 2, f2bf(a));
        }
      });
}

// FX_OP_DENSE_GU: layer-0 gate/up + SiLU over all workers (HF DeepseekV2MLP,
// modeling_deepseek.py:381-398, with numpy_ref's rounding points).
__device__ void op_dense_gu(const fx_stage& s, const FxEnv& env) {
  float* xs = (float*)(env.lds + LDS_XS);
  float* red = (float*)(env.lds + LDS_RED);
  const int K = s.k, I = s.n_rows;
  load_vec_sc1(xs, (const void*)s.x, K);
  rmsnorm_inplace(xs, (const uint16_t*)s.w_norm, K, s.eps, red);
  if (s.aux[6] && env.worker == 0) store_vec_sc1((void*)s.aux[6], xs, K);
  int p0, p1;
  range_split(I, env.nworkers, env.worker, p0, p1);
  gate_up_pairs((const uint16_t*)s.w, I, K, xs, p0, p1, (void*)s.out, 0);
}

// ------------------------------------------------------------------------------------------------
// Router softmax + top-k on one wave (harness/numpy_ref.py:205-235): lane e holds logit e; the
// softmax sum is the xor butterfly over pow2ceil(E) lanes; top-k by repeated argmax, lowest
// index on ties. Returns the selected ids (ids[k]) and weights on every lane.

__device__ __forceinline__ void softmax_topk_wave(const float* logits, int E, int topk, float scaling, int* ids,
                                                  float* wts, float* probs) {
  const int lane = lane_id();
  float l = lane < E ? logits[lane] : -__builtin_inff();
  float m = wave_max(l);
  float p = lane < E ? exp_s(l - m) : 0.0f;
  int nl = 1;
  while (nl < E) nl <<= 1;
  float sum = butterfly(p, nl);
  p = p / sum;
  if (probs && lane < E) probs[lane] = p;
  float rem = lane < E ? p : -__builtin_inff();
  for (int k = 0; k < topk; ++k) {
    float v = wave_max(rem);
    unsigned long long bal = __ballot(rem == v);
    int idx = __builtin_ctzll(bal);
    float pw = __shfl(p, idx, 64);
    if (lane == 0) { ids[k] = idx; wts[k] = pw * scaling; }
    if (lane == idx) rem = -__builtin_inff();
  }
}

// FX_OP_MOE_ROUTER: per XCD, h = rmsnorm(x_res), logits rows split over the XCD's workers.
__device__ void op_moe_router(const fx_stage& s, const FxEnv& env) {
  if (env.xcd >= s.topk) return;   // forced-expert slots need no routing
  float* xs = (float*)(env.lds + LDS_XS);
  float* red = (float*)(env.lds + LDS_RED);
  const int K = s.k, E = s.n_rows;
  load_vec_sc1(xs, (const void*)s.x, K);
  rmsnorm_inplace(xs, (const uint16_t*)s.w_norm, K, s.eps, red);
  void* lx = (void*)s.out;   // f32 [8][E]
  const int per = (E + env.xworkers - 1) / env.xworkers;   // rows: rank, rank + xworkers, ...
  gemv_groups<4, 4>(
      (const uint16_t*)s.w, K, xs, 1,
      [&](int g, int i) {
        int r = env.xrank + i * env.xworkers;
        return (i < per && r < E) ? r : -1;
      },
      [&](int g, const int* row, const bool* valid, const float* acc) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (valid[i] && lane_id() == i) stcf(lx, env.xcd * E + row[i], acc[i]);
      });
}

// FX_OP_MOE_W13: per XCD, slot = XCD. harness/numpy_ref.py:256-292 (moe_w13 + the silu-mul).
__device__ void op_moe_w13(const fx_stage& s, const FxEnv& env) {
  float* xs = (float*)(env.lds + LDS_XS);
  float* red = (float*)(env.lds + LDS_RED);
  int* misc = (int*)(env.lds + LDS_MISC);
  const int K = s.k, I = s.n_rows, E = s.aux_i0;
  const int slot = env.xcd;
  const int topk = s.topk;
  if (wave_id() == 0) {
    int* ids = (int*)(env.lds + LDS_MISC + 128);
    float* wts = (float*)(env.lds + LDS_MISC + 256);
    int e;
    const bool need_route = slot < topk || (env.xcd == 0 && env.xrank == 0);
    if (need_route) {
      float* lg = red + 256;
      float* probs = red + 512;
      for (int i = lane_id(); i < E; i += 64) lg[i] = ldcf((const void*)s.aux[0], env.xcd * E + i);
      softmax_topk_wave(lg, E, topk, s.scaling, ids, wts, probs);
      e = slot < topk ? ids[slot] : E + (slot - topk);
      if (env.xcd == 0 && env.xrank == 0) {
        // router outputs (numpy_ref.moe_router layout): topk_w, routing, mask, logits, route_log
        const int n_slots = s.n_slots, n_total = E + s.n_forced;
        const int lane = lane_id();
        for (int k = lane; k < n_slots; k += 64) {
          int id = k < topk ? ids[k] : E + (k - topk);
          float wv = k < topk ? wts[k] : 1.0f;
          stcf((void*)s.aux[1], k, wv);
          // route_log [prow rows][aux_i1 MoE layers][n_slots], row = step - (n_prompt - 1): the decode
          // iterations only, as the reference logs them (route_log [32, 26, 8] at [step - 1023])
          const int row = env.step - (env.n_prompt - 1);
          if (s.aux[5] && s.layer >= 1 && row >= 0 && row < s.prow)
            stc4((void*)s.aux[5], (uint32_t)(((row * s.aux_i1) + (s.layer - 1)) * n_slots + k) * 4, (uint32_t)id);
        }
        for (int x = lane; x < n_total; x += 64) {
          int r = 0;
          for (int k = 0; k < n_slots; ++k) {
            int id = k < topk ? ids[k] : E + (k - topk);
            if (id == x) r = k + 1;
          }
          stc4((void*)s.aux[2], x * 4, (uint32_t)r);
        }
        for (int x = lane; x <= n_total; x += 64) {
          int v = -1;
          if (x < n_slots) v = x < topk ? ids[x] : E + (x - topk);
          if (x == n_total) v = n_slots;
          stc4((void*)s.aux[3], x * 4, (uint32_t)v);
        }
        for (int x = lane; x < E; x += 64) stcf((void*)s.aux[4], x, lg[x]);
      }
    } else {
      e = E + (slot - topk);
    }
    if (lane_id() == 0) misc[0] = e;
    if (env.xrank == 0 && lane_id() == 0) stc4((void*)s.aux[7], slot * 4, (uint32_t)e);
  }
  load_vec_sc1(xs, (const void*)s.x, K);
  rmsnorm_inplace(xs, (const uint16_t*)s.w_norm, K, s.eps, red);
  if (s.aux[6] && env.xcd == 0 && env.xrank == 0) store_vec_sc1((void*)s.aux[6], xs, K);
  const int e = misc[0];
  int p0, p1;
  range_split(I, env.xworkers, env.xrank, p0, p1);
  const uint16_t* W = (const uint16_t*)s.w + (size_t)e * 2 * I * K;
  gate_up_pairs(W, I, K, xs, p0, p1, (void*)s.out, (uint32_t)slot * I * 2);
}

// FX_OP_MOE_W2: per XCD, out8[slot] = bf16(W2[e] act8[slot]) (harness/numpy_ref.py:275-292).
__device__ void op_moe_w2(const fx_stage& s, const FxEnv& env) {
  float* xs = (float*)(env.lds + LDS_XS);
  int* misc = (int*)(env.lds + LDS_MISC);
  const int I = s.k, H = s.n_rows;
  const int slot = env.xcd;
  if (threadIdx.x == 0) misc[0] = (int)ldc4((const void*)s.aux[7], slot * 4);
  load_vec_sc1(xs, (const uint8_t*)s.x + (size_t)slot * I * 2, I);
  __syncthreads();
  const int e = misc[0];
  const uint16_t* W = (const uint16_t*)s.w + (size_t)e * H * I;
  void* out = (void*)s.out;
  int r0, r1;
  range_split(H, env.xworkers, env.xrank, r0, r1);
  const int ngroups = (r1 - r0 + 3) / 4;
  gemv_groups<4, 3>(
      W, I, xs, ngroups, [&](int g, int i) { int r = r0 + g * 4 + i; return r < r1 ? r : -1; },
      [&](int g, const int* row, const bool* valid, const float* acc) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (valid[i] && lane_id() == i) stc2(out, (uint32_t)(slot * H + row[i]) * 2, f2bf(acc[i]));
      });
}

// FX_OP_MOE_COMBINE (standalone form; inside the decode it is the next layer's input prologue)
__device__ void op_moe_combine(const fx_stage& s, const FxEnv& env) {
  const int H = s.n_rows;
  int r0, r1;
  range_split(H / 8, env.nworkers, env.worker, r0, r1);
  float* w = (float*)(env.lds + LDS_MISC + 512);
  if (threadIdx.x < (unsigned)s.n_slots) w[threadIdx.x] = ldcf((const void*)s.aux[1], threadIdx.x);
  __syncthreads();
  for (int c = r0 + (int)threadIdx.x; c < r1; c += FX_THREADS) {
    const int i = c * 8;
    u32x4 v = ldc16((const void*)s.x, (uint32_t)i * 2);
    float acc[8] = {bf_lo(v.x), bf_hi(v.x), bf_lo(v.y), bf_hi(v.y), bf_lo(v.z), bf_hi(v.z), bf_lo(v.w), bf_hi(v.w)};
    for (int k = 0; k < s.n_slots; ++k) {
      u32x4 o = ldc16((const void*)s.aux[0], (uint32_t)(k * H + i) * 2);
      float ov[8] = {bf_lo(o.x), bf_hi(o.x), bf_lo(o.y), bf_hi(o.y), bf_lo(o.z), bf_hi(o.z), bf_lo(o.w), bf_hi(o.w)};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float t = ov[e] * w[k];
        acc[e] = acc[e] + t;
      }
    }
    u32x4 r;
    r.x = pack2(acc[0], acc[1]); r.y = pack2(acc[2], acc[3]);
    r.z = pack2(acc[4], acc[5]); r.w = pack2(acc[6], acc[7]);
    stc16((void*)s.out, (uint32_t)i * 2, r);
  }
}

// FX_OP_ARGMAX: tokens[step + 1] (the reduce of argmax_partial; fleet/graph_plan.py:598-602)
__device__ void op_argmax(const fx_stage& s, const FxEnv& env) {
  if (env.worker != 0 || wave_id() != 0) return;
  if (env.step + 1 < env.n_prompt) return;
  int64_t tok = argmax_reduce((const void*)s.aux[3], env.nworkers);
  if (lane_id() == 0) {
    u32x2 t;
    t.x = (uint32_t)tok;
    t.y = (uint32_t)((uint64_t)tok >> 32);
    stc8(env.tokens, (uint32_t)(env.step + 1) * 8, t);
  }
}

// ------------------------------------------------------------------------------------------------
// MLA (harness/numpy_ref.py:85-174). Heads are split over XCDs: XCD x owns heads
// [x * nh/8, (x + 1) * nh/8); the kernels below assume nh = 16 (two heads per XCD), d_c = 512,
// d_r = 64, d_n = 128 (checked on the host).

__device__ __forceinline__ void rope64_store(const float* xin, const uint16_t* cosr, const uint16_t* sinr, void* dst,
                                             uint32_t dst_off, int i) {
  // i in [0, 64): de-interleave, x*cos + rotate_half(x)*sin, bf16 at every op
  float xd = i < 32 ? xin[2 * i] : xin[2 * (i - 32) + 1];
  float rot = i < 32 ? -xin[2 * i + 1] : xin[2 * (i - 32)];
  float a = bf16r(xd * bf2f(cosr[i]));
  float b = bf16r(rot * bf2f(sinr[i]));
  stc2(dst, dst_off + (uint32_t)i * 2, f2bf(a + b));
}

// FX_OP_MLA_PREP (harness/numpy_ref.py:85-103): tasks per XCD: hp*4 ql_nope column blocks of 128,
// then one task for the cache row (c_kv norm, k_pe rope) and the XCD's q_pe rows.
__device__ void op_mla_prep(const fx_stage& s, const FxEnv& env) {
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

// FX_OP_MLA_ATTEND (harness/numpy_ref.py:110-149) for the XCD's two heads, one split per task,
// tiles of 32 positions; the last task of the XCD to finish merges its heads' partials
// (harness/numpy_ref.py:152-165) into o_merged (aux4, bf16 [nh][d_c]).
#define ATT_T 32
#define ATT_ROW 584   // bf16 elements per staged row: 576 + 8 pad (1168 bytes)

__device__ void attend_merge(const fx_stage& s, const FxEnv& env);

__device__ void op_mla_attend(const fx_stage& s, const FxEnv& env) {
  const int nh = s.n_rows, d_c = s.d_c, d_r = s.d_r, prow = s.prow;
  const int hp = 2;
  const int h0 = env.xcd * hp;
  const int step = env.step;
  const int split = s.split, n_splits = s.n_splits;
  const float scale = s.scale;
  float* ql = (float*)(env.lds + LDS_XS);                 // [2][512]
  float* qp = ql + 2 * 512;                               // [2][64]
  float* sp = qp + 2 * 64;                                // [2][32][5] partial scores
  float* sl = sp + 2 * 32 * 5;                            // [2][32] scores
  float* pb = sl + 64;                                    // [2][32] bf16(p)
  float* pp = pb + 64;                                    // [2][32] p
  float* hs = pp + 64;                                    // [2][4] m, l, alpha, psum
  uint16_t* tile = (uint16_t*)(env.lds + LDS_TILE);       // [32][ATT_ROW]
  const uint16_t* ckv = (const uint16_t*)s.aux[0];
  const uint16_t* kpe = (const uint16_t*)s.aux[1];
  void* part = (void*)s.out;
  bool did_task = false;
  for (int j = env.xrank; j < n_splits; j += env.xworkers) {
    did_task = true;
    __syncthreads();
    // q rows of the XCD's heads
    for (int i = threadIdx.x; i < hp * d_c / 8; i += FX_THREADS) {
      const int hh = i / (d_c / 8), c = (i % (d_c / 8)) * 8;
      u32x4 v = ldc16((const void*)s.x, (uint32_t)((h0 + hh) * d_c + c) * 2);
      float* d = ql + hh * 512 + c;
      d[0] = bf_lo(v.x); d[1] = bf_hi(v.x); d[2] = bf_lo(v.y); d[3] = bf_hi(v.y);
      d[4] = bf_lo(v.z); d[5] = bf_hi(v.z); d[6] = bf_lo(v.w); d[7] = bf_hi(v.w);
    }
    if (threadIdx.x < hp * d_r) {
      const int hh = threadIdx.x / d_r, r = threadIdx.x % d_r;
      qp[hh * 64 + r] = bf2f(ldc2((const void*)s.aux[2], (uint32_t)((h0 + hh) * d_r + r) * 2));
    }
    if (threadIdx.x < hp) { hs[threadIdx.x * 4 + 0] = -__builtin_inff(); hs[threadIdx.x * 4 + 1] = 0.0f; }
    const int lo = j * split;
    int hi = lo + split;
    if (hi > step + 1) hi = step + 1;
    // accumulators: thread -> head h = tid >> 7, columns 4 * (tid & 127) .. + 3
    const int ph = threadIdx.x >> 7, pc = (threadIdx.x & 127) * 4;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    __syncthreads();
    for (int t0 = lo; t0 < hi; t0 += ATT_T) {
      const int nt = (t0 + ATT_T < hi ? t0 + ATT_T : hi) - t0;
      // stage rows t0 .. t0+nt-1 (never a row past `step`)
      for (int q = threadIdx.x; q < nt * 72; q += FX_THREADS) {
        const int r = q / 72, c = q % 72;
        u32x4 v = c < 64 ? ld16(ckv + (size_t)(t0 + r) * d_c + c * 8) : ld16(kpe + (size_t)(t0 + r) * d_r + (c - 64) * 8);
        *(u32x4*)(tile + r * ATT_ROW + c * 8) = v;
      }
      __syncthreads();
      // scores: thread (h, t, k): chain k over columns [128k, 128k + 128); k == 0 also the rope chain
      {
        const int h = threadIdx.x >> 7, t = (threadIdx.x >> 2) & 31, k = threadIdx.x & 3;
        float a = 0.0f, b = 0.0f;
        if (t < nt) {
          const uint16_t* kr = tile + t * ATT_ROW;
          const float* qr = ql + h * 512;
          for (int c = k * 128; c < k * 128 + 128; c += 8) {
            u32x4 kv = *(const u32x4*)(kr + c);
            a = __builtin_fmaf(qr[c + 0], bf_lo(kv.x), a);
            a = __builtin_fmaf(qr[c + 1], bf_hi(kv.x), a);
            a = __builtin_fmaf(qr[c + 2], bf_lo(kv.y), a);
            a = __builtin_fmaf(qr[c + 3], bf_hi(kv.y), a);
            a = __builtin_fmaf(qr[c + 4], bf_lo(kv.z), a);
            a = __builtin_fmaf(qr[c + 5], bf_hi(kv.z), a);
            a = __builtin_fmaf(qr[c + 6], bf_lo(kv.w), a);
            a = __builtin_fmaf(qr[c + 7], bf_hi(kv.w), a);
          }
          if (k == 0) {
            const float* qpr = qp + h * 64;
            for (int r = 0; r < 64; r += 8) {
              u32x4 kv = *(const u32x4*)(kr + 512 + r);
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
      // softmax of the tile: wave 0, lane = h * 32 + t
      if (threadIdx.x < 64) {
        const int h = threadIdx.x >> 5, t = threadIdx.x & 31;
        float sc = -__builtin_inff();
        if (t < nt) {
          const float* q = sp + (h * 32 + t) * 5;
          float v = q[0] + q[1];
          v = v + q[2];
          v = v + q[3];
          v = v + q[4];
          sc = v * scale;
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
        const float alpha = hs[h * 4 + 2];
        float l = hs[h * 4 + 1];
        l = l * alpha + psum;
        hs[h * 4 + 1] = l;
        hs[h * 4 + 0] = hs[h * 4 + 3];
      }
      // value product: sequential over positions
      {
        const float alpha = hs[ph * 4 + 2];
        float tp[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int t = 0; t < nt; ++t) {
          const float pv = pb[ph * 32 + t];
          u32x2 kv = *(const u32x2*)(tile + t * ATT_ROW + pc);
          tp[0] = __builtin_fmaf(pv, bf_lo(kv.x), tp[0]);
          tp[1] = __builtin_fmaf(pv, bf_hi(kv.x), tp[1]);
          tp[2] = __builtin_fmaf(pv, bf_lo(kv.y), tp[2]);
          tp[3] = __builtin_fmaf(pv, bf_hi(kv.y), tp[3]);
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          float a = acc[c] * alpha;
          acc[c] = a + tp[c];
        }
      }
      __syncthreads();
    }
    // outputs: o = acc / l, lse = m + log(l); an empty split stores o = 0, lse = -inf
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
    uint32_t old = __hip_atomic_fetch_add(&env.sync[FX_CNT_ATTEND(env.xcd)], (uint32_t)done, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
    const bool last = old + done == (uint32_t)n_splits;
    if (last) flag_st(&env.sync[FX_CNT_ATTEND(env.xcd)], 0u);
    misc[0] = last ? 1 : 0;
  }
  __syncthreads();
  if (misc[0]) attend_merge(s, env);
}

// merge the live splits of the XCD's two heads: M = max lse, w_j = exp(lse_j - M),
// o = (sum_j w_j o_j, sequential fma) / (sum_j w_j, sequential) -> bf16
__device__ void attend_merge(const fx_stage& s, const FxEnv& env) {
  const int nh = s.n_rows, d_c = s.d_c, prow = s.prow;
  const int h0 = env.xcd * 2;
  const int live = (env.step + 1 + s.split - 1) / s.split;
  const void* part = (const void*)s.out;
  float* wj = (float*)(env.lds + LDS_TILE);   // [2][live]
  float* red = (float*)(env.lds + LDS_RED);
  // weights: wave h handles head h
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
  for (int j = 0; j < live; ++j) {
    const float w = wj[ph * live + j];
    u32x4 o = ldc16(part, (uint32_t)((j * nh + h0 + ph) * prow + pc) * 4);
    num[0] = __builtin_fmaf(w, __uint_as_float(o.x), num[0]);
    num[1] = __builtin_fmaf(w, __uint_as_float(o.y), num[1]);
    num[2] = __builtin_fmaf(w, __uint_as_float(o.z), num[2]);
    num[3] = __builtin_fmaf(w, __uint_as_float(o.w), num[3]);
  }
  const float den = red[ph];
  u32x2 r;
  r.x = pack2(num[0] / den, num[1] / den);
  r.y = pack2(num[2] / den, num[3] / den);
  stc8((void*)s.aux[4], (uint32_t)((h0 + ph) * d_c + pc) * 2, r);
}

// FX_OP_MLA_MERGE_UV: attn[h*d_v + v] = bf16(dot(o_merged[h], W_uv[h][v])) for the XCD's heads
// (harness/numpy_ref.py:168-174); the merge itself ran at the end of the attend stage.
__device__ void op_mla_merge_uv(const fx_stage& s, const FxEnv& env) {
  const int d_c = s.d_c, d_v = s.d_n;   // d_n field carries d_v (128) here
  const int hp = 2;
  const int h0 = env.xcd * hp;
  float* xs = (float*)(env.lds + LDS_XS);
  load_vec_sc1(xs, (const uint8_t*)s.x + (size_t)h0 * d_c * 2, hp * d_c);
  __syncthreads();
  int r0, r1;
  range_split(hp * d_v, env.xworkers, env.xrank, r0, r1);
  const uint16_t* W = (const uint16_t*)s.w + (size_t)h0 * d_v * d_c;
  void* out = (void*)s.out;
  const int ngroups = (r1 - r0 + 3) / 4;
  // the row r (0..hp*d_v) of this XCD uses o of head r / d_v: shift xs per row via a 2-pass split
  for (int hh = 0; hh < hp; ++hh) {
    int a = r0 > hh * d_v ? r0 : hh * d_v;
    int b = r1 < (hh + 1) * d_v ? r1 : (hh + 1) * d_v;
    if (a >= b) continue;
    const int ng = (b - a + 3) / 4;
    gemv_groups<4, 1>(
        W, d_c, xs + hh * d_c, ng, [&](int g, int i) { int r = a + g * 4 + i; return r < b ? r : -1; },
        [&](int g, const int* row, const bool* valid, const float* acc) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (valid[i] && lane_id() == i) stc2(out, (uint32_t)(h0 * d_v + row[i]) * 2, f2bf(acc[i]));
        });
  }
  (void)ngroups;
}

// ------------------------------------------------------------------------------------------------

__device__ void run_stage(const fx_stage& s, const FxEnv& env) {
  switch (s.op) {
    case FX_OP_GEMV: op_gemv(s, env); break;
    case FX_OP_MLA_PREP: op_mla_prep(s, env); break;
    case FX_OP_MLA_ATTEND: op_mla_attend(s, env); break;
    case FX_OP_MLA_MERGE_UV: op_mla_merge_uv(s, env); break;
    case FX_OP_MOE_ROUTER: op_moe_router(s, env); break;
    case FX_OP_MOE_W13: op_moe_w13(s, env); break;
    case FX_OP_MOE_W2: op_moe_w2(s, env); break;
    case FX_OP_MOE_COMBINE: op_moe_combine(s, env); break;
    case FX_OP_DENSE_GU: op_dense_gu(s, env); break;
    case FX_OP_ARGMAX: op_argmax(s, env); break;
    default: break;
  }
}
