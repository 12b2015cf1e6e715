// Batch-1 bf16 GEMV of the decode path (q_proj|kv_a, o_proj, the dense MLP, the LM head, the router,
// the experts, W_uv), harness/numpy_ref.py:295-313 and the reference's linear_gemv_mi300.cuh:143-252.
//
// A wave owns groups of R rows; lane l reads the 16-byte chunks c = l, l + 64, ... of each row
// (every load instruction of the wave covers 1 KiB of one row, fully coalesced), accumulates one fma
// per element in chunk order and the rows are closed by the xor butterfly: exactly the dot_lanes
// order of the spec (fx_device.h). Weights are streamed with non-temporal loads and the walk over
// a wave's groups is software-pipelined: the next group's R x NJ chunks are in flight while the
// current group is reduced, and the first group is issued by the caller before the input row is
// built (the weights do not depend on it), so the activation prologue hides under weight latency.
#pragma once
#include "fx_common.h"

template <int R, int NJ>
struct Tile {
  u32x4 w[R][NJ];
  int row[R];
};

template <int R, int NJ, class RowFn>
__device__ __forceinline__ void tile_load(Tile<R, NJ>& t, const uint16_t* __restrict__ W, int K, int g, RowFn& rowof) {
  const int lane = lane_id();
  const int nchunk = K >> 3;
  int first = -1;
#pragma unroll
  for (int i = 0; i < R; ++i) {
    t.row[i] = rowof(g, i);
    if (first < 0 && t.row[i] >= 0) first = t.row[i];
  }
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int c = lane + 64 * j;
    const int cc = c < nchunk ? c : nchunk - 1;
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int r = t.row[i] >= 0 ? t.row[i] : first;
      t.w[i][j] = ldw16(W + (size_t)r * K + (size_t)cc * 8);
    }
  }
}

template <int R, int NJ>
__device__ __forceinline__ void tile_dot(const Tile<R, NJ>& t, const float* xs, int K, float* acc) {
  const int lane = lane_id();
  const int nchunk = K >> 3;
#pragma unroll
  for (int i = 0; i < R; ++i) acc[i] = 0.0f;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int c = lane + 64 * j;
    if (c < nchunk) {
      const float4* xp = (const float4*)(xs + c * 8);
      const float4 a = xp[0], b = xp[1];
      const float xv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int i = 0; i < R; ++i) acc[i] = fma8(t.w[i][j], xv, acc[i]);
    }
  }
  const int nl = lanes_for(nchunk);
#pragma unroll
  for (int i = 0; i < R; ++i) acc[i] = butterfly(acc[i], nl);
}

// Issue the loads of this wave's first group (group index = wave id) into t0.
template <int R, int NJ, class RowFn>
__device__ __forceinline__ void gemv_prime(Tile<R, NJ>& t0, const uint16_t* W, int K, int ngroups, RowFn& rowof) {
  if (wave_id() < ngroups) tile_load(t0, W, K, wave_id(), rowof);
}

// Walk the wave's groups g = wave, wave + 4, ...; t0 holds group `wave` (gemv_prime). emit(g, rows,
// acc) sees the R results on every lane (row < 0: no row).
template <int R, int NJ, class RowFn, class EmitFn>
__device__ __forceinline__ void gemv_pipe(Tile<R, NJ>& t0, const uint16_t* W, int K, const float* xs, int ngroups,
                                          RowFn& rowof, EmitFn emit) {
  Tile<R, NJ> t1;
  float acc[R];
  int g = wave_id();
  while (g < ngroups) {
    const int g1 = g + FX_WAVES;
    if (g1 < ngroups) tile_load(t1, W, K, g1, rowof);
    tile_dot(t0, xs, K, acc);
    emit(g, t0.row, acc);
    if (g1 >= ngroups) break;
    const int g2 = g1 + FX_WAVES;
    if (g2 < ngroups) tile_load(t0, W, K, g2, rowof);
    tile_dot(t1, xs, K, acc);
    emit(g1, t1.row, acc);
    g = g2;
  }
}

// ------------------------------------------------------------------------------------------------
// input-row prologues: every thread takes 8-element chunks i = 8 * tid, 8 * (tid + 256), ...

__device__ __forceinline__ void unpack8(u32x4 v, float* d) {
  d[0] = bf_lo(v.x); d[1] = bf_hi(v.x); d[2] = bf_lo(v.y); d[3] = bf_hi(v.y);
  d[4] = bf_lo(v.z); d[5] = bf_hi(v.z); d[6] = bf_lo(v.w); d[7] = bf_hi(v.w);
}

__device__ __forceinline__ void load_vec_sc1(float* xs, const void* src, int K) {
  for (int i = threadIdx.x * 8; i < K; i += FX_THREADS * 8) unpack8(ldc16(src, (uint32_t)i * 2), xs + i);
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

// x + sum_s out8[s] * topk_w[s] for the 8 slots in slot order, mul then add, one bf16 rounding
// (harness/numpy_ref.py:316-321). All nine rows' chunks are loaded before any arithmetic.
#define FX_SLOTS 8
__device__ __forceinline__ void combine_chunk(const void* x, const void* out8, const float* w, int K, int i, float* dst) {
  u32x4 v = ldc16(x, (uint32_t)i * 2);
  u32x4 o[FX_SLOTS];
#pragma unroll
  for (int s = 0; s < FX_SLOTS; ++s) o[s] = ldc16(out8, (uint32_t)(s * K + i) * 2);
  float acc[8];
  unpack8(v, acc);
#pragma unroll
  for (int s = 0; s < FX_SLOTS; ++s) {
    float ov[8];
    unpack8(o[s], ov);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float t = ov[e] * w[s];
      acc[e] = acc[e] + t;
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) dst[e] = acc[e];
}

// slot weights into LDS (one sc1 load per slot); ends with __syncthreads
__device__ __forceinline__ void load_slot_weights(float* w, const void* topk_w) {
  if (threadIdx.x < FX_SLOTS) w[threadIdx.x] = ldcf(topk_w, threadIdx.x);
  __syncthreads();
}

// rmsnorm in place on xs (harness/numpy_ref.py:54-60): var = dot_lanes(x, x) / K,
// rs = 1 / sqrt(var + eps), y = bf16(w * bf16(x * rs)). Starts and ends with __syncthreads.
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
    float w8[8];
    unpack8(ld16(wn + i), w8);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float xn = bf16r(xs[i + e] * rs);
      xs[i + e] = bf16r(w8[e] * xn);
    }
  }
  __syncthreads();
}

// greedy id from the per-worker (max, index) pairs: the lowest index among the maxima (one wave)
__device__ __forceinline__ int64_t argmax_reduce(const void* amax, int nworkers) {
  float best = -__builtin_inff();
  int best_i = 0x7fffffff;
  float v[4];
  int id[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int w = lane_id() + 64 * k;
    const int ww = w < nworkers ? w : 0;
    v[k] = ldcf(amax, 2 * ww);
    id[k] = (int)ldc4(amax, (2 * ww + 1) * 4);
    if (w >= nworkers) v[k] = -__builtin_inff();
  }
#pragma unroll
  for (int k = 0; k < 4; ++k)
    if (v[k] > best || (v[k] == best && id[k] < best_i)) { best = v[k]; best_i = id[k]; }
  for (int off = 1; off < 64; off <<= 1) {
    float ov = shfl_xor_f(best, off);
    int oi = __shfl_xor(best_i, off, 64);
    if (ov > best || (ov == best && oi < best_i)) { best = ov; best_i = oi; }
  }
  return best_i;
}

// ------------------------------------------------------------------------------------------------
// FX_OP_GEMV

template <int NJ>
__device__ __forceinline__ void op_gemv_t(const fx_stage& s, FxEnv& env) {
  constexpr int R = NJ <= 4 ? 4 : 1;
  float* xs = (float*)(env.lds + LDS_XS);
  float* red = (float*)(env.lds + LDS_RED);
  float* rres = (float*)(env.lds + LDS_RES);
  const uint16_t* W = (const uint16_t*)s.w;
  const int K = s.k;
  int r0, r1;
  range_split(s.n_rows, env.nworkers, env.worker, r0, r1);
  const int ngroups = (r1 - r0 + R - 1) / R;
  auto rowof = [&](int g, int i) { const int r = r0 + g * R + i; return r < r1 ? r : -1; };
  Tile<R, NJ> t0;
  gemv_prime(t0, W, K, ngroups, rowof);
  const bool residual = (s.flags & FX_F_RESIDUAL) != 0;
  if (residual)
    for (int i = threadIdx.x; i < r1 - r0; i += FX_THREADS) rres[i] = bf2f(ldc2((const void*)s.res, (uint32_t)(r0 + i) * 2));
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
    const uint16_t* erow = (const uint16_t*)s.aux[0] + (size_t)misc[0] * K;
    for (int i = threadIdx.x * 8; i < K; i += FX_THREADS * 8) unpack8(ld16(erow + i), xs + i);
  } else if (s.in_kind == FX_IN_COMBINE) {
    float* w = (float*)(env.lds + LDS_MISC + 384);
    load_slot_weights(w, (const void*)s.aux[1]);
    for (int i = threadIdx.x * 8; i < K; i += FX_THREADS * 8) {
      float a[8];
      combine_chunk((const void*)s.x, (const void*)s.aux[0], w, K, i, a);
#pragma unroll
      for (int e = 0; e < 8; ++e) xs[i + e] = bf16r(a[e]);
    }
  } else {
    load_vec_sc1(xs, (const void*)s.x, K);
  }
  if ((s.flags & FX_F_WRITE_X) && env.worker == 0) store_vec_sc1((void*)s.aux[2], xs, K);
  if (s.flags & FX_F_NORM) rmsnorm_inplace(xs, (const uint16_t*)s.w_norm, K, s.eps, red);
  else __syncthreads();
  // ---- rows
  void* out = (void*)s.out;
  const bool want_max = (s.flags & FX_F_ARGMAX) != 0;
  float best = -__builtin_inff();
  int best_i = 0x7fffffff;
  gemv_pipe(t0, W, K, xs, ngroups, rowof, [&](int g, const int* row, const float* acc) {
    const int lane = lane_id();
#pragma unroll
    for (int i = 0; i < R; ++i) {
      if (row[i] < 0) continue;
      float v = acc[i];
      if (residual) v = v + rres[row[i] - r0];
      const uint32_t b = f2bf(v);
      if (lane == i) stc2(out, (uint32_t)row[i] * 2, b);
      if (want_max) {
        const float fv = bf2f(b);
        if (fv > best || (fv == best && row[i] < best_i)) { best = fv; best_i = row[i]; }
      }
    }
  });
  if (want_max) {
    float* rv = red + 16;
    int* ri = (int*)(red + 32);
    if (lane_id() == 0) { rv[wave_id()] = best; ri[wave_id()] = best_i; }
    __syncthreads();
    if (threadIdx.x == 0) {
      float b = rv[0];
      int bi = ri[0];
      for (int w = 1; w < FX_WAVES; ++w)
        if (rv[w] > b || (rv[w] == b && ri[w] < bi)) { b = rv[w]; bi = ri[w]; }
      stcf((void*)s.aux[3], 2 * env.worker, b);
      stc4((void*)s.aux[3], (2 * env.worker + 1) * 4, (uint32_t)bi);
    }
  }
}

__device__ __forceinline__ void op_gemv(const fx_stage& s, FxEnv& env) {
  const int nj = ((s.k >> 3) + 63) / 64;
  if (nj <= 1) op_gemv_t<1>(s, env);
  else if (nj <= 3) op_gemv_t<3>(s, env);
  else if (nj <= 4) op_gemv_t<4>(s, env);
  else op_gemv_t<22>(s, env);
}

// ------------------------------------------------------------------------------------------------
// gate|up pairs with SiLU (harness/numpy_ref.py:256-292 fused): act[i] = bf16(silu(g) * u),
// g = bf16(W[i] h), u = bf16(W[I + i] h). Pairs [p0, p1) of the I pairs of W (2I rows); a group
// is 2 pairs = rows (p, I + p, p + 1, I + p + 1).

struct PairRows {
  int p0, p1, I;
  __device__ __forceinline__ int operator()(int g, int i) const {
    const int p = p0 + g * 2 + (i >> 1);
    if (p >= p1) return -1;
    return (i & 1) ? I + p : p;
  }
};

__device__ __forceinline__ void gate_up_emit(void* act, uint32_t act_off, const int* row, const float* acc) {
  const int lane = lane_id();
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    if (row[2 * q] < 0) continue;
    const float gv = bf16r(acc[2 * q]);
    const float uv = bf16r(acc[2 * q + 1]);
    const float a = silu_s(gv) * uv;
    if (lane == q) stc2(act, act_off + (uint32_t)row[2 * q] * 2, f2bf(a));
  }
}

// FX_OP_DENSE_GU: layer-0 gate/up + SiLU over all workers (HF DeepseekV2MLP,
// modeling_deepseek.py:381-398, with numpy_ref's rounding points).
__device__ __forceinline__ void op_dense_gu(const fx_stage& s, FxEnv& env) {
  float* xs = (float*)(env.lds + LDS_XS);
  float* red = (float*)(env.lds + LDS_RED);
  const int K = s.k, I = s.n_rows;
  const uint16_t* W = (const uint16_t*)s.w;
  PairRows rowof;
  range_split(I, env.nworkers, env.worker, rowof.p0, rowof.p1);
  rowof.I = I;
  const int ngroups = (rowof.p1 - rowof.p0 + 1) / 2;
  Tile<4, 4> t0;
  gemv_prime(t0, W, K, ngroups, rowof);
  load_vec_sc1(xs, (const void*)s.x, K);
  rmsnorm_inplace(xs, (const uint16_t*)s.w_norm, K, s.eps, red);
  if (s.aux[6] && env.worker == 0) store_vec_sc1((void*)s.aux[6], xs, K);
  void* act = (void*)s.out;
  gemv_pipe(t0, W, K, xs, ngroups, rowof, [&](int g, const int* row, const float* acc) { gate_up_emit(act, 0, row, acc); });
}
