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
  static constexpr int kRows = R;
  using Row = Tile<1, NJ>;   // one row of the same chunking
  u32x4 w[R][NJ];
  int row[R];
};

// FP8 weights (OCP e4m3fn codes, one f32 scale per row): a row of K codes, then the output is
// scale[row] * dot_lanes16(codes, x): chunk c of 16 contiguous codes (16 bytes) -> lane c % 64,
// one fma per element in order, the xor butterfly, then one multiply by the row's scale.
struct Fp8W {
  const uint8_t* q;   // codes [rows][K]
  const float* s;     // scale [rows]
};
template <int R, int NJ>
struct TileQ {
  static constexpr int kRows = R;
  using Row = TileQ<1, NJ>;
  u32x4 w[R][NJ];
  int row[R];
  float sc[R];
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
  fx_issue_here();
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
  if (nchunk >= 64) {
#pragma unroll
    for (int i = 0; i < R; ++i) acc[i] = butterfly64(acc[i]);
  } else {
    const int nl = lanes_for(nchunk);
#pragma unroll
    for (int i = 0; i < R; ++i) acc[i] = butterfly(acc[i], nl);
  }
}

template <int R, int NJ, class RowFn>
__device__ __forceinline__ void tile_load(TileQ<R, NJ>& t, const Fp8W& W, int K, int g, RowFn& rowof) {
  const int lane = lane_id();
  const int nchunk = K >> 4;
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
      t.w[i][j] = ldw16(W.q + (size_t)r * K + (size_t)cc * 16);
    }
  }
#pragma unroll
  for (int i = 0; i < R; ++i) t.sc[i] = W.s[t.row[i] >= 0 ? t.row[i] : first];
  fx_issue_here();
}

// the 16 codes of a chunk as f32 (the hardware's OCP e4m3fn conversion, byte k = element k)
__device__ __forceinline__ void unpack16_fp8(u32x4 v, float* d) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[k], false);
    const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[k], true);
    d[4 * k + 0] = lo[0];
    d[4 * k + 1] = lo[1];
    d[4 * k + 2] = hi[0];
    d[4 * k + 3] = hi[1];
  }
}

template <int R, int NJ>
__device__ __forceinline__ void tile_dot(const TileQ<R, NJ>& t, const float* xs, int K, float* acc) {
  const int lane = lane_id();
  const int nchunk = K >> 4;
#pragma unroll
  for (int i = 0; i < R; ++i) acc[i] = 0.0f;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int c = lane + 64 * j;
    if (c < nchunk) {
      const float4* xp = (const float4*)(xs + c * 16);
      const float4 a = xp[0], b = xp[1], e = xp[2], f = xp[3];
      const float xv[16] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w, e.x, e.y, e.z, e.w, f.x, f.y, f.z, f.w};
#pragma unroll
      for (int i = 0; i < R; ++i) {
        float wv[16];
        unpack16_fp8(t.w[i][j], wv);
#pragma unroll
        for (int k = 0; k < 16; ++k) acc[i] = __builtin_fmaf(wv[k], xv[k], acc[i]);
      }
    }
  }
  if (nchunk >= 64) {
#pragma unroll
    for (int i = 0; i < R; ++i) acc[i] = butterfly64(acc[i]) * t.sc[i];
  } else {
    const int nl = lanes_for(nchunk);
#pragma unroll
    for (int i = 0; i < R; ++i) acc[i] = butterfly(acc[i], nl) * t.sc[i];
  }
}

// Issue the loads of this wave's first group (group index = wave id) into t0.
template <class TileT, class WT, class RowFn>
__device__ __forceinline__ void gemv_prime(TileT& t0, const WT& W, int K, int ngroups, RowFn& rowof) {
  if (wave_id() < ngroups) tile_load(t0, W, K, wave_id(), rowof);
}

// The rolling walk: tile_dot of group k that, as soon as chunk column j of every row has been
// consumed, re-fills those registers with chunk j of group gn (the wave's group two tiles ahead),
// so the next tile's loads leave during this dot instead of after it, with no more registers than
// two tiles. Each row's dot is tile_dot's (chunks in increasing j, one fma per element, the same
// butterfly); a lane past the row's last chunk computes on the last chunk and keeps its sum
// unchanged (a select, not a branch: the loads are unconditional, so the compiler's load counters
// stay exact). `rows` receives the reduced group's rows; t then describes group gn.
__device__ __forceinline__ void roll_fence(float* acc, int n) {
  // the chunk's fmas are complete before the loads that reuse its registers are issued
  for (int i = 0; i < n; ++i) asm volatile("" : "+v"(acc[i])::"memory");
}
template <int R, int NJ, class RowFn>
__device__ __forceinline__ void tile_dot_roll(Tile<R, NJ>& t, const float* xs, int K, float* acc, int* rows,
                                              const uint16_t* __restrict__ W, int gn, RowFn& rowof) {
  const int lane = lane_id();
  const int nchunk = K >> 3;
  int nrow[R];
  int first = -1;
#pragma unroll
  for (int i = 0; i < R; ++i) {
    rows[i] = t.row[i];
    nrow[i] = rowof(gn, i);
    if (first < 0 && nrow[i] >= 0) first = nrow[i];
    acc[i] = 0.0f;
  }
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int c = lane + 64 * j;
    const bool on = c < nchunk;
    const int cc = on ? c : nchunk - 1;
    const float4* xp = (const float4*)(xs + cc * 8);
    const float4 a = xp[0], b = xp[1];
    const float xv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const float v = fma8(t.w[i][j], xv, acc[i]);
      acc[i] = on ? v : acc[i];
    }
    roll_fence(acc, R);
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int r = nrow[i] >= 0 ? nrow[i] : first;
      t.w[i][j] = ldw16(W + (size_t)r * K + (size_t)cc * 8);
    }
    fx_issue_here();
  }
#pragma unroll
  for (int i = 0; i < R; ++i) t.row[i] = nrow[i];
  if (nchunk >= 64) {
#pragma unroll
    for (int i = 0; i < R; ++i) acc[i] = butterfly64(acc[i]);
  } else {
    const int nl = lanes_for(nchunk);
#pragma unroll
    for (int i = 0; i < R; ++i) acc[i] = butterfly(acc[i], nl);
  }
}
template <int R, int NJ, class RowFn>
__device__ __forceinline__ void tile_dot_roll(TileQ<R, NJ>& t, const float* xs, int K, float* acc, int* rows,
                                              const Fp8W& W, int gn, RowFn& rowof) {
  const int lane = lane_id();
  const int nchunk = K >> 4;
  int nrow[R];
  int first = -1;
#pragma unroll
  for (int i = 0; i < R; ++i) {
    rows[i] = t.row[i];
    nrow[i] = rowof(gn, i);
    if (first < 0 && nrow[i] >= 0) first = nrow[i];
    acc[i] = 0.0f;
  }
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int c = lane + 64 * j;
    const bool on = c < nchunk;
    const int cc = on ? c : nchunk - 1;
    const float4* xp = (const float4*)(xs + cc * 16);
    const float4 a = xp[0], b = xp[1], e = xp[2], f = xp[3];
    const float xv[16] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w, e.x, e.y, e.z, e.w, f.x, f.y, f.z, f.w};
#pragma unroll
    for (int i = 0; i < R; ++i) {
      float wv[16];
      unpack16_fp8(t.w[i][j], wv);
      float v = acc[i];
#pragma unroll
      for (int k = 0; k < 16; ++k) v = __builtin_fmaf(wv[k], xv[k], v);
      acc[i] = on ? v : acc[i];
    }
    roll_fence(acc, R);
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int r = nrow[i] >= 0 ? nrow[i] : first;
      t.w[i][j] = ldw16(W.q + (size_t)r * K + (size_t)cc * 16);
    }
    fx_issue_here();
  }
  if (nchunk >= 64) {
#pragma unroll
    for (int i = 0; i < R; ++i) acc[i] = butterfly64(acc[i]) * t.sc[i];
  } else {
    const int nl = lanes_for(nchunk);
#pragma unroll
    for (int i = 0; i < R; ++i) acc[i] = butterfly(acc[i], nl) * t.sc[i];
  }
  roll_fence(acc, R);
#pragma unroll
  for (int i = 0; i < R; ++i) {
    t.row[i] = nrow[i];
    t.sc[i] = W.s[nrow[i] >= 0 ? nrow[i] : first];
  }
  fx_issue_here();
}
// gemv_pipe_x's walk with rolling dots: t0 holds group `wave` (gemv_prime) and the group WS ahead is
// requested here. While both tiles have a group two ahead, each dot requests it (unconditionally);
// the last groups are reduced by tile_dot, as in gemv_pipe_x. The rolling loop is entered only on
// the path that requested t1, so every path into it has the same loads in flight (the compiler's
// load counts at the loop head are then exact instead of those of the shortest path).
template <int WS = FX_WAVES, class TileT, class WT, class RowFn, class XsFn, class EmitFn>
__device__ __forceinline__ void gemv_pipe_roll(TileT& t0, const WT& W, int K, XsFn xsof, int ngroups, RowFn& rowof,
                                               EmitFn emit) {
  TileT t1;
  float acc[TileT::kRows];
  int rows[TileT::kRows];
  int g = wave_id();
  if (g + 3 * WS < ngroups) {
    tile_load(t1, W, K, g + WS, rowof);
    do {
      tile_dot_roll(t0, xsof(g), K, acc, rows, W, g + 2 * WS, rowof);
      emit(g, rows, acc);
      tile_dot_roll(t1, xsof(g + WS), K, acc, rows, W, g + 3 * WS, rowof);
      emit(g + WS, rows, acc);
      g += 2 * WS;
    } while (g + 3 * WS < ngroups);
  } else if (g + WS < ngroups) {
    tile_load(t1, W, K, g + WS, rowof);
  }
  // t0 holds g, t1 holds g + WS; g + 2 WS (if any) is requested into t0 once t0 is reduced
  if (g < ngroups) {
    tile_dot(t0, xsof(g), K, acc);
    emit(g, t0.row, acc);
    if (g + WS < ngroups) {
      const int g2 = g + 2 * WS;
      if (g2 < ngroups) tile_load(t0, W, K, g2, rowof);
      tile_dot(t1, xsof(g + WS), K, acc);
      emit(g + WS, t1.row, acc);
      if (g2 < ngroups) {
        tile_dot(t0, xsof(g2), K, acc);
        emit(g2, t0.row, acc);
      }
    }
  }
}
// Walk the wave's groups g = wave, wave + WS, ... (WS: the waves that walk, 0 .. WS - 1); t0 holds
// group `wave` (gemv_prime). emit(g, rows, acc) sees the R results on every lane (row < 0: no row).
// FP8 tiles take the rolling walk above (FX_PIPE_ROLL_FP8, default on); bf16 tiles take it only
// with FX_PIPE_ROLL (default off: measured no faster in the decode, whose bf16 walks are 4 tiles per
// wave) and otherwise request tile k + 2 after tile k's whole dot (FX_PIPE_DEPTH 2) or rotate three
// tiles (FX_PIPE_DEPTH 3).
#ifndef FX_PIPE_ROLL
#define FX_PIPE_ROLL 0
#endif
#ifndef FX_PIPE_ROLL_FP8
#define FX_PIPE_ROLL_FP8 1
#endif
#ifndef FX_PIPE_DEPTH
#define FX_PIPE_DEPTH 2
#endif
template <class TileT>
struct RollOf {
  static constexpr bool value = FX_PIPE_ROLL;
};
template <int R, int NJ>
struct RollOf<TileQ<R, NJ>> {
  static constexpr bool value = FX_PIPE_ROLL_FP8;
};
template <int WS = FX_WAVES, class TileT, class WT, class RowFn, class XsFn, class EmitFn>
__device__ __forceinline__ void gemv_pipe_x(TileT& t0, const WT& W, int K, XsFn xsof, int ngroups, RowFn& rowof,
                                            EmitFn emit) {
  if constexpr (RollOf<TileT>::value) {
    gemv_pipe_roll<WS>(t0, W, K, xsof, ngroups, rowof, emit);
    return;
  }
  TileT t1;
  float acc[TileT::kRows];
  int g = wave_id();
#if FX_PIPE_DEPTH == 3
  static_assert(WS == FX_WAVES, "the 3-deep walk uses every wave");
  // three tiles in rotation: while one is reduced, the next two are in flight
  TileT t2;
  if (g + FX_WAVES < ngroups) tile_load(t1, W, K, g + FX_WAVES, rowof);
  while (g < ngroups) {
    if (g + 2 * FX_WAVES < ngroups) tile_load(t2, W, K, g + 2 * FX_WAVES, rowof);
    tile_dot(t0, xsof(g), K, acc);
    emit(g, t0.row, acc);
    g += FX_WAVES;
    if (g >= ngroups) break;
    if (g + 2 * FX_WAVES < ngroups) tile_load(t0, W, K, g + 2 * FX_WAVES, rowof);
    tile_dot(t1, xsof(g), K, acc);
    emit(g, t1.row, acc);
    g += FX_WAVES;
    if (g >= ngroups) break;
    if (g + 2 * FX_WAVES < ngroups) tile_load(t1, W, K, g + 2 * FX_WAVES, rowof);
    tile_dot(t2, xsof(g), K, acc);
    emit(g, t2.row, acc);
    g += FX_WAVES;
  }
#else
  while (g < ngroups) {
    const int g1 = g + WS;
    if (g1 < ngroups) tile_load(t1, W, K, g1, rowof);
    tile_dot(t0, xsof(g), K, acc);
    emit(g, t0.row, acc);
    if (g1 >= ngroups) break;
    const int g2 = g1 + WS;
    if (g2 < ngroups) tile_load(t0, W, K, g2, rowof);
    tile_dot(t1, xsof(g1), K, acc);
    emit(g1, t1.row, acc);
    g = g2;
  }
#endif
}
// the same walk with one input row for every group
template <int WS = FX_WAVES, class TileT, class WT, class RowFn, class EmitFn>
__device__ __forceinline__ void gemv_pipe(TileT& t0, const WT& W, int K, const float* xs, int ngroups, RowFn& rowof,
                                          EmitFn emit) {
  gemv_pipe_x<WS>(t0, W, K, [=](int) { return xs; }, ngroups, rowof, emit);
}

// The same walk at the granularity of one chunk column: a slice is the R rows' chunk j (R KiB), and
// the wave keeps D slices in flight instead of two whole tiles, so a CU queues D x R x 4 KiB of weight
// loads rather than 2 x R x NJ x 4 KiB: its later polls wait behind less. The arithmetic is
// tile_dot's (each row's chunks in increasing j, then the butterfly). rowof(g, i) as for the tiles.
// The first D slices of group `wave` are issued by slices_prime.
template <int R, int D>
struct SliceRing {
  u32x4 w[D][R];
  int row[R];
};
template <int R, class RowFn>
__device__ __forceinline__ void slice_rows(int (&row)[R], int g, RowFn& rowof) {
#pragma unroll
  for (int i = 0; i < R; ++i) row[i] = rowof(g, i);
}
template <int R>
__device__ __forceinline__ void slice_load(u32x4 (&b)[R], const int (&row)[R], const uint16_t* __restrict__ W, int K, int j) {
  const int nchunk = K >> 3;
  const int c = lane_id() + 64 * j;
  const int cc = c < nchunk ? c : nchunk - 1;
  int first = row[0];
#pragma unroll
  for (int i = 1; i < R; ++i)
    if (first < 0) first = row[i];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int r = row[i] >= 0 ? row[i] : first;
    b[i] = ldw16(W + (size_t)r * K + (size_t)cc * 8);
  }
  fx_issue_here();
}
template <int R, int NJ, int D, class RowFn>
__device__ __forceinline__ void slices_prime(SliceRing<R, D>& q, const uint16_t* W, int K, int ngroups, RowFn& rowof) {
  if (wave_id() >= ngroups) return;
  slice_rows(q.row, wave_id(), rowof);
#pragma unroll
  for (int d = 0; d < D && d < NJ; ++d) slice_load(q.w[d], q.row, W, K, d);
}
template <int NJ, int WS = FX_WAVES, int R, int D, class RowFn, class XsFn, class EmitFn>
__device__ __forceinline__ void gemv_slices_x(SliceRing<R, D>& q, const uint16_t* W, int K, XsFn xsof, int ngroups,
                                              RowFn& rowof, EmitFn emit) {
  static_assert(NJ % D == 0, "a group's slices must fill the ring evenly");
  const int nchunk = K >> 3;
  int g = wave_id();
  int rown[R];
  while (g < ngroups) {
    const int gn = g + WS;
    if (gn < ngroups) slice_rows(rown, gn, rowof);
    const float* xs = xsof(g);
    float acc[R];
#pragma unroll
    for (int i = 0; i < R; ++i) acc[i] = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int c = lane_id() + 64 * j;
      if (c < nchunk) {
        const float4* xp = (const float4*)(xs + c * 8);
        const float4 a = xp[0], b = xp[1];
        const float xv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int i = 0; i < R; ++i) acc[i] = fma8(q.w[j % D][i], xv, acc[i]);
      }
      // refill the slice just consumed with the one D places further on
      if (j + D < NJ) slice_load(q.w[j % D], q.row, W, K, j + D);
      else if (gn < ngroups) slice_load(q.w[j % D], rown, W, K, j + D - NJ);
    }
    if (nchunk >= 64) {
#pragma unroll
      for (int i = 0; i < R; ++i) acc[i] = butterfly64(acc[i]);
    } else {
      const int nl = lanes_for(nchunk);
#pragma unroll
      for (int i = 0; i < R; ++i) acc[i] = butterfly(acc[i], nl);
    }
    emit(g, q.row, acc);
    if (gn >= ngroups) break;
#pragma unroll
    for (int i = 0; i < R; ++i) q.row[i] = rown[i];
    g = gn;
  }
}

// A GEMV stage's walk over its groups: the tiled pipeline (two whole tiles in flight per wave), or,
// built with FX_SLICE_D > 0, for the K = 2048 bf16 tiles the sliced one (FX_SLICE_D slices of 4 KiB
// in flight per wave). Same arithmetic either way. The sliced walk streams as fast as the tiled one
// on its own (harness/probes.py --gemv) but made the decode slower (1,696 / 1,703 against 1,680 /
// 1,674 us per token at ctx 1,024), so the default is the tiled walk.
#ifndef FX_SLICE_D
#define FX_SLICE_D 0
#endif
template <class TileT>
struct Walker {
  TileT t0;
  template <class WT, class RowFn>
  __device__ __forceinline__ void prime(const WT& W, int K, int ngroups, RowFn& rowof) {
    gemv_prime(t0, W, K, ngroups, rowof);
  }
  template <class WT, class RowFn, class EmitFn>
  __device__ __forceinline__ void run(const WT& W, int K, const float* xs, int ngroups, RowFn& rowof, EmitFn emit) {
    gemv_pipe(t0, W, K, xs, ngroups, rowof, emit);
  }
};
#if FX_SLICE_D > 0
template <>
struct Walker<Tile<4, 4>> {
  SliceRing<4, FX_SLICE_D> q;
  template <class RowFn>
  __device__ __forceinline__ void prime(const uint16_t* W, int K, int ngroups, RowFn& rowof) {
    slices_prime<4, 4>(q, W, K, ngroups, rowof);
  }
  template <class RowFn, class EmitFn>
  __device__ __forceinline__ void run(const uint16_t* W, int K, const float* xs, int ngroups, RowFn& rowof, EmitFn emit) {
    gemv_slices_x<4>(q, W, K, [=](int) { return xs; }, ngroups, rowof, emit);
  }
};
#endif

// ------------------------------------------------------------------------------------------------
// input-row prologues: every thread takes 8-element chunks i = 8 * tid, 8 * (tid + 256), ...

__device__ __forceinline__ void unpack8(u32x4 v, float* d) {
  d[0] = bf_lo(v.x); d[1] = bf_hi(v.x); d[2] = bf_lo(v.y); d[3] = bf_hi(v.y);
  d[4] = bf_lo(v.z); d[5] = bf_hi(v.z); d[6] = bf_lo(v.w); d[7] = bf_hi(v.w);
}

// xs[0, K) <- the K bf16 values of a packet vector (K / 2 packets, K a multiple of 4): thread t
// takes pairs t, t + 256, ... (4 values each). Ends before any __syncthreads: the caller syncs.
template <int N>
__device__ __forceinline__ void poll_row_n(float* xs, const void* src, int K, uint32_t tag, uint32_t* err) {
  u32x4 v[N];
  const int npairs = K >> 2;
  pk_wait_pairs<N>(src, fx_tid(), FX_THREADS, npairs, tag, err, v);
#pragma unroll
  for (int n = 0; n < N; ++n) {
    const int q = fx_tid() + n * FX_THREADS;
    if (q < npairs) {
      xs[4 * q + 0] = bf_lo(v[n].x);
      xs[4 * q + 1] = bf_hi(v[n].x);
      xs[4 * q + 2] = bf_lo(v[n].z);
      xs[4 * q + 3] = bf_hi(v[n].z);
    }
  }
}
__device__ __forceinline__ void poll_row(float* xs, const void* src, int K, uint32_t tag, uint32_t* err) {
  if (K <= 4 * FX_THREADS) poll_row_n<1>(xs, src, K, tag, err);
  else if (K <= 8 * FX_THREADS) poll_row_n<2>(xs, src, K, tag, err);
  else if (K <= 16 * FX_THREADS) poll_row_n<4>(xs, src, K, tag, err);
  else poll_row_n<12>(xs, src, K, tag, err);
}

// plain (non-packet) copy of a bf16 row to a dump buffer
__device__ __forceinline__ void store_vec_sc1(void* dst, const float* xs, int K) {
  for (int i = fx_tid() * 8; i < K; i += FX_THREADS * 8) {
    u32x4 v;
    v.x = pack2(xs[i + 0], xs[i + 1]);
    v.y = pack2(xs[i + 2], xs[i + 3]);
    v.z = pack2(xs[i + 4], xs[i + 5]);
    v.w = pack2(xs[i + 6], xs[i + 7]);
    stc16(dst, (uint32_t)i * 2, v);
  }
}

// rmsnorm in place on xs (harness/numpy_ref.py:54-60): var = dot_lanes(x, x) / K,
// rs = 1 / sqrt(var + eps), y = bf16(w * bf16(x * rs)). Starts and ends with __syncthreads.
// wchunk(i): the 8 bf16 norm weights of elements i .. i + 8.
template <class WChunk>
__device__ __forceinline__ void rmsnorm_body(float* xs, int K, float eps, float* red, WChunk wchunk) {
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
  for (int i = fx_tid() * 8; i < K; i += FX_THREADS * 8) {
    float w8[8];
    unpack8(wchunk(i), w8);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float xn = bf16r(xs[i + e] * rs);
      xs[i + e] = bf16r(w8[e] * xn);
    }
  }
  __syncthreads();
}
__device__ __forceinline__ void rmsnorm_inplace(float* xs, const uint16_t* wn, int K, float eps, float* red) {
  rmsnorm_body(xs, K, eps, red, [&](int i) { return ld16(wn + i); });
}
// The same with the norm weights requested ahead (norm_prefetch, before the stage polls its input:
// their load latency then hides under the wait instead of following the input). K <= 8 * FX_THREADS:
// thread t's only chunk is elements 8t .. 8t + 8.
struct NormW {
  u32x4 w;
};
__device__ __forceinline__ NormW norm_prefetch(const uint16_t* wn, int K) {
  NormW n;
  n.w = u32x4{0u, 0u, 0u, 0u};
  if (fx_tid() * 8 < K) n.w = ld16(wn + fx_tid() * 8);
  fx_issue_here();
  return n;
}
__device__ __forceinline__ void rmsnorm_pre(float* xs, const NormW& n, int K, float eps, float* red) {
  rmsnorm_body(xs, K, eps, red, [&](int) { return n.w; });
}
// either, by K
__device__ __forceinline__ void rmsnorm_staged(float* xs, const NormW& n, const uint16_t* wn, int K, float eps, float* red) {
  if (K <= 8 * FX_THREADS) rmsnorm_pre(xs, n, K, eps, red);
  else rmsnorm_inplace(xs, wn, K, eps, red);
}

// The input row and its RMSNorm on ONE wave: a stage's control wave, which has no weight loads in
// flight, so its polls return as soon as the packets exist (a wave's loads complete in issue order:
// a poll behind a weight tile waits for the tile). Same arithmetic as rmsnorm_body: var =
// sumsq_wave / K, rs = 1 / sqrt(var + eps), y = bf16(w * bf16(x * rs)). K <= 2048, a multiple of 8;
// the caller syncs before other waves read xs.
struct NormWave {
  u32x4 w[4];   // chunks lane, lane + 64, lane + 128, lane + 192 of the norm weights
};
__device__ __forceinline__ NormWave norm_prefetch_wave(const uint16_t* wn, int K) {
  NormWave n;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = lane_id() + 64 * j;
    n.w[j] = c * 8 < K ? ld16(wn + c * 8) : u32x4{0u, 0u, 0u, 0u};
  }
  fx_issue_here();
  return n;
}
__device__ __forceinline__ void poll_norm_wave(float* xs, const void* src, int K, float eps, const NormWave& n,
                                               uint32_t tag, uint32_t* err) {
  u32x4 v[8];
  const int npairs = K >> 2;
  pk_wait_pairs<8>(src, lane_id(), 64, npairs, tag, err, v);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int q = lane_id() + 64 * j;
    if (q < npairs) {
      xs[4 * q + 0] = bf_lo(v[j].x);
      xs[4 * q + 1] = bf_hi(v[j].x);
      xs[4 * q + 2] = bf_lo(v[j].z);
      xs[4 * q + 3] = bf_hi(v[j].z);
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  const float ss = sumsq_wave(xs, K);
  const float rs = 1.0f / sqrtf(ss / (float)K + eps);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int i = (lane_id() + 64 * j) * 8;
    if (i < K) {
      float w8[8];
      unpack8(n.w[j], w8);
#pragma unroll
      for (int e = 0; e < 8; ++e) xs[i + e] = bf16r(w8[e] * bf16r(xs[i + e] * rs));
    }
  }
}

// greedy id from the per-worker (max, index) packet pairs: the lowest index among the maxima (one
// wave; result on every lane)
__device__ __forceinline__ int64_t argmax_reduce(const void* amax, int nworkers, uint32_t tag, uint32_t* err) {
  u32x4 v[4];
  pk_wait_pairs<4>(amax, lane_id(), 64, nworkers, tag, err, v);
  float best = -__builtin_inff();
  int best_i = 0x7fffffff;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    if (lane_id() + 64 * k >= nworkers) continue;
    const float fv = __uint_as_float(v[k].x);
    const int id = (int)v[k].z;
    if (fv > best || (fv == best && id < best_i)) { best = fv; best_i = id; }
  }
  for (int off = 1; off < 64; off <<= 1) {
    float ov = shfl_xor_f(best, off);
    int oi = __shfl_xor(best_i, off, 64);
    if (ov > best || (ov == best && oi < best_i)) { best = ov; best_i = oi; }
  }
  return best_i;
}

// token of this iteration: tokens[step] inside the prompt, else the previous head's argmax (worker
// 0 stores it to tokens[step]); kept in env.token. amax_tag: the previous head's output tag.
__device__ __forceinline__ void embed_token(const void* amax, uint32_t amax_tag, FxEnv& env) {
  int64_t* misc = (int64_t*)(env.lds + LDS_MISC);
  if (wave_id() == 0) {
    int64_t tok;
    if (env.step < env.n_prompt) {
      u32x2 t = ldc8(env.tokens, (uint32_t)env.step * 8);
      tok = (int64_t)(((uint64_t)t.y << 32) | t.x);
    } else {
      tok = argmax_reduce(amax, env.nworkers, amax_tag, env.err);
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
  env.token = misc[0];
  __syncthreads();
}

// ------------------------------------------------------------------------------------------------
// FX_OP_GEMV: rows in groups of 4, groups split over all workers

#ifndef FX_GEMV_R
#define FX_GEMV_R 4
#endif
// TileT / WT: bf16 tiles over a bf16 matrix, or FP8 tiles over codes + per-row scales (Fp8W)
template <class TileT, class WT>
__device__ __forceinline__ void op_gemv_w(const fx_stage& s, FxEnv& env, const WT& W) {
  constexpr int R = TileT::kRows;
  float* xs = (float*)(env.lds + LDS_XS);
  float* red = (float*)(env.lds + LDS_RED);
  float* rres = (float*)(env.lds + LDS_RES);
  const int K = s.k;
  int g0, g1;
  if (s.flags & FX_F_SKIP_XCD) {
    // the workers of XCDs 0..6 (rank r of XCD x is worker r * 7 + x of 224)
    if (env.xcd == FX_XCDS - 1) return;
    range_split((s.n_rows + 3) >> 2, env.nworkers - FX_XWORKERS, env.xrank * (FX_XCDS - 1) + env.xcd, g0, g1);
  } else if (s.flags & FX_F_LOW16) {
    // ranks 0..15 of every XCD: workers 0..127 (worker = rank * 8 + XCD)
    if (env.xrank >= FX_XWORKERS / 2) return;
    range_split((s.n_rows + 3) >> 2, env.nworkers / 2, env.worker, g0, g1);
  } else {
    range_split((s.n_rows + 3) >> 2, env.nworkers, env.worker, g0, g1);
  }
  const int r0 = g0 * 4, r1 = g1 * 4 < s.n_rows ? g1 * 4 : s.n_rows;
  const int ngroups = (r1 - r0 + R - 1) / R;
  auto rowof = [&](int g, int i) { const int r = r0 + g * R + i; return r < r1 ? r : -1; };
  Walker<TileT> wk;
  wk.prime(W, K, ngroups, rowof);
  const bool norm = (s.flags & FX_F_NORM) != 0;
  const NormW nw = norm && K <= 8 * FX_THREADS ? norm_prefetch((const uint16_t*)s.w_norm, K) : NormW{};
  const bool out_ll = (s.flags & FX_F_OUT_LL) != 0;
  const bool residual = (s.flags & FX_F_RESIDUAL) != 0;
  const bool res_embed = (s.flags & FX_F_RES_EMBED) != 0;
  // ---- token, input row, residual rows
  if (s.in_kind == FX_IN_EMBED) {
    embed_token((const void*)s.aux[3], tag_in(s, env, 1), env);
    const uint16_t* erow = (const uint16_t*)s.aux[0] + (size_t)env.token * K;
    for (int i = fx_tid() * 8; i < K; i += FX_THREADS * 8) unpack8(ld16(erow + i), xs + i);
  } else {
    poll_row(xs, (const void*)s.x, K, tag_in(s, env, 0), env.err);
  }
  if (residual && fx_tid() < ((r1 - r0 + 3) >> 2)) {
    u32x4 v[1];
    pk_wait_pairs<1>((const void*)s.res, (r0 >> 2) + fx_tid(), 0, (r1 + 3) >> 2, tag_in(s, env, 2), env.err, v);
    const int i = 4 * fx_tid();
    rres[i + 0] = bf_lo(v[0].x);
    rres[i + 1] = bf_hi(v[0].x);
    rres[i + 2] = bf_lo(v[0].z);
    rres[i + 3] = bf_hi(v[0].z);
  }
  if (res_embed) {
    const uint16_t* erow = (const uint16_t*)s.aux[0] + (size_t)env.token * s.n_rows;
    for (int i = fx_tid(); i < r1 - r0; i += FX_THREADS) rres[i] = bf2f(erow[r0 + i]);
  }
  prof_mark(env, 1);
  if (norm) rmsnorm_staged(xs, nw, (const uint16_t*)s.w_norm, K, s.eps, red);
  else __syncthreads();
  prof_mark(env, 4);
  // ---- rows
  void* out = (void*)s.out;
  const bool want_max = (s.flags & FX_F_ARGMAX) != 0;
  const bool add_res = residual || res_embed;
  // The LM head (argmax) keeps its rows' bf16 results in LDS past the input row and stores them
  // once its walk is done: a store among the walk's weight loads slows the stream (a 400-row walk
  // per CU: 59.6 us without stores, 64.8 with one per row or per tile). The same bits reach `out`.
  const bool defer = want_max && !out_ll && (r1 - r0) <= 2 * (LDS_XS_FLOATS - K);
  uint16_t* lo16 = (uint16_t*)(xs + K);
  float best = -__builtin_inff();
  int best_i = 0x7fffffff;
  wk.run(W, K, xs, ngroups, rowof, [&](int g, const int* row, const float* acc) {
    const int lane = lane_id();
#pragma unroll
    for (int i = 0; i < R; ++i) {
      if (row[i] < 0) continue;
      float v = acc[i];
      if (add_res) v = v + rres[row[i] - r0];
      const uint32_t b = f2bf(v);
      if (out_ll) {
        if (lane == 0) rres[FX_MAX_OUT_ROWS / 2 + row[i] - r0] = bf2f(b);
      } else if (defer) {
        if (lane == i) lo16[row[i] - r0] = (uint16_t)b;
      } else if (lane == i) {
        stc2(out, (uint32_t)row[i] * 2, b);
      }
      if (want_max) {
        const float fv = bf2f(b);
        if (fv > best || (fv == best && row[i] < best_i)) { best = fv; best_i = row[i]; }
      }
    }
  });
  prof_mark(env, 5);
  if (defer) {
    // rows [r0, r1) as 8-byte stores (r0 is a multiple of 4), the last < 4 rows one by one
    __syncthreads();
    const int n = r1 - r0;
    for (int t = fx_tid(); 4 * t < n; t += FX_THREADS) {
      const int q = 4 * t;
      if (q + 4 <= n) {
        u32x2 v;
        v.x = (uint32_t)lo16[q] | ((uint32_t)lo16[q + 1] << 16);
        v.y = (uint32_t)lo16[q + 2] | ((uint32_t)lo16[q + 3] << 16);
        stc8(out, (uint32_t)(r0 + q) * 2, v);
      } else {
        for (int k = q; k < n; ++k) stc2(out, (uint32_t)(r0 + k) * 2, lo16[k]);
      }
    }
  }
  if (out_ll) {
    __syncthreads();
    const float* o = rres + FX_MAX_OUT_ROWS / 2;
    const uint32_t tag = tag_out(env);
    for (int t = fx_tid(); 4 * t < r1 - r0; t += FX_THREADS)
      pk_put2(out, (uint32_t)((r0 >> 1) + 2 * t), pack2(o[4 * t], o[4 * t + 1]), pack2(o[4 * t + 2], o[4 * t + 3]), tag);
  }
  if (want_max) {
    float* rv = red + 16;
    int* ri = (int*)(red + 32);
    if (lane_id() == 0) { rv[wave_id()] = best; ri[wave_id()] = best_i; }
    __syncthreads();
    if (fx_tid() == 0) {
      float b = rv[0];
      int bi = ri[0];
      for (int w = 1; w < FX_WAVES; ++w)
        if (rv[w] > b || (rv[w] == b && ri[w] < bi)) { b = rv[w]; bi = ri[w]; }
      pk_put2((void*)s.aux[3], (uint32_t)(2 * env.worker), __float_as_uint(b), (uint32_t)bi, tag_out(env));
    }
  }
  prof_mark(env, 2);
}

template <int NJ>
__device__ __forceinline__ void op_gemv_t(const fx_stage& s, FxEnv& env) {
  constexpr int R = NJ <= 4 ? FX_GEMV_R : 1;
  op_gemv_w<Tile<R, NJ>>(s, env, (const uint16_t*)s.w);
}

// FX_F_FP8 (the LM head of an FP8 plan): w = the codes [n_rows][K] then one f32 scale per row;
// K <= 2048 (two 16-code chunks per lane); tiles of 8 rows, 16 KiB per wave as a bf16 tile of 4
__device__ __forceinline__ void op_gemv_fp8(const fx_stage& s, FxEnv& env) {
  const Fp8W W{(const uint8_t*)s.w, (const float*)((const uint8_t*)s.w + (size_t)s.n_rows * (size_t)s.k)};
  op_gemv_w<TileQ<8, 2>>(s, env, W);
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
// is 2 pairs = rows (p, I + p, p + 1, I + p + 1), whose two act values form one packet.

struct PairRows {
  int p0, p1, I;
  __device__ __forceinline__ int operator()(int g, int i) const {
    const int p = p0 + g * 2 + (i >> 1);
    if (p >= p1) return -1;
    return (i & 1) ? I + p : p;
  }
};

// act packet of the group (pairs row[0], row[2]) at packet index pkt_base + row[0] / 2
__device__ __forceinline__ void gate_up_emit(void* act, uint32_t pkt_base, const int* row, const float* acc,
                                             uint32_t tag) {
  float a[2] = {0.0f, 0.0f};
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    if (row[2 * q] < 0) continue;
    const float gv = bf16r(acc[2 * q]);
    const float uv = bf16r(acc[2 * q + 1]);
    a[q] = silu_s(gv) * uv;
  }
  if (lane_id() == 0 && row[0] >= 0) pk_put(act, pkt_base + (uint32_t)(row[0] >> 1), pack2(a[0], a[1]), tag);
}

// FX_OP_DENSE_GU: layer-0 gate/up + SiLU over all workers (HF DeepseekV2MLP,
// modeling_deepseek.py:381-398, with numpy_ref's rounding points).
__device__ __forceinline__ void op_dense_gu(const fx_stage& s, FxEnv& env) {
  float* xs = (float*)(env.lds + LDS_XS);
  float* red = (float*)(env.lds + LDS_RED);
  const int K = s.k, I = s.n_rows;
  const uint16_t* W = (const uint16_t*)s.w;
  PairRows rowof;
  int q0, q1;
  range_split(I >> 1, env.nworkers, env.worker, q0, q1);
  rowof.p0 = 2 * q0;
  rowof.p1 = 2 * q1;
  rowof.I = I;
  const int ngroups = q1 - q0;
  // the worker's 2 (q1 - q0) pairs (an even count: every tile's rows exist) walked as tiles of one
  // gate/up pair by the rolling walk, as the expert gate|up stage's routed groups: pair g2 is
  // p0 + g2, half g2 & 1 of group g2 >> 1
  auto rowof2 = [&](int g2, int i) { return rowof(g2 >> 1, ((g2 & 1) << 1) | i); };
  Tile<2, 4> t0;
  gemv_prime(t0, W, K, 2 * ngroups, rowof2);
  const NormW nw = K <= 8 * FX_THREADS ? norm_prefetch((const uint16_t*)s.w_norm, K) : NormW{};
  poll_row(xs, (const void*)s.x, K, tag_in(s, env, 0), env.err);
  prof_mark(env, 1);
  rmsnorm_staged(xs, nw, (const uint16_t*)s.w_norm, K, s.eps, red);
  if (s.aux[6] && env.worker == 0) store_vec_sc1((void*)s.aux[6], xs, K);
  void* act = (void*)s.out;
  const uint32_t tag = tag_out(env);
  // act values of the worker's groups into LDS, published after the stream
  float* actl = (float*)(env.lds + LDS_RES);
  gemv_pipe_roll(t0, W, K, [&](int) { return (const float*)xs; }, 2 * ngroups, rowof2,
                 [&](int g2, const int* row, const float* acc) {
                   const float gv = bf16r(acc[0]);
                   const float uv = bf16r(acc[1]);
                   if (lane_id() == 0) actl[g2] = row[0] >= 0 ? silu_s(gv) * uv : 0.0f;
                 });
  __syncthreads();
  if (fx_tid() < ngroups)
    pk_put(act, (uint32_t)(q0 + fx_tid()), pack2(actl[2 * fx_tid()], actl[2 * fx_tid() + 1]), tag);
  prof_mark(env, 2);
}
