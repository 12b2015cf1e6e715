// MoE operators: router, expert gate|up + SiLU, expert down fused with the combine; the argmax
// reduce. harness/numpy_ref.py:205-292, 316-321; the reference's moe_router_mi300.cuh:115-354,
// gang_moe_w13_gemv_mi300.cuh:101-219, gang_moe_w2_silu_mi300.cuh and moe_mul_sum_add.
// Slot s of the 8 (top-6 routed, then the two shared experts E, E+1 at weight 1.0). Gate|up and down
// are both spread over every worker for every slot (pair groups / 8 output rows each), shared slots
// first; the combine of a row happens where its eight slot values are.
#pragma once
#include <type_traits>

#include "fx_gemv.h"

// bf16 expert gate|up: routed groups walked as tiles of one gate/up pair with the rolling walk
#ifndef FX_W13_ROW2
#define FX_W13_ROW2 1
#endif

#define FX_SLOTS 8

// Router softmax + top-k on one wave: lane e holds logit e; the softmax sum is the xor butterfly
// over pow2ceil(E) lanes; top-k by repeated argmax, lowest index on ties (numpy_ref.py:216-227).
// ids[k], wts[k] (LDS) are written by lane 0.
__device__ __forceinline__ void softmax_topk_wave(const float* logits, int E, int topk, float scaling, int* ids,
                                                  float* wts, float* probs) {
  const int lane = lane_id();
  const float l = lane < E ? logits[lane] : -__builtin_inff();
  const float m = wave_max(l);
  float p = lane < E ? exp_s(l - m) : 0.0f;
  int nl = 1;
  while (nl < E) nl <<= 1;
  const float sum = butterfly(p, nl);
  p = p / sum;
  if (probs && lane < E) probs[lane] = p;
  float rem = lane < E ? p : -__builtin_inff();
  for (int k = 0; k < topk; ++k) {
    const float v = wave_max(rem);
    const unsigned long long bal = __ballot(rem == v);
    const int idx = __builtin_ctzll(bal);
    const float pw = __shfl(p, idx, 64);
    if (lane == 0) { ids[k] = idx; wts[k] = pw * scaling; }
    if (lane == idx) rem = -__builtin_inff();
  }
}

// wave 0: the E router logits (packets, f32) into lg[0, E)
__device__ __forceinline__ void poll_logits_wave(float* lg, const void* src, int E, uint32_t tag, uint32_t* err) {
  u32x4 v[1];
  pk_wait_pairs<1>(src, lane_id(), 0, E >> 1, tag, err, v);
  if (2 * lane_id() < E) {
    lg[2 * lane_id()] = __uint_as_float(v[0].x);
    lg[2 * lane_id() + 1] = __uint_as_float(v[0].z);
  }
}

// expert of each slot and its combine weight: ids/wts (LDS, n_slots entries) from the E logits
// (wave 0; the caller syncs)
__device__ __forceinline__ void route_slots_wave(const float* lg, const fx_stage& s, int* ids, float* wts, float* probs) {
  const int E = s.aux_i0 > 0 ? s.aux_i0 : s.n_rows;
  softmax_topk_wave(lg, E, s.topk, s.scaling, ids, wts, probs);
  if (lane_id() < s.n_forced) {
    ids[s.topk + lane_id()] = E + lane_id();
    wts[s.topk + lane_id()] = 1.0f;
  }
}

// FX_OP_MOE_ROUTER: h = rmsnorm(x_res), logits[e] = dot_lanes(W_gate[e], h) on worker e.
__device__ __forceinline__ void op_moe_router(const fx_stage& s, FxEnv& env) {
  const int E = s.n_rows;
  if (env.worker >= E) return;
  float* xs = (float*)(env.lds + LDS_XS);
  float* red = (float*)(env.lds + LDS_RED);
  const int K = s.k;
  const uint16_t* W = (const uint16_t*)s.w;
  const int e = env.worker;
  auto rowof = [&](int g, int i) { return e; };
  Tile<1, 4> t0;
  gemv_prime(t0, W, K, 1, rowof);
  const NormW nw = K <= 8 * FX_THREADS ? norm_prefetch((const uint16_t*)s.w_norm, K) : NormW{};
  poll_row(xs, (const void*)s.x, K, tag_in(s, env, 0), env.err);
  prof_mark(env, 1);
  rmsnorm_staged(xs, nw, (const uint16_t*)s.w_norm, K, s.eps, red);
  const uint32_t tag = tag_out(env);
  gemv_pipe(t0, W, K, xs, 1, rowof, [&](int g, const int* row, const float* acc) {
    if (lane_id() == 0) pk_put((void*)s.out, (uint32_t)e, __float_as_uint(acc[0]), tag);
  });
  prof_mark(env, 2);
}

// FX_OP_MOE_W13 over every worker: the shared slots' pair groups (2 pairs each) and the routed
// slots' pair groups are each split evenly over the workers; shared slots first, so their weights
// stream while the router logits are still on their way. With FX_F_ROUTER the stage also computes the router (row e on worker e, W_gate in `res`) and
// reads the logits back from its own packets. act8[slot][i] = bf16(silu(bf16(W13[e][i] h)) *
// bf16(W13[e][I + i] h)).
// w13_prime issues the loads that need nothing from the stage's inputs (each wave's first shared
// group, the router row, the norm weights); w13_main does the rest. The stage runs them back to
// back; a GEMV stage flagged FX_F_PAIR runs w13_prime of the next stage before its own work (run_pair).
template <class TileT>
struct W13Pre {
  TileT t0;          // the wave's first shared group
  Tile<1, 4> tr;     // the router row (worker e < E, wave 0)
  NormW nw;
};
// the worker's shared groups [a0, a1) and routed groups [b0, b1) (pair groups of 4 rows: p, I + p,
// p + 1, I + p + 1; PG = I / 2 per slot). The shared slots' nsh * PG groups and the routed slots'
// topk * PG groups are each split evenly over the workers, so every worker streams the same number
// of rows (within one group)
struct W13Split {
  int a0, a1, b0, b1;
};
__device__ __forceinline__ W13Split w13_split(const fx_stage& s, const FxEnv& env) {
  W13Split q;
  const int PG = s.n_rows >> 1;
  range_split(s.n_forced * PG, env.nworkers, env.worker, q.a0, q.a1);
  range_split(s.topk * PG, env.nworkers, env.worker, q.b0, q.b1);
  return q;
}
template <class TileT, class WT>
__device__ __forceinline__ void w13_prime(const fx_stage& s, const FxEnv& env, const WT& W, W13Pre<TileT>& p) {
  const int K = s.k, I = s.n_rows, E = s.aux_i0, PG = I >> 1;
  const W13Split q = w13_split(s, env);
  const size_t ex = (size_t)2 * I;
  auto rowA = [&](int g, int i) {
    const int a = q.a0 + g;
    const int e = E + a / PG;
    const int pp = 2 * (a % PG) + (i >> 1);
    return (int)(e * ex + ((i & 1) ? I + pp : pp));
  };
  gemv_prime(p.t0, W, K, q.a1 - q.a0, rowA);
  const bool rrow = (s.flags & FX_F_ROUTER) && env.worker < E;
  auto rowR = [&](int g, int i) { return env.worker; };
  if (rrow && wave_id() == 0) tile_load(p.tr, (const uint16_t*)s.res, K, 0, rowR);
  p.nw = K <= 8 * FX_THREADS ? norm_prefetch((const uint16_t*)s.w_norm, K) : NormW{};
}
template <class TileT, class WT>
__device__ __forceinline__ void w13_main(const fx_stage& s, FxEnv& env, const WT& W, W13Pre<TileT>& p) {
  float* xs = (float*)(env.lds + LDS_XS);
  float* red = (float*)(env.lds + LDS_RED);
  int* ids = (int*)(env.lds + LDS_MISC + 128);
  float* wts = (float*)(env.lds + LDS_MISC + 256);
  const int K = s.k, I = s.n_rows, E = s.aux_i0;
  const int topk = s.topk;
  const bool router = (s.flags & FX_F_ROUTER) != 0;
  const bool writer = env.worker == 0;
  float* lg = red + 256;
  const int PG = I >> 1;
  const W13Split q = w13_split(s, env);
  const int a0 = q.a0, b0 = q.b0;
  const int nA = q.a1 - q.a0, nB = q.b1 - q.b0;
  const size_t ex = (size_t)2 * I;   // rows per expert
  auto rowA = [&](int g, int i) {
    const int a = a0 + g;
    const int e = E + a / PG;
    const int pp = 2 * (a % PG) + (i >> 1);
    return (int)(e * ex + ((i & 1) ? I + pp : pp));
  };
  auto rowB = [&](int g, int i) {
    const int r = b0 + g;
    const int e = ids[r / PG];
    const int pp = 2 * (r % PG) + (i >> 1);
    return (int)(e * ex + ((i & 1) ? I + pp : pp));
  };
  TileT& t0 = p.t0;
  const bool rrow = router && env.worker < E;
  Tile<1, 4>& tr = p.tr;
  const NormW& nw = p.nw;
  poll_row(xs, (const void*)s.x, K, tag_in(s, env, 1), env.err);
  prof_mark(env, 1);
  rmsnorm_staged(xs, nw, (const uint16_t*)s.w_norm, K, s.eps, red);
  const uint32_t tag = tag_out(env);
  if (rrow && wave_id() == 0) {
    float acc[1];
    tile_dot(tr, xs, K, acc);
    if (lane_id() == 0) pk_put((void*)s.aux[0], (uint32_t)env.worker, __float_as_uint(acc[0]), tag);
  }
  if (s.aux[6] && writer) store_vec_sc1((void*)s.aux[6], xs, K);
  prof_mark(env, 4);
  void* act = (void*)s.out;
  const int half = I >> 1;
  // act values of the worker's groups: LDS [shared groups, then routed groups][2], published after
  // each stream; group a / r of a slot's PG groups is act packet slot * half + (a or r) % PG
  float* actl = (float*)(env.lds + LDS_RES);
  auto emit = [&](int base, int g, const float* acc) {
    float a[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const float gv = bf16r(acc[2 * q]);
      const float uv = bf16r(acc[2 * q + 1]);
      a[q] = silu_s(gv) * uv;
    }
    if (lane_id() == 0) {
      actl[2 * (base + g)] = a[0];
      actl[2 * (base + g) + 1] = a[1];
    }
  };
  gemv_pipe(t0, W, K, xs, nA, rowA, [&](int g, const int* row, const float* acc) { emit(0, g, acc); });
  prof_mark(env, 5);
  // routed slots: the top-k of the logits, on the last wave (groups g = wave, wave + 4, ..: it has
  // the fewest shared groups, so it polls the logits while the others finish theirs)
  if (wave_id() == FX_WAVES - 1) {
    prof_mark_wave(env, 7);
    poll_logits_wave(lg, (const void*)s.aux[0], E, router ? tag : tag_in(s, env, 0), env.err);
    prof_mark_wave(env, 6);
    float* probs = red + 512;
    route_slots_wave(lg, s, ids, wts, probs);
    if (writer) {
      // router outputs in numpy_ref.moe_router's layout: topk_w, routing, mask, logits, route_log, sel
      const int n_slots = s.n_slots, n_total = E + s.n_forced;
      const int lane = lane_id();
      const int row = env.step - (env.n_prompt - 1);
      for (int k = lane; k < n_slots; k += 64) {
        stcf((void*)s.aux[1], k, wts[k]);
        if (s.aux[7]) stc4((void*)s.aux[7], k * 4, (uint32_t)ids[k]);
        // route_log [prow][aux_i1][n_slots] at row step - (n_prompt - 1): the decode iterations,
        // as the reference logs them (route_log [32, 26, 8] at [step - 1023])
        if (s.aux[5] && s.layer >= 1 && row >= 0 && row < s.prow)
          stc4((void*)s.aux[5], (uint32_t)(((row * s.aux_i1) + (s.layer - 1)) * n_slots + k) * 4, (uint32_t)ids[k]);
      }
      for (int x = lane; x < n_total; x += 64) {
        int r = 0;
        for (int k = 0; k < n_slots; ++k)
          if (ids[k] == x) r = k + 1;
        stc4((void*)s.aux[2], x * 4, (uint32_t)r);
      }
      for (int x = lane; x <= n_total; x += 64) {
        int v = -1;
        if (x < n_slots) v = ids[x];
        if (x == n_total) v = n_slots;
        stc4((void*)s.aux[3], x * 4, (uint32_t)v);
      }
      for (int x = lane; x < E; x += 64) stcf((void*)s.aux[4], x, lg[x]);
    }
  }
  __syncthreads();
  if (fx_tid() < nA) {
    const int a = a0 + fx_tid();
    pk_put(act, (uint32_t)((topk + a / PG) * half + a % PG), pack2(actl[2 * fx_tid()], actl[2 * fx_tid() + 1]),
           tag);
  }
  // the routing stays in LDS for the expert-down stage that follows on this worker
  env.route_tag = router ? tag : tag_in(s, env, 0);
  // The routed groups are walked by whole waves up to a multiple of the wave count; one group left
  // over (the split gives every other worker 17 at V2-Lite's shapes) is split by rows, row w on wave
  // w, its loads requested ahead of the walk: the worker then ends a quarter tile after its
  // 16-group neighbours instead of a whole tile. Each row's dot is the same as in a 4-row tile.
  const int nrem = nB % FX_WAVES;
  const int nB4 = nrem == 1 && TileT::kRows == FX_WAVES ? nB - 1 : nB;
  float* remv = red + 896;   // the split group's 4 row values
  typename TileT::Row tq;
  auto rowQ = [&](int, int) { return rowB(nB4, wave_id()); };
  if (nB4 < nB) tile_load(tq, W, K, 0, rowQ);
  if constexpr (FX_W13_ROW2 && std::is_same<TileT, Tile<4, 4>>::value) {
    // bf16: the routed groups walked as tiles of one pair (gate p, up p; half of a group, 8 KiB per
    // wave) by the rolling walk: a worker's routed share is a short stream, which smaller tiles
    // with the next tile requested during the dot finish sooner. Pair g2 is half g2 & 1 of group
    // g2 >> 1; its act value is emit's for that half.
    auto rowB2 = [&](int g2, int i) { return rowB(g2 >> 1, ((g2 & 1) << 1) | i); };
    Tile<2, 4> u0;
    gemv_prime(u0, W, K, 2 * nB4, rowB2);
    gemv_pipe_roll(u0, W, K, [&](int) { return (const float*)xs; }, 2 * nB4, rowB2,
                   [&](int g2, const int* row, const float* acc) {
                     const float a = silu_s(bf16r(acc[0])) * bf16r(acc[1]);
                     if (lane_id() == 0) actl[2 * (nA + (g2 >> 1)) + (g2 & 1)] = a;
                   });
  } else {
    gemv_prime(t0, W, K, nB4, rowB);
    gemv_pipe(t0, W, K, xs, nB4, rowB, [&](int g, const int* row, const float* acc) { emit(nA, g, acc); });
  }
  if (nB4 < nB) {
    float acc[1];
    tile_dot(tq, xs, K, acc);
    if (lane_id() == 0) remv[wave_id()] = acc[0];
  }
  __syncthreads();
  if (fx_tid() < nB) {
    const int r = b0 + fx_tid();
    const int i = nA + fx_tid();
    if (fx_tid() == nB4) {
      // rows gate p, up p, gate p + 1, up p + 1 of the split group: emit's arithmetic
      float a[2];
#pragma unroll
      for (int q = 0; q < 2; ++q) a[q] = silu_s(bf16r(remv[2 * q])) * bf16r(remv[2 * q + 1]);
      actl[2 * i] = a[0];
      actl[2 * i + 1] = a[1];
    }
    pk_put(act, (uint32_t)((r / PG) * half + r % PG), pack2(actl[2 * i], actl[2 * i + 1]), tag);
  }
  prof_mark(env, 2);
}

// bf16 weights, or FP8 (kFp8, stages flagged FX_F_FP8: the codes [E + n_forced][2 I][K], then their
// per-row f32 scales)
template <bool kFp8>
__device__ __forceinline__ void op_moe_w13(const fx_stage& s, FxEnv& env) {
  if constexpr (kFp8) {
    const size_t rows = (size_t)(s.aux_i0 + s.n_forced) * 2 * s.n_rows;
    const Fp8W W{(const uint8_t*)s.w, (const float*)((const uint8_t*)s.w + rows * (size_t)s.k)};
    W13Pre<TileQ<4, 2>> p;
    w13_prime(s, env, W, p);
    w13_main(s, env, W, p);
  } else {
    const uint16_t* W = (const uint16_t*)s.w;
    W13Pre<Tile<4, 4>> p;
    w13_prime(s, env, W, p);
    w13_main(s, env, W, p);
  }
}

// FX_OP_MOE_W2 with the combine: worker w owns output rows [r0, r0 + 8) of every slot; group g is
// 4 rows of one slot. The shared slots' activations (finished first by the gate|up stage) are
// awaited and consumed first, then the routed ones; x_new[n] = bf16(x[n] + sum_s out8[s][n] * w_s),
// multiply then add, in slot order (harness/numpy_ref.py:316-321).
#define W2_ROWS 8
template <class TileT, class WT>
__device__ __forceinline__ void op_moe_w2_t(const fx_stage& s, FxEnv& env, const WT& W) {
  float* xs = (float*)(env.lds + LDS_XS);        // act8 [8][I]
  float* red = (float*)(env.lds + LDS_RED);
  int* ids = (int*)(env.lds + LDS_MISC + 128);
  float* wts = (float*)(env.lds + LDS_MISC + 256);
  float* rres = (float*)(env.lds + LDS_RES);     // x rows [8], then out8 [8 slots][8 rows] at +16
  const int I = s.k, H = s.n_rows;
  const int nslots = FX_SLOTS;
  const int nsh = s.n_forced, topk = s.topk;
  const int E = s.aux_i0;
  int c0, c1;
  range_split(H / W2_ROWS, env.nworkers, env.worker, c0, c1);
  const int r0 = c0 * W2_ROWS;
  const int nrow = (c1 - c0) * W2_ROWS;          // 8 (H = 2048, 256 workers)
  const int quads = nrow >> 2;
  const int nA = nsh * quads, nB = topk * quads;
  auto rowA = [&](int g, int i) { return (E + g / quads) * H + r0 + (g % quads) * 4 + i; };
  auto rowB = [&](int g, int i) { return ids[g / quads] * H + r0 + (g % quads) * 4 + i; };
  TileT t0;
  gemv_prime(t0, W, I, nA, rowA);
  // the usual split (2 quads per worker: one shared and three routed groups per wave): the routed
  // tiles of the wave are requested as soon as the routing is known (the third once the shared
  // tile is consumed), before the routed activations are awaited, so the down weights stream
  // while the slowest gate|up worker finishes
  const bool whole = nA == FX_WAVES && nB == 3 * FX_WAVES;
  // the routing: left in LDS by the gate|up stage of this layer on this worker (persistent kernel),
  // else from the logits
  const bool routed_here = env.route_tag == tag_in(s, env, 1);
  if (!routed_here && wave_id() == 0) {
    float* lg = red + 256;
    poll_logits_wave(lg, (const void*)s.aux[0], E, tag_in(s, env, 1), env.err);
    route_slots_wave(lg, s, ids, wts, nullptr);
  }
  TileT tr0, tr1;
  if (whole) {
    if (!routed_here) __syncthreads();   // ids
    const int w = wave_id();
    tile_load(tr0, W, I, w, rowB);
    tile_load(tr1, W, I, w + FX_WAVES, rowB);
  }
  if (fx_tid() < (nrow >> 2)) {
    u32x4 v[1];
    pk_wait_pairs<1>((const void*)s.res, (r0 >> 2) + fx_tid(), 0, (r0 + nrow) >> 2, tag_in(s, env, 2), env.err, v);
    const int i = 4 * fx_tid();
    rres[i + 0] = bf_lo(v[0].x);
    rres[i + 1] = bf_hi(v[0].x);
    rres[i + 2] = bf_lo(v[0].z);
    rres[i + 3] = bf_hi(v[0].z);
  }
  // shared slots' activations (slots topk .. topk + nsh - 1 of act8)
  const uint32_t tact = tag_in(s, env, 0);
  poll_row(xs + topk * I, (const uint8_t*)s.x + (size_t)topk * I * 4, nsh * I, tact, env.err);
  prof_mark(env, 1);
  __syncthreads();
  float* o8 = rres + 16;
  auto emit = [&](int slot_base, int g, const float* acc) {
    if (lane_id() == 0) {
      const int sl = slot_base + g / quads;
#pragma unroll
      for (int i = 0; i < 4; ++i) o8[sl * W2_ROWS + (g % quads) * 4 + i] = bf16r(acc[i]);
    }
  };
  if (whole) {
    float acc[4];
    const int g = wave_id();
    tile_dot(t0, xs + (topk + g / quads) * I, I, acc);
    emit(topk, g, acc);
    // the third routed tile reuses the shared tile's registers
    tile_load(t0, W, I, g + 2 * FX_WAVES, rowB);
    prof_mark(env, 4);
    poll_row(xs, (const void*)s.x, topk * I, tact, env.err);
    __syncthreads();
    prof_mark(env, 5);
    tile_dot(tr0, xs + (g / quads) * I, I, acc);
    emit(0, g, acc);
    tile_dot(tr1, xs + ((g + FX_WAVES) / quads) * I, I, acc);
    emit(0, g + FX_WAVES, acc);
    tile_dot(t0, xs + ((g + 2 * FX_WAVES) / quads) * I, I, acc);
    emit(0, g + 2 * FX_WAVES, acc);
  } else {
    gemv_pipe_x(t0, W, I, [&](int g) { return (const float*)(xs + (topk + g / quads) * I); }, nA, rowA,
                [&](int g, const int* row, const float* acc) { emit(topk, g, acc); });
    prof_mark(env, 4);
    // routed slots
    gemv_prime(t0, W, I, nB, rowB);
    poll_row(xs, (const void*)s.x, topk * I, tact, env.err);
    __syncthreads();
    prof_mark(env, 5);
    gemv_pipe_x(t0, W, I, [&](int g) { return (const float*)(xs + (g / quads) * I); }, nB, rowB,
                [&](int g, const int* row, const float* acc) { emit(0, g, acc); });
  }
  __syncthreads();
  if (fx_tid() < nrow) {
    const int r = fx_tid();
    float acc = rres[r];
    for (int sl = 0; sl < nslots; ++sl) {
      const float t = o8[sl * W2_ROWS + r] * wts[sl];
      acc = acc + t;
    }
    red[r] = bf16r(acc);
    if (s.aux[1])
      for (int sl = 0; sl < nslots; ++sl) stc2((void*)s.aux[1], (uint32_t)(sl * H + r0 + r) * 2, f2bf(o8[sl * W2_ROWS + r]));
  }
  __syncthreads();
  if (fx_tid() < (nrow >> 1))
    pk_put((void*)s.out, (uint32_t)((r0 >> 1) + fx_tid()), pack2(red[2 * fx_tid()], red[2 * fx_tid() + 1]),
           tag_out(env));
  prof_mark(env, 2);
}

// bf16 weights, or FP8 (kFp8, stages flagged FX_F_FP8: the codes [E + n_forced][H][I], then their
// per-row f32 scales)
template <bool kFp8>
__device__ __forceinline__ void op_moe_w2(const fx_stage& s, FxEnv& env) {
  if constexpr (kFp8) {
    const size_t rows = (size_t)(s.aux_i0 + s.n_forced) * s.n_rows;
    const Fp8W W{(const uint8_t*)s.w, (const float*)((const uint8_t*)s.w + rows * (size_t)s.k)};
    op_moe_w2_t<TileQ<4, 2>>(s, env, W);
  } else {
    op_moe_w2_t<Tile<4, 3>>(s, env, (const uint16_t*)s.w);
  }
}

// FX_OP_ARGMAX: tokens[step + 1] (the reduce of argmax_partial; fleet/graph_plan.py:598-602)
__device__ __forceinline__ void op_argmax(const fx_stage& s, FxEnv& env) {
  if (env.worker != 0 || wave_id() != 0) return;
  if (env.step + 1 < env.n_prompt) return;
  const int64_t tok = argmax_reduce((const void*)s.aux[3], env.nworkers, tag_in(s, env, 0), env.err);
  if (lane_id() == 0) {
    u32x2 t;
    t.x = (uint32_t)tok;
    t.y = (uint32_t)((uint64_t)tok >> 32);
    stc8(env.tokens, (uint32_t)(env.step + 1) * 8, t);
  }
}
