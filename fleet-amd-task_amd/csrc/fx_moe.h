// MoE operators: router, expert gate|up + SiLU, expert down, combine; the argmax reduce.
// harness/numpy_ref.py:205-292, 316-321; the reference's moe_router_mi300.cuh:115-354,
// gang_moe_w13_gemv_mi300.cuh:101-219, gang_moe_w2_silu_mi300.cuh and moe_mul_sum_add.
// Slot s of the 8 (top-6 routed, then the two shared experts E, E+1 at weight 1.0) runs on XCD s.
#pragma once
#include "fx_gemv.h"

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

// FX_OP_MOE_ROUTER: per XCD, h = rmsnorm(x_res), logits rows e = rank, rank + 31, ... of the XCD's
// workers into logits_x[xcd] (each routed XCD computes its own copy).
__device__ __forceinline__ void op_moe_router(const fx_stage& s, FxEnv& env) {
  if (env.xcd >= s.topk) return;   // forced-expert slots need no routing
  float* xs = (float*)(env.lds + LDS_XS);
  float* red = (float*)(env.lds + LDS_RED);
  const int K = s.k, E = s.n_rows;
  const uint16_t* W = (const uint16_t*)s.w;
  const int per = (E + env.xworkers - 1) / env.xworkers;
  auto rowof = [&](int g, int i) { const int r = env.xrank + i * env.xworkers; return (i < per && r < E) ? r : -1; };
  Tile<4, 4> t0;
  gemv_prime(t0, W, K, 1, rowof);
  load_vec_sc1(xs, (const void*)s.x, K);
  rmsnorm_inplace(xs, (const uint16_t*)s.w_norm, K, s.eps, red);
  void* lx = (void*)s.out;
  gemv_pipe(t0, W, K, xs, 1, rowof, [&](int g, const int* row, const float* acc) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (row[i] >= 0 && lane_id() == i) stcf(lx, env.xcd * E + row[i], acc[i]);
  });
}

// FX_OP_MOE_W13: per XCD, slot = XCD; the slot's expert from the XCD's router logits, then
// act8[slot][i] = bf16(silu(bf16(W13[e][i] h)) * bf16(W13[e][I + i] h)) over the XCD's workers.
__device__ __forceinline__ void op_moe_w13(const fx_stage& s, FxEnv& env) {
  float* xs = (float*)(env.lds + LDS_XS);
  float* red = (float*)(env.lds + LDS_RED);
  int* misc = (int*)(env.lds + LDS_MISC);
  int* ids = (int*)(env.lds + LDS_MISC + 128);
  float* wts = (float*)(env.lds + LDS_MISC + 256);
  const int K = s.k, I = s.n_rows, E = s.aux_i0;
  const int slot = env.xcd;
  const int topk = s.topk;
  const bool routed = slot < topk;
  const bool writer = env.xcd == 0 && env.xrank == 0;
  float* lg = red + 256;
  // the input row and this XCD's logits are independent loads: issue both first
  if (routed || writer)
    for (int i = threadIdx.x; i < E; i += FX_THREADS) lg[i] = ldcf((const void*)s.aux[0], env.xcd * E + i);
  load_vec_sc1(xs, (const void*)s.x, K);
  __syncthreads();
  if (wave_id() == 0) {
    int e = E + (slot - topk);
    if (routed || writer) {
      float* probs = red + 512;
      softmax_topk_wave(lg, E, topk, s.scaling, ids, wts, probs);
      if (routed) e = ids[slot];
      if (writer) {
        // router outputs in numpy_ref.moe_router's layout: topk_w, routing, mask, logits, route_log
        const int n_slots = s.n_slots, n_total = E + s.n_forced;
        const int lane = lane_id();
        const int row = env.step - (env.n_prompt - 1);
        for (int k = lane; k < n_slots; k += 64) {
          const int id = k < topk ? ids[k] : E + (k - topk);
          stcf((void*)s.aux[1], k, k < topk ? wts[k] : 1.0f);
          // route_log [prow][aux_i1][n_slots] at row step - (n_prompt - 1): the decode iterations,
          // as the reference logs them (route_log [32, 26, 8] at [step - 1023])
          if (s.aux[5] && s.layer >= 1 && row >= 0 && row < s.prow)
            stc4((void*)s.aux[5], (uint32_t)(((row * s.aux_i1) + (s.layer - 1)) * n_slots + k) * 4, (uint32_t)id);
        }
        for (int x = lane; x < n_total; x += 64) {
          int r = 0;
          for (int k = 0; k < n_slots; ++k) {
            const int id = k < topk ? ids[k] : E + (k - topk);
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
    }
    if (lane_id() == 0) misc[0] = e;
    if (env.xrank == 0 && lane_id() == 0) stc4((void*)s.aux[7], slot * 4, (uint32_t)e);
  }
  __syncthreads();
  const int e = misc[0];
  env.moe_e = e;
  const uint16_t* W = (const uint16_t*)s.w + (size_t)e * 2 * I * K;
  PairRows rowof;
  range_split(I, env.xworkers, env.xrank, rowof.p0, rowof.p1);
  rowof.I = I;
  const int ngroups = (rowof.p1 - rowof.p0 + 1) / 2;
  Tile<4, 4> t0;
  gemv_prime(t0, W, K, ngroups, rowof);
  rmsnorm_inplace(xs, (const uint16_t*)s.w_norm, K, s.eps, red);
  if (s.aux[6] && writer) store_vec_sc1((void*)s.aux[6], xs, K);
  void* act = (void*)s.out;
  const uint32_t off = (uint32_t)slot * I * 2;
  gemv_pipe(t0, W, K, xs, ngroups, rowof, [&](int g, const int* row, const float* acc) { gate_up_emit(act, off, row, acc); });
}

// FX_OP_MOE_W2: per XCD, out8[slot] = bf16(W2[e] act8[slot]). Inside the persistent kernel the
// expert is the one this workgroup's W13 stage chose; a standalone launch reads it from sel.
__device__ __forceinline__ void op_moe_w2(const fx_stage& s, FxEnv& env) {
  float* xs = (float*)(env.lds + LDS_XS);
  int* misc = (int*)(env.lds + LDS_MISC);
  const int I = s.k, H = s.n_rows;
  const int slot = env.xcd;
  int e = env.moe_e;
  if (e < 0) {
    if (threadIdx.x == 0) misc[0] = (int)ldc4((const void*)s.aux[7], slot * 4);
    __syncthreads();
    e = misc[0];
  }
  const uint16_t* W = (const uint16_t*)s.w + (size_t)e * H * I;
  int r0, r1;
  range_split(H, env.xworkers, env.xrank, r0, r1);
  const int ngroups = (r1 - r0 + 3) / 4;
  auto rowof = [&](int g, int i) { const int r = r0 + g * 4 + i; return r < r1 ? r : -1; };
  Tile<4, 3> t0;
  gemv_prime(t0, W, I, ngroups, rowof);
  load_vec_sc1(xs, (const uint8_t*)s.x + (size_t)slot * I * 2, I);
  __syncthreads();
  void* out = (void*)s.out;
  gemv_pipe(t0, W, I, xs, ngroups, rowof, [&](int g, const int* row, const float* acc) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (row[i] >= 0 && lane_id() == i) stc2(out, (uint32_t)(slot * H + row[i]) * 2, f2bf(acc[i]));
  });
}

// FX_OP_MOE_COMBINE (standalone form; inside the decode it is the next GEMV's input prologue)
__device__ __forceinline__ void op_moe_combine(const fx_stage& s, FxEnv& env) {
  const int H = s.n_rows;
  int c0, c1;
  range_split(H / 8, env.nworkers, env.worker, c0, c1);
  float* w = (float*)(env.lds + LDS_MISC + 384);
  load_slot_weights(w, (const void*)s.aux[1]);
  for (int c = c0 + (int)threadIdx.x; c < c1; c += FX_THREADS) {
    const int i = c * 8;
    float a[8];
    combine_chunk((const void*)s.x, (const void*)s.aux[0], w, H, i, a);
    u32x4 r;
    r.x = pack2(a[0], a[1]);
    r.y = pack2(a[2], a[3]);
    r.z = pack2(a[4], a[5]);
    r.w = pack2(a[6], a[7]);
    stc16((void*)s.out, (uint32_t)i * 2, r);
  }
}

// FX_OP_ARGMAX: tokens[step + 1] (the reduce of argmax_partial; fleet/graph_plan.py:598-602)
__device__ __forceinline__ void op_argmax(const fx_stage& s, FxEnv& env) {
  if (env.worker != 0 || wave_id() != 0) return;
  if (env.step + 1 < env.n_prompt) return;
  const int64_t tok = argmax_reduce((const void*)s.aux[3], env.nworkers);
  if (lane_id() == 0) {
    u32x2 t;
    t.x = (uint32_t)tok;
    t.y = (uint32_t)((uint64_t)tok >> 32);
    stc8(env.tokens, (uint32_t)(env.step + 1) * 8, t);
  }
}
