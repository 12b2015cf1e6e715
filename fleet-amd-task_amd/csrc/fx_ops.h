// Operators of the decode task table (one fx_stage each), as device functions executed by one
// worker workgroup (256 threads) for its share of the stage. The same code runs inside the
// persistent kernel and in the per-stage launcher of the kernel suite.
//   fx_gemv.h  GEMV (qkva, o_proj, dense down, LM head + argmax), dense gate|up + SiLU
//   fx_moe.h   router, expert gate|up + SiLU, expert down + combine, argmax reduce
//   fx_mla.h   MLA prep (norm, RoPE, cache append, W_uk absorb), split-KV attend, LSE merge + W_uv
//   fx_attn.h  split-KV attend on the matrix cores (FX_F_MFMA), and with its merge on one XCD (FX_F_XCD)
#pragma once
#include "fx_attn.h"
#include "fx_moe.h"

// kFp8: the kernel variant whose expert stages read FP8 weights (a plan's expert stages are all
// bf16 or all FP8; the launch picks the variant, so each kernel holds one expert path)
template <bool kFp8 = false>
__device__ __forceinline__ void run_stage(const fx_stage& s, FxEnv& env) {
  switch (s.op) {
    case FX_OP_GEMV:
      if constexpr (kFp8) {
        if (s.flags & FX_F_FP8) { op_gemv_fp8(s, env); break; }
      }
      op_gemv(s, env);
      break;
    case FX_OP_MLA_PREP: op_mla_prep(s, env); break;
    case FX_OP_MLA_ATTEND:
      // FX_F_XCD: the attention runs inside the merge stage that follows
      if (s.flags & FX_F_XCD) break;
      if (s.flags & FX_F_MFMA) op_mla_attend_mfma(s, env);
      else op_mla_attend(s, env);
      break;
    case FX_OP_MLA_MERGE_UV:
      if (s.flags & FX_F_XCD) op_mla_attend_merge_xcd(s, env);
      else op_mla_merge_uv(s, env);
      break;
    case FX_OP_MOE_ROUTER: op_moe_router(s, env); break;
    case FX_OP_MOE_W13: op_moe_w13<kFp8>(s, env); break;
    case FX_OP_MOE_W2: op_moe_w2<kFp8>(s, env); break;
    case FX_OP_DENSE_GU: op_dense_gu(s, env); break;
    case FX_OP_ARGMAX: op_argmax(s, env); break;
    default: break;
  }
}

// A GEMV stage flagged FX_F_PAIR and the MOE_W13 stage after it as one operator: the expert
// stage's first weight loads (w13_prime: its shared groups, the router row, the norm weights) are
// issued before the GEMV's own, so they stream while the GEMV waits for its input (o_proj waits for
// the attention chain, with the HBM otherwise idle) and the expert stage starts with them in
// registers and no weight loads queued ahead of its polls. `pst_next`: the second stage's profile
// stamps; env.sidx / env.pst are switched to the second stage for its part.
template <bool kFp8, class TileT, class WT>
__device__ __forceinline__ void run_pair_w(const fx_stage& g, const fx_stage& m, FxEnv& env, uint64_t* pst_next,
                                           const WT& W) {
  W13Pre<TileT> p;
  w13_prime(m, env, W, p);
  run_stage<kFp8>(g, env);
  prof_mark(env, 3);
  env.sidx = env.sidx + 1;
  env.pst = pst_next;
  prof_mark(env, 0);
  w13_main(m, env, W, p);
}
template <bool kFp8>
__device__ __forceinline__ void run_pair(const fx_stage& g, const fx_stage& m, FxEnv& env, uint64_t* pst_next) {
  if constexpr (kFp8) {
    const size_t rows = (size_t)(m.aux_i0 + m.n_forced) * 2 * m.n_rows;
    const Fp8W W{(const uint8_t*)m.w, (const float*)((const uint8_t*)m.w + rows * (size_t)m.k)};
    run_pair_w<kFp8, TileQ<4, 2>>(g, m, env, pst_next, W);
  } else {
    run_pair_w<kFp8, Tile<4, 4>>(g, m, env, pst_next, (const uint16_t*)m.w);
  }
}
