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
