// Per-workgroup state, packet tags and the LDS layout shared by the operators and the runtime.
#pragma once
#include "fx_device.h"
#include "../../include/fleet_mi355x.h"

// 256 workers, one per CU: worker w runs on XCD w % 8 and is rank w / 8 of the 32 of its XCD.
#define FX_WORKERS 256
#define FX_XWORKERS 32

struct FxEnv {
  int worker, nworkers;   // global worker index and count
  int xcd, xrank, xworkers;
  int step, iter;
  int n_prompt;
  uint32_t tbase;         // tag base of this iteration: epoch0 + iter * n_stages
  int sidx;               // index of the running stage in the table
  int64_t token;          // token of this iteration (set by the embed prologue; -1 before)
  int64_t* tokens;
  uint32_t* err;          // the run's error flag
  uint64_t* pst;          // profile stamps of this stage and worker, or null
  char* lds;
  uint32_t route_tag;     // tag of the router logits whose routing (expert ids, weights) is in LDS, 0: none
};

// tag that packet input k of stage s carries / that this stage's outputs carry
__device__ __forceinline__ uint32_t tag_in(const fx_stage& s, const FxEnv& e, int k) {
  return e.tbase + (uint32_t)(s.src[k] + 1);
}
__device__ __forceinline__ uint32_t tag_out(const FxEnv& e) { return e.tbase + (uint32_t)(e.sidx + 1); }

// profile stamp `slot` of the running stage (thread 0 only)
__device__ __forceinline__ void prof_mark(const FxEnv& e, int slot) {
  if (e.pst && fx_tid() == 0) e.pst[slot] = __builtin_amdgcn_s_memrealtime();
}
// the same from the calling wave's lane 0 (a stamp taken on a wave other than wave 0)
__device__ __forceinline__ void prof_mark_wave(const FxEnv& e, int slot) {
  if (e.pst && lane_id() == 0) e.pst[slot] = __builtin_amdgcn_s_memrealtime();
}

// LDS layout (bytes)
#define LDS_XS 0                         // f32 [11264]  GEMV input row
#define LDS_XS_FLOATS 11264
#define LDS_RED (45056)                  // f32 [1024]   reductions / small tables
#define LDS_MISC (LDS_RED + 4096)        // scalars: token, expert, slot weights
#define LDS_RES (LDS_MISC + 512)         // f32 [128]    residual / output values of the worker's rows
#define LDS_TILE (LDS_MISC + 1024)       // attention tile / merge tables (<= 37.5 KiB)
#define LDS_STAGE (FX_LDS_BYTES - 256)   // end of the operators' LDS (the last 256 B unused)
// the persistent kernel's task table (every stage, then the epilogue) past the operators' LDS
#define FX_TABLE_MAX 300
#define FX_LDS_TOTAL (FX_LDS_BYTES + FX_TABLE_MAX * 208)
#define FX_MAX_OUT_ROWS 128

__device__ __forceinline__ void range_split(int n, int parts, int i, int& lo, int& hi) {
  lo = (int)(((long long)n * i) / parts);
  hi = (int)(((long long)n * (i + 1)) / parts);
}
