// Per-workgroup state, sync-area and LDS layouts shared by the operators and the runtime.
#pragma once
#include "fx_device.h"
#include "../../include/fleet_mi355x.h"

// Work split: 248 workers = 256 CUs minus one scheduler per XCD; worker w sits on XCD w % 8 and is
// rank w / 8 of the 31 workers of its XCD.
struct FxEnv {
  int worker, nworkers;   // global worker index and count
  int xcd, xrank, xworkers;
  int step, iter;
  int n_prompt;
  int moe_e;              // expert of this XCD's slot chosen by the last MOE_W13 stage (-1: unknown)
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

// LDS layout (bytes)
#define LDS_XS 0                         // f32 [11264]  GEMV input row
#define LDS_RED (45056)                  // f32 [1024]   reductions / small tables
#define LDS_MISC (LDS_RED + 4096)        // scalars: token, expert, slot weights, residual rows
#define LDS_RES (LDS_MISC + 512)         // f32 [64]     residual values of the worker's rows
#define LDS_TILE (LDS_MISC + 1024)       // attention tile / merge tables (<= 37.5 KiB)
#define LDS_STAGE (FX_LDS_BYTES - 256)   // the current fx_stage (persistent kernel)
#define FX_MAX_RES_ROWS 64

__device__ __forceinline__ void range_split(int n, int parts, int i, int& lo, int& hi) {
  lo = (int)(((long long)n * i) / parts);
  hi = (int)(((long long)n * (i + 1)) / parts);
}
