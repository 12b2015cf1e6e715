// Persistent decode runtime for gfx950 (MI355X) and the C ABI of include/fleet_mi355x.h.
//
// One cooperative launch of 256 workgroups, one per CU (the 96 KiB of dynamic LDS each admits one
// per CU), with blockIdx b on XCD b % 8 (checked at fx_create). Every workgroup is a worker: it
// walks the task table, iteration by iteration, and runs its share of each stage (fx_ops.h). There
// is no barrier between stages: each stage publishes its outputs as tagged packets
// (fleet_mi355x.h, "dataflow") and each consumer polls only the packets it reads, after issuing its
// own weight loads, so a stage starts as soon as its inputs exist and weight streaming overlaps the
// wait. Values that are not packets (cache rows, attention partials) are stored with the sc1
// policy and completed (s_waitcnt) before the packet that announces them. No counter is shared by
// two writers and no cache-maintenance instruction is issued.
//
// Replaces the fork runtime's prepare / scheduler / worker kernels and event counters
// (docs/fleet/03-runtime.md:125-313, fleet/patches/sched_xcd.patch) with a static task table.
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstring>
#include <cstdlib>
#include <string>
#include <vector>

#include "fx_ops.h"
#include "fx_prefill.h"

#include <rocblas/rocblas.h>

#define FX_BLOCKS 256
static_assert(sizeof(fx_stage) == 208, "fx_stage layout is part of the ABI (fleet/runtime.py FxStage)");
static_assert(FX_BLOCKS == FX_WORKERS, "one worker per CU");
#define FX_ERR_WORDS 64

struct FxRunArgs {
  const fx_stage* stages;
  int n_stages;
  const fx_stage* epi;
  int n_epi;
  int iters, step0, n_prompt;
  int64_t* tokens;
  uint32_t* err;
  uint64_t* timing;
  uint64_t* prof;      // [n_stages][256][FX_PROF_SLOTS] stamps of iteration prof_iter, or null
  int prof_iter;
  uint32_t epoch0;
};

__device__ __forceinline__ void env_init(FxEnv& env, char* lds, int64_t* tokens, uint32_t* err, int n_prompt) {
  const int b = blockIdx.x;
  env.worker = b;
  env.nworkers = FX_WORKERS;
  env.xcd = b & 7;
  env.xrank = b >> 3;
  env.xworkers = FX_XWORKERS;
  env.n_prompt = n_prompt;
  env.tokens = tokens;
  env.err = err;
  env.lds = lds;
  env.pst = nullptr;
  env.token = -1;
  env.route_tag = 0;
}

template <bool kFp8>
__device__ __forceinline__ void persistent_body(const FxRunArgs& a) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  const int b = blockIdx.x;
  FxEnv env;
  env_init(env, lds, a.tokens, a.err, a.n_prompt);
  // the task table (stages, then the epilogue) is copied into LDS once per launch: a stage starts
  // with one barrier (the operators reuse the same LDS regions) and reads its descriptor from LDS
  fx_stage* table = (fx_stage*)(lds + FX_LDS_BYTES);
  {
    const int w0 = a.n_stages * (int)(sizeof(fx_stage) / 16), w1 = a.n_epi * (int)(sizeof(fx_stage) / 16);
    u32x4* dst = (u32x4*)table;
    for (int i = threadIdx.x; i < w0; i += FX_THREADS) dst[i] = ld16((const u32x4*)a.stages + i);
    for (int i = threadIdx.x; i < w1; i += FX_THREADS) dst[w0 + i] = ld16((const u32x4*)a.epi + i);
  }
  for (int it = 0; it < a.iters; ++it) {
    env.iter = it;
    env.step = a.step0 + it;
    env.tbase = a.epoch0 + (uint32_t)(it * a.n_stages);
    env.token = -1;
    if (b == 0 && threadIdx.x == 0 && a.timing) a.timing[it] = __builtin_amdgcn_s_memrealtime();
    const bool prof = a.prof && it == a.prof_iter;
    for (int s = 0; s < a.n_stages; ++s) {
      __syncthreads();
      const fx_stage* sst = table + s;
      if ((sst->flags & FX_F_HEAD) && (env.step + 1 < env.n_prompt)) continue;
      env.sidx = s;
      env.pst = prof ? a.prof + ((size_t)s * FX_BLOCKS + b) * FX_PROF_SLOTS : nullptr;
      prof_mark(env, 0);
      if (sst->flags & FX_F_PAIR) {
        // this GEMV and the expert gate|up stage after it as one operator (fx_load_plan checked the
        // pair): the second stage's profile stamps and index are its own
        run_pair<kFp8>(*sst, table[s + 1], env,
                       prof ? a.prof + ((size_t)(s + 1) * FX_BLOCKS + b) * FX_PROF_SLOTS : nullptr);
        ++s;
      } else {
        run_stage<kFp8>(*sst, env);
      }
      if (prof) {
        __syncthreads();
        prof_mark(env, 3);
      }
    }
  }
  env.pst = nullptr;
  env.iter = a.iters;
  env.step = a.step0 + a.iters - 1;
  env.tbase = a.epoch0 + (uint32_t)(a.iters * a.n_stages);
  for (int s = 0; s < a.n_epi; ++s) {
    __syncthreads();
    env.sidx = a.n_stages + s;
    run_stage<kFp8>(table[a.n_stages + s], env);
  }
  if (b == 0 && threadIdx.x == 0 && a.timing) a.timing[a.iters] = __builtin_amdgcn_s_memrealtime();
}

// The decode launch (iterations that end in the LM head + argmax) and the prefill launch (prompt
// positions only: the head stages are skipped) run the same body; they are two symbols so that a
// kernel trace attributes prefill and decode time separately.
__global__ void __launch_bounds__(FX_THREADS) fx_persistent(FxRunArgs a) { persistent_body<false>(a); }
__global__ void __launch_bounds__(FX_THREADS) fx_prefill(FxRunArgs a) { persistent_body<false>(a); }
// the same with FP8 expert weights (plans whose expert stages carry FX_F_FP8)
__global__ void __launch_bounds__(FX_THREADS) fx_persistent_fp8(FxRunArgs a) { persistent_body<true>(a); }
__global__ void __launch_bounds__(FX_THREADS) fx_prefill_fp8(FxRunArgs a) { persistent_body<true>(a); }

// one stage as a standalone launch (kernel suite): same work split; packet inputs carry
// tbase + src[k] + 1, outputs tbase + sidx + 1
__global__ void __launch_bounds__(FX_THREADS) fx_stage_kernel(fx_stage st, int step, int n_prompt, uint32_t tbase, int sidx,
                                                            int64_t* tokens, uint32_t* err) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  FxEnv env;
  env_init(env, lds, tokens, err, n_prompt);
  env.iter = 0;
  env.step = step;
  env.tbase = tbase;
  env.sidx = sidx;
  if (tokens) env.token = tokens[step];
  run_stage(st, env);
}

__global__ void fx_xcc_map(uint32_t* out) {
  extern __shared__ char lds[];
  lds[threadIdx.x] = 0;
  if (threadIdx.x == 0) out[blockIdx.x] = xcc_id();
}

// ------------------------------------------------------------------------------------------------
// seeded generator: Philox4x32-10 (Salmon et al., SC'11) + Box-Muller with the spec's log and a
// polynomial sin/cos on the quadrant-reduced angle; the CPU oracle implements the same sequence.

__device__ __forceinline__ void philox(uint64_t seed, uint64_t block, uint32_t stream, uint32_t out[4]) {
  uint32_t c0 = (uint32_t)block, c1 = (uint32_t)(block >> 32), c2 = stream, c3 = 0x5EEDu;
  uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    uint64_t p0 = (uint64_t)0xD2511F53u * c0, p1 = (uint64_t)0xCD9E8D57u * c2;
    uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0;
    uint32_t n1 = (uint32_t)p1;
    uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
    uint32_t n3 = (uint32_t)p0;
    c0 = n0; c1 = n1; c2 = n2; c3 = n3;
    if (r < 9) { k0 += 0x9E3779B9u; k1 += 0xBB67AE85u; }
  }
  out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

__device__ __forceinline__ void sincos_quarter(float f, float* s, float* c) {
  const float HALF_PI = 1.57079637f;
  float t = f * HALF_PI;
  float z = t * t;
  float ps = -2.5052108e-8f;
  ps = ps * z + 2.7557319e-6f;
  ps = ps * z + -1.9841270e-4f;
  ps = ps * z + 8.3333333e-3f;
  ps = ps * z + -1.6666667e-1f;
  ps = ps * z + 1.0f;
  *s = ps * t;
  float pc = 2.0876757e-9f;
  pc = pc * z + -2.7557319e-7f;
  pc = pc * z + 2.4801587e-5f;
  pc = pc * z + -1.3888889e-3f;
  pc = pc * z + 4.1666668e-2f;
  pc = pc * z + -0.5f;
  pc = pc * z + 1.0f;
  *c = pc;
}

__device__ __forceinline__ void box_muller(uint32_t a, uint32_t b, float* z0, float* z1) {
  const float INV24 = 5.96046448e-08f;
  float u1 = (float)((a >> 8) + 1u) * INV24;
  float u2 = (float)(b >> 8) * INV24;
  float r = sqrtf(-2.0f * log_s(u1));
  float v = u2 * 4.0f;
  int q = (int)v;
  float f = v - (float)q;
  float s, c;
  sincos_quarter(f, &s, &c);
  float cs, sn;
  switch (q) {
    case 0: cs = c; sn = s; break;
    case 1: cs = -s; sn = c; break;
    case 2: cs = -c; sn = -s; break;
    default: cs = s; sn = -c; break;
  }
  *z0 = r * cs;
  *z1 = r * sn;
}

// contiguous source range [offset, offset + n): one thread per Philox block of 4 elements
__global__ void fx_gen_kernel(uint16_t* dst, uint64_t n, uint64_t seed, uint32_t stream, float scale, uint64_t offset) {
  const uint64_t first = offset & ~3ull;
  const uint64_t nblocks = (offset + n - first + 3) / 4;
  for (uint64_t bk = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; bk < nblocks; bk += (uint64_t)gridDim.x * blockDim.x) {
    const uint64_t base = first + bk * 4;
    uint32_t r[4];
    philox(seed, base >> 2, stream, r);
    float z[4];
    box_muller(r[0], r[1], &z[0], &z[1]);
    box_muller(r[2], r[3], &z[2], &z[3]);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint64_t i = base + k;
      if (i < offset || i >= offset + n) continue;
      dst[i - offset] = (uint16_t)f2bf(z[k] * scale);
    }
  }
}

// strided rows: one thread per element (each regenerates its Philox block)
__global__ void fx_gen2d_kernel(uint16_t* dst, uint64_t rows, uint64_t row_len, uint64_t dst_stride, uint64_t src_offset,
                                uint64_t src_stride, uint64_t seed, uint32_t stream, float scale) {
  const uint64_t total = rows * row_len;
  for (uint64_t e = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (uint64_t)gridDim.x * blockDim.x) {
    const uint64_t r = e / row_len, j = e % row_len;
    const uint64_t i = src_offset + r * src_stride + j;
    uint32_t w[4];
    philox(seed, i >> 2, stream, w);
    float z[4];
    box_muller(w[0], w[1], &z[0], &z[1]);
    box_muller(w[2], w[3], &z[2], &z[3]);
    dst[r * dst_stride + j] = (uint16_t)f2bf(z[i & 3] * scale);
  }
}

__global__ void fx_fill_kernel(uint16_t* dst, uint64_t n, uint16_t v) {
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x) dst[i] = v;
}

// ------------------------------------------------------------------------------------------------
// The allocation-free attention entry (fx_mla_attend_merge_noalloc): the split partials and the
// per-worker done packets live in this file-scope array, one copy per GPU, for the whole process.
// Host code never passes `scratch` itself to a kernel: fx_create resolves its device address on the
// context's device (hipGetSymbolAddress) and every launch uses that address.
#define FX_NOALLOC_PROW 516
#define FX_NOALLOC_PARTIAL_BYTES ((size_t)FX_NOALLOC_MAX_SPLITS * 16 * FX_NOALLOC_PROW * 4)
#define FX_NOALLOC_DONE_BYTES ((size_t)FX_WORKERS * 8)
static __device__ __align__(256) uint8_t scratch[FX_NOALLOC_PARTIAL_BYTES + FX_NOALLOC_DONE_BYTES];

// ------------------------------------------------------------------------------------------------
// C ABI

struct fx_ctx {
  int device;
  int cus;
  std::string err;
  uint32_t* err_flag = nullptr;
  uint64_t* timing = nullptr;
  int timing_cap = 0;
  int last_iters = 0;
  uint32_t epoch = 1;              // packet tags start above 0, the tag of zeroed packet buffers
  int64_t next_step = -1;          // step0 + iters of the last launch of the loaded plan (-1: none)
  fx_stage* d_stages = nullptr;
  int n_stages = 0;
  fx_stage* d_epi = nullptr;
  int n_epi = 0;
  std::vector<fx_stage> h_stages, h_epi;
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  hipEvent_t marks[FX_MAX_MARKS] = {};
  uint64_t* prof = nullptr;
  size_t prof_words = 0;
  int prof_iter = -1;
  rocblas_handle blas = nullptr;   // the prefill's GEMMs (created on first use)
  bool fp8 = false;                // the loaded plan's expert stages read FP8 weights
  uint8_t* scratch = nullptr;      // device address of this device's `scratch` array
};

static int fail(fx_ctx* c, int code, const std::string& msg) {
  if (c) c->err = msg;
  return code;
}
#define HIPCHK(c, x)                                                                    \
  do {                                                                                  \
    hipError_t e_ = (x);                                                                \
    if (e_ != hipSuccess) return fail((c), FX_E_HIP, std::string(#x) + ": " + hipGetErrorString(e_)); \
  } while (0)

extern "C" {

int fx_abi_version(void) { return FX_ABI_VERSION; }

const char* fx_last_error(fx_ctx* c) { return c ? c->err.c_str() : "no context"; }

int fx_create(int device, fx_ctx** out) {
  if (!out) return FX_E_ARG;
  *out = nullptr;
  fx_ctx* c = new fx_ctx();
  c->device = device;
  hipError_t e = hipSetDevice(device);
  if (e != hipSuccess) { delete c; return FX_E_HIP; }
  hipDeviceProp_t pr;
  if (hipGetDeviceProperties(&pr, device) != hipSuccess) { delete c; return FX_E_HIP; }
  c->cus = pr.multiProcessorCount;
  if (std::strncmp(pr.gcnArchName, "gfx950", 6) != 0 || pr.multiProcessorCount != FX_BLOCKS ||
      pr.sharedMemPerBlock < (size_t)FX_LDS_TOTAL) {
    *out = c;
    return fail(c, FX_E_DEVICE, std::string("expected a gfx950 with 256 CUs, got ") + pr.gcnArchName + " with " +
                                    std::to_string(pr.multiProcessorCount) + " CUs");
  }
  *out = c;
  HIPCHK(c, hipFuncSetAttribute((const void*)fx_persistent, hipFuncAttributeMaxDynamicSharedMemorySize, FX_LDS_TOTAL));
  HIPCHK(c, hipFuncSetAttribute((const void*)fx_prefill, hipFuncAttributeMaxDynamicSharedMemorySize, FX_LDS_TOTAL));
  HIPCHK(c, hipFuncSetAttribute((const void*)fx_persistent_fp8, hipFuncAttributeMaxDynamicSharedMemorySize, FX_LDS_TOTAL));
  HIPCHK(c, hipFuncSetAttribute((const void*)fx_prefill_fp8, hipFuncAttributeMaxDynamicSharedMemorySize, FX_LDS_TOTAL));
  HIPCHK(c, hipFuncSetAttribute((const void*)fx_stage_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, FX_LDS_BYTES));
  HIPCHK(c, hipFuncSetAttribute((const void*)fx_xcc_map, hipFuncAttributeMaxDynamicSharedMemorySize, FX_LDS_BYTES));
  HIPCHK(c, hipMalloc(&c->err_flag, FX_ERR_WORDS * 4));
  HIPCHK(c, hipMemset(c->err_flag, 0, FX_ERR_WORDS * 4));
  c->timing_cap = FX_MAX_ITERS + 1;
  HIPCHK(c, hipMalloc(&c->timing, sizeof(uint64_t) * c->timing_cap));
  HIPCHK(c, hipEventCreate(&c->ev0));
  HIPCHK(c, hipEventCreate(&c->ev1));
  // the allocation-free entry's scratch on this device (the context's device is current here)
  HIPCHK(c, hipGetSymbolAddress((void**)&c->scratch, HIP_SYMBOL(scratch)));
  // the work split assumes block b runs on XCD b % 8 (round-robin dispatch); verify it once
  uint32_t* d = nullptr;
  HIPCHK(c, hipMalloc(&d, FX_BLOCKS * 4));
  hipLaunchKernelGGL(fx_xcc_map, dim3(FX_BLOCKS), dim3(64), FX_LDS_BYTES, 0, d);
  HIPCHK(c, hipGetLastError());
  uint32_t h[FX_BLOCKS];
  HIPCHK(c, hipMemcpy(h, d, sizeof(h), hipMemcpyDeviceToHost));
  HIPCHK(c, hipFree(d));
  for (int b = 0; b < FX_BLOCKS; ++b)
    if (h[b] != (uint32_t)(b % 8))
      return fail(c, FX_E_DEVICE, "block " + std::to_string(b) + " ran on XCD " + std::to_string(h[b]));
  return FX_OK;
}

int fx_destroy(fx_ctx* c) {
  if (!c) return FX_OK;
  if (c->err_flag) (void)hipFree(c->err_flag);
  if (c->timing) (void)hipFree(c->timing);
  if (c->d_stages) (void)hipFree(c->d_stages);
  if (c->d_epi) (void)hipFree(c->d_epi);
  if (c->ev0) (void)hipEventDestroy(c->ev0);
  if (c->ev1) (void)hipEventDestroy(c->ev1);
  for (hipEvent_t e : c->marks)
    if (e) (void)hipEventDestroy(e);
  if (c->prof) (void)hipFree(c->prof);
  if (c->blas) (void)rocblas_destroy_handle(c->blas);
  delete c;
  return FX_OK;
}

int fx_device_info(fx_ctx* c, int32_t* cus, int32_t* xcds, int32_t* workers, int32_t* lds_bytes) {
  if (!c) return FX_E_ARG;
  if (cus) *cus = c->cus;
  if (xcds) *xcds = FX_XCDS;
  if (workers) *workers = FX_WORKERS;
  if (lds_bytes) *lds_bytes = FX_LDS_BYTES;
  return FX_OK;
}

int fx_malloc(fx_ctx* c, size_t n, void** p) {
  if (!p) return fail(c, FX_E_ARG, "null out pointer");
  HIPCHK(c, hipMalloc(p, n ? n : 16));
  return FX_OK;
}
int fx_free(fx_ctx* c, void* p) {
  HIPCHK(c, hipFree(p));
  return FX_OK;
}
int fx_memcpy_htod(fx_ctx* c, void* dst, const void* src, size_t n) {
  HIPCHK(c, hipMemcpy(dst, src, n, hipMemcpyHostToDevice));
  return FX_OK;
}
int fx_memcpy_dtoh(fx_ctx* c, void* dst, const void* src, size_t n) {
  HIPCHK(c, hipMemcpy(dst, src, n, hipMemcpyDeviceToHost));
  return FX_OK;
}
int fx_memcpy_dtod(fx_ctx* c, void* dst, const void* src, size_t n) {
  HIPCHK(c, hipMemcpy(dst, src, n, hipMemcpyDeviceToDevice));
  return FX_OK;
}
int fx_memset(fx_ctx* c, void* dst, int v, size_t n) {
  HIPCHK(c, hipMemset(dst, v, n));
  return FX_OK;
}
int fx_synchronize(fx_ctx* c) {
  HIPCHK(c, hipDeviceSynchronize());
  return FX_OK;
}

// host-side checks of one stage against what its device code assumes
static int check_stage(fx_ctx* c, const fx_stage& s, int idx, int n_total) {
  auto bad = [&](const std::string& m) { return fail(c, FX_E_ARG, "stage " + std::to_string(idx) + ": " + m); };
  for (int k = 0; k < 4; ++k)
    if (s.src[k] < -n_total || s.src[k] >= n_total) return bad("packet source out of range");
  if ((s.flags & FX_F_MFMA) && s.op != FX_OP_MLA_ATTEND && s.op != FX_OP_MLA_MERGE_UV)
    return bad("FX_F_MFMA marks the attention and its merge only");
  if ((s.flags & FX_F_XLOCAL) && s.op != FX_OP_MLA_PREP) return bad("FX_F_XLOCAL marks the MLA prep only");
  if ((s.flags & FX_F_XCD) && s.op != FX_OP_MLA_ATTEND && s.op != FX_OP_MLA_MERGE_UV)
    return bad("FX_F_XCD marks the attention and its merge only");
  if ((s.flags & FX_F_XCD) && (s.flags & FX_F_MFMA)) return bad("FX_F_XCD and FX_F_MFMA exclude each other");
  if ((s.flags & FX_F_SKIP_XCD) && (s.op != FX_OP_GEMV || (s.flags & FX_F_ARGMAX)))
    return bad("FX_F_SKIP_XCD marks a GEMV without argmax only");
  if ((s.flags & FX_F_LOW16) && (s.op != FX_OP_GEMV || (s.flags & (FX_F_ARGMAX | FX_F_SKIP_XCD))))
    return bad("FX_F_LOW16 marks a GEMV without argmax or FX_F_SKIP_XCD only");
  if (s.flags & FX_F_FP8) {
    const bool head = s.op == FX_OP_GEMV && (s.flags & FX_F_ARGMAX) && s.in_kind == FX_IN_VEC;
    if (s.op != FX_OP_MOE_W13 && s.op != FX_OP_MOE_W2 && !head)
      return bad("FP8 weights are read by the expert stages and the LM head only");
    if (s.k % 16 || (s.k / 16 + 63) / 64 > 2) return bad("FP8 K must be a multiple of 16, at most 2048");
  }
  switch (s.op) {
    case FX_OP_GEMV: {
      if (!s.w || !s.out || s.n_rows <= 0 || s.k <= 0 || s.k % 8) return bad("gemv shape/pointers");
      const int nj = (s.k / 8 + 63) / 64;
      if (!(nj <= 4 || nj == 22)) return bad("gemv K not supported: " + std::to_string(s.k));
      if (s.k > 11264) return bad("gemv K exceeds the LDS row");
      if (s.in_kind == FX_IN_VEC && (!s.x || s.k % 4)) return bad("gemv input");
      if (s.in_kind == FX_IN_EMBED && (!s.aux[0] || !s.aux[3] || !s.aux[4])) return bad("embed table / amax / tokens");
      if ((s.flags & FX_F_NORM) && !s.w_norm) return bad("norm weight");
      if ((s.flags & FX_F_RESIDUAL) && !s.res) return bad("residual");
      if ((s.flags & FX_F_RES_EMBED) && !s.aux[0]) return bad("embedding residual");
      const int groups = (s.n_rows + 3) / 4;
      const int gworkers = (s.flags & FX_F_LOW16) ? FX_WORKERS / 2 : FX_WORKERS;
      const int rows_max = 4 * ((groups + gworkers - 1) / gworkers);
      if ((s.flags & (FX_F_OUT_LL | FX_F_RESIDUAL | FX_F_RES_EMBED)) && rows_max > FX_MAX_OUT_ROWS / 2)
        return bad("rows per worker exceed the LDS row table");
      if ((s.flags & FX_F_OUT_LL) && s.n_rows % 4) return bad("packet output needs rows in multiples of 4");
      if ((s.flags & FX_F_ARGMAX) && !s.aux[3]) return bad("amax");
      break;
    }
    case FX_OP_MLA_PREP:
    case FX_OP_MLA_ATTEND:
    case FX_OP_MLA_MERGE_UV:
      if (s.n_rows != 16 || s.d_c != 512 || s.d_r != 64 || s.d_n != 128) return bad("MLA dims must be 16 x (512, 64, 128)");
      if (!s.x || !s.out || (s.op != FX_OP_MLA_ATTEND && !s.w)) return bad("MLA pointers");
      if (s.op == FX_OP_MLA_PREP && (!s.aux[0] || !s.aux[1] || !s.aux[2] || !s.aux[3] || !s.aux[4] || !s.aux[5] || !s.w_norm))
        return bad("prep pointers");
      if (s.op == FX_OP_MLA_ATTEND) {
        if (!s.aux[0] || !s.aux[1] || !s.aux[2] || !s.aux[5] || !s.aux[6]) return bad("attend pointers");
        if (s.split <= 0 || s.split % 32 || s.n_splits <= 0 || s.prow < s.d_c + 1 || s.prow % 4) return bad("attend splits");
        if ((long long)s.n_splits * s.split < s.s_max) return bad("splits do not cover s_max");
      }
      if (s.op == FX_OP_MLA_MERGE_UV) {
        if (!s.aux[6] || s.split <= 0) return bad("merge pointers");
        if (s.n_splits * 4 > 37 * 1024) return bad("too many splits for the merge table");
        if (s.flags & FX_F_XCD) {
          if (!s.aux[0] || !s.aux[1] || !s.aux[2] || !s.aux[3] || !s.aux[5]) return bad("single-XCD attention pointers");
          if (s.split % 32 || s.n_splits <= 0 || s.prow < s.d_c + 1 || s.prow % 4) return bad("attend splits");
          if ((long long)s.n_splits * s.split < s.s_max) return bad("splits do not cover s_max");
        }
      }
      break;
    case FX_OP_MOE_ROUTER:
      if (!s.w || !s.x || !s.out || !s.w_norm || s.n_rows > 64 || s.n_rows % 2 || s.k != 2048) return bad("router");
      break;
    case FX_OP_MOE_W13:
      if (!s.w || !s.x || !s.out || !s.w_norm || !s.aux[0] || !s.aux[1] || !s.aux[2] || !s.aux[3] || !s.aux[4])
        return bad("w13 pointers");
      if (s.n_slots != FX_XCDS || s.topk + s.n_forced != s.n_slots || s.aux_i0 > 64 || s.aux_i0 % 2 || s.k != 2048 ||
          s.n_rows % 4)
        return bad("w13 shape");
      if ((s.flags & FX_F_ROUTER) && !s.res) return bad("w13 router weights");
      if (((s.n_rows / 2 + FX_WORKERS - 1) / FX_WORKERS) * s.n_slots > 64) return bad("w13 groups per worker");
      break;
    case FX_OP_MOE_W2:
      if (!s.w || !s.x || !s.out || !s.res || !s.aux[0] || (s.k / 8 + 63) / 64 > 3 || s.k % 8) return bad("w2");
      if (s.n_slots != FX_XCDS || s.topk + s.n_forced != s.n_slots || s.aux_i0 > 64 || s.aux_i0 % 2) return bad("w2 slots");
      if (s.n_rows != 8 * FX_WORKERS || s.n_slots * s.k > 11264) return bad("w2 rows / input row");
      break;
    case FX_OP_DENSE_GU:
      if (!s.w || !s.x || !s.out || !s.w_norm || s.k != 2048 || s.n_rows % 4) return bad("dense gate/up");
      if (2 * ((s.n_rows / 2 + FX_WORKERS - 1) / FX_WORKERS) > FX_MAX_OUT_ROWS) return bad("dense gate/up rows per worker");
      break;
    case FX_OP_ARGMAX:
      if (!s.aux[3] || !s.aux[4]) return bad("argmax");
      break;
    default:
      return bad("unknown op " + std::to_string(s.op));
  }
  return FX_OK;
}

int fx_load_plan(fx_ctx* c, const fx_stage* st, int32_t n, const fx_stage* epi, int32_t n_epi) {
  if (!c) return FX_E_ARG;
  if (n <= 0 || !st) return fail(c, FX_E_ARG, "empty plan");
  if (n_epi < 0 || n + n_epi > FX_TABLE_MAX)
    return fail(c, FX_E_ARG, "the plan has " + std::to_string(n) + " stages + " + std::to_string(n_epi) +
                                 " epilogue stages; the persistent kernel holds at most " + std::to_string(FX_TABLE_MAX));
  for (int i = 0; i < n; ++i) {
    int r = check_stage(c, st[i], i, n);
    if (r) return r;
  }
  for (int i = 0; i < n_epi; ++i) {
    int r = check_stage(c, epi[i], n + i, n);
    if (r) return r;
  }
  // FX_F_PAIR: a GEMV that the persistent kernel runs together with the MOE_W13 stage after it
  for (int i = 0; i < n + n_epi; ++i) {
    const fx_stage& t = i < n ? st[i] : epi[i - n];
    if (!(t.flags & FX_F_PAIR)) continue;
    const std::string at = "stage " + std::to_string(i) + ": FX_F_PAIR ";
    if (i >= n - 1) return fail(c, FX_E_ARG, at + "needs a MOE_W13 stage after it in the plan");
    if (t.op != FX_OP_GEMV || (t.flags & (FX_F_ARGMAX | FX_F_HEAD | FX_F_SKIP_XCD | FX_F_FP8)))
      return fail(c, FX_E_ARG, at + "is for a plain GEMV stage");
    if (st[i + 1].op != FX_OP_MOE_W13 || (st[i + 1].flags & (FX_F_HEAD | FX_F_PAIR)))
      return fail(c, FX_E_ARG, at + "needs a MOE_W13 stage after it");
  }
  // a plan's expert stages are all bf16 or all FP8: the launch picks the kernel variant
  int n_fp8 = 0, n_exp = 0;
  for (int i = 0; i < n; ++i)
    if (st[i].op == FX_OP_MOE_W13 || st[i].op == FX_OP_MOE_W2) {
      ++n_exp;
      n_fp8 += (st[i].flags & FX_F_FP8) != 0;
    }
  if (n_fp8 && n_fp8 != n_exp) return fail(c, FX_E_ARG, "a plan's expert stages must be all bf16 or all FP8");
  // an FP8 LM head runs in the FP8 kernel variant, which the launch picks from the expert stages
  for (int i = 0; i < n + n_epi; ++i) {
    const fx_stage& t = i < n ? st[i] : epi[i - n];
    if (t.op == FX_OP_GEMV && (t.flags & FX_F_FP8) && (n_exp == 0 || n_fp8 != n_exp))
      return fail(c, FX_E_ARG, "an FP8 LM head needs FP8 expert stages in the same plan");
  }
  if (c->d_stages) { HIPCHK(c, hipFree(c->d_stages)); c->d_stages = nullptr; }
  if (c->d_epi) { HIPCHK(c, hipFree(c->d_epi)); c->d_epi = nullptr; }
  HIPCHK(c, hipMalloc(&c->d_stages, sizeof(fx_stage) * n));
  HIPCHK(c, hipMemcpy(c->d_stages, st, sizeof(fx_stage) * n, hipMemcpyHostToDevice));
  if (n_epi > 0) {
    HIPCHK(c, hipMalloc(&c->d_epi, sizeof(fx_stage) * n_epi));
    HIPCHK(c, hipMemcpy(c->d_epi, epi, sizeof(fx_stage) * n_epi, hipMemcpyHostToDevice));
  }
  c->n_stages = n;
  c->n_epi = n_epi;
  c->fp8 = n_fp8 > 0;
  c->next_step = -1;
  c->h_stages.assign(st, st + n);
  c->h_epi.assign(epi ? epi : st, epi ? epi + n_epi : st);
  return FX_OK;
}

int fx_launch(fx_ctx* c, int32_t iters, int32_t step0, int32_t n_prompt, int64_t* tokens, void* stream) {
  if (!c) return FX_E_ARG;
  if (!c->d_stages) return fail(c, FX_E_STATE, "no plan loaded");
  if (iters <= 0 || iters > FX_MAX_ITERS || step0 < 0 || !tokens) return fail(c, FX_E_ARG, "iters/step0/tokens");
  if (n_prompt < 1) return fail(c, FX_E_ARG, "n_prompt must be at least 1");
  // past the prompt, an iteration's token is the previous iteration's argmax: a launch may start
  // there only where the previous launch of this plan ended
  if (step0 >= n_prompt && step0 != c->next_step)
    return fail(c, FX_E_ARG, "a launch starting at step " + std::to_string(step0) + " (past the prompt of " +
                                 std::to_string(n_prompt) + ") must continue the previous launch, which ended at " +
                                 std::to_string(c->next_step));
  for (const fx_stage& s : c->h_stages) {
    if (s.s_max > 0 && step0 + iters > s.s_max) return fail(c, FX_E_ARG, "steps exceed the cache length s_max");
  }
  const uint64_t total = (uint64_t)c->n_stages * (uint64_t)iters;
  hipStream_t s = (hipStream_t)stream;
  if ((uint64_t)c->epoch + total + (uint64_t)c->n_stages + 1 > 0xFFFFFFF0ull)
    return fail(c, FX_E_STATE, "packet tags exhausted for this context: recreate it and zero the plan's packet buffers");
  FxRunArgs a;
  a.stages = c->d_stages;
  a.n_stages = c->n_stages;
  a.epi = c->d_epi;
  a.n_epi = c->n_epi;
  a.iters = iters;
  a.step0 = step0;
  a.n_prompt = n_prompt;
  a.tokens = tokens;
  a.err = c->err_flag;
  a.timing = c->timing;
  a.prof = nullptr;
  a.prof_iter = -1;
  if (c->prof_iter >= 0 && c->prof_iter < iters) {
    const size_t words = (size_t)c->n_stages * FX_BLOCKS * FX_PROF_SLOTS;
    if (c->prof_words < words) {
      HIPCHK(c, hipStreamSynchronize(s));
      if (c->prof) HIPCHK(c, hipFree(c->prof));
      HIPCHK(c, hipMalloc(&c->prof, words * 8));
      c->prof_words = words;
    }
    HIPCHK(c, hipMemsetAsync(c->prof, 0, words * 8, s));
    a.prof = c->prof;
    a.prof_iter = c->prof_iter;
  }
  a.epoch0 = c->epoch;
  void* args[] = {&a};
  // every iteration skips the head (all positions inside the prompt): the prefill symbol
  const bool prefill = (int64_t)step0 + iters < (int64_t)n_prompt;
  const void* fn = c->fp8 ? (prefill ? (const void*)fx_prefill_fp8 : (const void*)fx_persistent_fp8)
                          : (prefill ? (const void*)fx_prefill : (const void*)fx_persistent);
  HIPCHK(c, hipEventRecord(c->ev0, s));
  HIPCHK(c, hipLaunchCooperativeKernel(fn, dim3(FX_BLOCKS), dim3(FX_THREADS), args, FX_LDS_TOTAL, s));
  HIPCHK(c, hipEventRecord(c->ev1, s));
  c->epoch += (uint32_t)total;
  c->last_iters = iters;
  c->next_step = (int64_t)step0 + iters;
  return FX_OK;
}

int fx_finish(fx_ctx* c, void* stream) {
  if (!c) return FX_E_ARG;
  HIPCHK(c, hipStreamSynchronize((hipStream_t)stream));
  uint32_t err = 0;
  HIPCHK(c, hipMemcpy(&err, c->err_flag, 4, hipMemcpyDeviceToHost));
  if (err) return fail(c, FX_E_STATE, "a synchronisation wait timed out inside the persistent kernel; create a new context");
  return FX_OK;
}

int fx_run(fx_ctx* c, int32_t iters, int32_t step0, int32_t n_prompt, int64_t* tokens, void* stream) {
  const int r = fx_launch(c, iters, step0, n_prompt, tokens, stream);
  if (r) return r;
  return fx_finish(c, stream);
}

int fx_mark(fx_ctx* c, int32_t idx, void* stream) {
  if (!c || idx < 0 || idx >= FX_MAX_MARKS) return fail(c, FX_E_ARG, "mark index");
  if (!c->marks[idx]) HIPCHK(c, hipEventCreate(&c->marks[idx]));
  HIPCHK(c, hipEventRecord(c->marks[idx], (hipStream_t)stream));
  return FX_OK;
}

int fx_marks_ms(fx_ctx* c, int32_t i, int32_t j, float* ms) {
  if (!c || !ms || i < 0 || j < 0 || i >= FX_MAX_MARKS || j >= FX_MAX_MARKS || !c->marks[i] || !c->marks[j])
    return fail(c, FX_E_ARG, "mark index");
  HIPCHK(c, hipEventElapsedTime(ms, c->marks[i], c->marks[j]));
  return FX_OK;
}

int fx_set_profile(fx_ctx* c, int32_t iter) {
  if (!c) return FX_E_ARG;
  c->prof_iter = iter;
  return FX_OK;
}

int fx_read_profile(fx_ctx* c, uint64_t* buf, int32_t n) {
  if (!c || !buf) return -1;
  if (!c->prof) return 0;
  size_t m = (size_t)c->n_stages * FX_BLOCKS * FX_PROF_SLOTS;
  if ((size_t)n < m) m = (size_t)n;
  if (hipMemcpy(buf, c->prof, m * 8, hipMemcpyDeviceToHost) != hipSuccess) return -1;
  return (int)m;
}

int fx_last_run_ms(fx_ctx* c, float* ms) {
  if (!c || !ms) return FX_E_ARG;
  if (!c->last_iters) return fail(c, FX_E_STATE, "no run yet");
  HIPCHK(c, hipEventElapsedTime(ms, c->ev0, c->ev1));
  return FX_OK;
}

int fx_read_timing(fx_ctx* c, uint64_t* buf, int32_t n) {
  if (!c || !buf) return -1;
  if (!c->timing) return 0;
  int m = c->last_iters + 1;
  if (n < m) m = n;
  if (hipMemcpy(buf, c->timing, sizeof(uint64_t) * m, hipMemcpyDeviceToHost) != hipSuccess) return -1;
  return m;
}

int fx_run_stage(fx_ctx* c, const fx_stage* st, int32_t step, uint32_t tbase, int32_t sidx, void* stream) {
  if (!c || !st) return FX_E_ARG;
  int r = check_stage(c, *st, 0, 1 << 20);
  if (r) return r;
  if (st->flags & FX_F_FP8) return fail(c, FX_E_ARG, "FP8 expert stages run in the persistent kernel only");
  hipStream_t s = (hipStream_t)stream;
  // the embed prologue reads tokens[step]; the argmax reduce always stores tokens[step + 1]
  const int n_prompt = st->op == FX_OP_ARGMAX ? 0 : (1 << 30);
  const bool uses_tokens = st->op == FX_OP_ARGMAX ||
                           (st->op == FX_OP_GEMV && (st->in_kind == FX_IN_EMBED || (st->flags & FX_F_RES_EMBED)));
  int64_t* tokens = uses_tokens ? (int64_t*)st->aux[4] : nullptr;
  void* args[] = {(void*)st, &step, (void*)&n_prompt, &tbase, &sidx, &tokens, &c->err_flag};
  HIPCHK(c, hipLaunchCooperativeKernel((const void*)fx_stage_kernel, dim3(FX_BLOCKS), dim3(FX_THREADS), args, FX_LDS_BYTES, s));
  HIPCHK(c, hipStreamSynchronize(s));
  uint32_t err = 0;
  HIPCHK(c, hipMemcpy(&err, c->err_flag, 4, hipMemcpyDeviceToHost));
  if (err) return fail(c, FX_E_STATE, "a packet wait timed out in the stage launch; create a new context");
  return FX_OK;
}

// The attention pair of the kernel suite (an MLA_ATTEND stage, then its MLA_MERGE_UV stage) with
// the split partials and the done packets in this device's `scratch` instead of caller buffers:
// no allocation on any path. The attend stage runs with (tbase, sidx), the merge with
// (tbase, sidx + 1) reading the attend stage's outputs; the stages' partials / done pointers are
// ignored. At most FX_NOALLOC_MAX_SPLITS splits. Calls that overlap on one GPU race on `scratch`.
int fx_mla_attend_merge_noalloc(fx_ctx* c, const fx_stage* attend, const fx_stage* merge, int32_t step,
                                uint32_t tbase, int32_t sidx, void* stream) {
  if (!c || !attend || !merge) return FX_E_ARG;
  if (!c->scratch) return fail(c, FX_E_STATE, "the context has no scratch address");
  if (attend->op != FX_OP_MLA_ATTEND || merge->op != FX_OP_MLA_MERGE_UV)
    return fail(c, FX_E_ARG, "fx_mla_attend_merge_noalloc takes an MLA_ATTEND stage and an MLA_MERGE_UV stage");
  if ((attend->flags & (FX_F_MFMA | FX_F_XCD)) != (merge->flags & (FX_F_MFMA | FX_F_XCD)))
    return fail(c, FX_E_ARG, "the attend and merge stages must use the same attention kernel (FX_F_MFMA, FX_F_XCD)");
  if (attend->n_splits <= 0 || attend->n_splits > FX_NOALLOC_MAX_SPLITS || merge->n_splits != attend->n_splits ||
      merge->split != attend->split)
    return fail(c, FX_E_ARG, "n_splits must be in [1, " + std::to_string(FX_NOALLOC_MAX_SPLITS) +
                                 "] and equal on both stages (the scratch holds that many splits' partials)");
  if (attend->prow != FX_NOALLOC_PROW || merge->prow != FX_NOALLOC_PROW)
    return fail(c, FX_E_ARG, "partials rows must be 516 floats (d_c = 512)");
  if (step < 0 || (long long)step >= (long long)attend->n_splits * attend->split)
    return fail(c, FX_E_ARG, "step outside the splits");
  fx_stage a = *attend, m = *merge;
  const uint64_t part = (uint64_t)c->scratch, done = part + FX_NOALLOC_PARTIAL_BYTES;
  a.out = part;
  a.aux[6] = done;
  m.x = part;
  m.aux[6] = done;
  // no slice-exchange buffer: the merge reads every column itself (the exchange packets would be
  // caller memory beyond this entry's inputs and outputs)
  if (!(merge->flags & FX_F_XCD)) m.aux[7] = 0;
  // the merge waits for the attention's done packets; the single-XCD merge runs the attention itself
  // and waits for the attention's inputs
  const bool xcd = (merge->flags & FX_F_XCD) != 0;
  m.src[0] = xcd ? attend->src[0] : sidx;
  int r = check_stage(c, a, 0, 1 << 20);
  if (r) return r;
  r = check_stage(c, m, 1, 1 << 20);
  if (r) return r;
  hipStream_t s = (hipStream_t)stream;
  // stale done packets of an earlier call could carry the tags this call waits for: zero them with a
  // fill kernel (no memset node, so the call can be captured)
  hipLaunchKernelGGL(fx_fill_kernel, dim3(1), dim3(256), 0, s, (uint16_t*)done, (uint64_t)(FX_NOALLOC_DONE_BYTES / 2),
                     (uint16_t)0);
  HIPCHK(c, hipGetLastError());
  int32_t n_prompt = 1 << 30, sidx_m = sidx + 1;
  int64_t* no_tokens = nullptr;
  void* args_a[] = {(void*)&a, &step, &n_prompt, &tbase, &sidx, &no_tokens, &c->err_flag};
  if (!xcd)
    HIPCHK(c, hipLaunchCooperativeKernel((const void*)fx_stage_kernel, dim3(FX_BLOCKS), dim3(FX_THREADS), args_a,
                                         FX_LDS_BYTES, s));
  void* args_m[] = {(void*)&m, &step, &n_prompt, &tbase, &sidx_m, &no_tokens, &c->err_flag};
  HIPCHK(c, hipLaunchCooperativeKernel((const void*)fx_stage_kernel, dim3(FX_BLOCKS), dim3(FX_THREADS), args_m,
                                       FX_LDS_BYTES, s));
  HIPCHK(c, hipStreamSynchronize(s));
  uint32_t err = 0;
  HIPCHK(c, hipMemcpy(&err, c->err_flag, 4, hipMemcpyDeviceToHost));
  if (err) return fail(c, FX_E_STATE, "a packet wait timed out in the attention launch; create a new context");
  return FX_OK;
}

int fx_time_stages(fx_ctx* c, const fx_stage* st, int32_t n, int32_t reps, int32_t step, uint32_t tbase, int32_t sidx,
                   void* stream, float* us) {
  if (!c || !st || n <= 0 || reps <= 0 || !us) return fail(c, FX_E_ARG, "time_stages arguments");
  for (int i = 0; i < n; ++i) {
    int r = check_stage(c, st[i], i, 1 << 20);
    if (r) return r;
    if (st[i].flags & FX_F_FP8) return fail(c, FX_E_ARG, "FP8 expert stages run in the persistent kernel only");
  }
  hipStream_t s = (hipStream_t)stream;
  int n_prompt = 1 << 30;
  HIPCHK(c, hipEventRecord(c->ev0, s));
  for (int rep = 0; rep < reps; ++rep)
    for (int i = 0; i < n; ++i) {
      const bool uses_tokens = st[i].op == FX_OP_ARGMAX ||
                               (st[i].op == FX_OP_GEMV && (st[i].in_kind == FX_IN_EMBED || (st[i].flags & FX_F_RES_EMBED)));
      int64_t* tokens = uses_tokens ? (int64_t*)st[i].aux[4] : nullptr;
      void* args[] = {(void*)&st[i], &step, &n_prompt, &tbase, &sidx, &tokens, &c->err_flag};
      HIPCHK(c, hipLaunchCooperativeKernel((const void*)fx_stage_kernel, dim3(FX_BLOCKS), dim3(FX_THREADS), args,
                                           FX_LDS_BYTES, s));
    }
  HIPCHK(c, hipEventRecord(c->ev1, s));
  HIPCHK(c, hipEventSynchronize(c->ev1));
  float ms = 0.0f;
  HIPCHK(c, hipEventElapsedTime(&ms, c->ev0, c->ev1));
  *us = 1000.0f * ms / (float)(reps * n);
  uint32_t err = 0;
  HIPCHK(c, hipMemcpy(&err, c->err_flag, 4, hipMemcpyDeviceToHost));
  if (err) return fail(c, FX_E_STATE, "a packet wait timed out in a timed stage launch; create a new context");
  return FX_OK;
}

int fx_gen_normal_bf16(fx_ctx* c, void* dst, uint64_t rows, uint64_t row_len, uint64_t dst_stride, uint64_t src_offset,
                       uint64_t src_stride, uint64_t seed, uint32_t stream, float scale) {
  if (!dst) return fail(c, FX_E_ARG, "null dst");
  if (rows == 0 || row_len == 0) return FX_OK;
  if (rows == 1 || (dst_stride == row_len && src_stride == row_len)) {
    const uint64_t n = rows * row_len;
    uint64_t blocks = (n + 3) / 4 + 1;
    uint64_t grid = (blocks + 255) / 256;
    if (grid > 65536) grid = 65536;
    hipLaunchKernelGGL(fx_gen_kernel, dim3((unsigned)grid), dim3(256), 0, 0, (uint16_t*)dst, n, seed, stream, scale,
                       src_offset);
  } else {
    uint64_t grid = (rows * row_len + 255) / 256;
    if (grid > 65536) grid = 65536;
    hipLaunchKernelGGL(fx_gen2d_kernel, dim3((unsigned)grid), dim3(256), 0, 0, (uint16_t*)dst, rows, row_len, dst_stride,
                       src_offset, src_stride, seed, stream, scale);
  }
  HIPCHK(c, hipGetLastError());
  return FX_OK;
}

int fx_fill_u16(fx_ctx* c, void* dst, uint64_t n, uint16_t v) {
  if (!dst) return fail(c, FX_E_ARG, "null dst");
  if (n == 0) return FX_OK;
  uint64_t grid = (n + 255) / 256;
  if (grid > 65536) grid = 65536;
  hipLaunchKernelGGL(fx_fill_kernel, dim3((unsigned)grid), dim3(256), 0, 0, (uint16_t*)dst, n, v);
  HIPCHK(c, hipGetLastError());
  return FX_OK;
}

// ------------------------------------------------------------------------------------------------
// batched prefill: rocBLAS GEMMs and the row kernels of fx_prefill.h

#define PF_CHECK(c, cond, msg) \
  do {                         \
    if (!(cond)) return fail((c), FX_E_ARG, msg); \
  } while (0)

static bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

int fx_gemm(fx_ctx* c, int32_t trans_a, int32_t trans_b, int32_t M, int32_t N, int32_t K, float alpha, const void* A,
            int64_t lda, int64_t stride_a, const void* B, int64_t ldb, int64_t stride_b, float beta, const void* C,
            int64_t ldc, int64_t stride_c, void* D, int64_t ldd, int64_t stride_d, int32_t d_f32, int32_t batch,
            void* stream) {
  if (!c) return FX_E_ARG;
  PF_CHECK(c, M > 0 && N > 0 && K > 0 && batch > 0, "fx_gemm: empty shape");
  PF_CHECK(c, A && B && D && (beta == 0.0f || C), "fx_gemm: null operand");
  PF_CHECK(c, lda >= (trans_a ? M : K) && ldb >= (trans_b ? K : N) && ldd >= N && (beta == 0.0f || ldc >= N),
           "fx_gemm: leading dimension smaller than the row");
  if (!c->blas) {
    if (rocblas_create_handle(&c->blas) != rocblas_status_success) return fail(c, FX_E_HIP, "rocblas_create_handle");
  }
  if (rocblas_set_stream(c->blas, (hipStream_t)stream) != rocblas_status_success)
    return fail(c, FX_E_HIP, "rocblas_set_stream");
  // row-major D[M,N] = op(A) op(B) is column-major D^T[N,M] = op(B)^T op(A)^T: B first
  const rocblas_datatype dt = d_f32 ? rocblas_datatype_f32_r : rocblas_datatype_bf16_r;
  rocblas_status st = rocblas_gemm_strided_batched_ex(
      c->blas, trans_b ? rocblas_operation_transpose : rocblas_operation_none,
      trans_a ? rocblas_operation_transpose : rocblas_operation_none, N, M, K, &alpha, B, rocblas_datatype_bf16_r, ldb,
      stride_b, A, rocblas_datatype_bf16_r, lda, stride_a, &beta, beta == 0.0f ? D : C, dt, beta == 0.0f ? ldd : ldc,
      beta == 0.0f ? stride_d : stride_c, D, dt, ldd, stride_d, batch, rocblas_datatype_f32_r, rocblas_gemm_algo_standard,
      0, 0);
  if (st != rocblas_status_success)
    return fail(c, FX_E_HIP, std::string("rocblas_gemm_strided_batched_ex: ") + rocblas_status_to_string(st));
  return FX_OK;
}

int fx_pf_embed(fx_ctx* c, const int64_t* tokens, const void* W, void* x, int32_t M, int32_t H, void* stream) {
  if (!c) return FX_E_ARG;
  PF_CHECK(c, tokens && W && x && M > 0 && H > 0 && H % 8 == 0 && al16(W) && al16(x), "fx_pf_embed: arguments");
  hipLaunchKernelGGL(pf_embed_kernel, dim3(M), dim3(PF_THREADS), 0, (hipStream_t)stream, tokens, (const uint16_t*)W,
                     (uint16_t*)x, H);
  HIPCHK(c, hipGetLastError());
  return FX_OK;
}

int fx_pf_rmsnorm(fx_ctx* c, const void* x, int64_t ldx, const void* w, void* y, int64_t ldy, int32_t M, int32_t K,
                  float eps, void* stream) {
  if (!c) return FX_E_ARG;
  PF_CHECK(c, x && w && y && M > 0 && K > 0 && K % 8 == 0 && K <= 16384 && ldx >= K && ldy >= K && ldx % 8 == 0 &&
                  ldy % 8 == 0 && al16(x) && al16(y) && al16(w),
           "fx_pf_rmsnorm: arguments");
  const size_t lds = (size_t)(((K + 63) & ~63) + 64) * 4;
  hipLaunchKernelGGL(pf_rmsnorm_kernel, dim3(M), dim3(PF_THREADS), lds, (hipStream_t)stream, (const uint16_t*)x, ldx,
                     (const uint16_t*)w, (uint16_t*)y, ldy, K, eps);
  HIPCHK(c, hipGetLastError());
  return FX_OK;
}

int fx_pf_prep(fx_ctx* c, const void* qkva, int64_t ldq, const void* w_kv_norm, const void* cos, const void* sin,
               void* c_kv, void* k_pe, void* q_pe, int32_t pos0, int32_t M, int32_t s_max, int32_t n_heads,
               int32_t d_n, int32_t d_c, float eps, void* stream) {
  if (!c) return FX_E_ARG;
  PF_CHECK(c, qkva && w_kv_norm && cos && sin && c_kv && k_pe && q_pe && M > 0 && pos0 >= 0 && pos0 + M <= s_max &&
                  n_heads > 0 && n_heads <= 64 && d_n > 0 && d_c > 0 && d_c % 8 == 0 && d_c <= 4096 &&
                  ldq >= (int64_t)n_heads * (d_n + 64) + d_c + 64 && al16(w_kv_norm),
           "fx_pf_prep: arguments");
  const size_t lds = (size_t)(d_c + (1 + n_heads) * 64 + 64) * 4;
  hipLaunchKernelGGL(pf_prep_kernel, dim3(M), dim3(PF_THREADS), lds, (hipStream_t)stream, (const uint16_t*)qkva, ldq,
                     (const uint16_t*)w_kv_norm, (const uint16_t*)cos, (const uint16_t*)sin, (uint16_t*)c_kv,
                     (uint16_t*)k_pe, (uint16_t*)q_pe, pos0, n_heads, d_n, d_c, eps);
  HIPCHK(c, hipGetLastError());
  return FX_OK;
}

int fx_pf_softmax(fx_ctx* c, const void* S, int64_t ldS, int64_t strideS, void* P, int64_t ldP, int64_t strideP,
                  void* l, int64_t strideL, int32_t M, int32_t heads, int32_t n_cols, int32_t key0, float scale,
                  void* stream) {
  if (!c) return FX_E_ARG;
  PF_CHECK(c, S && P && l && M > 0 && heads > 0 && heads <= 65535 && n_cols > 0 && key0 >= 0 && ldS >= n_cols &&
                  ldP >= n_cols && strideL >= M,
           "fx_pf_softmax: arguments");
  hipLaunchKernelGGL(pf_softmax_kernel, dim3(M, heads), dim3(PF_THREADS), 0, (hipStream_t)stream, (const float*)S, ldS,
                     strideS, (uint16_t*)P, ldP, strideP, (float*)l, strideL, n_cols, key0, scale);
  HIPCHK(c, hipGetLastError());
  return FX_OK;
}

int fx_pf_attn_out(fx_ctx* c, const void* O, const void* l, void* obf, int32_t M, int32_t heads, int32_t d,
                   void* stream) {
  if (!c) return FX_E_ARG;
  PF_CHECK(c, O && l && obf && M > 0 && heads > 0 && heads <= 65535 && d > 0, "fx_pf_attn_out: arguments");
  hipLaunchKernelGGL(pf_attn_out_kernel, dim3(M, heads), dim3(PF_THREADS), 0, (hipStream_t)stream, (const float*)O,
                     (const float*)l, (uint16_t*)obf, M, d);
  HIPCHK(c, hipGetLastError());
  return FX_OK;
}

int fx_pf_silu(fx_ctx* c, const void* gu, void* act, int32_t rows, int32_t I, void* stream) {
  if (!c) return FX_E_ARG;
  PF_CHECK(c, gu && act && rows >= 0 && I > 0, "fx_pf_silu: arguments");
  if (rows == 0) return FX_OK;
  hipLaunchKernelGGL(pf_silu_kernel, dim3(rows), dim3(PF_THREADS), 0, (hipStream_t)stream, (const uint16_t*)gu,
                     (uint16_t*)act, I);
  HIPCHK(c, hipGetLastError());
  return FX_OK;
}

int fx_pf_route(fx_ctx* c, const void* logits, void* ids, void* wts, int32_t M, int32_t E, int32_t topk,
                int32_t n_shared, float scaling, void* stream) {
  if (!c) return FX_E_ARG;
  PF_CHECK(c, logits && ids && wts && M > 0 && E > 0 && E <= 64 && topk > 0 && topk <= E && n_shared >= 0 &&
                  topk + n_shared <= 16,
           "fx_pf_route: arguments");
  hipLaunchKernelGGL(pf_route_kernel, dim3(M), dim3(64), 0, (hipStream_t)stream, (const float*)logits, E, topk,
                     n_shared, scaling, (int32_t*)ids, (float*)wts);
  HIPCHK(c, hipGetLastError());
  return FX_OK;
}

int fx_pf_gather(fx_ctx* c, const void* src, const void* idx, void* dst, int32_t rows, int32_t H, void* stream) {
  if (!c) return FX_E_ARG;
  PF_CHECK(c, src && idx && dst && rows >= 0 && H > 0 && H % 8 == 0 && al16(src) && al16(dst), "fx_pf_gather: arguments");
  if (rows == 0) return FX_OK;
  hipLaunchKernelGGL(pf_gather_kernel, dim3(rows), dim3(PF_THREADS), 0, (hipStream_t)stream, (const uint16_t*)src,
                     (const int32_t*)idx, (uint16_t*)dst, H);
  HIPCHK(c, hipGetLastError());
  return FX_OK;
}

int fx_pf_combine(fx_ctx* c, const void* x_mid, const void* og, const void* inv, const void* w, void* x_res, int32_t M,
                  int32_t H, int32_t slots, void* stream) {
  if (!c) return FX_E_ARG;
  PF_CHECK(c, x_mid && og && inv && w && x_res && M > 0 && H > 0 && slots > 0, "fx_pf_combine: arguments");
  hipLaunchKernelGGL(pf_combine_kernel, dim3(M), dim3(PF_THREADS), 0, (hipStream_t)stream, (const uint16_t*)x_mid,
                     (const uint16_t*)og, (const int32_t*)inv, (const float*)w, (uint16_t*)x_res, H, slots);
  HIPCHK(c, hipGetLastError());
  return FX_OK;
}

// FP8 rows from bf16 rows (weight-only quantization): scale = max|w| / 448 (1 for an all-zero row),
// codes = e4m3fn(w / scale) rounded to nearest even, saturated at 448; dst holds the rows' codes,
// then their f32 scales.
int fx_quantize_fp8(fx_ctx* c, const void* src, void* dst, int64_t rows, int32_t K, void* stream) {
  if (!c) return FX_E_ARG;
  PF_CHECK(c, src && dst && rows > 0 && rows <= 0x7fffffff && K > 0 && K % 16 == 0 && al16(src) && al16(dst),
           "fx_quantize_fp8: arguments");
  hipLaunchKernelGGL(fx_quant_fp8_kernel, dim3((unsigned)rows), dim3(PF_THREADS), 0, (hipStream_t)stream,
                     (const uint16_t*)src, (uint8_t*)dst, (float*)((uint8_t*)dst + rows * K), K);
  HIPCHK(c, hipGetLastError());
  return FX_OK;
}

// bf16 rows from FP8 rows (codes then scales, as fx_quantize_fp8 writes them)
int fx_dequantize_fp8(fx_ctx* c, const void* src, void* dst, int64_t rows, int32_t K, void* stream) {
  if (!c) return FX_E_ARG;
  PF_CHECK(c, src && dst && rows > 0 && rows <= 0x7fffffff && K > 0 && K % 16 == 0 && al16(src) && al16(dst),
           "fx_dequantize_fp8: arguments");
  hipLaunchKernelGGL(fx_dequant_fp8_kernel, dim3((unsigned)rows), dim3(PF_THREADS), 0, (hipStream_t)stream,
                     (const uint8_t*)src, (const float*)((const uint8_t*)src + rows * K), (uint16_t*)dst, K);
  HIPCHK(c, hipGetLastError());
  return FX_OK;
}

}  // extern "C"
