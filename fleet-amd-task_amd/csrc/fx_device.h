// Device primitives of the gfx950 decode path: bf16, the FP32 arithmetic spec (fixed summation
// orders, own exp/log), coherent (agent-scope, sc1) activation access and weight streaming.
//
// Arithmetic spec shared with the CPU oracle (oracle/fleet_oracle.c), all FP32 IEEE RNE, compiled
// with -ffp-contract=off so every written multiply and add rounds on its own:
//   bf16r        round to nearest even                      (harness/numpy_ref.py:36-42)
//   dot_lanes    chunk c of 8 contiguous elements -> lane c % 64, one fma per element in increasing
//                c, then an xor butterfly over min(64, pow2ceil(chunks)) lanes, offsets 1, 2, .., 32
//   exp_s/log_s  Cody-Waite range reduction + Taylor polynomial (below)
//   silu_s       x / (1 + exp_s(-x))                           (harness/numpy_ref.py:248-253)
//
// Coherence model (measured on MI355X): the eight XCD L2s are not coherent with each other and the
// agent-scope fences (buffer_wbl2 / buffer_inv) cost microseconds when 256 workgroups issue them.
// Every value one workgroup writes and another reads is therefore stored and loaded with the sc1
// cache policy (agent-coherent, bypassing the non-coherent cache levels) and ordered with
// s_waitcnt; weights and other read-only tensors use ordinary (non-temporal) loads.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define FX_THREADS 256
#define FX_WAVES 4
#define FX_XCDS 8
#define FX_LDS_BYTES (96 * 1024)
#define FX_TIMEOUT_TICKS (200ull * 1000 * 1000)   // 2 s of s_memrealtime: a wait this long fails the run

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ------------------------------------------------------------------------------------------------
// bf16

__device__ __forceinline__ float bf2f(uint32_t u16) { return __uint_as_float(u16 << 16); }
__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ uint32_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  u = u + 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}
__device__ __forceinline__ float bf16r(float f) { return bf2f(f2bf(f)); }
__device__ __forceinline__ uint32_t pack2(float lo, float hi) { return f2bf(lo) | (f2bf(hi) << 16); }

// ------------------------------------------------------------------------------------------------
// spec exp / log / silu (identical operation sequence to oracle/fleet_oracle.c)

__device__ __forceinline__ float exp_s(float x) {
  if (!(x >= -87.0f)) return 0.0f;
  if (x > 88.0f) return __uint_as_float(0x7f800000u);
  const float LOG2E = 1.44269504088896341f;
  const float LN2_HI = 0.693145751953125f;
  const float LN2_LO = 1.42860682030941723e-06f;
  float t = x * LOG2E;
  float n = __builtin_rintf(t);
  float r = x - n * LN2_HI;
  r = r - n * LN2_LO;
  float p = 1.3888889e-3f;
  p = p * r + 8.3333333e-3f;
  p = p * r + 4.1666668e-2f;
  p = p * r + 1.6666667e-1f;
  p = p * r + 0.5f;
  p = p * r + 1.0f;
  p = p * r + 1.0f;
  int ni = (int)n;
  float scale = __uint_as_float((uint32_t)(ni + 127) << 23);
  return p * scale;
}

__device__ __forceinline__ float log_s(float x) {
  uint32_t u = __float_as_uint(x);
  int e = (int)((u >> 23) & 0xffu) - 127;
  float m = __uint_as_float((u & 0x007fffffu) | 0x3f800000u);
  if (m > 1.41421356f) { m = m * 0.5f; e = e + 1; }
  float f = m - 1.0f;
  float s = f / (2.0f + f);
  float z = s * s;
  float p = 0.22222222f;
  p = p * z + 0.28571429f;
  p = p * z + 0.4f;
  p = p * z + 0.66666669f;
  p = p * z + 2.0f;
  float lm = s * p;
  const float LN2 = 0.693147182f;
  return (float)e * LN2 + lm;
}

__device__ __forceinline__ float silu_s(float x) { return x / (1.0f + exp_s(-x)); }

// ------------------------------------------------------------------------------------------------
// coherent (sc1) access to activations through buffer resources; byte offsets

// The base must be the same on every lane of the wave (every caller passes a stage-table pointer or
// a kernel argument plus a uniform offset; per-lane addressing goes in the byte offset). It is made
// provably uniform here: the stage table lives in LDS, so its pointers arrive in vector registers,
// and without this the compiler wraps every buffer access in a loop over the distinct bases.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p) {
  const uint64_t a = (uint64_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  void* u = (void*)(((uint64_t)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(u, (short)0, 0x7fffffff, 0x00020000);
}
#define FX_SC1 16
__device__ __forceinline__ u32x4 ldc16(const void* base, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(rsrc(base), off, 0, FX_SC1);
}
__device__ __forceinline__ u32x2 ldc8(const void* base, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b64(rsrc(base), off, 0, FX_SC1);
}
__device__ __forceinline__ uint32_t ldc4(const void* base, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(rsrc(base), off, 0, FX_SC1);
}
__device__ __forceinline__ uint32_t ldc2(const void* base, uint32_t off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rsrc(base), off, 0, FX_SC1);
}
__device__ __forceinline__ void stc16(void* base, uint32_t off, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, rsrc(base), off, 0, FX_SC1);
}
__device__ __forceinline__ void stc8(void* base, uint32_t off, u32x2 v) {
  __builtin_amdgcn_raw_buffer_store_b64(v, rsrc(base), off, 0, FX_SC1);
}
__device__ __forceinline__ void stc4(void* base, uint32_t off, uint32_t v) {
  __builtin_amdgcn_raw_buffer_store_b32(v, rsrc(base), off, 0, FX_SC1);
}
__device__ __forceinline__ void stc2(void* base, uint32_t off, uint32_t v) {
  __builtin_amdgcn_raw_buffer_store_b16((unsigned short)v, rsrc(base), off, 0, FX_SC1);
}
// XCD-local stores (sc0): the data stays in this XCD's L2, where the sc1 loads of workgroups on the
// same XCD find it (a flag round trip this way takes ~0.63 us, idle or under a full-chip weight
// stream, against 1.0 / 2.8 us with sc1 stores); workgroups on other XCDs do not see it until the
// line leaves the L2. Used only for data whose every reader runs on the writer's XCD.
#define FX_SC0 1
__device__ __forceinline__ void stl16(void* base, uint32_t off, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, rsrc(base), off, 0, FX_SC0);
}
__device__ __forceinline__ void stl8(void* base, uint32_t off, u32x2 v) {
  __builtin_amdgcn_raw_buffer_store_b64(v, rsrc(base), off, 0, FX_SC0);
}
__device__ __forceinline__ void stl4(void* base, uint32_t off, uint32_t v) {
  __builtin_amdgcn_raw_buffer_store_b32(v, rsrc(base), off, 0, FX_SC0);
}
__device__ __forceinline__ float ldcf(const void* base, uint32_t idx) { return __uint_as_float(ldc4(base, idx * 4)); }
__device__ __forceinline__ void stcf(void* base, uint32_t idx, float v) { stc4(base, idx * 4, __float_as_uint(v)); }

// flags (agent scope, relaxed)
__device__ __forceinline__ uint32_t flag_ld(const uint32_t* p) {
  return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void flag_st(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void wait_mem() { __builtin_amdgcn_s_waitcnt(0); }

// ------------------------------------------------------------------------------------------------
// packets: 8 bytes = 32-bit payload | 32-bit tag of the producing stage. Stored and loaded with
// sc1, two packets per 16-byte access (the tag of each packet is checked on its own).

// local: every reader of the packet runs on this XCD (stored with sc0, see stl16)
__device__ __forceinline__ void pk_put(void* base, uint32_t pkt, uint32_t payload, uint32_t tag, bool local = false) {
  u32x2 v;
  v.x = payload;
  v.y = tag;
  if (local) stl8(base, pkt * 8u, v);
  else stc8(base, pkt * 8u, v);
}
// packets pkt, pkt + 1 (pkt even)
__device__ __forceinline__ void pk_put2(void* base, uint32_t pkt, uint32_t p0, uint32_t p1, uint32_t tag,
                                        bool local = false) {
  u32x4 v;
  v.x = p0;
  v.y = tag;
  v.z = p1;
  v.w = tag;
  if (local) stl16(base, pkt * 8u, v);
  else stc16(base, pkt * 8u, v);
}

// Wait until packets pkt, pkt + 1 (pkt even) carry `tag`; returns them (payloads in .x, .z).
// Gives up after FX_TIMEOUT_TICKS and raises the run's error flag; once the flag is up every wait
// returns at once, so the grid drains.
__device__ __forceinline__ u32x4 pk_wait2(const void* base, uint32_t pkt, uint32_t tag, uint32_t* err) {
  u32x4 v = ldc16(base, pkt * 8u);
  if (v.y == tag && v.w == tag) return v;
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  for (uint32_t spin = 1;; ++spin) {
    __builtin_amdgcn_s_sleep(1);
    v = ldc16(base, pkt * 8u);
    if (v.y == tag && v.w == tag) break;
    if ((spin & 63u) == 0) {
      if (__builtin_amdgcn_s_memrealtime() - t0 > FX_TIMEOUT_TICKS) {
        __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      if (__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) break;
    }
  }
  return v;
}
// Poll the packet pairs q = first + n * stride (n < N, q < npairs; pair q = packets 2q, 2q + 1)
// until each carries `tag`; out[n] receives pair n (payloads in .x, .z). Every round issues the
// loads of all pending pairs before checking any of them.
template <int N>
__device__ __forceinline__ void pk_wait_pairs(const void* base, int first, int stride, int npairs, uint32_t tag,
                                              uint32_t* err, u32x4* out) {
  uint32_t pending = 0;
#pragma unroll
  for (int n = 0; n < N; ++n)
    if (first + n * stride < npairs) pending |= 1u << n;
  uint64_t t0 = 0;
  for (uint32_t round = 0; pending != 0u; ++round) {
#pragma unroll
    for (int n = 0; n < N; ++n)
      if (pending & (1u << n)) out[n] = ldc16(base, (uint32_t)(first + n * stride) * 16u);
#pragma unroll
    for (int n = 0; n < N; ++n)
      if ((pending & (1u << n)) && out[n].y == tag && out[n].w == tag) pending &= ~(1u << n);
    if (pending == 0u) break;
    if (round == 0) t0 = __builtin_amdgcn_s_memrealtime();
    __builtin_amdgcn_s_sleep(1);
    if ((round & 15u) == 15u) {
      if (__builtin_amdgcn_s_memrealtime() - t0 > FX_TIMEOUT_TICKS) {
        __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      if (__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) break;
    }
  }
}

// Poll the single packets first + n * stride (n < N, index < npkts) until each carries `tag`
// (every round issues the loads of all pending packets before checking any of them).
template <int N>
__device__ __forceinline__ void pk_wait_singles(const void* base, int first, int stride, int npkts, uint32_t tag,
                                                uint32_t* err) {
  uint32_t pending = 0;
#pragma unroll
  for (int n = 0; n < N; ++n)
    if (first + n * stride < npkts) pending |= 1u << n;
  uint64_t t0 = 0;
  for (uint32_t round = 0; pending != 0u; ++round) {
    u32x2 v[N];
#pragma unroll
    for (int n = 0; n < N; ++n)
      if (pending & (1u << n)) v[n] = ldc8(base, (uint32_t)(first + n * stride) * 8u);
#pragma unroll
    for (int n = 0; n < N; ++n)
      if ((pending & (1u << n)) && v[n].y == tag) pending &= ~(1u << n);
    if (pending == 0u) break;
    if (round == 0) t0 = __builtin_amdgcn_s_memrealtime();
    __builtin_amdgcn_s_sleep(1);
    if ((round & 15u) == 15u) {
      if (__builtin_amdgcn_s_memrealtime() - t0 > FX_TIMEOUT_TICKS) {
        __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      if (__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) break;
    }
  }
}

// one packet (any index): payload
__device__ __forceinline__ uint32_t pk_wait1(const void* base, uint32_t pkt, uint32_t tag, uint32_t* err) {
  u32x2 v = ldc8(base, pkt * 8u);
  if (v.y == tag) return v.x;
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  for (uint32_t spin = 1;; ++spin) {
    __builtin_amdgcn_s_sleep(1);
    v = ldc8(base, pkt * 8u);
    if (v.y == tag) break;
    if ((spin & 63u) == 0) {
      if (__builtin_amdgcn_s_memrealtime() - t0 > FX_TIMEOUT_TICKS) {
        __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      if (__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) break;
    }
  }
  return v.x;
}

// weights: read-only for the whole dispatch, streamed once -> non-temporal 16-byte loads. Global
// (address space 1) loads, not flat: a flat load also counts against the LDS counter, so every LDS
// access would wait for the weight loads still in flight.
typedef const __attribute__((address_space(1))) u32x4* gptr16;
__device__ __forceinline__ u32x4 ldw16(const void* p) { return __builtin_nontemporal_load((gptr16)p); }
// Keeps the loads issued before it where the source issues them. Without it the compiler may sink a
// prefetch (the next weight tile, the next cache rows) past the packet polls and barriers that
// follow, down to its first use: the load then starts only when its data is needed and its whole
// latency is exposed. An empty asm with a memory clobber is a compiler-only fence: it emits no
// instruction and no wait.
__device__ __forceinline__ void fx_issue_here() { asm volatile("" ::: "memory"); }
__device__ __forceinline__ u32x4 ld16(const void* p) { return *(gptr16)p; }

// ------------------------------------------------------------------------------------------------
// identity

__device__ __forceinline__ uint32_t xcc_id() {
  uint32_t x;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
  return x & 15u;
}
// The thread index as a value the compiler cannot hoist out of the persistent kernel's loops: the
// empty volatile asm makes every use a fresh value, so each per-thread address is computed inside
// the stage that uses it instead of living in registers (or scratch) across every stage of the
// iteration. The operators use fx_tid() wherever they would use threadIdx.x.
__device__ __forceinline__ int fx_tid() {
  int t = (int)__builtin_amdgcn_workitem_id_x();
  asm volatile("" : "+v"(t));
  return t;
}
__device__ __forceinline__ int lane_id() { return fx_tid() & 63; }
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(fx_tid() >> 6); }

// ------------------------------------------------------------------------------------------------
// reductions

__device__ __forceinline__ float shfl_xor_f(float v, int m) { return __shfl_xor(v, m, 64); }

// Value of lane (lane ^ o) for o = 1, 2, 4, 8 (DPP inside a row of 16), 16 and 32 (the gfx950 row
// swaps), all on the VALU: no LDS instruction, so no wait on outstanding flat/LDS counters.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
template <int O>
__device__ __forceinline__ float xor_lane(float v) {
  if constexpr (O == 1) return dpp_mov<0xB1>(v);          // quad_perm [1,0,3,2]
  else if constexpr (O == 2) return dpp_mov<0x4E>(v);     // quad_perm [2,3,0,1]
  else if constexpr (O == 4) {
    // row_half_mirror (lane i of 8 <- 7 - i = i ^ 7), then quad_perm [3,2,1,0] (i <- i ^ 3): i ^ 4
    return dpp_mov<0x1B>(dpp_mov<0x141>(v));
  } else if constexpr (O == 8) return dpp_mov<0x128>(v);  // row_ror:8 (lane ^ 8 inside 16)
  else if constexpr (O == 16) {
    // odd rows of the first operand <-> even rows of the second: [0] = rows (0, 0, 2, 2), [1] = (1, 1, 3, 3)
    const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v),
                                                    false, false);
    return __builtin_bit_cast(float, (fx_tid() & 16) ? r[0] : r[1]);
  } else {
    // upper half of the first operand <-> lower half of the second
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v),
                                                    false, false);
    return __builtin_bit_cast(float, (fx_tid() & 32) ? r[0] : r[1]);
  }
}

// Both outputs of the row swap of v with itself (as floats in o0, o1): per lane, one holds the
// lane's own value and the other its partner's (lane ^ 16, or lane ^ 32). Each output goes through
// a scalar (__uint_as_float by value): __builtin_bit_cast of a vector element reads the vector's
// first element whatever the index, so both outputs would come out as the first.
template <int O>
__device__ __forceinline__ void swap_pair(float v, float& o0, float& o1) {
  const unsigned a = __float_as_uint(v);
  if constexpr (O == 16) {
    const auto t = __builtin_amdgcn_permlane16_swap(a, a, false, false);
    const unsigned t0 = t[0], t1 = t[1];
    o0 = __uint_as_float(t0);
    o1 = __uint_as_float(t1);
  } else {
    const auto t = __builtin_amdgcn_permlane32_swap(a, a, false, false);
    const unsigned t0 = t[0], t1 = t[1];
    o0 = __uint_as_float(t0);
    o1 = __uint_as_float(t1);
  }
}
// v + xor_lane<O>(v) on every lane. For O = 16 / 32 the sum of the swap's two outputs is the lane's
// own value plus its partner's on every lane: IEEE addition is commutative, so this is bit for bit
// the same sum, without the per-lane select of xor_lane.
template <int O>
__device__ __forceinline__ float add_xor(float v) {
  if constexpr (O == 16 || O == 32) {
    float o0, o1;
    swap_pair<O>(v, o0, o1);
    return o0 + o1;
  } else {
    return v + xor_lane<O>(v);
  }
}
// max(v, xor_lane<O>(v)) on every lane (the same select-free form; max is commutative)
template <int O>
__device__ __forceinline__ float max_xor(float v) {
  if constexpr (O == 16 || O == 32) {
    float o0, o1;
    swap_pair<O>(v, o0, o1);
    return fmaxf(o0, o1);
  } else {
    return fmaxf(v, xor_lane<O>(v));
  }
}

// xor butterfly over the lowest `nl` lanes of each 64-lane group (spec order 1, 2, 4, ..): the
// balanced pairwise tree over lanes; every lane ends with the same sum
__device__ __forceinline__ float butterfly(float v, int nl) {
  if (nl > 1) v = add_xor<1>(v);
  if (nl > 2) v = add_xor<2>(v);
  if (nl > 4) v = add_xor<4>(v);
  if (nl > 8) v = add_xor<8>(v);
  if (nl > 16) v = add_xor<16>(v);
  if (nl > 32) v = add_xor<32>(v);
  return v;
}
// the same over all 64 lanes, with no test (nl is a runtime value in butterfly: each test would be
// a branch per row and level)
__device__ __forceinline__ float butterfly64(float v) {
  v = add_xor<1>(v);
  v = add_xor<2>(v);
  v = add_xor<4>(v);
  v = add_xor<8>(v);
  v = add_xor<16>(v);
  return add_xor<32>(v);
}
__device__ __forceinline__ int lanes_for(int nchunk) {
  int nl = 1;
  while (nl < nchunk && nl < 64) nl <<= 1;
  return nl;
}
__device__ __forceinline__ float wave_max(float v) {
  v = max_xor<1>(v);
  v = max_xor<2>(v);
  v = max_xor<4>(v);
  v = max_xor<8>(v);
  v = max_xor<16>(v);
  return max_xor<32>(v);
}

// 8 fma of a bf16 chunk (4 words) with 8 f32 values, chunk order e = 0..7
__device__ __forceinline__ float fma8(u32x4 w, const float* x, float acc) {
  acc = __builtin_fmaf(bf_lo(w.x), x[0], acc);
  acc = __builtin_fmaf(bf_hi(w.x), x[1], acc);
  acc = __builtin_fmaf(bf_lo(w.y), x[2], acc);
  acc = __builtin_fmaf(bf_hi(w.y), x[3], acc);
  acc = __builtin_fmaf(bf_lo(w.z), x[4], acc);
  acc = __builtin_fmaf(bf_hi(w.z), x[5], acc);
  acc = __builtin_fmaf(bf_lo(w.w), x[6], acc);
  acc = __builtin_fmaf(bf_hi(w.w), x[7], acc);
  return acc;
}

// dot_lanes of a vector held in LDS (f32, K values) with itself: one wave, result on all lanes
__device__ __forceinline__ float sumsq_wave(const float* xs, int K) {
  const int lane = lane_id();
  const int nchunk = K >> 3;
  float acc = 0.0f;
  for (int c = lane; c < nchunk; c += 64) {
    const float* p = xs + c * 8;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc = __builtin_fmaf(p[e], p[e], acc);
  }
  return butterfly(acc, lanes_for(nchunk));
}
