// Hardware probes of the gfx950 memory system that the decode kernel's design rests on
// (the reference's env/hw/probes/stream_read.cu, chase.cu and fence_probe.cu, re-written for
// MI355X): the HBM stream rate of the GEMV load pattern as a function of bytes per workgroup and
// loads in flight, the latency of one dependent load per cache policy (idle and under a streaming
// load), and the round trip of a flag between two workgroups on the same or different XCDs.
// Every loop is bounded; nothing here waits on a condition without a tick limit.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <vector>

#include "fx_gemv.h"

#define PROBE_LIMIT (100ull * 1000 * 1000)   // 1 s of s_memrealtime ticks: every wait gives up after it

typedef uint32_t u32x4p __attribute__((ext_vector_type(4)));

// ---- stream: block b reads [b * bytes, (b + 1) * bytes) of src with the GEMV pattern: each wave
// issues `depth` 1 KiB loads (64 lanes x 16 B) before consuming them; stamps per block.
// pattern 0: load d of a wave reads the d-th KiB of its D KiB block; pattern 1: the GEMV tile order,
// D / 4 KiB-chunks of 4 rows of 4 KiB, chunk-major (load d: row d % 4, KiB d / 4); pattern 2: as 1
// with rows 2, 3 taken from the second half of the block (two streams, the gate | up pair layout).
template <int D>
__device__ void stream_body(const uint8_t* src, uint64_t bytes, uint64_t* ticks, uint32_t* sink, int pattern) {
  const uint8_t* base = src + (uint64_t)blockIdx.x * bytes;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  uint32_t acc = 0;
  const uint64_t step = (uint64_t)nw * D * 1024;
  for (uint64_t off = (uint64_t)wave * D * 1024; off < bytes; off += step) {
    u32x4p v[D];
#pragma unroll
    for (int d = 0; d < D; ++d) {
      uint64_t o;
      if (pattern == 0) o = off + (uint64_t)d * 1024;
      else if (pattern == 1) o = off + (uint64_t)(d % 4) * (D / 4) * 1024 + (uint64_t)(d / 4) * 1024;
      else {
        const int r = d % 4;
        o = (off >> 1) + (uint64_t)(r >> 1) * (bytes >> 1) + (uint64_t)(r & 1) * (D / 4) * 1024 + (uint64_t)(d / 4) * 1024;
      }
      o += lane * 16;
      if (o + 16 > bytes) o = lane * 16;
      v[d] = __builtin_nontemporal_load((const u32x4p*)(base + o));
    }
#pragma unroll
    for (int d = 0; d < D; ++d) acc += v[d].x ^ v[d].y ^ v[d].z ^ v[d].w;
  }
  __syncthreads();
  if (threadIdx.x == 0) ticks[blockIdx.x] = __builtin_amdgcn_s_memrealtime() - t0;
  if (acc == 0x12345678u) sink[0] = acc;
}

// double-buffered walk (the GEMV pipeline): tile = D loads of 1 KiB; the next tile is issued before
// the current one is consumed, so between D and 2D loads are in flight per wave
template <int D>
__device__ void stream_db(const uint8_t* src, uint64_t bytes, uint64_t* ticks, uint32_t* sink) {
  const uint8_t* base = src + (uint64_t)blockIdx.x * bytes;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  uint32_t acc = 0;
  const uint64_t step = (uint64_t)nw * D * 1024;
  auto load = [&](u32x4p* v, uint64_t off) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      uint64_t o = off + (uint64_t)d * 1024 + lane * 16;
      if (o + 16 > bytes) o = lane * 16;
      v[d] = __builtin_nontemporal_load((const u32x4p*)(base + o));
    }
  };
  auto use = [&](const u32x4p* v) {
#pragma unroll
    for (int d = 0; d < D; ++d) acc += v[d].x ^ v[d].y ^ v[d].z ^ v[d].w;
  };
  u32x4p a[D], b[D];
  uint64_t off = (uint64_t)wave * D * 1024;
  if (off < bytes) load(a, off);
  while (off < bytes) {
    const uint64_t o1 = off + step;
    if (o1 < bytes) load(b, o1);
    use(a);
    if (o1 >= bytes) break;
    const uint64_t o2 = o1 + step;
    if (o2 < bytes) load(a, o2);
    use(b);
    off = o2;
  }
  __syncthreads();
  if (threadIdx.x == 0) ticks[blockIdx.x] = __builtin_amdgcn_s_memrealtime() - t0;
  if (acc == 0x12345678u) sink[0] = acc;
}

// direct-to-LDS walk: each wave owns a ring of D 1 KiB slots in LDS; load d of the wave's block goes
// to slot d % D via global_load_lds (no VGPRs held), the wave waits until the oldest slot has landed
// (vmcnt(D - 1)), reads it back with ds_read_b128 and refills the slot with load d + D.
#define VMCNT(n) (0x0F70 | ((n) & 15) | (((n) >> 4) << 14))
template <int D>
__device__ void stream_lds(const uint8_t* src, uint64_t bytes, uint64_t* ticks, uint32_t* sink) {
  extern __shared__ __attribute__((aligned(16))) char lds_ring[];
  const uint8_t* base = src + (uint64_t)blockIdx.x * bytes;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __attribute__((address_space(3))) char* ring = (__attribute__((address_space(3))) char*)lds_ring + wave * D * 1024;
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  uint32_t acc = 0;
  // the wave's loads: KiB k = wave, wave + nw, ... of the block
  const int nk = (int)(bytes >> 10);
  int issued = 0, k0 = wave;
  auto issue = [&](int k, int slot) {
    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(base + (uint64_t)k * 1024 + lane * 16),
                                     (__attribute__((address_space(3))) void*)(ring + slot * 1024), 16, 0, 0);
  };
#pragma unroll
  for (int d = 0; d < D; ++d) {
    const int k = wave + d * nw;
    if (k < nk) issue(k, d);
  }
  int d = 0;
  for (int k = k0; k < nk; k += nw, ++d) {
    __builtin_amdgcn_s_waitcnt(VMCNT(D - 1));
    const int slot = d % D;
    const u32x4p v = *(__attribute__((address_space(3))) u32x4p*)(ring + slot * 1024 + lane * 16);
    acc += v.x ^ v.y ^ v.z ^ v.w;
    const int kn = k + D * nw;
    // the slot is refilled only after its value is in registers
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
    if (kn < nk) issue(kn, slot);
    else __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(base + lane * 16),
                                          (__attribute__((address_space(3))) void*)(ring + slot * 1024), 16, 0, 0);
  }
  __builtin_amdgcn_s_waitcnt(VMCNT(0));
  __syncthreads();
  if (threadIdx.x == 0) ticks[blockIdx.x] = __builtin_amdgcn_s_memrealtime() - t0;
  if (acc == 0x12345678u) sink[0] = acc;
  (void)issued;
}

__global__ void fxp_stream_kernel(const uint8_t* src, uint64_t bytes, int depth, uint64_t* ticks, uint32_t* sink,
                                  int pattern) {
  if (pattern == 4) {
    if (depth == 8) stream_lds<8>(src, bytes, ticks, sink);
    else if (depth == 16) stream_lds<16>(src, bytes, ticks, sink);
    else stream_lds<32>(src, bytes, ticks, sink);
    return;
  }
  if (pattern == 3) {
    if (depth == 4) stream_db<4>(src, bytes, ticks, sink);
    else if (depth == 8) stream_db<8>(src, bytes, ticks, sink);
    else stream_db<16>(src, bytes, ticks, sink);
    return;
  }
  switch (depth) {
    case 4: stream_body<4>(src, bytes, ticks, sink, pattern); break;
    case 8: stream_body<8>(src, bytes, ticks, sink, pattern); break;
    case 16: stream_body<16>(src, bytes, ticks, sink, pattern); break;
    default: stream_body<32>(src, bytes, ticks, sink, pattern); break;
  }
}

// ---- chase: block 0 lane 0 follows idx[] for `hops` dependent loads with the chosen policy;
// blocks 1.. stream-read `load` (if non-null) until block 0 is done or a tick limit passes.
__device__ __forceinline__ uint32_t ld_policy(const uint32_t* p, uint32_t i, int mode) {
  if (mode == 1) return __builtin_amdgcn_raw_buffer_load_b32(rsrc(p), i * 4, 0, FX_SC1);
  if (mode == 2) return __builtin_nontemporal_load(p + i);
  return __hip_atomic_load(const_cast<uint32_t*>(p + i), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
}

__global__ void fxp_chase_kernel(const uint32_t* idx, uint32_t hops, int mode, const uint8_t* load, uint64_t load_bytes,
                                 uint32_t* done, uint64_t* out) {
  if (blockIdx.x == 0) {
    if (threadIdx.x == 0) {
      uint32_t j = 0;
      // warm the first access (TLB), then time
      j = ld_policy(idx, j, mode);
      const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
      for (uint32_t h = 0; h < hops; ++h) j = ld_policy(idx, j, mode);
      const uint64_t t1 = __builtin_amdgcn_s_memrealtime();
      out[0] = t1 - t0;
      out[1] = j;
      __hip_atomic_store(done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    return;
  }
  if (!load) return;
  const uint64_t per = load_bytes / gridDim.x;
  const uint8_t* base = load + (uint64_t)blockIdx.x * per;
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  uint32_t acc = 0;
  for (int rep = 0; rep < 1000; ++rep) {
    for (uint64_t off = threadIdx.x * 16; off + 16 * 8 * blockDim.x <= per; off += 16 * 8 * blockDim.x) {
      u32x4p v[8];
#pragma unroll
      for (int d = 0; d < 8; ++d) v[d] = __builtin_nontemporal_load((const u32x4p*)(base + off + (uint64_t)d * 16 * blockDim.x));
#pragma unroll
      for (int d = 0; d < 8; ++d) acc += v[d].x;
    }
    if (__hip_atomic_load(done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ||
        __builtin_amdgcn_s_memrealtime() - t0 > PROBE_LIMIT)
      break;
  }
  if (acc == 0x12345678u) out[2] = acc;
}

// ---- ping-pong between block a and block b (cooperative launch of `grid` blocks): a stores
// flag[0] = i, b waits for it and stores flag[32] = i, a waits; `rounds` round trips, stamped by a.
// Other blocks stream-read `load` while the exchange runs (if non-null).
// mode 0: agent-scope relaxed atomics; 1: buffer loads with sc0 and plain buffer stores; 2: buffer
// loads and stores with sc1 (the packet policy of the decode kernel); 3: plain buffer stores, and
// loads after an invalidate of the CU's L1 (buffer_inv sc0); 4: buffer loads and stores with sc0;
// 5: stores with sc1, loads with sc0; 6: stores with sc0, loads with sc1. Modes 1 and 3..5 are meant
// for a and b on one XCD.
__device__ __forceinline__ uint32_t pp_ld(const uint32_t* p, int mode) {
  if (mode == 0) return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, 64, 0x00020000);
  if (mode == 1 || mode == 4 || mode == 5) return __builtin_amdgcn_raw_buffer_load_b32(r, 0, 0, 1);
  if (mode == 3) {
    asm volatile("buffer_inv sc0" ::: "memory");
    return __builtin_amdgcn_raw_buffer_load_b32(r, 0, 0, 0);
  }
  return __builtin_amdgcn_raw_buffer_load_b32(r, 0, 0, 16);
}
__device__ __forceinline__ void pp_st(uint32_t* p, uint32_t v, int mode) {
  if (mode == 0) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); return; }
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, 64, 0x00020000);
  if (mode == 2 || mode == 5) __builtin_amdgcn_raw_buffer_store_b32(v, r, 0, 0, 16);
  else if (mode == 4 || mode == 6) __builtin_amdgcn_raw_buffer_store_b32(v, r, 0, 0, 1);
  else __builtin_amdgcn_raw_buffer_store_b32(v, r, 0, 0, 0);
}
__global__ void fxp_pingpong_kernel(uint32_t* flag, int a, int b, uint32_t rounds, int mode, const uint8_t* load,
                                    uint64_t load_bytes, uint64_t* out) {
  const int blk = blockIdx.x;
  if (blk == a || blk == b) {
    if (threadIdx.x != 0) return;
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    bool ok = true;
    for (uint32_t i = 1; i <= rounds && ok; ++i) {
      if (blk == a) {
        pp_st(&flag[0], i, mode);
        while (pp_ld(&flag[32], mode) != i)
          if (__builtin_amdgcn_s_memrealtime() - t0 > PROBE_LIMIT) { ok = false; break; }
      } else {
        while (pp_ld(&flag[0], mode) != i)
          if (__builtin_amdgcn_s_memrealtime() - t0 > PROBE_LIMIT) { ok = false; break; }
        pp_st(&flag[32], i, mode);
      }
    }
    out[blk == a ? 3 : 4] = xcc_id();
    if (blk == a) {
      out[0] = __builtin_amdgcn_s_memrealtime() - t0;
      out[1] = ok ? 1 : 0;
      __hip_atomic_store(&flag[64], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    return;
  }
  if (!load) return;
  const uint64_t per = load_bytes / gridDim.x;
  const uint8_t* base = load + (uint64_t)blk * per;
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  uint32_t acc = 0;
  for (int rep = 0; rep < 1000; ++rep) {
    for (uint64_t off = threadIdx.x * 16; off + 16 * 8 * blockDim.x <= per; off += 16 * 8 * blockDim.x) {
      u32x4p v[8];
#pragma unroll
      for (int d = 0; d < 8; ++d) v[d] = __builtin_nontemporal_load((const u32x4p*)(base + off + (uint64_t)d * 16 * blockDim.x));
#pragma unroll
      for (int d = 0; d < 8; ++d) acc += v[d].x;
    }
    if (__hip_atomic_load(&flag[64], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ||
        __builtin_amdgcn_s_memrealtime() - t0 > PROBE_LIMIT)
      break;
  }
  if (acc == 0x12345678u) out[2] = acc;
}

// ---- loaded round trip: blocks a and b ping-pong a flag with sc1 stores and loads (the decode
// kernel's packet policy) for `rounds` round trips while every other block streams its share of
// `load` without a pause: a wave keeps between D and 2D 1 KiB non-temporal loads in flight
// (double-buffered tiles, wrapping over the block's share), so D sets the depth of the memory
// queues the flag's stores and loads meet. Per streaming block: bytes read and ticks until it saw
// the stop flag (bounded by PROBE_LIMIT like every wait here).
template <int D>
__device__ void loaded_stream(const uint8_t* base, uint64_t per, const uint32_t* stop, uint64_t* bytes_out,
                              uint64_t* ticks_out, int work) {
  __shared__ uint64_t wave_bytes[16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const uint64_t step = (uint64_t)nw * D * 1024;
  const uint64_t span = per - per % step;
  uint32_t acc = 0;
  uint64_t off = (uint64_t)wave * D * 1024, nbytes = 0;
  auto load = [&](u32x4p* v, uint64_t o0) {
#pragma unroll
    for (int d = 0; d < D; ++d)
      v[d] = __builtin_nontemporal_load((const u32x4p*)(base + o0 + (uint64_t)d * 1024 + lane * 16));
  };
  // `work` dependent fmas per KiB loaded: the VALU time a GEMV tile spends per KiB
  float f = (float)lane;
  auto use = [&](const u32x4p* v) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      acc += v[d].x ^ v[d].y ^ v[d].z ^ v[d].w;
      for (int k = 0; k < work; ++k) f = __builtin_fmaf(f, 0.999f, __uint_as_float(v[d].x & 0x3f800000u));
    }
  };
  auto next = [&](uint64_t o) { o += step; return o >= span ? o - span : o; };
  u32x4p a[D], b[D];
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  load(a, off);
  for (uint32_t it = 0;; ++it) {
    off = next(off);
    load(b, off);
    use(a);
    off = next(off);
    load(a, off);
    use(b);
    nbytes += 2 * D * 1024;
    if ((it & 7) == 7 && (__hip_atomic_load(stop, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ||
                          __builtin_amdgcn_s_memrealtime() - t0 > PROBE_LIMIT))
      break;
  }
  use(a);
  if (lane == 0) wave_bytes[wave] = nbytes;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t tot = 0;
    for (int w = 0; w < nw; ++w) tot += wave_bytes[w];
    bytes_out[blockIdx.x] = tot;
    ticks_out[blockIdx.x] = __builtin_amdgcn_s_memrealtime() - t0;
  }
  if (acc == 0x12345678u || f == 1234.5f) bytes_out[gridDim.x] = acc;
}

// waves 1 .. of a ping-pong block stream their block's share the same way (self < 0: they exit),
// so the flag's loads share the CU with a stream; no block-wide barrier (wave 0 is elsewhere)
template <int D>
__device__ void self_stream(const uint8_t* base, uint64_t per, const uint32_t* stop) {
  const int lane = threadIdx.x & 63, wave = (threadIdx.x >> 6) - 1, nw = (blockDim.x >> 6) - 1;
  const uint64_t step = (uint64_t)nw * D * 1024;
  const uint64_t span = per - per % step;
  uint32_t acc = 0;
  uint64_t off = (uint64_t)wave * D * 1024;
  auto load = [&](u32x4p* v, uint64_t o0) {
#pragma unroll
    for (int d = 0; d < D; ++d)
      v[d] = __builtin_nontemporal_load((const u32x4p*)(base + o0 + (uint64_t)d * 1024 + lane * 16));
  };
  auto use = [&](const u32x4p* v) {
#pragma unroll
    for (int d = 0; d < D; ++d) acc += v[d].x ^ v[d].y ^ v[d].z ^ v[d].w;
  };
  auto next = [&](uint64_t o) { o += step; return o >= span ? o - span : o; };
  u32x4p a[D], b[D];
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  load(a, off);
  for (uint32_t it = 0;; ++it) {
    off = next(off);
    load(b, off);
    use(a);
    off = next(off);
    load(a, off);
    use(b);
    if ((it & 7) == 7 && (__hip_atomic_load(stop, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ||
                          __builtin_amdgcn_s_memrealtime() - t0 > PROBE_LIMIT))
      break;
  }
  use(a);
  if (acc == 0x12345678u) *(uint32_t*)(base) = acc;
}

__global__ void __launch_bounds__(256) fxp_loaded_kernel(uint32_t* flag, int a, int b, uint32_t rounds, int depth,
                                                         int work, const uint8_t* load, uint64_t load_bytes,
                                                         uint64_t* bytes_out, uint64_t* ticks_out, uint64_t* out) {
  const int blk = blockIdx.x;
  if (blk == a || blk == b) {
    // work < 0: waves 1 .. of the ping-pong blocks stream too (depth -work)
    if (threadIdx.x >= 64) {
      if (work < 0 && load) {
        const uint64_t per = load_bytes / gridDim.x;
        const uint8_t* base = load + (uint64_t)blk * per;
        if (work == -4) self_stream<4>(base, per, &flag[64]);
        else if (work == -8) self_stream<8>(base, per, &flag[64]);
        else self_stream<16>(base, per, &flag[64]);
      }
      return;
    }
    if (threadIdx.x == 0) {
      // a short idle delay so the streams are running before the first round trip
      const uint64_t ts = __builtin_amdgcn_s_memrealtime();
      while (__builtin_amdgcn_s_memrealtime() - ts < 2000) __builtin_amdgcn_s_sleep(8);
      const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
      bool ok = true;
      for (uint32_t i = 1; i <= rounds && ok; ++i) {
        if (blk == a) {
          pp_st(&flag[0], i, 2);
          while (pp_ld(&flag[32], 2) != i)
            if (__builtin_amdgcn_s_memrealtime() - t0 > PROBE_LIMIT) { ok = false; break; }
        } else {
          while (pp_ld(&flag[0], 2) != i)
            if (__builtin_amdgcn_s_memrealtime() - t0 > PROBE_LIMIT) { ok = false; break; }
          pp_st(&flag[32], i, 2);
        }
      }
      if (blk == a) {
        out[0] = __builtin_amdgcn_s_memrealtime() - t0;
        out[1] = ok ? 1 : 0;
        __hip_atomic_store(&flag[64], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    return;
  }
  if (!load || depth == 0) return;
  const uint64_t per = load_bytes / gridDim.x;
  const uint8_t* base = load + (uint64_t)blk * per;
  if (work < 0) work = 0;
  if (depth == 1) loaded_stream<1>(base, per, &flag[64], bytes_out, ticks_out, work);
  else if (depth == 2) loaded_stream<2>(base, per, &flag[64], bytes_out, ticks_out, work);
  else if (depth == 4) loaded_stream<4>(base, per, &flag[64], bytes_out, ticks_out, work);
  else if (depth == 8) loaded_stream<8>(base, per, &flag[64], bytes_out, ticks_out, work);
  else if (depth == 16) loaded_stream<16>(base, per, &flag[64], bytes_out, ticks_out, work);
  else loaded_stream<24>(base, per, &flag[64], bytes_out, ticks_out, work);
}

// ---- the decode GEMV's own walk (fx_gemv.h: Tile<4, 4> over K = 2048, double-buffered, groups of 4
// rows, wave w taking groups w, w + 4, ...) over `rows_per_block` rows per block of W, timed.
// mode 0: tile_dot (the real dot_lanes work); mode 1: the same loads, each tile folded by one xor
// per word (no dot); mode 2: as 1 with every load instruction of a tile reading the next KiB of the
// tile's 16 contiguous KiB (instead of row-interleaved); modes 3, 4: the sliced walk (gemv_slices_x)
// with 2 / 4 slices (4 rows x 1 KiB) in flight per wave; mode 5: the rolling walk (gemv_pipe_roll:
// each chunk column of a tile re-filled with the tile two ahead once its fmas are done); modes 6, 7:
// FP8 rows of K codes (TileQ<4, 2>, the expert stages' FP8 tiles), tile_dot and rolling; modes 8, 9:
// mode 0 with each row's bf16 result stored to `out` as the LM head stores its logits (one 2-byte
// sc1 store per row from lane i, mode 8) or as one 8-byte store of the tile's 4 rows (mode 9); mode
// 10: results into LDS, 8-byte stores after the walk; modes 11, 12: tiles of 2 rows, two-tile and
// rolling walks; modes 13, 14: tiles of 1 row, rolling and two-tile walks.
template <int MODE>
__device__ __forceinline__ void gemv_walk(const uint16_t* W, int K, int r0, int ngroups, const float* xs, float& sink,
                                          void* out) {
  auto rowof = [&](int g, int i) { return r0 + g * 4 + i; };
  if constexpr (MODE == 13 || MODE == 14) {
    // tiles of 1 row (4 KiB per wave): rolling (13) and two-tile (14) walks
    auto row1 = [&](int g, int i) { return r0 + g; };
    Tile<1, 4> t0;
    const int ng1 = ngroups * 4;
    gemv_prime(t0, W, K, ng1, row1);
    auto em = [&](int, const int*, const float* acc) { sink += acc[0]; };
    if constexpr (MODE == 14) gemv_pipe(t0, W, K, xs, ng1, row1, em);
    else gemv_pipe_roll(t0, W, K, [&](int) { return xs; }, ng1, row1, em);
  } else if constexpr (MODE == 11 || MODE == 12) {
    // tiles of 2 rows (8 KiB per wave): the two-tile walk (11) and the rolling walk (12)
    auto row2 = [&](int g, int i) { return r0 + g * 2 + i; };
    Tile<2, 4> t0;
    const int ng2 = ngroups * 2;
    gemv_prime(t0, W, K, ng2, row2);
    auto em = [&](int, const int*, const float* acc) { sink += acc[0] + acc[1]; };
    if constexpr (MODE == 11) gemv_pipe(t0, W, K, xs, ng2, row2, em);
    else gemv_pipe_roll(t0, W, K, [&](int) { return xs; }, ng2, row2, em);
  } else if constexpr (MODE == 10) {
    // the LM head's deferred stores: results into LDS per tile, 8-byte stores after the walk
    __shared__ uint16_t lo16[400];
    Tile<4, 4> t0;
    gemv_prime(t0, W, K, ngroups, rowof);
    gemv_pipe(t0, W, K, xs, ngroups, rowof, [&](int, const int* row, const float* acc) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (lane_id() == i) lo16[row[i] - r0] = (uint16_t)f2bf(acc[i]);
    });
    __syncthreads();
    const int n = ngroups * 4;
    for (int t = threadIdx.x; 4 * t < n && 4 * t < 400; t += 256) {
      u32x2 v;
      v.x = (uint32_t)lo16[4 * t] | ((uint32_t)lo16[4 * t + 1] << 16);
      v.y = (uint32_t)lo16[4 * t + 2] | ((uint32_t)lo16[4 * t + 3] << 16);
      stc8(out, (uint32_t)(r0 + 4 * t) * 2, v);
    }
  } else if constexpr (MODE == 8 || MODE == 9) {
    Tile<4, 4> t0;
    gemv_prime(t0, W, K, ngroups, rowof);
    gemv_pipe(t0, W, K, xs, ngroups, rowof, [&](int, const int* row, const float* acc) {
      const int lane = lane_id();
      uint32_t b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) b[i] = f2bf(acc[i]);
      if constexpr (MODE == 8) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (lane == i) stc2(out, (uint32_t)row[i] * 2, b[i]);
      } else {
        u32x2 v;
        v.x = b[0] | (b[1] << 16);
        v.y = b[2] | (b[3] << 16);
        if (lane == 0) stc8(out, (uint32_t)row[0] * 2, v);
      }
    });
  } else if constexpr (MODE == 0) {
    Tile<4, 4> t0;
    gemv_prime(t0, W, K, ngroups, rowof);
    gemv_pipe(t0, W, K, xs, ngroups, rowof, [&](int, const int*, const float* acc) { sink += acc[0] + acc[1] + acc[2] + acc[3]; });
  } else if constexpr (MODE == 5) {
    Tile<4, 4> t0;
    gemv_prime(t0, W, K, ngroups, rowof);
    gemv_pipe_roll(t0, W, K, [&](int) { return xs; }, ngroups, rowof,
                   [&](int, const int*, const float* acc) { sink += acc[0] + acc[1] + acc[2] + acc[3]; });
  } else if constexpr (MODE == 6 || MODE == 7) {
    // codes [rows][K] at W (scales: any words of the buffer; only the timing is used)
    const Fp8W Q{(const uint8_t*)W, (const float*)W};
    auto rowq = [&](int g, int i) { return r0 + g * 4 + i; };
    TileQ<4, 2> t0;
    gemv_prime(t0, Q, K, ngroups, rowq);
    auto em = [&](int, const int*, const float* acc) { sink += acc[0] + acc[1] + acc[2] + acc[3]; };
    if constexpr (MODE == 6) gemv_pipe(t0, Q, K, xs, ngroups, rowq, em);
    else gemv_pipe_roll(t0, Q, K, [&](int) { return xs; }, ngroups, rowq, em);
  } else if constexpr (MODE >= 3) {
    // the sliced walk with 2 (mode 3) or 4 (mode 4) slices of 4 KiB in flight per wave
    constexpr int D = MODE == 3 ? 2 : 4;
    SliceRing<4, D> q;
    slices_prime<4, 4>(q, W, K, ngroups, rowof);
    gemv_slices_x<4>(q, W, K, [&](int) { return xs; }, ngroups, rowof,
                     [&](int, const int*, const float* acc) { sink += acc[0] + acc[1] + acc[2] + acc[3]; });
  } else {
    auto load = [&](u32x4* v, int g) {
      const uint8_t* base = (const uint8_t*)(W + (size_t)(r0 + g * 4) * K);
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int kib = MODE == 1 ? i * 4 + j : j * 4 + i;
          v[j * 4 + i] = *(const u32x4*)__builtin_assume_aligned(base + (size_t)kib * 1024 + lane_id() * 16, 16);
        }
    };
    uint32_t acc = 0;
    u32x4 a[16], b[16];
    int g = wave_id();
    if (g < ngroups) load(a, g);
    while (g < ngroups) {
      const int g1 = g + FX_WAVES;
      if (g1 < ngroups) load(b, g1);
#pragma unroll
      for (int k = 0; k < 16; ++k) acc ^= a[k].x ^ a[k].y ^ a[k].z ^ a[k].w;
      if (g1 >= ngroups) break;
      const int g2 = g1 + FX_WAVES;
      if (g2 < ngroups) load(a, g2);
#pragma unroll
      for (int k = 0; k < 16; ++k) acc ^= b[k].x ^ b[k].y ^ b[k].z ^ b[k].w;
      g = g2;
    }
    sink += (float)(acc & 1u);
  }
}
__global__ void __launch_bounds__(256) fxp_gemv_kernel(const uint16_t* W, int K, int rows_per_block, int mode,
                                                       uint64_t* ticks, float* out) {
  __shared__ float xs[2048];
  for (int i = threadIdx.x; i < K; i += 256) xs[i] = 0.001f * (float)(i % 7);
  __syncthreads();
  const int r0 = blockIdx.x * rows_per_block, ngroups = rows_per_block / 4;
  float sink = 0.0f;
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  if (mode == 0) gemv_walk<0>(W, K, r0, ngroups, xs, sink, out);
  else if (mode == 1) gemv_walk<1>(W, K, r0, ngroups, xs, sink, out);
  else if (mode == 2) gemv_walk<2>(W, K, r0, ngroups, xs, sink, out);
  else if (mode == 3) gemv_walk<3>(W, K, r0, ngroups, xs, sink, out);
  else if (mode == 4) gemv_walk<4>(W, K, r0, ngroups, xs, sink, out);
  else if (mode == 5) gemv_walk<5>(W, K, r0, ngroups, xs, sink, out);
  else if (mode == 6) gemv_walk<6>(W, K, r0, ngroups, xs, sink, out);
  else if (mode == 7) gemv_walk<7>(W, K, r0, ngroups, xs, sink, out);
  else if (mode == 8) gemv_walk<8>(W, K, r0, ngroups, xs, sink, out);
  else if (mode == 9) gemv_walk<9>(W, K, r0, ngroups, xs, sink, out);
  else if (mode == 10) gemv_walk<10>(W, K, r0, ngroups, xs, sink, out);
  else if (mode == 11) gemv_walk<11>(W, K, r0, ngroups, xs, sink, out);
  else if (mode == 12) gemv_walk<12>(W, K, r0, ngroups, xs, sink, out);
  else if (mode == 13) gemv_walk<13>(W, K, r0, ngroups, xs, sink, out);
  else gemv_walk<14>(W, K, r0, ngroups, xs, sink, out);
  __syncthreads();
  if (threadIdx.x == 0) ticks[blockIdx.x] = __builtin_amdgcn_s_memrealtime() - t0;
  if (sink == 1234.5f) out[0] = sink;
}

// ---- lane exchange check: out[lane * 6 + k] = the value xor_lane<2^k> returns on `lane` when every
// lane holds its own index (must be lane ^ 2^k)
// ---- FP8 decode: the 256 codes through the hardware's packed FP8 -> f32 conversion (lane l: codes
// 4l .. 4l + 3 as one 32-bit word; word_sel false takes bytes 0, 1, true bytes 2, 3)
__global__ void fxp_fp8_kernel(float* out) {
  const int l = threadIdx.x & 63;
  const int src = (4 * l) | ((4 * l + 1) << 8) | ((4 * l + 2) << 16) | ((4 * l + 3) << 24);
  const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(src, false);
  const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(src, true);
  out[4 * l + 0] = lo[0];
  out[4 * l + 1] = lo[1];
  out[4 * l + 2] = hi[0];
  out[4 * l + 3] = hi[1];
}

__global__ void fxp_lanes_kernel(float* out) {
  const float v = (float)(threadIdx.x & 63);
  const int l = threadIdx.x & 63;
  out[l * 6 + 0] = xor_lane<1>(v);
  out[l * 6 + 1] = xor_lane<2>(v);
  out[l * 6 + 2] = xor_lane<4>(v);
  out[l * 6 + 3] = xor_lane<8>(v);
  out[l * 6 + 4] = xor_lane<16>(v);
  out[l * 6 + 5] = xor_lane<32>(v);
}

// ---- shader clock: block 0 runs a dependent VALU chain of `iters` fmas between two stamps of the
// core clock (s_memtime) and the 100 MHz real-time clock; the other blocks stream `load` meanwhile
// (if non-null). out = {core ticks, real ticks, fma chain result bits}
__global__ void fxp_clock_kernel(int iters, const uint8_t* load, uint64_t load_bytes, uint32_t* done, uint64_t* out) {
  if (blockIdx.x == 0) {
    if (threadIdx.x >= 64) return;
    float a = (float)threadIdx.x, b = 1.0000001f;
    const uint64_t c0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
    for (int i = 0; i < iters; ++i) a = __builtin_fmaf(a, b, 1.0f);
    const uint64_t c1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    if (threadIdx.x == 0) {
      out[0] = c1 - c0;
      out[1] = r1 - r0;
      out[2] = __float_as_uint(a);
      __hip_atomic_store(done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    return;
  }
  if (!load) return;
  const uint64_t per = load_bytes / gridDim.x;
  const uint8_t* base = load + (uint64_t)blockIdx.x * per;
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  uint32_t acc = 0;
  for (int rep = 0; rep < 1000; ++rep) {
    for (uint64_t off = threadIdx.x * 16; off + 16 * 8 * blockDim.x <= per; off += 16 * 8 * blockDim.x) {
      u32x4p v[8];
#pragma unroll
      for (int d = 0; d < 8; ++d) v[d] = __builtin_nontemporal_load((const u32x4p*)(base + off + (uint64_t)d * 16 * blockDim.x));
#pragma unroll
      for (int d = 0; d < 8; ++d) acc += v[d].x;
    }
    if (__hip_atomic_load(done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ||
        __builtin_amdgcn_s_memrealtime() - t0 > PROBE_LIMIT)
      break;
  }
  if (acc == 0x12345678u) out[3] = acc;
}

// ---- VALU issue rate of FMA chains, one wave per SIMD (256 threads, one workgroup): 1024 v_fmac_f32
// per lane as one dependent chain, or as 2 / 4 / 8 independent chains interleaved instruction by
// instruction (each chain itself dependent). out[v] = core cycles (s_memtime) of variant v on wave 0.
__global__ void __launch_bounds__(256) fxp_valu_kernel(uint64_t* out, float* sink) {
  float a0 = (float)threadIdx.x, a1 = a0 + 1.0f, a2 = a0 + 2.0f, a3 = a0 + 3.0f, a4 = a0 + 4.0f, a5 = a0 + 5.0f,
        a6 = a0 + 6.0f, a7 = a0 + 7.0f;
  const float b = 1.0000001f, c = 0.5f;
  uint64_t t[5];
  __syncthreads();
  t[0] = __builtin_amdgcn_s_memtime();
  asm volatile(".rept 1024\n v_fmac_f32 %0, %1, %2\n .endr" : "+v"(a0) : "v"(b), "v"(c));
  t[1] = __builtin_amdgcn_s_memtime();
  asm volatile(".rept 512\n v_fmac_f32 %0, %2, %3\n v_fmac_f32 %1, %2, %3\n .endr" : "+v"(a0), "+v"(a1) : "v"(b), "v"(c));
  t[2] = __builtin_amdgcn_s_memtime();
  asm volatile(".rept 256\n v_fmac_f32 %0, %4, %5\n v_fmac_f32 %1, %4, %5\n v_fmac_f32 %2, %4, %5\n v_fmac_f32 %3, %4, %5\n .endr"
               : "+v"(a0), "+v"(a1), "+v"(a2), "+v"(a3) : "v"(b), "v"(c));
  t[3] = __builtin_amdgcn_s_memtime();
  asm volatile(".rept 128\n v_fmac_f32 %0, %8, %9\n v_fmac_f32 %1, %8, %9\n v_fmac_f32 %2, %8, %9\n v_fmac_f32 %3, %8, %9\n"
               " v_fmac_f32 %4, %8, %9\n v_fmac_f32 %5, %8, %9\n v_fmac_f32 %6, %8, %9\n v_fmac_f32 %7, %8, %9\n .endr"
               : "+v"(a0), "+v"(a1), "+v"(a2), "+v"(a3), "+v"(a4), "+v"(a5), "+v"(a6), "+v"(a7) : "v"(b), "v"(c));
  t[4] = __builtin_amdgcn_s_memtime();
  if (threadIdx.x == 0)
    for (int v = 0; v < 4; ++v) out[v] = t[v + 1] - t[v];
  sink[threadIdx.x] = a0 + a1 + a2 + a3 + a4 + a5 + a6 + a7;
}

// ---- instruction fetch: block 0 (256 threads, one wave per SIMD) runs a straight-line block of
// 4096 v_fmac_f32 in the 8-byte encoding (32 KiB of code) twice; the first pass fetches the code
// (cold), the second finds it in the instruction cache. out[0], out[1] = core cycles of the two
// passes on wave 0. The other blocks stream-read `load` meanwhile (if non-null), as in the clock probe.
__global__ void __launch_bounds__(256) fxp_icache_kernel(const uint8_t* load, uint64_t load_bytes, uint32_t* done,
                                                         uint64_t* out, float* sink) {
  if (blockIdx.x == 0) {
    float a = (float)threadIdx.x;
    const float b = 1.0000001f, c = 0.5f;
    uint64_t t[3];
    __syncthreads();
#pragma unroll 1
    for (int pass = 0; pass < 2; ++pass) {
      t[pass] = __builtin_amdgcn_s_memtime();
      asm volatile(".rept 4096\n v_fmac_f32_e64 %0, %1, %2\n .endr" : "+v"(a) : "v"(b), "v"(c));
    }
    t[2] = __builtin_amdgcn_s_memtime();
    if (threadIdx.x == 0) {
      out[0] = t[1] - t[0];
      out[1] = t[2] - t[1];
      __hip_atomic_store(done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    sink[threadIdx.x] = a;
    return;
  }
  if (!load) return;
  const uint64_t per = load_bytes / gridDim.x;
  const uint8_t* base = load + (uint64_t)blockIdx.x * per;
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  uint32_t acc = 0;
  for (int rep = 0; rep < 1000; ++rep) {
    for (uint64_t off = threadIdx.x * 16; off + 16 * 8 * blockDim.x <= per; off += 16 * 8 * blockDim.x) {
      u32x4p v[8];
#pragma unroll
      for (int d = 0; d < 8; ++d) v[d] = __builtin_nontemporal_load((const u32x4p*)(base + off + (uint64_t)d * 16 * blockDim.x));
#pragma unroll
      for (int d = 0; d < 8; ++d) acc += v[d].x;
    }
    if (__hip_atomic_load(done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ||
        __builtin_amdgcn_s_memrealtime() - t0 > PROBE_LIMIT)
      break;
  }
  if (acc == 0x12345678u) out[3] = acc;
}

// ---- v_dot2c_f32_bf16 on given operands: d[i] = dot2(a[i], b[i]) + c[i], a and b two bf16 each
// (low half = element 0); the host compares the results with candidate rounding models.
typedef __bf16 fxp_bf16x2 __attribute__((ext_vector_type(2)));
__global__ void fxp_dot2_kernel(const uint32_t* a, const uint32_t* b, const float* c, float* d, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  d[i] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(fxp_bf16x2, a[i]), __builtin_bit_cast(fxp_bf16x2, b[i]), c[i],
                                         false);
}

// ---- direct-to-LDS layout: one wave loads 2 KiB of src (u32 index values) with two 16-byte
// global_load_lds at LDS offsets 0 and 1024 (the second from src + 1024 + 16 * (63 - lane), lanes
// reversed), then copies the 2 KiB of LDS to dst as they lie
__global__ void fxp_lds_dma_kernel(const uint32_t* src, uint32_t* dst) {
  __shared__ __attribute__((aligned(16))) uint32_t buf[512];
  const int lane = threadIdx.x;
  for (int i = lane; i < 512; i += 64) buf[i] = 0xFFFFFFFFu;
  __syncthreads();
  __attribute__((address_space(3))) char* l = (__attribute__((address_space(3))) char*)(void*)buf;
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)((const char*)src + lane * 16),
                                   (__attribute__((address_space(3))) void*)l, 16, 0, 0);
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)((const char*)src + 1024 + (63 - lane) * 16),
                                   (__attribute__((address_space(3))) void*)(l + 1024), 16, 0, 0);
  __builtin_amdgcn_s_waitcnt(VMCNT(0));
  __syncthreads();
  for (int i = lane; i < 512; i += 64) dst[i] = buf[i];
}

// ---- MFMA bf16 semantics: case = blockIdx.x, one wave runs one v_mfma_f32_16x16x32_bf16 on
// A[case] [16][32], B[case] [32][16] (k rows), C[case] [16][16] and stores D[case] [16][16]. The
// assumed operand layout: lane l holds A[l % 16][8 (l / 16) + i] and B[8 (l / 16) + i][l % 16] for
// i < 8, C and D [4 (l / 16) + j][l % 16] for j < 4 (checked by exact integer cases on the host).
typedef __bf16 fxp_bf16x8 __attribute__((ext_vector_type(8)));
typedef float fxp_f32x4 __attribute__((ext_vector_type(4)));
__global__ void fxp_mfma_kernel(const uint16_t* A, const uint16_t* B, const float* C, float* D) {
  const size_t cs = blockIdx.x;
  const int l = threadIdx.x & 63, r = l & 15, g = l >> 4;
  const uint16_t* a = A + cs * 512;
  const uint16_t* b = B + cs * 512;
  fxp_bf16x8 av, bv;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    av[i] = __builtin_bit_cast(__bf16, a[r * 32 + 8 * g + i]);
    bv[i] = __builtin_bit_cast(__bf16, b[(8 * g + i) * 16 + r]);
  }
  fxp_f32x4 cv;
#pragma unroll
  for (int j = 0; j < 4; ++j) cv[j] = C[cs * 256 + (4 * g + j) * 16 + r];
  const fxp_f32x4 dv = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, cv, 0, 0, 0);
#pragma unroll
  for (int j = 0; j < 4; ++j) D[cs * 256 + (4 * g + j) * 16 + r] = dv[j];
}

// ---- LDS transpose read: LDS holds u16 index values lds[i] = i (8 KiB); lane l issues
// ds_read_b64_tr_b16 at byte offset off[l] (8-byte aligned, < 8 KiB - 8); out[l][0..3] = what it got
typedef short fxp_i16x4 __attribute__((ext_vector_type(4)));
__global__ void fxp_ldstr_kernel(const uint32_t* off, uint16_t* out) {
  __shared__ __attribute__((aligned(16))) uint16_t buf[4096];
  const int l = threadIdx.x & 63;
  for (int i = l; i < 4096; i += 64) buf[i] = (uint16_t)i;
  __syncthreads();
  uint32_t o = off[l];
  if (o > 8192 - 8) o = 0;
  o &= ~7u;
  const fxp_i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) fxp_i16x4*)(
      (__attribute__((address_space(3))) char*)(void*)buf + o));
#pragma unroll
  for (int j = 0; j < 4; ++j) out[l * 4 + j] = (uint16_t)v[j];
}

extern "C" {

// all functions: 0 on success, else the hipError_t value
int fxp_stream(const void* src, uint64_t bytes_per_block, int blocks, int threads, int depth, int pattern,
               uint64_t* ticks_host, float* ms) {
  uint64_t* d_ticks = nullptr;
  uint32_t* sink = nullptr;
  hipEvent_t e0, e1;
  hipError_t e;
  if ((e = hipMalloc(&d_ticks, 8 * blocks)) != hipSuccess) return e;
  if ((e = hipMalloc(&sink, 64)) != hipSuccess) return e;
  (void)hipEventCreate(&e0);
  (void)hipEventCreate(&e1);
  (void)hipEventRecord(e0, 0);
  const unsigned shm = pattern == 4 ? (unsigned)(threads / 64) * depth * 1024 : 0;
  if (shm > 64 * 1024) (void)hipFuncSetAttribute((const void*)fxp_stream_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  hipLaunchKernelGGL(fxp_stream_kernel, dim3(blocks), dim3(threads), shm, 0, (const uint8_t*)src, bytes_per_block, depth,
                     d_ticks, sink, pattern);
  (void)hipEventRecord(e1, 0);
  if ((e = hipEventSynchronize(e1)) != hipSuccess) return e;
  (void)hipEventElapsedTime(ms, e0, e1);
  e = hipMemcpy(ticks_host, d_ticks, 8 * blocks, hipMemcpyDeviceToHost);
  (void)hipFree(d_ticks);
  (void)hipFree(sink);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  return e;
}

int fxp_chase(const uint32_t* idx, uint32_t hops, int mode, const void* load, uint64_t load_bytes, int blocks,
              uint64_t* out_host) {
  uint32_t* done = nullptr;
  uint64_t* out = nullptr;
  hipError_t e;
  if ((e = hipMalloc(&done, 256)) != hipSuccess) return e;
  if ((e = hipMalloc(&out, 64)) != hipSuccess) return e;
  (void)hipMemset(done, 0, 256);
  (void)hipMemset(out, 0, 64);
  void* args[] = {(void*)&idx, &hops, &mode, (void*)&load, &load_bytes, &done, &out};
  if ((e = hipLaunchCooperativeKernel((const void*)fxp_chase_kernel, dim3(blocks), dim3(256), args, 0, 0)) != hipSuccess)
    return e;
  if ((e = hipDeviceSynchronize()) != hipSuccess) return e;
  e = hipMemcpy(out_host, out, 24, hipMemcpyDeviceToHost);
  (void)hipFree(done);
  (void)hipFree(out);
  return e;
}

int fxp_pingpong(int a, int b, uint32_t rounds, int mode, const void* load, uint64_t load_bytes, int blocks,
                 uint64_t* out_host) {
  uint32_t* flag = nullptr;
  uint64_t* out = nullptr;
  hipError_t e;
  if ((e = hipMalloc(&flag, 1024)) != hipSuccess) return e;
  if ((e = hipMalloc(&out, 64)) != hipSuccess) return e;
  (void)hipMemset(flag, 0, 1024);
  (void)hipMemset(out, 0, 64);
  void* args[] = {&flag, &a, &b, &rounds, &mode, (void*)&load, &load_bytes, &out};
  if ((e = hipLaunchCooperativeKernel((const void*)fxp_pingpong_kernel, dim3(blocks), dim3(256), args, 0, 0)) != hipSuccess)
    return e;
  if ((e = hipDeviceSynchronize()) != hipSuccess) return e;
  e = hipMemcpy(out_host, out, 40, hipMemcpyDeviceToHost);
  (void)hipFree(flag);
  (void)hipFree(out);
  return e;
}

// out_host[0] = round-trip ticks for `rounds`, [1] = 1 if every round completed, [2] = bytes the
// streaming blocks read, [3] = their mean ticks until they stopped
int fxp_loaded(int a, int b, uint32_t rounds, int depth, int work, const void* load, uint64_t load_bytes, int blocks,
               int threads, uint64_t* out_host) {
  if (depth != 0 && depth != 1 && depth != 2 && depth != 4 && depth != 8 && depth != 16 && depth != 24) return -1;
  if (a < 0 || b < 0 || a >= blocks || b >= blocks || a == b || threads % 64 || threads > 256 || threads < 128) return -1;
  if (work < 0 && work != -4 && work != -8 && work != -16) return -1;
  uint32_t* flag = nullptr;
  uint64_t *out = nullptr, *bo = nullptr, *to = nullptr;
  hipError_t e;
  if ((e = hipMalloc(&flag, 1024)) != hipSuccess) return e;
  if ((e = hipMalloc(&out, 64)) != hipSuccess) return e;
  if ((e = hipMalloc(&bo, (blocks + 1) * 8)) != hipSuccess) return e;
  if ((e = hipMalloc(&to, blocks * 8)) != hipSuccess) return e;
  (void)hipMemset(flag, 0, 1024);
  (void)hipMemset(out, 0, 64);
  (void)hipMemset(bo, 0, (blocks + 1) * 8);
  (void)hipMemset(to, 0, blocks * 8);
  void* args[] = {&flag, &a, &b, &rounds, &depth, &work, (void*)&load, &load_bytes, &bo, &to, &out};
  if ((e = hipLaunchCooperativeKernel((const void*)fxp_loaded_kernel, dim3(blocks), dim3(threads), args, 0, 0)) !=
      hipSuccess)
    return e;
  if ((e = hipDeviceSynchronize()) != hipSuccess) return e;
  uint64_t o[2];
  std::vector<uint64_t> hb(blocks), ht(blocks);
  if ((e = hipMemcpy(o, out, 16, hipMemcpyDeviceToHost)) != hipSuccess) return e;
  if ((e = hipMemcpy(hb.data(), bo, blocks * 8, hipMemcpyDeviceToHost)) != hipSuccess) return e;
  if ((e = hipMemcpy(ht.data(), to, blocks * 8, hipMemcpyDeviceToHost)) != hipSuccess) return e;
  uint64_t tb = 0, tt = 0, n = 0;
  for (int i = 0; i < blocks; ++i)
    if (i != a && i != b && ht[i]) { tb += hb[i]; tt += ht[i]; ++n; }
  out_host[0] = o[0];
  out_host[1] = o[1];
  out_host[2] = tb;
  out_host[3] = n ? tt / n : 0;
  (void)hipFree(flag);
  (void)hipFree(out);
  (void)hipFree(bo);
  (void)hipFree(to);
  return 0;
}

// the GEMV walk over rows_per_block * blocks rows of W [rows][K] (K = 2048, rows_per_block a multiple
// of 4): per-block ticks and the launch's event time
int fxp_gemv(const void* W, int K, int rows_per_block, int blocks, int mode, uint64_t* ticks_host, float* ms) {
  if (K != 2048 || rows_per_block % 4 || mode < 0 || mode > 14 || blocks <= 0) return -1;
  if (mode == 10 && rows_per_block > 400) return -1;
  uint64_t* d_ticks = nullptr;
  float* out = nullptr;
  hipEvent_t e0, e1;
  hipError_t e;
  if ((e = hipMalloc(&d_ticks, 8 * blocks)) != hipSuccess) return e;
  // the walks' outputs (modes 8, 9: one bf16 per row)
  if ((e = hipMalloc(&out, (size_t)rows_per_block * blocks * 2 + 64)) != hipSuccess) return e;
  (void)hipEventCreate(&e0);
  (void)hipEventCreate(&e1);
  (void)hipEventRecord(e0, 0);
  hipLaunchKernelGGL(fxp_gemv_kernel, dim3(blocks), dim3(256), 0, 0, (const uint16_t*)W, K, rows_per_block, mode,
                     d_ticks, out);
  (void)hipEventRecord(e1, 0);
  if ((e = hipEventSynchronize(e1)) != hipSuccess) return e;
  (void)hipEventElapsedTime(ms, e0, e1);
  e = hipMemcpy(ticks_host, d_ticks, 8 * blocks, hipMemcpyDeviceToHost);
  (void)hipFree(d_ticks);
  (void)hipFree(out);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  return e;
}

int fxp_dot2(const uint32_t* a_host, const uint32_t* b_host, const float* c_host, float* d_host, int n) {
  uint32_t *a = nullptr, *b = nullptr;
  float *c = nullptr, *d = nullptr;
  hipError_t e;
  const size_t by = (size_t)n * 4;
  if ((e = hipMalloc(&a, by)) != hipSuccess) return e;
  if ((e = hipMalloc(&b, by)) != hipSuccess) return e;
  if ((e = hipMalloc(&c, by)) != hipSuccess) return e;
  if ((e = hipMalloc(&d, by)) != hipSuccess) return e;
  if ((e = hipMemcpy(a, a_host, by, hipMemcpyHostToDevice)) != hipSuccess) return e;
  if ((e = hipMemcpy(b, b_host, by, hipMemcpyHostToDevice)) != hipSuccess) return e;
  if ((e = hipMemcpy(c, c_host, by, hipMemcpyHostToDevice)) != hipSuccess) return e;
  hipLaunchKernelGGL(fxp_dot2_kernel, dim3((n + 255) / 256), dim3(256), 0, 0, a, b, c, d, n);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  if ((e = hipDeviceSynchronize()) != hipSuccess) return e;
  e = hipMemcpy(d_host, d, by, hipMemcpyDeviceToHost);
  (void)hipFree(a);
  (void)hipFree(b);
  (void)hipFree(c);
  (void)hipFree(d);
  return e;
}

int fxp_icache(const void* load, uint64_t load_bytes, uint64_t* out_host) {
  uint64_t* out = nullptr;
  uint32_t* done = nullptr;
  float* sink = nullptr;
  hipError_t e;
  if ((e = hipMalloc(&out, 64)) != hipSuccess) return e;
  if ((e = hipMalloc(&done, 256)) != hipSuccess) return e;
  if ((e = hipMalloc(&sink, 1024)) != hipSuccess) return e;
  (void)hipMemset(done, 0, 256);
  void* args[] = {(void*)&load, &load_bytes, &done, &out, &sink};
  if ((e = hipLaunchCooperativeKernel((const void*)fxp_icache_kernel, dim3(256), dim3(256), args, 0, 0)) != hipSuccess)
    return e;
  if ((e = hipDeviceSynchronize()) != hipSuccess) return e;
  e = hipMemcpy(out_host, out, 16, hipMemcpyDeviceToHost);
  (void)hipFree(out);
  (void)hipFree(done);
  (void)hipFree(sink);
  return e;
}

int fxp_valu(uint64_t* out_host) {
  uint64_t* out = nullptr;
  float* sink = nullptr;
  hipError_t e;
  if ((e = hipMalloc(&out, 64)) != hipSuccess) return e;
  if ((e = hipMalloc(&sink, 1024)) != hipSuccess) return e;
  hipLaunchKernelGGL(fxp_valu_kernel, dim3(1), dim3(256), 0, 0, out, sink);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  if ((e = hipDeviceSynchronize()) != hipSuccess) return e;
  e = hipMemcpy(out_host, out, 32, hipMemcpyDeviceToHost);
  (void)hipFree(out);
  (void)hipFree(sink);
  return e;
}

int fxp_lanes(float* out_host) {
  float* d = nullptr;
  hipError_t e;
  if ((e = hipMalloc(&d, 64 * 6 * 4)) != hipSuccess) return e;
  hipLaunchKernelGGL(fxp_lanes_kernel, dim3(1), dim3(64), 0, 0, d);
  if ((e = hipDeviceSynchronize()) != hipSuccess) return e;
  e = hipMemcpy(out_host, d, 64 * 6 * 4, hipMemcpyDeviceToHost);
  (void)hipFree(d);
  return e;
}

int fxp_clock(int iters, const void* load, uint64_t load_bytes, uint64_t* out_host) {
  uint32_t* done = nullptr;
  uint64_t* out = nullptr;
  hipError_t e;
  if ((e = hipMalloc(&done, 256)) != hipSuccess) return e;
  if ((e = hipMalloc(&out, 64)) != hipSuccess) return e;
  (void)hipMemset(done, 0, 256);
  void* args[] = {&iters, (void*)&load, &load_bytes, &done, &out};
  if ((e = hipLaunchCooperativeKernel((const void*)fxp_clock_kernel, dim3(256), dim3(256), args, 0, 0)) != hipSuccess) return e;
  if ((e = hipDeviceSynchronize()) != hipSuccess) return e;
  e = hipMemcpy(out_host, out, 24, hipMemcpyDeviceToHost);
  (void)hipFree(done);
  (void)hipFree(out);
  return e;
}

int fxp_fp8(float* out_host) {
  float* d = nullptr;
  hipError_t e;
  if ((e = hipMalloc(&d, 256 * 4)) != hipSuccess) return e;
  hipLaunchKernelGGL(fxp_fp8_kernel, dim3(1), dim3(64), 0, 0, d);
  if ((e = hipDeviceSynchronize()) != hipSuccess) return e;
  e = hipMemcpy(out_host, d, 256 * 4, hipMemcpyDeviceToHost);
  (void)hipFree(d);
  return e;
}

int fxp_lds_dma(uint32_t* out_host) {
  uint32_t *src = nullptr, *dst = nullptr;
  hipError_t e;
  if ((e = hipMalloc(&src, 2048)) != hipSuccess) return e;
  if ((e = hipMalloc(&dst, 2048)) != hipSuccess) return e;
  uint32_t h[512];
  for (int i = 0; i < 512; ++i) h[i] = (uint32_t)i;
  if ((e = hipMemcpy(src, h, 2048, hipMemcpyHostToDevice)) != hipSuccess) return e;
  hipLaunchKernelGGL(fxp_lds_dma_kernel, dim3(1), dim3(64), 0, 0, (const uint32_t*)src, dst);
  if ((e = hipDeviceSynchronize()) != hipSuccess) return e;
  e = hipMemcpy(out_host, dst, 2048, hipMemcpyDeviceToHost);
  (void)hipFree(src);
  (void)hipFree(dst);
  return e;
}

// n_cases MFMA cases (host arrays: A, B n_cases * 512 bf16 bits, C, D n_cases * 256 f32)
int fxp_mfma(const uint16_t* A, const uint16_t* B, const float* C, float* D, int n_cases) {
  if (n_cases <= 0 || n_cases > (1 << 20)) return (int)hipErrorInvalidValue;
  uint16_t *dA = nullptr, *dB = nullptr;
  float *dC = nullptr, *dD = nullptr;
  hipError_t e;
  const size_t n = (size_t)n_cases;
  if ((e = hipMalloc(&dA, n * 1024)) != hipSuccess) return e;
  if ((e = hipMalloc(&dB, n * 1024)) != hipSuccess) return e;
  if ((e = hipMalloc(&dC, n * 1024)) != hipSuccess) return e;
  if ((e = hipMalloc(&dD, n * 1024)) != hipSuccess) return e;
  if ((e = hipMemcpy(dA, A, n * 1024, hipMemcpyHostToDevice)) != hipSuccess) return e;
  if ((e = hipMemcpy(dB, B, n * 1024, hipMemcpyHostToDevice)) != hipSuccess) return e;
  if ((e = hipMemcpy(dC, C, n * 1024, hipMemcpyHostToDevice)) != hipSuccess) return e;
  hipLaunchKernelGGL(fxp_mfma_kernel, dim3(n_cases), dim3(64), 0, 0, (const uint16_t*)dA, (const uint16_t*)dB,
                     (const float*)dC, dD);
  if ((e = hipDeviceSynchronize()) != hipSuccess) return e;
  e = hipMemcpy(D, dD, n * 1024, hipMemcpyDeviceToHost);
  (void)hipFree(dA);
  (void)hipFree(dB);
  (void)hipFree(dC);
  (void)hipFree(dD);
  return e;
}

// one wave of ds_read_b64_tr_b16 at the 64 byte offsets off_host; out_host: 64 x 4 u16
int fxp_ldstr(const uint32_t* off_host, uint16_t* out_host) {
  uint32_t* d_off = nullptr;
  uint16_t* d_out = nullptr;
  hipError_t e;
  if ((e = hipMalloc(&d_off, 256)) != hipSuccess) return e;
  if ((e = hipMalloc(&d_out, 512)) != hipSuccess) return e;
  if ((e = hipMemcpy(d_off, off_host, 256, hipMemcpyHostToDevice)) != hipSuccess) return e;
  hipLaunchKernelGGL(fxp_ldstr_kernel, dim3(1), dim3(64), 0, 0, (const uint32_t*)d_off, d_out);
  if ((e = hipDeviceSynchronize()) != hipSuccess) return e;
  e = hipMemcpy(out_host, d_out, 512, hipMemcpyDeviceToHost);
  (void)hipFree(d_off);
  (void)hipFree(d_out);
  return e;
}

}  // extern "C"
