// Batched prefill kernels: the row-wise work between the GEMMs of a prompt's forward pass over
// M positions at once (the GEMMs themselves are rocBLAS calls, fx_gemm). Every kernel takes one
// row per workgroup (the router one row per wave) and rounds at the decode spec's points with
// the decode path's own device functions (rmsnorm_inplace, rope64, exp_s, silu_s,
// softmax_topk_wave), so a row's norm, RoPE, SiLU and routing are the decode's functions of the
// same inputs; only the GEMM and attention reductions run in another order.
#pragma once
#include "fx_ops.h"

#define PF_THREADS 256

// x[m] = W_embed[tokens[m]] (H bf16 per row, H % 8 == 0)
__global__ void __launch_bounds__(PF_THREADS) pf_embed_kernel(const int64_t* tokens, const uint16_t* W, uint16_t* x,
                                                             int H) {
  const size_t m = blockIdx.x;
  const uint16_t* src = W + (size_t)tokens[m] * H;
  for (int i = threadIdx.x * 8; i < H; i += PF_THREADS * 8) *(u32x4*)(x + m * H + i) = ld16(src + i);
}

// y[m] = rmsnorm(x[m]) with weight w (numpy_ref.py:54-60, the decode's rmsnorm_inplace); rows of K
// bf16 at strides ldx / ldy (elements, multiples of 8)
__global__ void __launch_bounds__(PF_THREADS) pf_rmsnorm_kernel(const uint16_t* x, int64_t ldx, const uint16_t* w,
                                                               uint16_t* y, int64_t ldy, int K, float eps) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  float* xs = (float*)lds;
  float* red = xs + ((K + 63) & ~63);
  const uint16_t* xr = x + (size_t)blockIdx.x * ldx;
  for (int i = threadIdx.x * 8; i < K; i += PF_THREADS * 8) unpack8(ld16(xr + i), xs + i);
  rmsnorm_inplace(xs, w, K, eps, red);
  uint16_t* yr = y + (size_t)blockIdx.x * ldy;
  for (int i = threadIdx.x * 8; i < K; i += PF_THREADS * 8) {
    u32x4 v;
    v.x = pack2(xs[i + 0], xs[i + 1]);
    v.y = pack2(xs[i + 2], xs[i + 3]);
    v.z = pack2(xs[i + 4], xs[i + 5]);
    v.w = pack2(xs[i + 6], xs[i + 7]);
    *(u32x4*)(yr + i) = v;
  }
}

// MLA prep of row m at position pos0 + m (numpy_ref.py:85-103): the latent c = rmsnorm(qkva[m,
// q_out : q_out + d_c]) and k_pe = rope(qkva[m, q_out + d_c :]) into the caches at that position,
// q_pe[m][h] = rope(q[m, h, d_n :]). q_out = nh * (d_n + 64), d_r = 64.
__global__ void __launch_bounds__(PF_THREADS) pf_prep_kernel(const uint16_t* qkva, int64_t ldq, const uint16_t* wkv,
                                                            const uint16_t* cos, const uint16_t* sin, uint16_t* ckv,
                                                            uint16_t* kpe, uint16_t* qpe, int pos0, int nh, int d_n,
                                                            int d_c, float eps) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  const int d_r = 64;
  float* xs = (float*)lds;                 // [d_c]
  float* raw = xs + d_c;                   // [1 + nh][64]: k_pe, then q_pe per head
  float* red = raw + (1 + nh) * d_r;       // [64]
  const int m = blockIdx.x, pos = pos0 + m;
  const int q_out = nh * (d_n + d_r);
  const uint16_t* row = qkva + (size_t)m * ldq;
  for (int i = threadIdx.x; i < d_c; i += PF_THREADS) xs[i] = bf2f(row[q_out + i]);
  for (int t = threadIdx.x; t < (1 + nh) * d_r; t += PF_THREADS) {
    const int v = t / d_r, i = t % d_r;
    raw[t] = bf2f(v == 0 ? row[q_out + d_c + i] : row[(v - 1) * (d_n + d_r) + d_n + i]);
  }
  rmsnorm_inplace(xs, wkv, d_c, eps, red);
  const uint16_t* cr = cos + (size_t)pos * d_r;
  const uint16_t* sr = sin + (size_t)pos * d_r;
  for (int i = threadIdx.x; i < d_c; i += PF_THREADS) ckv[(size_t)pos * d_c + i] = (uint16_t)f2bf(xs[i]);
  for (int t = threadIdx.x; t < (1 + nh) * d_r; t += PF_THREADS) {
    const int v = t / d_r, i = t % d_r;
    const uint16_t r = (uint16_t)f2bf(rope64(raw + v * d_r, cr, sr, i));
    if (v == 0) kpe[(size_t)pos * d_r + i] = r;
    else qpe[((size_t)m * nh + (v - 1)) * d_r + i] = r;
  }
}

// block-wide reductions over PF_THREADS (fixed order: wave butterflies, then wave 0 over the waves)
__device__ __forceinline__ float pf_block_max(float v, float* red) {
  v = wave_max(v);
  __syncthreads();
  if (lane_id() == 0) red[wave_id()] = v;
  __syncthreads();
  float r = red[0];
  for (int w = 1; w < PF_THREADS / 64; ++w) r = fmaxf(r, red[w]);
  return r;
}
__device__ __forceinline__ float pf_block_sum(float v, float* red) {
  v = butterfly(v, 64);
  __syncthreads();
  if (lane_id() == 0) red[wave_id()] = v;
  __syncthreads();
  float r = red[0];
  for (int w = 1; w < PF_THREADS / 64; ++w) r = r + red[w];
  return r;
}

// causal softmax of score row i of head blockIdx.y: keys j < key0 + i + 1; p_j = exp(s_j * scale -
// max), P = bf16(p) (0 past the last key, up to n_cols), l = sum of p (FP32)
__global__ void __launch_bounds__(PF_THREADS) pf_softmax_kernel(const float* S, int64_t ldS, int64_t strideS,
                                                               uint16_t* P, int64_t ldP, int64_t strideP, float* l,
                                                               int64_t strideL, int n_cols, int key0, float scale) {
  __shared__ float red[PF_THREADS / 64];
  const int i = blockIdx.x, h = blockIdx.y;
  const int n = key0 + i + 1 < n_cols ? key0 + i + 1 : n_cols;
  const float* row = S + h * strideS + (size_t)i * ldS;
  uint16_t* prow = P + h * strideP + (size_t)i * ldP;
  float mx = -__builtin_inff();
  for (int j = threadIdx.x; j < n; j += PF_THREADS) mx = fmaxf(mx, row[j] * scale);
  mx = pf_block_max(mx, red);
  float sum = 0.0f;
  for (int j = threadIdx.x; j < n_cols; j += PF_THREADS) {
    float p = 0.0f;
    if (j < n) p = exp_s(row[j] * scale - mx);
    prow[j] = (uint16_t)f2bf(p);
    sum = sum + p;
  }
  sum = pf_block_sum(sum, red);
  if (threadIdx.x == 0) l[h * strideL + i] = sum;
}

// obf[h][i][c] = bf16(O[h][i][c] / l[h][i]) (d columns, d % 4 == 0)
__global__ void __launch_bounds__(PF_THREADS) pf_attn_out_kernel(const float* O, const float* l, uint16_t* obf, int M,
                                                                int d) {
  const int i = blockIdx.x, h = blockIdx.y;
  const float li = l[(size_t)h * M + i];
  const size_t base = ((size_t)h * M + i) * d;
  for (int c = threadIdx.x; c < d; c += PF_THREADS) obf[base + c] = (uint16_t)f2bf(O[base + c] / li);
}

// act[r][i] = bf16(silu(g) * u), g = gu[r][i], u = gu[r][I + i] (the decode's gate|up epilogue)
__global__ void __launch_bounds__(PF_THREADS) pf_silu_kernel(const uint16_t* gu, uint16_t* act, int I) {
  const size_t r = blockIdx.x;
  for (int i = threadIdx.x; i < I; i += PF_THREADS) {
    const float g = bf2f(gu[r * 2 * I + i]);
    const float u = bf2f(gu[r * 2 * I + I + i]);
    act[r * I + i] = (uint16_t)f2bf(silu_s(g) * u);
  }
}

// router of row m (one wave): softmax of the E logits, top-k by repeated argmax (lowest index on
// ties), weights p * scaling; then the n_sh forced shared experts E.. at weight 1.0
__global__ void __launch_bounds__(64) pf_route_kernel(const float* logits, int E, int topk, int n_sh, float scaling,
                                                     int32_t* ids, float* wts) {
  __shared__ int sid[16];
  __shared__ float sw[16];
  const int m = blockIdx.x, slots = topk + n_sh;
  softmax_topk_wave(logits + (size_t)m * E, E, topk, scaling, sid, sw, nullptr);
  __syncthreads();
  const int lane = lane_id();
  if (lane < topk) {
    ids[(size_t)m * slots + lane] = sid[lane];
    wts[(size_t)m * slots + lane] = sw[lane];
  } else if (lane < slots) {
    ids[(size_t)m * slots + lane] = E + lane - topk;
    wts[(size_t)m * slots + lane] = 1.0f;
  }
}

// dst[r] = src[idx[r]] (rows of H bf16)
__global__ void __launch_bounds__(PF_THREADS) pf_gather_kernel(const uint16_t* src, const int32_t* idx, uint16_t* dst,
                                                              int H) {
  const size_t r = blockIdx.x;
  const uint16_t* s = src + (size_t)idx[r] * H;
  for (int i = threadIdx.x * 8; i < H; i += PF_THREADS * 8) *(u32x4*)(dst + r * H + i) = ld16(s + i);
}

// x_res[m] = bf16(x_mid[m] + sum over slots s in order of og[inv[m][s]] * w[m][s]) (numpy_ref.py:
// 316-321, multiply then add, as the decode's combine)
__global__ void __launch_bounds__(PF_THREADS) pf_combine_kernel(const uint16_t* x_mid, const uint16_t* og,
                                                               const int32_t* inv, const float* w, uint16_t* x_res,
                                                               int H, int slots) {
  const size_t m = blockIdx.x;
  for (int c = threadIdx.x; c < H; c += PF_THREADS) {
    float acc = bf2f(x_mid[m * H + c]);
    for (int s = 0; s < slots; ++s) {
      const float t = bf2f(og[(size_t)inv[m * slots + s] * H + c]) * w[m * slots + s];
      acc = acc + t;
    }
    x_res[m * H + c] = (uint16_t)f2bf(acc);
  }
}

// OCP e4m3fn code of a finite f32 (round to nearest even, saturated at +-448; -0 keeps its sign)
__device__ __forceinline__ uint32_t f32_to_e4m3(float v) {
  const uint32_t u = __float_as_uint(v);
  const uint32_t sign = (u >> 24) & 0x80u;
  const float a = fabsf(v);
  uint32_t code;
  if (!(a < 448.0f)) {
    code = 0x7Eu;
  } else if (a < 0.015625f) {                       // below the smallest normal 2^-6: units of 2^-9
    code = (uint32_t)__builtin_rintf(a * 512.0f);  // 0 .. 8 (8 is the smallest normal, code 0x08)
  } else {
    const uint32_t ua = __float_as_uint(a);
    const int e = (int)(ua >> 23) - 127;            // -6 .. 8
    const uint32_t m = ua & 0x7FFFFFu;
    uint32_t q = (m + 0x7FFFFu + ((m >> 20) & 1u)) >> 20;   // 3 mantissa bits, RNE (may carry to 8)
    uint32_t ex = (uint32_t)(e + 7);
    if (q == 8u) { q = 0u; ex += 1u; }
    code = (ex << 3) | q;
    if (code > 0x7Eu) code = 0x7Eu;
  }
  return sign | code;
}

__global__ void __launch_bounds__(PF_THREADS) fx_quant_fp8_kernel(const uint16_t* src, uint8_t* q, float* s, int K) {
  __shared__ float red[PF_THREADS / 64];
  const size_t r = blockIdx.x;
  const uint16_t* row = src + r * K;
  float amax = 0.0f;
  for (int j = threadIdx.x; j < K; j += PF_THREADS) amax = fmaxf(amax, fabsf(bf2f(row[j])));
  amax = pf_block_max(amax, red);
  const float scale = amax > 0.0f ? amax / 448.0f : 1.0f;
  for (int j = threadIdx.x; j < K; j += PF_THREADS) q[r * K + j] = (uint8_t)f32_to_e4m3(bf2f(row[j]) / scale);
  if (threadIdx.x == 0) s[r] = scale;
}

// dst[r][j] = bf16(e4m3(codes[r][j]) * scale[r]): FP8 rows back to bf16 (the batched prefill's GEMMs)
__global__ void __launch_bounds__(PF_THREADS) fx_dequant_fp8_kernel(const uint8_t* q, const float* s, uint16_t* dst,
                                                                   int K) {
  const size_t r = blockIdx.x;
  const float sc = s[r];
  for (int j = threadIdx.x * 16; j < K; j += PF_THREADS * 16) {
    float v[16];
    unpack16_fp8(*(const u32x4*)(q + r * K + j), v);
#pragma unroll
    for (int k = 0; k < 16; ++k) dst[r * K + j + k] = (uint16_t)f2bf(v[k] * sc);
  }
}
