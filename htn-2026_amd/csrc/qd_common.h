// Shared device helpers for the Qwen3 decode kernels (gfx950 / CDNA4, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define QD_OK 0
#define QD_EARG (-1)      // a shape / pointer / size argument is invalid
#define QD_EWS (-2)       // workspace too small
#define QD_ESTATE (-3)    // plan / graph state invalid

typedef uint16_t bf16_t;  // raw bf16 bits everywhere in the ABI

// ---------------------------------------------------------------- bf16 <-> fp32
__device__ __forceinline__ float bf2f(uint32_t b) { return __uint_as_float(b << 16); }
__device__ __forceinline__ float bflo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bfhi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// round-to-nearest-even fp32 -> bf16 bits (NaN stays a quiet NaN)
__device__ __forceinline__ uint32_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u >> 16) | 0x40u;
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}
// value rounded through bf16 (the reference materialises this intermediate as a bf16 tensor)
__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }
__device__ __forceinline__ uint32_t pack2(float lo, float hi) { return f2bf(lo) | (f2bf(hi) << 16); }

// ---------------------------------------------------------------- wave64 reductions
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}
// sum over the 16 lanes of a DPP row (lanes 16r .. 16r+15)
__device__ __forceinline__ float row16_sum(float v) {
#pragma unroll
  for (int m = 8; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// dot of 8 bf16 pairs held in two uint4 (fp32 accumulate, exact products)
__device__ __forceinline__ float dot8(const uint4 a, const uint4 b, float acc) {
  acc = fmaf(bflo(a.x), bflo(b.x), acc); acc = fmaf(bfhi(a.x), bfhi(b.x), acc);
  acc = fmaf(bflo(a.y), bflo(b.y), acc); acc = fmaf(bfhi(a.y), bfhi(b.y), acc);
  acc = fmaf(bflo(a.z), bflo(b.z), acc); acc = fmaf(bfhi(a.z), bfhi(b.z), acc);
  acc = fmaf(bflo(a.w), bflo(b.w), acc); acc = fmaf(bfhi(a.w), bfhi(b.w), acc);
  return acc;
}

// Qwen3RMSNorm's output element: weight * bf16(x * rstd), rounded to bf16
__device__ __forceinline__ float norm_elem(float x, float rstd, float w) { return rbf(rbf(x * rstd) * w); }

// torch silu in fp32 opmath: x / (1 + exp(-x)) (HIP's own expf, IEEE divide)
__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + expf(-g)); }

// rsqrt(mean + eps) as torch computes it on the CPU: 1 / sqrt(v), each correctly rounded
__device__ __forceinline__ float rstd_of(float sumsq, int n, float eps) {
  return 1.0f / sqrtf(sumsq / (float)n + eps);
}

// streaming 128-bit load (weights are read once per step): non-temporal hint
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_stream(const uint4* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

static inline int qd_err(hipError_t e) { return e == hipSuccess ? QD_OK : (int)e; }
