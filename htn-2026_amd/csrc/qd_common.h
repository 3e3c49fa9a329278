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

// round-to-nearest-even fp32 -> bf16 bits: one v_cvt_pk_bf16_f32 (IEEE RNE, NaN stays NaN)
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
__device__ __forceinline__ uint32_t f2bf(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}
// value rounded through bf16 (the reference materialises this intermediate as a bf16 tensor)
__device__ __forceinline__ float rbf(float f) { return static_cast<float>(static_cast<__bf16>(f)); }
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

// ---------------------------------------------------------------- wave64 reductions
// DPP moves within a row of 16 lanes (no LDS crossbar): quad_perm [1,0,3,2], quad_perm
// [2,3,0,1], row_half_mirror, row_mirror -- after the four adds every lane holds its row's sum.
#define QD_DPP(v, ctrl) \
  __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, (v)), (ctrl), 0xF, 0xF, true))
__device__ __forceinline__ float row16_sum_dpp(float v) {
  v += QD_DPP(v, 0xB1);
  v += QD_DPP(v, 0x4E);
  v += QD_DPP(v, 0x141);
  v += QD_DPP(v, 0x140);
  return v;
}
// v of lane ^ 16 / lane ^ 32 with gfx950's v_permlane16_swap / v_permlane32_swap (one VALU op
// each instead of an LDS-crossbar ds_bpermute).  With both operands = v, permlane16_swap
// returns (v with its odd rows replaced by the even rows, v with its even rows replaced by the
// odd rows); permlane32_swap does the same for the two 32-lane halves.  Every lane must be
// active.
__device__ __forceinline__ float lane_xor16(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return __builtin_bit_cast(float, (threadIdx.x & 16) ? r[0] : r[1]);
}
__device__ __forceinline__ float lane_xor32(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __builtin_bit_cast(float, (threadIdx.x & 32) ? r[0] : r[1]);
}
__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum_dpp(v);
  v += lane_xor16(v);
  v += lane_xor32(v);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, lane_xor32(v));
  v = fmaxf(v, lane_xor16(v));
  v = fmaxf(v, QD_DPP(v, 0xB1));
  v = fmaxf(v, QD_DPP(v, 0x4E));
  v = fmaxf(v, QD_DPP(v, 0x141));
  v = fmaxf(v, QD_DPP(v, 0x140));
  return v;
}
// sum over the 16 lanes of a DPP row (lanes 16r .. 16r+15)
__device__ __forceinline__ float row16_sum(float v) { return row16_sum_dpp(v); }

// dot of 8 bf16 pairs held in two uint4, fp32 accumulate: v_dot2_f32_bf16 multiplies two bf16
// pairs exactly and adds them to the fp32 accumulator (4 VALU ops per 16 bytes instead of
// unpack + 8 FMAs)
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), acc, false);
}
__device__ __forceinline__ float dot8(const uint4 a, const uint4 b, float acc) {
  acc = dot2(a.x, b.x, acc);
  acc = dot2(a.y, b.y, acc);
  acc = dot2(a.z, b.z, acc);
  acc = dot2(a.w, b.w, acc);
  return acc;
}

// One term of a 128-wide q/k head's sum of squares: dims d (x1) and d + 64 (x2), the
// rotate_half partners, as one explicit fma.  The decode attention unit (lane d holds both) and
// qk_norm_rope_kernel (16 lanes per head) add the 64 terms in the same balanced order, so the
// two compute identical statistics.
__device__ __forceinline__ float sq_pair(float x1, float x2) { return fmaf(x1, x1, x2 * x2); }

// Qwen3RMSNorm's output element: weight * bf16(x * rstd), rounded to bf16
__device__ __forceinline__ float norm_elem(float x, float rstd, float w) { return rbf(rbf(x * rstd) * w); }

// sum of squares of 8 packed bf16 values, in one fixed expression order (every RMSNorm
// prologue uses this, so statistics agree across kernels that partition a row alike)
__device__ __forceinline__ float sumsq8(const uint4 v) {
  return bflo(v.x) * bflo(v.x) + bfhi(v.x) * bfhi(v.x) + bflo(v.y) * bflo(v.y) +
         bfhi(v.y) * bfhi(v.y) + bflo(v.z) * bflo(v.z) + bfhi(v.z) * bfhi(v.z) +
         bflo(v.w) * bflo(v.w) + bfhi(v.w) * bfhi(v.w);
}

// y = bf16(bf16(v * rstd) * g) for 8 packed values
__device__ __forceinline__ uint4 norm8(const uint4 v, const uint4 g, float rstd) {
  uint4 o;
  o.x = pack2(norm_elem(bflo(v.x), rstd, bflo(g.x)), norm_elem(bfhi(v.x), rstd, bfhi(g.x)));
  o.y = pack2(norm_elem(bflo(v.y), rstd, bflo(g.y)), norm_elem(bfhi(v.y), rstd, bfhi(g.y)));
  o.z = pack2(norm_elem(bflo(v.z), rstd, bflo(g.z)), norm_elem(bfhi(v.z), rstd, bfhi(g.z)));
  o.w = pack2(norm_elem(bflo(v.w), rstd, bflo(g.w)), norm_elem(bfhi(v.w), rstd, bfhi(g.w)));
  return o;
}

// torch silu in fp32 opmath: x / (1 + exp(-x)) (HIP's own expf, IEEE divide)
__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + expf(-g)); }

// bf16(silu_f(g)), the only form the SwiGLU paths use, at a fraction of its cost.  The quotient
// q = g * rcp(1 + exp2(-g log2 e)) on the hardware exp2 and reciprocal (each within 1 ulp)
// differs from silu_f's by at most 21 x 2^-23 relative for |g| <= 16: the exponent's rounding
// carries |g| x 2^-23 into exp, the two hardware ops 2^-23 each, the roundings of t, d and q
// the rest, and silu_f's own expf and roundings 2 x 2^-23.  That is at most 42 fp32 ulps
// (adjacent bit patterns), so the two round to the same bf16 unless q's low 16 bits lie within
// 64 of 0x8000 (a bf16 rounding midpoint).  Those inputs (~0.2 % of them), |g| > 16, infinities
// and NaN take silu_f itself, so the result is silu_f's bf16 for every g
// (tests/test_gpu_kernels.py checks all 65,536 bf16 inputs against the table of silu_f's).
__device__ __forceinline__ float silu_rbf(float g) {
  const float d = 1.0f + __builtin_amdgcn_exp2f(-g * 1.44269504f);
  const float q = g * __builtin_amdgcn_rcpf(d);
  const uint32_t m = (__float_as_uint(q) & 0xffffu) - (0x8000u - 64u);   // <= 128: near a midpoint
  if (__builtin_expect(!(fabsf(g) <= 16.0f) || m <= 128u, 0)) return rbf(silu_f(g));
  return rbf(q);
}

// rsqrt(mean + eps) as torch computes it on the CPU: 1 / sqrt(v), each correctly rounded
__device__ __forceinline__ float rstd_of(float sumsq, int n, float eps) {
  return 1.0f / sqrtf(sumsq / (float)n + eps);
}

// Workgroup barrier that orders LDS only.  __syncthreads() is a full workgroup fence: it makes
// the wave wait for every outstanding global load (s_waitcnt vmcnt(0)) before the barrier, which
// would serialise a kernel's weight stream behind its activation prologue.  LDS visibility needs
// only lgkmcnt(0).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// LDS byte address of a __shared__ object
__device__ __forceinline__ uint32_t lds_u32(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
// lane l's 16 bytes at base + voff go to LDS byte lds + 16 l (wave-uniform lds).  Issued as
// inline asm so that the compiler, which would otherwise wait for every outstanding LDS DMA
// before any later LDS read, leaves the waits to the explicit vmcnt counts of the stage loop.
// The s_nop keeps a wait state between the compiler's M0 write and the load.
__device__ __forceinline__ void dma16(const void* base, uint32_t voff, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "{m0}"(lds)
               : "memory");
}
template <int N>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// wait until at most PER * C of this wave's loads are outstanding, C = min(n, CMAX)
template <int PER, int CMAX>
__device__ __forceinline__ void wait_stages(int n) {
  if constexpr (CMAX == 0) {
    wait_vm<0>();
  } else {
    if (n >= CMAX) wait_vm<PER * CMAX>();
    else wait_stages<PER, CMAX - 1>(n);
  }
}

// plain 128-bit global load
__device__ __forceinline__ uint4 ld_plain(const uint4* p) { return *p; }

// streaming 128-bit load (weights are read once per step): non-temporal hint
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_stream(const uint4* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

static inline int qd_err(hipError_t e) { return e == hipSuccess ? QD_OK : (int)e; }
