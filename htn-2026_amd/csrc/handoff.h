// Cross-workgroup hand-off words of the persistent decode step (mega.hip, B = 1): every
// produced value travels in 32-bit words (two bf16, or one
// fp32 / index) written with agent-coherent stores and read with agent-coherent loads (the
// cache policy of agent-scope relaxed atomics: single-copy atomic per word, coherent across the
// XCDs' L2s).  A word holds its payload inverted (~payload), so 0 means "not written yet": a
// consumer waits until every word it loaded is nonzero.  The one payload whose inverse is 0,
// 0xFFFFFFFF (two bf16 NaNs, or an fp32 NaN), is stored as 0xFFFFFFFE, still NaN.
// Waits are bounded: after HW_SPIN_LIMIT polls, or once any wait has failed, a wait sets the
// error word and returns, so a launch completes with garbage instead of hanging.
#pragma once

#include "qd_common.h"

constexpr uint32_t HW_SPIN_LIMIT = 1u << 20;   // polls per wait (~1 s) before giving up
constexpr int HW_CPOL = 16;   // buffer-op cache policy of the words: sc1, as agent-scope atomics

__device__ __forceinline__ uint32_t hw_enc(uint32_t payload) {
  return ~(payload == 0xFFFFFFFFu ? 0xFFFFFFFEu : payload);
}
__device__ __forceinline__ void hw_put(uint32_t* p, uint32_t payload) {
  __hip_atomic_store(p, hw_enc(payload), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// two words in one store (p 8-byte aligned)
__device__ __forceinline__ void hw_put2(uint32_t* p, uint32_t lo, uint32_t hi) {
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), ((uint64_t)hw_enc(hi) << 32) | hw_enc(lo),
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool hw_ready(uint32_t v) { return v != 0u; }
__device__ __forceinline__ bool hw_ready(uint64_t v) {
  return (uint32_t)v != 0u && (uint32_t)(v >> 32) != 0u;
}
// one word (uint32_t) or two (uint64_t, 8-byte aligned), as stored
template <typename T>
__device__ __forceinline__ T hw_raw(const T* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Slow path of a wait: poll until every word is written; bounded, and a failed wait anywhere
// makes every later wait give up within 64 polls.
template <typename T>
__device__ __noinline__ T hw_spin(const T* p, uint32_t* err) {
  T v = hw_raw(p);
  for (uint32_t it = 1; !hw_ready(v); ++it) {
    if ((it & 63) == 0) {
      if (__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) break;
      if (it >= HW_SPIN_LIMIT) {
        __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
    }
    __builtin_amdgcn_s_sleep(1);
    v = hw_raw(p);
  }
  return v;
}

// the payload(s) of v, loaded from p, once written
template <typename T>
__device__ __forceinline__ T hw_wait(T v, const T* p, uint32_t* err) {
  if (!hw_ready(v)) v = hw_spin(p, err);
  return ~v;
}

// zero this workgroup's share of words [0, n) (n even, dst 8-byte aligned), NT threads
template <int NT>
__device__ __forceinline__ void hw_clear(uint32_t* dst, int64_t n, int wg, int P) {
  const int64_t a = (n / 2) * wg / P, b = (n / 2) * (wg + 1) / P;
  uint64_t* d = reinterpret_cast<uint64_t*>(dst);
  for (int64_t i = a + threadIdx.x; i < b; i += NT)
    __hip_atomic_store(d + i, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- four words at once (16-byte buffer loads / stores with the words' cache policy)
typedef unsigned int hw_u4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bool hw_ready4(const uint4& v) {
  return v.x != 0u && v.y != 0u && v.z != 0u && v.w != 0u;
}
__device__ __forceinline__ uint4 hw_load4(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so) {
  const hw_u4 v = __builtin_amdgcn_raw_buffer_load_b128(r, vo, so, HW_CPOL);
  return make_uint4(v.x, v.y, v.z, v.w);
}
// poll four words (at vo + so of r) until all are written; bounded like hw_spin
__device__ __noinline__ uint4 hw_spin4(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so,
                                       uint32_t* err) {
  uint4 v = hw_load4(r, vo, so);
  for (uint32_t it = 1; !hw_ready4(v); ++it) {
    if ((it & 63) == 0) {
      if (__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) break;
      if (it >= HW_SPIN_LIMIT) {
        __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
    }
    __builtin_amdgcn_s_sleep(1);
    v = hw_load4(r, vo, so);
  }
  return v;
}
// the payloads of four words v loaded from (r, vo, so), once written
__device__ __forceinline__ uint4 hw_wait4(uint4 v, __amdgpu_buffer_rsrc_t r, uint32_t vo,
                                          uint32_t so, uint32_t* err) {
  if (!hw_ready4(v)) v = hw_spin4(r, vo, so, err);
  return make_uint4(~v.x, ~v.y, ~v.z, ~v.w);
}
// four words (p 16-byte aligned) in two 8-byte stores
__device__ __forceinline__ void hw_put4(uint32_t* p, uint32_t a, uint32_t b, uint32_t c,
                                        uint32_t d) {
  hw_put2(p, a, b);
  hw_put2(p + 2, c, d);
}

// threadIdx.x behind an empty asm: values derived from it are recomputed where they are used
// instead of being hoisted out of a persistent kernel's layer loop (where they would hold
// registers across every phase)
__device__ __forceinline__ int hw_tid() {
  int t = (int)threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}
