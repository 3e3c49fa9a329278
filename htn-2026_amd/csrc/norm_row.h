// One row of the residual-add + RMSNorm over split partials, run by a workgroup of the
// persistent batched step (mega_batch.hip).
#pragma once

#include "handoff.h"

// RMSNorm of row `row` by threads 0..255 (every thread of the workgroup reaches the barriers),
// with part_add_rmsnorm_kernel<S>'s chunking and reduction order, so the same bits.  S > 0:
// acc = the S split partials part[S][B][H] summed in split order, r' = bf16(res + bf16(acc))
// written back to res; S == 0: r' = res (add_rmsnorm_kernel without an addend).  The partials
// are hand-off words (handoff.h), waited for and decoded; y = bf16(bf16(r' * rstd) * w) as
// hand-off words (HWOUT) or plain bf16 rows; err is the error word of the waits.
template <int S, bool HWOUT, int H>
__device__ void norm_row(const uint32_t* part, int B, int row, bf16_t* res,
                         const bf16_t* __restrict__ w, void* y, float eps, float* red,
                         uint32_t* err) {
  constexpr int NCH = H / 8;                   // 16-byte chunks of a row
  constexpr int J = (NCH + 255) / 256;         // chunks per thread
  const int tid = threadIdx.x;
  uint4* rr = reinterpret_cast<uint4*>(res + (int64_t)row * H);
  const uint4* wr = reinterpret_cast<const uint4*>(w);
  float ss = 0.f;
  uint4 rv[J], gv[J];
  if (tid < 256) {
    if constexpr (S > 0) {
      // every split's words of both chunks are requested at once, and re-requested together
      // until all have arrived (one round trip per poll, not one per word)
      const uint64_t* base = reinterpret_cast<const uint64_t*>(part + (int64_t)row * H);
      const int64_t split_stride = (int64_t)B * H / 2;        // uint64 pairs per split
      uint64_t raw[J][S][4];
      auto fetch = [&]() {
#pragma unroll
        for (int j = 0; j < J; ++j) {
          const int c = tid + 256 * j;
#pragma unroll
          for (int s = 0; s < S; ++s)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              raw[j][s][e] = c < NCH ? hw_raw(base + s * split_stride + 4 * c + e) : ~0ull;
        }
      };
      auto ready = [&]() {
        bool ok = true;
#pragma unroll
        for (int j = 0; j < J; ++j)
#pragma unroll
          for (int s = 0; s < S; ++s)
#pragma unroll
            for (int e = 0; e < 4; ++e) ok = ok && hw_ready(raw[j][s][e]);
        return ok;
      };
      fetch();
      if (!ready()) {
        for (uint32_t it = 1; !ready(); ++it) {
          if ((it & 63) == 0) {
            if (__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) break;
            if (it >= HW_SPIN_LIMIT) {
              __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
              break;
            }
          }
          __builtin_amdgcn_s_sleep(1);
          fetch();
        }
      }
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const int c = tid + 256 * j;
        if (c < NCH) {
          float a[8];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint64_t v = ~raw[j][0][e];
            a[2 * e] = __uint_as_float((uint32_t)v);
            a[2 * e + 1] = __uint_as_float((uint32_t)(v >> 32));
          }
#pragma unroll
          for (int s = 1; s < S; ++s)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const uint64_t v = ~raw[j][s][e];
              a[2 * e] += __uint_as_float((uint32_t)v);
              a[2 * e + 1] += __uint_as_float((uint32_t)(v >> 32));
            }
          const uint4 r = rr[c];
          uint4 o;
          o.x = pack2(bflo(r.x) + rbf(a[0]), bfhi(r.x) + rbf(a[1]));
          o.y = pack2(bflo(r.y) + rbf(a[2]), bfhi(r.y) + rbf(a[3]));
          o.z = pack2(bflo(r.z) + rbf(a[4]), bfhi(r.z) + rbf(a[5]));
          o.w = pack2(bflo(r.w) + rbf(a[6]), bfhi(r.w) + rbf(a[7]));
          rv[j] = o;
          gv[j] = wr[c];
          ss += sumsq8(o);
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const int c = tid + 256 * j;
        if (c < NCH) {
          rv[j] = rr[c];
          gv[j] = wr[c];
          ss += sumsq8(rv[j]);
        }
      }
    }
  }
  // the 256 threads' sum as block_sum256: wave sums, then waves 0..3 in order
  ss = wave_sum(ss);
  if (tid < 256 && (tid & 63) == 0) red[tid >> 6] = ss;
  lds_barrier();
  const float rstd = rstd_of(red[0] + red[1] + red[2] + red[3], H, eps);
  if (tid < 256) {
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int c = tid + 256 * j;
      if (c < NCH) {
        const uint4 o = norm8(rv[j], gv[j], rstd);
        if constexpr (HWOUT) {
          hw_put4(static_cast<uint32_t*>(y) + (int64_t)row * (H / 2) + 4 * c, o.x, o.y, o.z, o.w);
        } else {
          reinterpret_cast<uint4*>(static_cast<bf16_t*>(y) + (int64_t)row * H)[c] = o;
        }
        if constexpr (S > 0) rr[c] = rv[j];
      }
    }
  }
  lds_barrier();                                // red is free again
}
