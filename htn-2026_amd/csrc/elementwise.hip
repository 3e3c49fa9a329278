// Row-wise kernels of the decode path: embedding gather, residual add + RMSNorm, per-head
// q/k RMSNorm + RoPE with the K/V cache write, SwiGLU, KV compaction of an accepted tree
// path, the synthetic-weight generator and the greedy argmax reduction.
//
// All of them are HBM/latency bound byte movers: 128-bit loads along a row, one workgroup
// (or one wave) per row/head, fp32 arithmetic with the reference's bf16 rounding points.
#include "qd_launch.h"

// ------------------------------------------------------------------ embedding gather
// x[i, :] = table[ids[i], :] -- a bit copy (F.embedding, engine.py:338; embed_ss fast.py:53-70).
// An id outside [0, vocab) writes a zero row instead of reading out of bounds (the host
// rejects such ids before they reach the device).
__global__ __launch_bounds__(256) void embed_kernel(const int64_t* __restrict__ ids,
                                                    const bf16_t* __restrict__ table,
                                                    bf16_t* __restrict__ out, int64_t vocab,
                                                    int64_t hidden, int64_t out_stride) {
  const int64_t i = blockIdx.x;
  const int64_t id = ids[i];
  const bool ok = id >= 0 && id < vocab;
  const int64_t nch = hidden / 8;
  const uint4* src = reinterpret_cast<const uint4*>(table + (ok ? id : 0) * hidden);
  uint4* dst = reinterpret_cast<uint4*>(out + i * out_stride);
  for (int64_t c = threadIdx.x; c < nch; c += blockDim.x) {
    uint4 v = ok ? src[c] : make_uint4(0, 0, 0, 0);
    dst[c] = v;
  }
}

void launch_embed(const int64_t* ids, const bf16_t* table, bf16_t* out, int64_t n, int64_t vocab,
                  int64_t hidden, int64_t out_stride, hipStream_t s) {
  if (n <= 0) return;
  embed_kernel<<<dim3((unsigned)n), dim3(256), 0, s>>>(ids, table, out, vocab, hidden, out_stride);
}

// The decode step's first launch also stages the step's RoPE row: every layer's attention then
// reads it from a fixed address instead of waiting for pos before fetching the table row.
__global__ __launch_bounds__(256) void embed_rope_kernel(const int64_t* __restrict__ ids,
                                                         const bf16_t* __restrict__ table,
                                                         bf16_t* __restrict__ out, int64_t vocab,
                                                         int64_t hidden, int64_t out_stride,
                                                         const bf16_t* __restrict__ cos_t,
                                                         const bf16_t* __restrict__ sin_t,
                                                         const int64_t* __restrict__ pos,
                                                         int64_t cap, bf16_t* rope_out) {
  const int64_t i = blockIdx.x;
  const int64_t id = ids[i];
  const bool ok = id >= 0 && id < vocab;
  const int64_t nch = hidden / 8;
  const uint4* src = reinterpret_cast<const uint4*>(table + (ok ? id : 0) * hidden);
  uint4* dst = reinterpret_cast<uint4*>(out + i * out_stride);
  for (int64_t c = threadIdx.x; c < nch; c += blockDim.x) dst[c] = ok ? src[c] : make_uint4(0, 0, 0, 0);
  if (i == 0 && threadIdx.x < 256) {
    const int64_t p = pos[0];
    if (p >= 0 && p < cap) {
      const int t = threadIdx.x;
      rope_out[t] = t < 128 ? cos_t[p * 128 + t] : sin_t[p * 128 + t - 128];
    }
  }
}

void launch_embed_rope(const int64_t* ids, const bf16_t* table, bf16_t* out, int64_t n,
                       int64_t vocab, int64_t hidden, int64_t out_stride, const bf16_t* cos_t,
                       const bf16_t* sin_t, const int64_t* pos, int64_t cap, bf16_t* rope_out,
                       hipStream_t s) {
  if (n <= 0) return;
  embed_rope_kernel<<<dim3((unsigned)n), dim3(256), 0, s>>>(ids, table, out, vocab, hidden,
                                                            out_stride, cos_t, sin_t, pos, cap,
                                                            rope_out);
}

// ------------------------------------------------------------------ residual add + RMSNorm
// r' = bf16(x + r) (x may be null: r' = r), y = bf16(bf16(r' * rstd) * w),
// rstd = 1 / sqrt(mean(r'^2) + eps) from the bf16-rounded residual (rmsnorm.py:15-32,
// TF:modeling_qwen3.py:59-64, 304-322).  One workgroup per row.
__device__ __forceinline__ float block_sum256(float v, float* red) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  if (l == 0) red[w] = v;
  __syncthreads();
  float t = red[0] + red[1] + red[2] + red[3];
  __syncthreads();
  return t;
}

constexpr int AR_MAXC = 4;   // 16-byte chunks per thread held in registers (hidden <= 8192)

__global__ __launch_bounds__(256) void add_rmsnorm_kernel(
    const bf16_t* __restrict__ x, const bf16_t* res, const bf16_t* __restrict__ w,
    bf16_t* res_out, bf16_t* __restrict__ y, int64_t hidden, int64_t in_stride,
    int64_t y_stride, float eps) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const int64_t nch = hidden / 8;
  const uint4* xr = x ? reinterpret_cast<const uint4*>(x + row * in_stride) : nullptr;
  const uint4* rr = reinterpret_cast<const uint4*>(res + row * in_stride);
  uint4* ro = res_out ? reinterpret_cast<uint4*>(res_out + row * in_stride) : nullptr;
  const uint4* wr = reinterpret_cast<const uint4*>(w);
  uint4* yr = reinterpret_cast<uint4*>(y + row * y_stride);
  auto add = [&](uint4 r, int64_t c) {
    if (xr) {
      const uint4 a = xr[c];
      r.x = pack2(bflo(a.x) + bflo(r.x), bfhi(a.x) + bfhi(r.x));
      r.y = pack2(bflo(a.y) + bflo(r.y), bfhi(a.y) + bfhi(r.y));
      r.z = pack2(bflo(a.z) + bflo(r.z), bfhi(a.z) + bfhi(r.z));
      r.w = pack2(bflo(a.w) + bflo(r.w), bfhi(a.w) + bfhi(r.w));
    }
    return r;
  };
  auto norm_out = [&](const uint4 r, const uint4 g, float rstd) {
    uint4 o;
    o.x = pack2(norm_elem(bflo(r.x), rstd, bflo(g.x)), norm_elem(bfhi(r.x), rstd, bfhi(g.x)));
    o.y = pack2(norm_elem(bflo(r.y), rstd, bflo(g.y)), norm_elem(bfhi(r.y), rstd, bfhi(g.y)));
    o.z = pack2(norm_elem(bflo(r.z), rstd, bflo(g.z)), norm_elem(bfhi(r.z), rstd, bfhi(g.z)));
    o.w = pack2(norm_elem(bflo(r.w), rstd, bflo(g.w)), norm_elem(bfhi(r.w), rstd, bfhi(g.w)));
    return o;
  };
  float ss = 0.f;
  if (nch <= 256 * AR_MAXC) {
    // the row (and the norm weights) stay in registers across the reduction: one pass of loads
    uint4 rv[AR_MAXC], gv[AR_MAXC];
#pragma unroll
    for (int j = 0; j < AR_MAXC; ++j) {
      const int64_t c = threadIdx.x + 256 * j;
      if (c < nch) {
        rv[j] = add(rr[c], c);
        gv[j] = wr[c];
        ss += sumsq8(rv[j]);
      }
    }
    const float rstd = rstd_of(block_sum256(ss, red), (int)hidden, eps);
#pragma unroll
    for (int j = 0; j < AR_MAXC; ++j) {
      const int64_t c = threadIdx.x + 256 * j;
      if (c < nch) {
        yr[c] = norm_out(rv[j], gv[j], rstd);
        if (ro && xr) ro[c] = rv[j];
      }
    }
    return;
  }
  for (int64_t c = threadIdx.x; c < nch; c += 256) ss += sumsq8(add(rr[c], c));
  const float rstd = rstd_of(block_sum256(ss, red), (int)hidden, eps);
  for (int64_t c = threadIdx.x; c < nch; c += 256) {
    const uint4 r = add(rr[c], c);
    yr[c] = norm_out(r, wr[c], rstd);
    // each thread writes back exactly the chunks it read, after its last read of them
    if (ro && xr) ro[c] = r;
  }
}

// Split-K partials + residual add + RMSNorm (the batched decode step's o / down projections
// end here): acc = sum of part[s][row] in split order (fp32), r' = bf16(res + bf16(acc))
// written back to res -- the residual epilogue's rounding points (gemv.py:50-51) -- and
// y = bf16(bf16(r' * rstd) * w).  One workgroup per row, hidden <= 8192.
// SC > 0: the split count as a compile-time constant, so every split's loads are issued before
// the first add (a runtime loop costs one round trip per split: 4.9 us per launch at 4 splits)
template <int SC>
__global__ __launch_bounds__(256) void part_add_rmsnorm_kernel(
    const float* __restrict__ part, int S_rt, int64_t rows, bf16_t* res, const bf16_t* __restrict__ w,
    bf16_t* __restrict__ y, int64_t hidden, float eps) {
  const int S = SC > 0 ? SC : S_rt;
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const int64_t nch = hidden / 8;
  uint4* rr = reinterpret_cast<uint4*>(res + row * hidden);
  const uint4* wr = reinterpret_cast<const uint4*>(w);
  uint4* yr = reinterpret_cast<uint4*>(y + row * hidden);
  float ss = 0.f;
  uint4 rv[AR_MAXC], gv[AR_MAXC];
#pragma unroll
  for (int j = 0; j < AR_MAXC; ++j) {
    const int64_t c = threadIdx.x + 256 * j;
    if (c < nch) {
      const float4* p = reinterpret_cast<const float4*>(part + row * hidden) + 2 * c;
      float4 a = p[0], b = p[1];
      if constexpr (SC > 0) {
        float4 pa[SC > 1 ? SC - 1 : 1], pb[SC > 1 ? SC - 1 : 1];
#pragma unroll
        for (int s = 1; s < SC; ++s) {
          const float4* ps = reinterpret_cast<const float4*>(part + ((int64_t)s * rows + row) * hidden) + 2 * c;
          pa[s - 1] = ps[0];
          pb[s - 1] = ps[1];
        }
#pragma unroll
        for (int s = 1; s < SC; ++s) {
          const float4 a2 = pa[s - 1], b2 = pb[s - 1];
          a.x += a2.x; a.y += a2.y; a.z += a2.z; a.w += a2.w;
          b.x += b2.x; b.y += b2.y; b.z += b2.z; b.w += b2.w;
        }
      } else {
        for (int s = 1; s < S; ++s) {
          const float4* ps = reinterpret_cast<const float4*>(part + ((int64_t)s * rows + row) * hidden) + 2 * c;
          const float4 a2 = ps[0], b2 = ps[1];
          a.x += a2.x; a.y += a2.y; a.z += a2.z; a.w += a2.w;
          b.x += b2.x; b.y += b2.y; b.z += b2.z; b.w += b2.w;
        }
      }
      const uint4 r = rr[c];
      uint4 o;
      o.x = pack2(bflo(r.x) + rbf(a.x), bfhi(r.x) + rbf(a.y));
      o.y = pack2(bflo(r.y) + rbf(a.z), bfhi(r.y) + rbf(a.w));
      o.z = pack2(bflo(r.z) + rbf(b.x), bfhi(r.z) + rbf(b.y));
      o.w = pack2(bflo(r.w) + rbf(b.z), bfhi(r.w) + rbf(b.w));
      rv[j] = o;
      gv[j] = wr[c];
      ss += sumsq8(o);
    }
  }
  const float rstd = rstd_of(block_sum256(ss, red), (int)hidden, eps);
#pragma unroll
  for (int j = 0; j < AR_MAXC; ++j) {
    const int64_t c = threadIdx.x + 256 * j;
    if (c < nch) {
      yr[c] = norm8(rv[j], gv[j], rstd);
      rr[c] = rv[j];                             // each thread writes back the chunks it read
    }
  }
}

// 256 < hidden / 8 <= 512 (hidden 2560: 320 chunks): chunks tid and tid + 256 of the row, with
// every load of both -- all splits' partials, the residual, the norm weights -- issued before
// the first add (the second chunk's address clamped to the first's where it lies past the row,
// its results dropped); the arithmetic and its order are part_add_rmsnorm_kernel's, so the bits
// are the same.  The guarded per-chunk loop above issues the second chunk's loads only after the
// first chunk's sums: two memory round trips instead of one.
template <int SC>
__global__ __launch_bounds__(256) void part_add_rmsnorm2_kernel(
    const float* __restrict__ part, int64_t rows, bf16_t* res, const bf16_t* __restrict__ w,
    bf16_t* __restrict__ y, int64_t hidden, float eps) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const int nch = (int)(hidden / 8);
  uint4* rr = reinterpret_cast<uint4*>(res + row * hidden);
  const uint4* wr = reinterpret_cast<const uint4*>(w);
  uint4* yr = reinterpret_cast<uint4*>(y + row * hidden);
  const int c0 = threadIdx.x, c1 = threadIdx.x + 256;
  const bool has1 = c1 < nch;
  const int cc[2] = {c0, has1 ? c1 : c0};
  float4 pv[2][SC][2];
  uint4 rv[2], gv[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
#pragma unroll
    for (int sp = 0; sp < SC; ++sp) {
      const float4* ps = reinterpret_cast<const float4*>(part + ((int64_t)sp * rows + row) * hidden) + 2 * cc[q];
      pv[q][sp][0] = ps[0];
      pv[q][sp][1] = ps[1];
    }
    rv[q] = rr[cc[q]];
    gv[q] = wr[cc[q]];
  }
  float ss = 0.f;
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    if (q == 1 && !has1) break;
    float4 a = pv[q][0][0], b = pv[q][0][1];
#pragma unroll
    for (int sp = 1; sp < SC; ++sp) {
      const float4 a2 = pv[q][sp][0], b2 = pv[q][sp][1];
      a.x += a2.x; a.y += a2.y; a.z += a2.z; a.w += a2.w;
      b.x += b2.x; b.y += b2.y; b.z += b2.z; b.w += b2.w;
    }
    const uint4 r = rv[q];
    uint4 o;
    o.x = pack2(bflo(r.x) + rbf(a.x), bfhi(r.x) + rbf(a.y));
    o.y = pack2(bflo(r.y) + rbf(a.z), bfhi(r.y) + rbf(a.w));
    o.z = pack2(bflo(r.z) + rbf(b.x), bfhi(r.z) + rbf(b.y));
    o.w = pack2(bflo(r.w) + rbf(b.z), bfhi(r.w) + rbf(b.w));
    rv[q] = o;
    ss += sumsq8(o);
  }
  const float rstd = rstd_of(block_sum256(ss, red), (int)hidden, eps);
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    if (q == 1 && !has1) break;
    yr[cc[q]] = norm8(rv[q], gv[q], rstd);
    rr[cc[q]] = rv[q];                           // each thread writes back the chunks it read
  }
}

void launch_part_add_rmsnorm(const float* part, int S, int64_t rows, bf16_t* res, const bf16_t* w,
                             bf16_t* y, int64_t hidden, float eps, hipStream_t s) {
  if (rows <= 0) return;
  const dim3 g((unsigned)rows), b(256);
  if (hidden / 8 > 256 && hidden / 8 <= 512) {
    switch (S) {
      case 1: part_add_rmsnorm2_kernel<1><<<g, b, 0, s>>>(part, rows, res, w, y, hidden, eps); return;
      case 2: part_add_rmsnorm2_kernel<2><<<g, b, 0, s>>>(part, rows, res, w, y, hidden, eps); return;
      case 4: part_add_rmsnorm2_kernel<4><<<g, b, 0, s>>>(part, rows, res, w, y, hidden, eps); return;
      case 6: part_add_rmsnorm2_kernel<6><<<g, b, 0, s>>>(part, rows, res, w, y, hidden, eps); return;
      default: break;
    }
  }
  switch (S) {
    case 1: part_add_rmsnorm_kernel<1><<<g, b, 0, s>>>(part, S, rows, res, w, y, hidden, eps); break;
    case 2: part_add_rmsnorm_kernel<2><<<g, b, 0, s>>>(part, S, rows, res, w, y, hidden, eps); break;
    case 4: part_add_rmsnorm_kernel<4><<<g, b, 0, s>>>(part, S, rows, res, w, y, hidden, eps); break;
    case 6: part_add_rmsnorm_kernel<6><<<g, b, 0, s>>>(part, S, rows, res, w, y, hidden, eps); break;
    default: part_add_rmsnorm_kernel<0><<<g, b, 0, s>>>(part, S, rows, res, w, y, hidden, eps); break;
  }
}

// Many rows (prefill chunks): the same per-row arithmetic -- chunk c of a row in thread c % 256,
// the thread's chunks summed in order, block_sum256 -- so the same bits, with each workgroup
// walking rows blockIdx.x, + gridDim.x, ... and the next row's loads (non-temporal) issued
// before the current row's reduction; the norm weights are loaded once per workgroup.  Used
// above QD_ARN_WG_PER_CU rows per CU.  Measured on MI355X (add + norm, hidden 2560): 32768 rows
// 105.1 us one row per workgroup, 99.8 us at 32 workgroups per CU (4 rows each; 102.2 at 4 and
// 102.0 at 16 per CU); at 8192 rows one row per workgroup stays best (26.3 us against 29.5 us
// at 8 per CU).
#ifndef QD_ARN_WG_PER_CU
#define QD_ARN_WG_PER_CU 32
#endif
constexpr int ARN_J = 2;                    // chunks per thread: hidden <= 4096

template <bool HAS_X>
__global__ __launch_bounds__(256) void add_rmsnorm_rows_kernel(
    const bf16_t* __restrict__ x, const bf16_t* res, const bf16_t* __restrict__ w,
    bf16_t* res_out, bf16_t* __restrict__ y, int64_t rows, int64_t hidden, int64_t in_stride,
    int64_t y_stride, float eps) {
  __shared__ float red[4];
  const int nch = (int)(hidden / 8);
  const int tid = threadIdx.x;
  const uint4* wr = reinterpret_cast<const uint4*>(w);
  uint4 gv[ARN_J], cr[ARN_J] = {}, cx[ARN_J] = {};
#pragma unroll
  for (int j = 0; j < ARN_J; ++j) {
    const int c = tid + 256 * j;
    gv[j] = c < nch ? wr[c] : make_uint4(0, 0, 0, 0);
  }
  auto issue = [&](int64_t row, uint4 (&r)[ARN_J], uint4 (&a)[ARN_J]) {
    const uint4* rr = reinterpret_cast<const uint4*>(res + row * in_stride);
#pragma unroll
    for (int j = 0; j < ARN_J; ++j) {
      const int c = tid + 256 * j;
      if (c < nch) {
        r[j] = ld_stream(rr + c);
        if (HAS_X) a[j] = ld_stream(reinterpret_cast<const uint4*>(x + row * in_stride) + c);
      }
    }
  };
  int64_t row = blockIdx.x;
  if (row >= rows) return;
  issue(row, cr, cx);
  for (; row < rows; row += gridDim.x) {
    uint4 nr[ARN_J] = {}, nx[ARN_J] = {};
    const int64_t next = row + gridDim.x;
    if (next < rows) issue(next, nr, nx);
    uint4 rv[ARN_J];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < ARN_J; ++j) {
      const int c = tid + 256 * j;
      if (c < nch) {
        uint4 r = cr[j];
        if (HAS_X) {
          const uint4 a = cx[j];
          r.x = pack2(bflo(a.x) + bflo(r.x), bfhi(a.x) + bfhi(r.x));
          r.y = pack2(bflo(a.y) + bflo(r.y), bfhi(a.y) + bfhi(r.y));
          r.z = pack2(bflo(a.z) + bflo(r.z), bfhi(a.z) + bfhi(r.z));
          r.w = pack2(bflo(a.w) + bflo(r.w), bfhi(a.w) + bfhi(r.w));
        }
        rv[j] = r;
        ss += sumsq8(r);
      }
    }
    const float rstd = rstd_of(block_sum256(ss, red), (int)hidden, eps);
    uint4* yr = reinterpret_cast<uint4*>(y + row * y_stride);
    uint4* ro = res_out ? reinterpret_cast<uint4*>(res_out + row * in_stride) : nullptr;
#pragma unroll
    for (int j = 0; j < ARN_J; ++j) {
      const int c = tid + 256 * j;
      if (c < nch) {
        const uint4 o = norm8(rv[j], gv[j], rstd);
        __builtin_nontemporal_store(*reinterpret_cast<const u32x4_t*>(&o),
                                    reinterpret_cast<u32x4_t*>(yr + c));
        if (HAS_X && ro) ro[c] = rv[j];
      }
    }
#pragma unroll
    for (int j = 0; j < ARN_J; ++j) {
      cr[j] = nr[j];
      cx[j] = nx[j];
    }
  }
}

static int64_t arn_cus() {
  static int64_t cus = -1;
  if (cus < 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
      (void)hipGetLastError();
      n = 256;
    }
    cus = n > 0 ? n : 256;
  }
  return cus;
}

// add_rmsnorm_kernel for 256 < hidden / 8 <= 512 with both chunks' loads issued first (as
// part_add_rmsnorm2_kernel; same arithmetic, same bits).
template <bool HAS_X>
__global__ __launch_bounds__(256) void add_rmsnorm2_kernel(
    const bf16_t* __restrict__ x, const bf16_t* res, const bf16_t* __restrict__ w,
    bf16_t* res_out, bf16_t* __restrict__ y, int64_t hidden, int64_t in_stride,
    int64_t y_stride, float eps) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const int nch = (int)(hidden / 8);
  const uint4* rr = reinterpret_cast<const uint4*>(res + row * in_stride);
  const uint4* wr = reinterpret_cast<const uint4*>(w);
  uint4* yr = reinterpret_cast<uint4*>(y + row * y_stride);
  const int c0 = threadIdx.x, c1 = threadIdx.x + 256;
  const bool has1 = c1 < nch;
  const int cc[2] = {c0, has1 ? c1 : c0};
  uint4 rv[2], xv[2], gv[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    rv[q] = rr[cc[q]];
    if (HAS_X) xv[q] = reinterpret_cast<const uint4*>(x + row * in_stride)[cc[q]];
    gv[q] = wr[cc[q]];
  }
  float ss = 0.f;
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    if (q == 1 && !has1) break;
    if (HAS_X) {
      uint4 r = rv[q];
      const uint4 a = xv[q];
      r.x = pack2(bflo(a.x) + bflo(r.x), bfhi(a.x) + bfhi(r.x));
      r.y = pack2(bflo(a.y) + bflo(r.y), bfhi(a.y) + bfhi(r.y));
      r.z = pack2(bflo(a.z) + bflo(r.z), bfhi(a.z) + bfhi(r.z));
      r.w = pack2(bflo(a.w) + bflo(r.w), bfhi(a.w) + bfhi(r.w));
      rv[q] = r;
    }
    ss += sumsq8(rv[q]);
  }
  const float rstd = rstd_of(block_sum256(ss, red), (int)hidden, eps);
  uint4* ro = res_out ? reinterpret_cast<uint4*>(res_out + row * in_stride) : nullptr;
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    if (q == 1 && !has1) break;
    yr[cc[q]] = norm8(rv[q], gv[q], rstd);
    if (HAS_X && ro) ro[cc[q]] = rv[q];
  }
}

void launch_add_rmsnorm(const bf16_t* x, const bf16_t* res, const bf16_t* w, bf16_t* res_out,
                        bf16_t* y, int64_t rows, int64_t hidden, int64_t in_stride,
                        int64_t y_stride, float eps, hipStream_t s) {
  if (rows <= 0) return;
  const int64_t grid = arn_cus() * QD_ARN_WG_PER_CU;
  if (rows > grid && hidden / 8 <= 256 * ARN_J) {
    if (x)
      add_rmsnorm_rows_kernel<true><<<dim3((unsigned)grid), dim3(256), 0, s>>>(
          x, res, w, res_out, y, rows, hidden, in_stride, y_stride, eps);
    else
      add_rmsnorm_rows_kernel<false><<<dim3((unsigned)grid), dim3(256), 0, s>>>(
          x, res, w, res_out, y, rows, hidden, in_stride, y_stride, eps);
    return;
  }
  if (hidden / 8 > 256 && hidden / 8 <= 512) {
    if (x)
      add_rmsnorm2_kernel<true><<<dim3((unsigned)rows), dim3(256), 0, s>>>(
          x, res, w, res_out, y, hidden, in_stride, y_stride, eps);
    else
      add_rmsnorm2_kernel<false><<<dim3((unsigned)rows), dim3(256), 0, s>>>(
          x, res, w, res_out, y, hidden, in_stride, y_stride, eps);
    return;
  }
  add_rmsnorm_kernel<<<dim3((unsigned)rows), dim3(256), 0, s>>>(x, res, w, res_out, y, hidden,
                                                                 in_stride, y_stride, eps);
}

// ------------------------------------------------------------------ q/k RMSNorm + RoPE + KV write
// 8 lanes per (token row, head in [0, Hq + 2 Hkv)): lane j holds dims 8j .. 8j+7 ("lo") and
// their rotate_half partners 64 + 8j .. ("hi"), two 16-byte loads, so the pair terms of the
// statistics and the rotation need no cross-lane moves and no lane computes a term twice.
// A 256-thread workgroup is 32 such groups: 16 heads x 2 runs of QKR_RPG consecutive token
// rows (one run per pair of waves, so row-dependent branches are wave-uniform).
// Per-head RMSNorm (q_norm / k_norm weights), then
//   o1 = bf16(bf16(y1 c1) + bf16(-y2 s1)),  o2 = bf16(bf16(y2 c2) + bf16(y1 s2))
// for each (d, d + 64) pair (fused.py:24-81, tree.py:26-69, TF:modeling_qwen3.py:140-170,
// 252-257).  The 64 sum-of-squares terms sq_pair(x_d, x_{d+64}) are added as a balanced binary
// tree in index order -- within the lane over its 8 pairs, then across lanes j = 0..7 -- the
// same tree wave_sum builds over lanes d = 0..63 in the decode attention unit, so the
// statistics are bit-identical to the decode step's.  rstd (an IEEE sqrt and divide) is
// computed once per lane for row j & 3 of the lane's run and broadcast within each quad.
// V heads are copied unnormalised into the cache.  Position of token t of row b:
//   POS_T t | POS_SHARED pos[0]+t | POS_ROW pos[b]+t | POS_CHUNK pos[b]+t (= slot)
//   POS_TREE: RoPE at pos[b] + depth[b*T + t], cache slot pos[b] + t.
__device__ __forceinline__ void unpack8(const uint4 v, float (&f)[8]) {
  f[0] = bflo(v.x); f[1] = bfhi(v.x); f[2] = bflo(v.y); f[3] = bfhi(v.y);
  f[4] = bflo(v.z); f[5] = bfhi(v.z); f[6] = bflo(v.w); f[7] = bfhi(v.w);
}
// two values rounded through bf16 with one conversion (the empty asm keeps the compiler from
// splitting it back into one conversion per value)
__device__ __forceinline__ void rbf2(float& a, float& b) {
  uint32_t p = pack2(a, b);
  asm("" : "+v"(p));
  a = bflo(p);
  b = bfhi(p);
}
// hide a packed word's origin from the optimiser, so values derived from it are recomputed
// where they are used instead of being kept live from an earlier use
__device__ __forceinline__ void opaque(uint4& v) {
  asm("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w));
}

constexpr int QKR_RPG = 4;              // token rows per 8-lane group
constexpr int QKR_ROWS = 2 * QKR_RPG;   // token rows per workgroup

// PART: the packed qkv rows are the split-K partials of the qkv projection, part[S][B*T][width]
// fp32 (the tiled GEMM's split layout): each value is their sum in split order rounded to
// bf16, the same bits gemm_split_reduce_kernel would have stored.
template <bool PART, int SC = 0>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(
    const bf16_t* __restrict__ qkv, int64_t qkv_stride, const bf16_t* __restrict__ qn,
    const bf16_t* __restrict__ kn, const bf16_t* __restrict__ cos_t,
    const bf16_t* __restrict__ sin_t, int64_t table_len, const int64_t* __restrict__ pos,
    const int64_t* __restrict__ depth, int mode, bf16_t* __restrict__ q_out,
    bf16_t* __restrict__ k_cache, bf16_t* __restrict__ v_cache, int64_t T, int Hq, int Hkv,
    int64_t cap, float eps, const float* __restrict__ part, int S, int64_t rows_total) {
  // grid (token blocks of QKR_ROWS, sequence b, head group of 16): no integer division
  const int grp = threadIdx.x >> 3, j = threadIdx.x & 7;
  const int head = (int)blockIdx.z * 16 + (grp & 15);
  const int64_t b = blockIdx.y;
  // The workgroup's QKR_ROWS RoPE rows, unpacked to fp32 once and shared by its 16 heads
  // through LDS: thread t stages 16-byte unit (t & 15) of the cos (t & 16 == 0) or sin row of
  // token row t >> 5 (clamped into the table; rows outside it are skipped below).  The unpack
  // is exact, so the arithmetic is the same as unpacking per head.
  __shared__ float4 rope_lds[QKR_ROWS][2][32];
  {
    const int r = (int)threadIdx.x >> 5, unit = threadIdx.x & 15, tab = (threadIdx.x >> 4) & 1;
    const int64_t tr = (int64_t)blockIdx.x * QKR_ROWS + r;
    const int64_t p0s = mode == POS_T ? 0 : mode == POS_SHARED ? pos[0] : pos[b];
    int64_t rp = mode == POS_TREE ? p0s + depth[b * T + (tr < T ? tr : T - 1)] : p0s + tr;
    rp = rp < 0 ? 0 : (rp >= table_len ? table_len - 1 : rp);
    const uint4 v = reinterpret_cast<const uint4*>((tab ? sin_t : cos_t) + rp * 128)[unit];
    rope_lds[r][tab][2 * unit] = make_float4(bflo(v.x), bfhi(v.x), bflo(v.y), bfhi(v.y));
    rope_lds[r][tab][2 * unit + 1] = make_float4(bflo(v.z), bfhi(v.z), bflo(v.w), bfhi(v.w));
  }
  __syncthreads();
  if (head >= Hq + 2 * Hkv) return;            // whole 8-lane groups leave together
  // the run's first row: uniform over the wave (waves 0-1 the first run, 2-3 the second), so
  // every row-dependent value below lives in scalar registers
  const int run = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 7);
  const int64_t t0 = (int64_t)blockIdx.x * QKR_ROWS + run * QKR_RPG;
  const bool vhead = head >= Hq + Hkv;
  uint4 xl[QKR_RPG], xh[QKR_RPG];
  if constexpr (PART) {
    const int64_t width = (int64_t)(Hq + 2 * Hkv) * 128;
#pragma unroll
    for (int i = 0; i < QKR_RPG; ++i) {
      const int64_t t = t0 + i < T ? t0 + i : T - 1;
      const int64_t col = (b * T + t) * width + (int64_t)head * 128 + 8 * j;
      float4 v[4];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const float4* p0 = reinterpret_cast<const float4*>(part + col + 64 * h);
        v[2 * h] = p0[0];
        v[2 * h + 1] = p0[1];
      }
      if constexpr (SC > 1) {
        // the split count at compile time: every split's loads issue before the first add
        float4 w[SC - 1][4];
#pragma unroll
        for (int sp = 1; sp < SC; ++sp)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const float4* ps = reinterpret_cast<const float4*>(part + (int64_t)sp * rows_total * width + col + 64 * h);
            w[sp - 1][2 * h] = ps[0];
            w[sp - 1][2 * h + 1] = ps[1];
          }
#pragma unroll
        for (int sp = 1; sp < SC; ++sp)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            v[e].x += w[sp - 1][e].x; v[e].y += w[sp - 1][e].y;
            v[e].z += w[sp - 1][e].z; v[e].w += w[sp - 1][e].w;
          }
      } else {
        for (int sp = 1; sp < S; ++sp) {
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const float4* ps = reinterpret_cast<const float4*>(part + (int64_t)sp * rows_total * width + col + 64 * h);
            const float4 a2 = ps[0], b2 = ps[1];
            float4& a = v[2 * h];
            float4& c = v[2 * h + 1];
            a.x += a2.x; a.y += a2.y; a.z += a2.z; a.w += a2.w;
            c.x += b2.x; c.y += b2.y; c.z += b2.z; c.w += b2.w;
          }
        }
      }
      xl[i] = make_uint4(pack2(v[0].x, v[0].y), pack2(v[0].z, v[0].w), pack2(v[1].x, v[1].y), pack2(v[1].z, v[1].w));
      xh[i] = make_uint4(pack2(v[2].x, v[2].y), pack2(v[2].z, v[2].w), pack2(v[3].x, v[3].y), pack2(v[3].z, v[3].w));
    }
  } else {
#pragma unroll
    for (int i = 0; i < QKR_RPG; ++i) {          // every row's 2 x 16 bytes in flight at once
      const int64_t t = t0 + i < T ? t0 + i : T - 1;
      const uint4* src = reinterpret_cast<const uint4*>(qkv + (b * T + t) * qkv_stride + (int64_t)head * 128);
      xl[i] = src[j];
      xh[i] = src[j + 8];
    }
  }
  // positions (RoPE row, cache slot) of the run's rows
  const int64_t p0 = mode == POS_T ? 0 : mode == POS_SHARED ? pos[0] : pos[b];
  int64_t rpos[QKR_RPG], slot[QKR_RPG];
#pragma unroll
  for (int i = 0; i < QKR_RPG; ++i) {
    const int64_t t = t0 + i;
    slot[i] = p0 + t;
    rpos[i] = mode == POS_TREE ? p0 + depth[b * T + (t < T ? t : T - 1)] : slot[i];
  }
  if (vhead) {                                 // V: copied into the cache as is
    const int64_t base = (b * Hkv + (head - Hq - Hkv)) * cap;
#pragma unroll
    for (int i = 0; i < QKR_RPG; ++i) {
      if (t0 + i >= T) break;                  // uniform over the wave
      if (slot[i] < 0 || slot[i] >= cap) continue;
      uint4* dst = reinterpret_cast<uint4*>(v_cache + (base + slot[i]) * 128);
      dst[j] = xl[i];
      dst[j + 8] = xh[i];
    }
    return;
  }
  float wl[8], wh[8];
  {
    const uint4* wsrc = reinterpret_cast<const uint4*>(head < Hq ? qn : kn);
    unpack8(wsrc[j], wl);
    unpack8(wsrc[j + 8], wh);
  }
  // statistics of every row of the run (all lanes active: DPP within the 8-lane group)
  float tot[QKR_RPG];
#pragma unroll
  for (int i = 0; i < QKR_RPG; ++i) {
    float a[8], c[8], sq[8];
    unpack8(xl[i], a);
    unpack8(xh[i], c);
#pragma unroll
    for (int e = 0; e < 8; ++e) sq[e] = sq_pair(a[e], c[e]);
    float s = ((sq[0] + sq[1]) + (sq[2] + sq[3])) + ((sq[4] + sq[5]) + (sq[6] + sq[7]));
    s += QD_DPP(s, 0xB1);                      // lanes j ^ 1
    s += QD_DPP(s, 0x4E);                      // lanes j ^ 2
    s += QD_DPP(s, 0x141);                     // the other quad of the 8 (row_half_mirror)
    tot[i] = s;
  }
#pragma unroll
  for (int i = 0; i < QKR_RPG; ++i) { opaque(xl[i]); opaque(xh[i]); }   // unpacked again per row
  // lane j computes rstd of row j & 3; quad_perm [i,i,i,i] hands row i's to every lane
  const int q = j & 3;
  const float tsel = q == 0 ? tot[0] : q == 1 ? tot[1] : q == 2 ? tot[2] : tot[3];
  const float rq = rstd_of(tsel, 128, eps);
  float rs[QKR_RPG];
  rs[0] = QD_DPP(rq, 0x00);
  rs[1] = QD_DPP(rq, 0x55);
  rs[2] = QD_DPP(rq, 0xAA);
  rs[3] = QD_DPP(rq, 0xFF);
  static_assert(QKR_RPG == 4, "one row per quad lane");
#pragma unroll
  for (int i = 0; i < QKR_RPG; ++i) {
    const int64_t t = t0 + i;
    if (t >= T) break;                         // uniform over the wave
    if (rpos[i] < 0 || rpos[i] >= table_len) continue;
    const int64_t row = b * T + t;
    // one packed word (dims 2k, 2k + 1 of the lane's lo and hi runs) at a time, each closed by a
    // scheduling barrier: interleaving all 16 dims would keep ~80 temporaries live and halve
    // the waves a SIMD can hold
    const uint32_t* X1 = reinterpret_cast<const uint32_t*>(&xl[i]);
    const uint32_t* X2 = reinterpret_cast<const uint32_t*>(&xh[i]);
    // cos / sin of dims 8j .. 8j + 7 (c1, s1) and 64 + 8j .. (c2, s2) of this row, fp32
    const float4* rl = rope_lds[run * QKR_RPG + i][0];
    const float4* sl = rope_lds[run * QKR_RPG + i][1];
    const float4 c1v[2] = {rl[2 * j], rl[2 * j + 1]}, c2v[2] = {rl[16 + 2 * j], rl[17 + 2 * j]};
    const float4 s1v[2] = {sl[2 * j], sl[2 * j + 1]}, s2v[2] = {sl[16 + 2 * j], sl[17 + 2 * j]};
    const float* c1 = reinterpret_cast<const float*>(c1v);
    const float* c2 = reinterpret_cast<const float*>(c2v);
    const float* s1 = reinterpret_cast<const float*>(s1v);
    const float* s2 = reinterpret_cast<const float*>(s2v);
    uint32_t ow[8];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      // norm: weight * bf16(x * rstd), rounded to bf16 (y1: the lo dims, y2: their partners)
      float y1a = bflo(X1[k]) * rs[i], y1b = bfhi(X1[k]) * rs[i];
      float y2a = bflo(X2[k]) * rs[i], y2b = bfhi(X2[k]) * rs[i];
      rbf2(y1a, y1b); rbf2(y2a, y2b);
      y1a *= wl[2 * k]; y1b *= wl[2 * k + 1];
      y2a *= wh[2 * k]; y2b *= wh[2 * k + 1];
      rbf2(y1a, y1b); rbf2(y2a, y2b);
      // rotation: o1 = bf16(y1 c1) + bf16(-y2 s1), o2 = bf16(y2 c2) + bf16(y1 s2)
      float p1a = y1a * c1[2 * k], p1b = y1b * c1[2 * k + 1];
      float q1a = -y2a * s1[2 * k], q1b = -y2b * s1[2 * k + 1];
      float p2a = y2a * c2[2 * k], p2b = y2b * c2[2 * k + 1];
      float q2a = y1a * s2[2 * k], q2b = y1b * s2[2 * k + 1];
      rbf2(p1a, p1b); rbf2(q1a, q1b); rbf2(p2a, p2b); rbf2(q2a, q2b);
      ow[k] = pack2(p1a + q1a, p1b + q1b);
      ow[4 + k] = pack2(p2a + q2a, p2b + q2b);
      __builtin_amdgcn_sched_barrier(0);
    }
    const uint4 ol = make_uint4(ow[0], ow[1], ow[2], ow[3]);
    const uint4 oh = make_uint4(ow[4], ow[5], ow[6], ow[7]);
    uint4* dst;
    if (head < Hq) {
      dst = reinterpret_cast<uint4*>(q_out + (row * Hq + head) * 128);   // q_out [B, T, Hq, 128]
    } else if (slot[i] >= 0 && slot[i] < cap) {
      dst = reinterpret_cast<uint4*>(k_cache + ((b * Hkv + (head - Hq)) * cap + slot[i]) * 128);
    } else {
      continue;
    }
    dst[j] = ol;
    dst[j + 8] = oh;
  }
}

void launch_qk_norm_rope(const bf16_t* qkv, int64_t qkv_stride, const bf16_t* qn, const bf16_t* kn,
                         const bf16_t* cos_t, const bf16_t* sin_t, int64_t table_len,
                         const int64_t* pos, const int64_t* depth, int mode, bf16_t* q_out,
                         bf16_t* k_cache, bf16_t* v_cache, int64_t B, int64_t T, int Hq, int Hkv,
                         int64_t cap, float eps, hipStream_t s) {
  if (B * T <= 0) return;
  const dim3 grid((unsigned)((T + QKR_ROWS - 1) / QKR_ROWS), (unsigned)B,
                  (unsigned)((Hq + 2 * Hkv + 15) / 16));
  qk_norm_rope_kernel<false><<<grid, dim3(256), 0, s>>>(qkv, qkv_stride, qn, kn, cos_t, sin_t,
                                                        table_len, pos, depth, mode, q_out, k_cache,
                                                        v_cache, T, Hq, Hkv, cap, eps, nullptr, 1,
                                                        B * T);
}

void launch_qk_norm_rope_part(const float* part, int S, const bf16_t* qn, const bf16_t* kn,
                              const bf16_t* cos_t, const bf16_t* sin_t, int64_t table_len,
                              const int64_t* pos, const int64_t* depth, int mode, bf16_t* q_out,
                              bf16_t* k_cache, bf16_t* v_cache, int64_t B, int64_t T, int Hq,
                              int Hkv, int64_t cap, float eps, hipStream_t s) {
  if (B * T <= 0) return;
  const dim3 grid((unsigned)((T + QKR_ROWS - 1) / QKR_ROWS), (unsigned)B,
                  (unsigned)((Hq + 2 * Hkv + 15) / 16));
  if (S == 2)
    qk_norm_rope_kernel<true, 2><<<grid, dim3(256), 0, s>>>(nullptr, 0, qn, kn, cos_t, sin_t,
                                                            table_len, pos, depth, mode, q_out,
                                                            k_cache, v_cache, T, Hq, Hkv, cap, eps,
                                                            part, S, B * T);
  else
    qk_norm_rope_kernel<true><<<grid, dim3(256), 0, s>>>(nullptr, 0, qn, kn, cos_t, sin_t, table_len,
                                                         pos, depth, mode, q_out, k_cache, v_cache,
                                                         T, Hq, Hkv, cap, eps, part, S, B * T);
}

// ------------------------------------------------------------------ SwiGLU
// act = bf16(bf16(silu(g)) * u) from packed [rows, 2*inter] (gate | up) (fused.py:101-110,
// TF:modeling_qwen3.py:81-83).
__global__ __launch_bounds__(256) void swiglu_kernel(const bf16_t* __restrict__ gu,
                                                     int64_t gu_stride, bf16_t* __restrict__ out,
                                                     int64_t out_stride, int64_t inter) {
  const int64_t row = blockIdx.y;
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (c >= inter / 8) return;
  const uint4 g = reinterpret_cast<const uint4*>(gu + row * gu_stride)[c];
  const uint4 u = reinterpret_cast<const uint4*>(gu + row * gu_stride + inter)[c];
  uint4 o;
#define SW(lo, hi, G, U) pack2(silu_rbf(lo(G)) * lo(U), silu_rbf(hi(G)) * hi(U))
  o.x = SW(bflo, bfhi, g.x, u.x);
  o.y = SW(bflo, bfhi, g.y, u.y);
  o.z = SW(bflo, bfhi, g.z, u.z);
  o.w = SW(bflo, bfhi, g.w, u.w);
#undef SW
  reinterpret_cast<uint4*>(out + row * out_stride)[c] = o;
}

void launch_swiglu(const bf16_t* gu, int64_t gu_stride, bf16_t* out, int64_t out_stride,
                   int64_t rows, int64_t inter, hipStream_t s) {
  if (rows <= 0) return;
  const unsigned gx = (unsigned)((inter / 8 + 255) / 256);
  swiglu_kernel<<<dim3(gx, (unsigned)rows), dim3(256), 0, s>>>(gu, gu_stride, out, out_stride,
                                                                inter);
}

// ------------------------------------------------------------------ KV compaction
// For the accepted tree path of row b (tree.py:145-164): for k = 1 .. cnt[b]-1,
// cache[base + k] <- cache[base + src[b, k]] in every layer, for K and V.  src[k] >= k, and
// each thread moves the same (head, 8-dim) position of every slot, so the in-order per-thread
// loop never reads a slot after it was overwritten.
__global__ __launch_bounds__(256) void kv_compact_kernel(bf16_t* k_all, bf16_t* v_all, int64_t B,
                                                         int Hkv, int64_t cap,
                                                         const int64_t* __restrict__ base,
                                                         const int32_t* __restrict__ src,
                                                         const int32_t* __restrict__ cnt,
                                                         int64_t T) {
  const int64_t layer = blockIdx.x, b = blockIdx.y;
  const int n = cnt[b];
  const int64_t bs = base[b];
  const int per = Hkv * 16;  // uint4 chunks per slot per tensor
  for (int c = threadIdx.x; c < 2 * per; c += blockDim.x) {
    bf16_t* buf = c < per ? k_all : v_all;
    const int cc = c < per ? c : c - per;
    const int h = cc / 16, d8 = cc % 16;
    uint4* head_base = reinterpret_cast<uint4*>(buf + (((layer * B + b) * Hkv + h) * cap) * 128);
    for (int k = 1; k < n && k < T; ++k) {
      const int sidx = src[b * T + k];
      if (sidx == k || sidx < 0 || sidx >= T) continue;
      const int64_t from = bs + sidx, to = bs + k;
      if (from >= cap || to >= cap) continue;
      head_base[to * 16 + d8] = head_base[from * 16 + d8];
    }
  }
}

void launch_kv_compact(bf16_t* k_all, bf16_t* v_all, int64_t L, int64_t B, int Hkv, int64_t cap,
                       const int64_t* base, const int32_t* src, const int32_t* cnt, int64_t T,
                       hipStream_t s) {
  if (L <= 0 || B <= 0) return;
  kv_compact_kernel<<<dim3((unsigned)L, (unsigned)B), dim3(256), 0, s>>>(k_all, v_all, B, Hkv,
                                                                           cap, base, src, cnt, T);
}

// ------------------------------------------------------------------ synthetic weights
// Counter-based generator (no reference counterpart: synthetic benchmark data).
//   h_w(i) = mix64(key + (2 i + w + 1) * 0x9E3779B97F4A7C15), key = seed << 32 | stream
//   value  = bf16_rne(float(sum of the 16-bit fields of h_0, h_1 - 262140) * scale)
// Integer arithmetic and one fp32 multiply, so the CPU restatement produces identical bits.
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
__device__ __forceinline__ int64_t fields16(uint64_t h) {
  return (int64_t)((h & 0xFFFF) + ((h >> 16) & 0xFFFF) + ((h >> 32) & 0xFFFF) + (h >> 48));
}
__device__ __forceinline__ uint32_t synth_one(uint64_t key, uint64_t i, float scale) {
  const uint64_t g = 0x9E3779B97F4A7C15ull;
  const uint64_t h0 = mix64(key + (2 * i + 1) * g);
  const uint64_t h1 = mix64(key + (2 * i + 2) * g);
  const float v = __fmul_rn((float)(fields16(h0) + fields16(h1) - 262140), scale);
  return f2bf(v);
}

__global__ __launch_bounds__(256) void synth_kernel(bf16_t* __restrict__ out, int64_t count,
                                                    uint64_t key, uint64_t start, float scale) {
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;  // 8 elements per thread
  const int64_t j0 = c * 8;
  if (j0 >= count) return;
  if (j0 + 8 <= count) {
    uint32_t v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = synth_one(key, start + (uint64_t)(j0 + e), scale);
    reinterpret_cast<uint4*>(out)[c] =
        make_uint4(v[0] | (v[1] << 16), v[2] | (v[3] << 16), v[4] | (v[5] << 16), v[6] | (v[7] << 16));
  } else {
    for (int64_t j = j0; j < count; ++j) out[j] = (bf16_t)synth_one(key, start + (uint64_t)j, scale);
  }
}

void launch_synth(bf16_t* out, int64_t count, uint64_t seed, uint64_t stream, uint64_t start,
                  float scale, hipStream_t s) {
  if (count <= 0) return;
  const int64_t threads = (count + 7) / 8;
  const uint64_t key = (seed << 32) | stream;
  synth_kernel<<<dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s>>>(out, count, key, start,
                                                                             scale);
}

__global__ __launch_bounds__(256) void fill_kernel(bf16_t* out, int64_t count, uint16_t value) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < count) out[i] = value;
}

void launch_fill(bf16_t* out, int64_t count, uint16_t value, hipStream_t s) {
  if (count <= 0) return;
  fill_kernel<<<dim3((unsigned)((count + 255) / 256)), dim3(256), 0, s>>>(out, count, value);
}

// ------------------------------------------------------------------ read-stream probe
// Reads n 16-byte chunks with non-temporal loads, grid-stride, four loads in flight per thread,
// folded into one word that is stored only if it equals a constant no data here produces (so
// the loads are not optimised away and nothing is written): the single-launch read rate the
// memory system gives a kernel of this size, the bound for any kernel that reads these bytes.
__global__ __launch_bounds__(256) void read_probe_kernel(const uint4* __restrict__ p, int64_t n,
                                                         uint32_t* sink) {
  int64_t i = (int64_t)blockIdx.x * 1024 + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * 1024;
  uint32_t acc = 0;
  for (; i < n; i += stride) {
    uint4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = i + u * 256 < n ? ld_stream(p + i + u * 256) : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int u = 0; u < 4; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  if (acc == 0x5EEDF00Du) sink[0] = acc;
}

void launch_read_probe(const void* buf, int64_t bytes, int grid, uint32_t* sink, hipStream_t s) {
  read_probe_kernel<<<dim3((unsigned)grid), dim3(256), 0, s>>>(static_cast<const uint4*>(buf),
                                                               bytes / 16, sink);
}

// ------------------------------------------------------------------ greedy argmax reduction
// tok[m] = index of the maximum over the per-tile (value, lowest index) partials of row m,
// lowest index on exact ties (gemv.py:147-154, fast.py:402-426); optionally pos[0] += 1.
__global__ __launch_bounds__(256) void argmax_reduce_kernel(const float* __restrict__ pval,
                                                            const int32_t* __restrict__ pidx,
                                                            int64_t nparts, int64_t* tok,
                                                            int64_t* pos_inc) {
  __shared__ float sv[256];
  __shared__ int32_t si[256];
  const int64_t m = blockIdx.x;
  float bv = -INFINITY;
  int32_t bi = 0x7FFFFFFF;
  for (int64_t p = threadIdx.x; p < nparts; p += 256) {
    const float v = pval[m * nparts + p];
    const int32_t i = pidx[m * nparts + p];
    if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
  }
  sv[threadIdx.x] = bv;
  si[threadIdx.x] = bi;
  __syncthreads();
  for (int off = 128; off > 0; off >>= 1) {
    if (threadIdx.x < off) {
      const float v = sv[threadIdx.x + off];
      const int32_t i = si[threadIdx.x + off];
      if (v > sv[threadIdx.x] || (v == sv[threadIdx.x] && i < si[threadIdx.x])) {
        sv[threadIdx.x] = v;
        si[threadIdx.x] = i;
      }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    tok[m] = si[0] == 0x7FFFFFFF ? 0 : (int64_t)si[0];
    if (pos_inc && m == 0) pos_inc[0] += 1;
  }
}

void launch_argmax_reduce(const float* pval, const int32_t* pidx, int64_t nparts, int64_t M,
                          int64_t* tok, int64_t* pos_inc, hipStream_t s) {
  if (M <= 0) return;
  argmax_reduce_kernel<<<dim3((unsigned)M), dim3(256), 0, s>>>(pval, pidx, nparts, tok, pos_inc);
}
