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
__global__ __launch_bounds__(256) void part_add_rmsnorm_kernel(
    const float* __restrict__ part, int S, int64_t rows, bf16_t* res, const bf16_t* __restrict__ w,
    bf16_t* __restrict__ y, int64_t hidden, float eps) {
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
      for (int s = 1; s < S; ++s) {
        const float4* ps = reinterpret_cast<const float4*>(part + ((int64_t)s * rows + row) * hidden) + 2 * c;
        const float4 a2 = ps[0], b2 = ps[1];
        a.x += a2.x; a.y += a2.y; a.z += a2.z; a.w += a2.w;
        b.x += b2.x; b.y += b2.y; b.z += b2.z; b.w += b2.w;
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

void launch_part_add_rmsnorm(const float* part, int S, int64_t rows, bf16_t* res, const bf16_t* w,
                             bf16_t* y, int64_t hidden, float eps, hipStream_t s) {
  if (rows <= 0) return;
  part_add_rmsnorm_kernel<<<dim3((unsigned)rows), dim3(256), 0, s>>>(part, S, rows, res, w, y,
                                                                      hidden, eps);
}

void launch_add_rmsnorm(const bf16_t* x, const bf16_t* res, const bf16_t* w, bf16_t* res_out,
                        bf16_t* y, int64_t rows, int64_t hidden, int64_t in_stride,
                        int64_t y_stride, float eps, hipStream_t s) {
  if (rows <= 0) return;
  add_rmsnorm_kernel<<<dim3((unsigned)rows), dim3(256), 0, s>>>(x, res, w, res_out, y, hidden,
                                                                 in_stride, y_stride, eps);
}

// ------------------------------------------------------------------ q/k RMSNorm + RoPE + KV write
// 16 lanes per (token row, head in [0, Hq + 2 Hkv)), 16 heads x 4 rows per workgroup: lane j
// of a head holds dims 8j .. 8j+7 as one 16-byte load, so a wave moves 1 KiB per access and
// the rotate_half partner of lane j (dims 64 apart) is lane j ^ 8 of the same DPP row.
// Per-head RMSNorm (q_norm / k_norm weights), then
//   o1 = bf16(bf16(y1 c1) + bf16(-y2 s1)),  o2 = bf16(bf16(y2 c2) + bf16(y1 s2))
// for each (d, d + 64) pair (fused.py:24-81, tree.py:26-69, TF:modeling_qwen3.py:140-170,
// 252-257).  The 64 sum-of-squares terms sq_pair(x_d, x_{d+64}) are added as a balanced binary
// tree in index order -- within the lane over its 8 pairs, then across lanes j = 0..7 -- the
// same tree wave_sum builds over lanes d = 0..63 in the decode attention unit, so the
// statistics are bit-identical to the decode step's.  V heads are copied unnormalised into
// the cache.  Position of token t of row b:
//   POS_T t | POS_SHARED pos[0]+t | POS_ROW pos[b]+t | POS_CHUNK pos[b]+t (= slot)
//   POS_TREE: RoPE at pos[b] + depth[b*T + t], cache slot pos[b] + t.
__device__ __forceinline__ uint32_t row_xor8(uint32_t v) {    // lane ^ 8 within a 16-lane row
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xF, 0xF, true);   // row_ror:8
}
__device__ __forceinline__ uint4 row_xor8(const uint4 v) {
  return make_uint4(row_xor8(v.x), row_xor8(v.y), row_xor8(v.z), row_xor8(v.w));
}
__device__ __forceinline__ void unpack8(const uint4 v, float (&f)[8]) {
  f[0] = bflo(v.x); f[1] = bfhi(v.x); f[2] = bflo(v.y); f[3] = bfhi(v.y);
  f[4] = bflo(v.z); f[5] = bfhi(v.z); f[6] = bflo(v.w); f[7] = bfhi(v.w);
}

constexpr int QKR_ROWS = 4;   // token rows per workgroup: their loads are issued together

// PART: the packed qkv rows are the split-K partials of the qkv projection, part[S][B*T][width]
// fp32 (the tiled GEMM's split layout): each value is their sum in split order rounded to
// bf16, the same bits gemm_split_reduce_kernel would have stored.
template <bool PART>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(
    const bf16_t* __restrict__ qkv, int64_t qkv_stride, const bf16_t* __restrict__ qn,
    const bf16_t* __restrict__ kn, const bf16_t* __restrict__ cos_t,
    const bf16_t* __restrict__ sin_t, int64_t table_len, const int64_t* __restrict__ pos,
    const int64_t* __restrict__ depth, int mode, bf16_t* __restrict__ q_out,
    bf16_t* __restrict__ k_cache, bf16_t* __restrict__ v_cache, int64_t T, int Hq, int Hkv,
    int64_t cap, float eps, const float* __restrict__ part, int S, int64_t rows_total) {
  // grid (token blocks of QKR_ROWS, sequence b, head group of 16): no integer division
  const int head = (int)blockIdx.z * 16 + (threadIdx.x >> 4);
  if (head >= Hq + 2 * Hkv) return;            // whole 16-lane groups leave together
  const int64_t b = blockIdx.y;
  const int64_t t0 = (int64_t)blockIdx.x * QKR_ROWS;
  const int j = threadIdx.x & 15;
  const bool vhead = head >= Hq + Hkv, lo = j < 8;
  uint4 xr[QKR_ROWS];
  if constexpr (PART) {
    const int64_t width = (int64_t)(Hq + 2 * Hkv) * 128;
#pragma unroll
    for (int i = 0; i < QKR_ROWS; ++i) {
      const int64_t t = t0 + i < T ? t0 + i : T - 1;
      const int64_t col = (b * T + t) * width + (int64_t)head * 128 + 8 * j;
      const float4* p0 = reinterpret_cast<const float4*>(part + col);
      float4 a = p0[0], c2 = p0[1];
      for (int sp = 1; sp < S; ++sp) {
        const float4* ps = reinterpret_cast<const float4*>(part + (int64_t)sp * rows_total * width + col);
        const float4 a2 = ps[0], b2 = ps[1];
        a.x += a2.x; a.y += a2.y; a.z += a2.z; a.w += a2.w;
        c2.x += b2.x; c2.y += b2.y; c2.z += b2.z; c2.w += b2.w;
      }
      xr[i] = make_uint4(pack2(a.x, a.y), pack2(a.z, a.w), pack2(c2.x, c2.y), pack2(c2.z, c2.w));
    }
  } else {
#pragma unroll
    for (int i = 0; i < QKR_ROWS; ++i) {         // every row's 16 bytes in flight at once
      const int64_t t = t0 + i < T ? t0 + i : T - 1;
      xr[i] = reinterpret_cast<const uint4*>(qkv + (b * T + t) * qkv_stride + (int64_t)head * 128)[j];
    }
  }
  const uint4 w = reinterpret_cast<const uint4*>(head < Hq ? qn : kn)[j];
#pragma unroll
  for (int i = 0; i < QKR_ROWS; ++i) {
    const int64_t t = t0 + i;
    if (t >= T) break;                         // uniform over the workgroup
    const int64_t row = b * T + t;
    int64_t rpos, slot;
    switch (mode) {
      case POS_T: rpos = slot = t; break;
      case POS_SHARED: rpos = slot = pos[0] + t; break;
      case POS_TREE: slot = pos[b] + t; rpos = pos[b] + depth[row]; break;
      default: rpos = slot = pos[b] + t; break;  // POS_ROW, POS_CHUNK
    }
    const uint4 x = xr[i];
    if (vhead) {                               // V: copied into the cache as is
      if (slot >= 0 && slot < cap)
        reinterpret_cast<uint4*>(v_cache + ((b * Hkv + (head - Hq - Hkv)) * cap + slot) * 128)[j] = x;
      continue;
    }
    if (rpos < 0 || rpos >= table_len) continue;   // per row: the whole group
    float xs[8], xp[8];
    unpack8(x, xs);
    unpack8(row_xor8(x), xp);                  // the partner dims (d +- 64)
    float sq[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) sq[e] = lo ? sq_pair(xs[e], xp[e]) : sq_pair(xp[e], xs[e]);
    float tot = ((sq[0] + sq[1]) + (sq[2] + sq[3])) + ((sq[4] + sq[5]) + (sq[6] + sq[7]));
    tot += QD_DPP(tot, 0xB1);                  // lanes j ^ 1
    tot += QD_DPP(tot, 0x4E);                  // lanes j ^ 2
    tot += QD_DPP(tot, 0x141);                 // the other 4-lane half of the 8 (row_half_mirror)
    const float r = rstd_of(tot, 128, eps);
    const uint4 y = norm8(x, w, r);            // bf16-rounded normed values of my dims
    float ys[8], yp[8], c[8], sn[8];
    unpack8(y, ys);
    unpack8(row_xor8(y), yp);
    unpack8(reinterpret_cast<const uint4*>(cos_t + rpos * 128)[j], c);
    unpack8(reinterpret_cast<const uint4*>(sin_t + rpos * 128)[j], sn);
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e)
      o[e] = lo ? rbf(ys[e] * c[e]) + rbf(-yp[e] * sn[e]) : rbf(ys[e] * c[e]) + rbf(yp[e] * sn[e]);
    const uint4 ov = make_uint4(pack2(o[0], o[1]), pack2(o[2], o[3]), pack2(o[4], o[5]),
                                pack2(o[6], o[7]));
    if (head < Hq) {
      reinterpret_cast<uint4*>(q_out + (row * Hq + head) * 128)[j] = ov;   // q_out [B, T, Hq, 128]
    } else if (slot >= 0 && slot < cap) {
      reinterpret_cast<uint4*>(k_cache + ((b * Hkv + (head - Hq)) * cap + slot) * 128)[j] = ov;
    }
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
  qk_norm_rope_kernel<true><<<grid, dim3(256), 0, s>>>(nullptr, 0, qn, kn, cos_t, sin_t, table_len,
                                                       pos, depth, mode, q_out, k_cache, v_cache, T,
                                                       Hq, Hkv, cap, eps, part, S, B * T);
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
#define SW(lo, hi, G, U) pack2(rbf(silu_f(lo(G))) * lo(U), rbf(silu_f(hi(G))) * hi(U))
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
