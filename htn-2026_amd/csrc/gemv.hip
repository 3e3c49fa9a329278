// Vector-ALU decode GEMV for 1..2 activation rows (batch B <= 2): the bf16 weight stream is
// the whole cost, so the design is about bytes in flight, not arithmetic.
//
//   out[b, n] = epi( sum_k xin[b, k] * W[n, k] )     fp32 accumulate (gemv.py:61-99, fast.py:99-158)
//   xin = NORM ? bf16(bf16(x * rstd) * norm_w) : x    (RMSNorm prologue, rmsnorm.py:26-31)
//   EPI_NONE   bf16(acc)
//   EPI_RES    bf16(res + bf16(acc))                  (residual add; res may alias out)
//   EPI_SWIGLU bf16(bf16(silu(bf16(acc_g))) * bf16(acc_u)), up rows at W + N*K
//
// Layout and schedule (gfx950, wave64):
//  * one wave owns RPW whole weight rows; lane l reads the 16-byte chunks l, l+64, l+128, ...
//    of a row, so every wave-wide load is 1 KiB contiguous (K % 512 == 0 for these shapes);
//  * the wave issues all loads of its first row(s) BEFORE the workgroup builds the normalised
//    activation in LDS, so the HBM latency overlaps the prologue; later rows are double-buffered;
//  * weights are loaded non-temporally (read once per step, never reused);
//  * the row dot is finished with a wave64 butterfly and one lane per batch row stores.
// No split-K: at B <= 2 there are enough rows (2560 .. 151936) to occupy all 256 CUs.
#include "qd_launch.h"

// The normalised activation rows go to LDS once per workgroup.  Barriers order LDS only, so
// the weight loads each wave issued before this prologue stay in flight across it.
template <int MB, int KCH, int NT>
__device__ __forceinline__ void stage_x(const bf16_t* __restrict__ x, int64_t x_stride,
                                        const bf16_t* __restrict__ norm_w, float eps, bool norm,
                                        uint4* xs, float* red) {
  constexpr int NCH = KCH * 64;  // 16-byte chunks per row
  const int nw = NT / 64;
  for (int b = 0; b < MB; ++b) {
    const uint4* xr = reinterpret_cast<const uint4*>(x + b * x_stride);
    float ss = 0.f;
    for (int c = threadIdx.x; c < NCH; c += NT) {
      const uint4 v = xr[c];
      xs[b * NCH + c] = v;
      ss += sumsq8(v);
    }
    if (!norm) continue;
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[b * nw + (threadIdx.x >> 6)] = ss;
  }
  lds_barrier();
  if (!norm) return;
  const uint4* wr = reinterpret_cast<const uint4*>(norm_w);
  for (int b = 0; b < MB; ++b) {
    float tot = 0.f;
    for (int q = 0; q < nw; ++q) tot += red[b * nw + q];
    const float rstd = rstd_of(tot, KCH * 512, eps);
    for (int c = threadIdx.x; c < NCH; c += NT) {
      xs[b * NCH + c] = norm8(xs[b * NCH + c], wr[c], rstd);
    }
  }
  lds_barrier();
}

template <int KCH, bool STREAM>
__device__ __forceinline__ void load_row(const bf16_t* __restrict__ w, int64_t n, uint4* dst) {
  const uint4* wr = reinterpret_cast<const uint4*>(w + n * (int64_t)(KCH * 512));
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < KCH; ++j) dst[j] = STREAM ? ld_stream(wr + lane + 64 * j) : wr[lane + 64 * j];
}

template <int MB, int KCH>
__device__ __forceinline__ void dot_row(const uint4* wv, const uint4* xs, float* acc) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int b = 0; b < MB; ++b) {
    float a = 0.f;
#pragma unroll
    for (int j = 0; j < KCH; ++j) a = dot8(wv[j], xs[b * KCH * 64 + lane + 64 * j], a);
    acc[b] = wave_sum(a);
  }
}

// One workgroup = NW waves; wave w owns rows [(blockIdx.x * NW + w) * RPW, ... + RPW).
// The first row's loads are issued before the LDS prologue, later rows one row ahead.
template <int MB, int KCH, int EPI, bool NORM, int RPW, int NW, bool STREAM>
__global__ __launch_bounds__(NW * 64) void gemv_kernel(const bf16_t* __restrict__ x,
                                                       int64_t x_stride,
                                                       const bf16_t* __restrict__ w, int N,
                                                       bf16_t* out, int64_t out_stride,
                                                       const bf16_t* res, int64_t res_stride,
                                                       const bf16_t* __restrict__ norm_w,
                                                       float eps) {
  constexpr bool SW = EPI == EPI_SWIGLU;
  extern __shared__ uint4 xs[];
  __shared__ float red[NW * MB];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row0 = ((int64_t)blockIdx.x * NW + wave) * RPW;
  uint4 wa[KCH], ua[SW ? KCH : 1], wb[RPW > 1 ? KCH : 1], ub[(RPW > 1 && SW) ? KCH : 1];
  if (row0 < N) {
    load_row<KCH, STREAM>(w, row0, wa);
    if constexpr (SW) load_row<KCH, STREAM>(w, row0 + N, ua);
  }
  stage_x<MB, KCH, NW * 64>(x, x_stride, norm_w, eps, NORM, xs, red);
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const int64_t n = row0 + r;
    if (n >= N) break;
    uint4* cw = (r & 1) ? wb : wa;
    uint4* cu = (r & 1) ? ub : ua;
    if (r + 1 < RPW && n + 1 < N) {
      load_row<KCH, STREAM>(w, n + 1, (r & 1) ? wa : wb);
      if constexpr (SW) load_row<KCH, STREAM>(w, n + 1 + N, (r & 1) ? ua : ub);
    }
    float ag[MB], au[MB];
    dot_row<MB, KCH>(cw, xs, ag);
    if constexpr (SW) dot_row<MB, KCH>(cu, xs, au);
    if (lane < MB) {
      const int b = lane;
      float y;
      if constexpr (EPI == EPI_RES) {
        y = bf2f(res[b * res_stride + n]) + rbf(ag[b]);
      } else if constexpr (SW) {
        y = silu_rbf(rbf(ag[b])) * rbf(au[b]);
      } else {
        y = ag[b];
      }
      out[b * out_stride + n] = (bf16_t)f2bf(y);
    }
  }
}

int gemv_supported(int64_t M, int64_t K) {
  return (M >= 1 && M <= 2) && (K == 2560 || K == 4096 || K == 9728);
}

template <int MB, int KCH, int RPW, int NW, bool STREAM>
static void gemv_go(const bf16_t* x, int64_t xs, const bf16_t* w, int64_t N, bf16_t* out,
                    int64_t os, const bf16_t* res, int64_t rs, const bf16_t* nw, float eps,
                    int epi, hipStream_t s) {
  const int64_t rows_per_wg = (int64_t)RPW * NW;
  const dim3 grid((unsigned)((N + rows_per_wg - 1) / rows_per_wg)), block(NW * 64);
  const size_t lds = (size_t)MB * KCH * 64 * sizeof(uint4);
  const bool norm = nw != nullptr;
#define GO(E, NM) \
  gemv_kernel<MB, KCH, E, NM, RPW, NW, STREAM><<<grid, block, lds, s>>>(x, xs, w, (int)N, out, os, res, rs, nw, eps)
  if (epi == EPI_RES) {
    if (norm) GO(EPI_RES, true); else GO(EPI_RES, false);
  } else if (epi == EPI_SWIGLU) {
    if (norm) GO(EPI_SWIGLU, true); else GO(EPI_SWIGLU, false);
  } else {
    if (norm) GO(EPI_NONE, true); else GO(EPI_NONE, false);
  }
#undef GO
}

// Per-shape launch configuration (rows per wave, waves per workgroup, streaming loads), chosen
// by sweeping rows/wave in {1,2,4} x waves/WG in {4,8,16} x {streaming, plain} loads on MI355X
// at B = 1 (hipGraph of 36 launches over distinct layers' weights):
//   qkv 6144x2560 -> 2 rows, 16 waves (7.9 us);  gate/up 2x9728x2560 -> 1 row, 8 waves (17.8 us)
//   o 2560x4096 -> 1 row, 4 waves (5.8 us);      down 2560x9728 -> 1 row, 4 waves (11.0 us)
template <int MB>
static void gemv_dispatch_k(const bf16_t* x, int64_t xs, const bf16_t* w, int64_t N, int64_t K,
                            bf16_t* out, int64_t os, const bf16_t* res, int64_t rs,
                            const bf16_t* nw, float eps, int epi, hipStream_t s) {
  if (K == 2560) {
    if (epi == EPI_SWIGLU) gemv_go<MB, 5, 1, 8, true>(x, xs, w, N, out, os, res, rs, nw, eps, epi, s);
    else gemv_go<MB, 5, 2, 16, true>(x, xs, w, N, out, os, res, rs, nw, eps, epi, s);
  } else if (K == 4096) {
    gemv_go<MB, 8, 1, 4, true>(x, xs, w, N, out, os, res, rs, nw, eps, epi, s);
  } else {
    gemv_go<MB, 19, 1, 4, true>(x, xs, w, N, out, os, res, rs, nw, eps, epi, s);
  }
}

void launch_gemv(const bf16_t* x, int64_t x_stride, const bf16_t* w, int64_t N, int64_t K,
                 bf16_t* out, int64_t out_stride, const bf16_t* res, int64_t res_stride,
                 const bf16_t* norm_w, float eps, int epi, int64_t M, hipStream_t s) {
  if (M == 1)
    gemv_dispatch_k<1>(x, x_stride, w, N, K, out, out_stride, res, res_stride, norm_w, eps, epi, s);
  else
    gemv_dispatch_k<2>(x, x_stride, w, N, K, out, out_stride, res, res_stride, norm_w, eps, epi, s);
}

// ------------------------------------------------------------------ LM head + greedy argmax
// Final RMSNorm prologue, bf16 logits of the tied embedding, per-workgroup (max, lowest index)
// partials; a second launch (argmax_reduce) picks the global (max, lowest index) per row and
// advances pos (fast.py:380-436; gemv.py:118-154).  RPW rows per wave, double-buffered.
constexpr int LM_RPW = 8;

int64_t lm_vec_parts(int64_t V) { return (V + 4 * LM_RPW - 1) / (4 * LM_RPW); }

template <int MB>
__global__ __launch_bounds__(256) void lm_vec_kernel(const bf16_t* __restrict__ x, int64_t x_stride,
                                                     const bf16_t* __restrict__ w, int V,
                                                     const bf16_t* __restrict__ norm_w, float eps,
                                                     float* pval, int32_t* pidx, float* logits) {
  constexpr int KCH = 5;  // K = 2560
  extern __shared__ uint4 xs[];
  __shared__ float red[4 * MB];
  __shared__ float wv_best[4][MB];
  __shared__ int32_t wi_best[4][MB];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row0 = ((int64_t)blockIdx.x * 4 + wave) * LM_RPW;
  uint4 buf[2][KCH];
  if (row0 < V) load_row<KCH, true>(w, row0, buf[0]);
  stage_x<MB, KCH, 256>(x, x_stride, norm_w, eps, true, xs, red);
  float bv[MB];
  int32_t bi[MB];
#pragma unroll
  for (int b = 0; b < MB; ++b) { bv[b] = -INFINITY; bi[b] = 0x7FFFFFFF; }
#pragma unroll
  for (int r = 0; r < LM_RPW; ++r) {
    const int64_t n = row0 + r;
    if (n >= V) break;
    if (r + 1 < LM_RPW && n + 1 < V) load_row<KCH, true>(w, n + 1, buf[(r + 1) & 1]);
    float acc[MB];
    dot_row<MB, KCH>(buf[r & 1], xs, acc);
#pragma unroll
    for (int b = 0; b < MB; ++b) {
      if (logits && lane == 0) logits[b * (int64_t)V + n] = acc[b];
      const float v = rbf(acc[b]);  // the reference's logits are bf16
      if (v > bv[b]) { bv[b] = v; bi[b] = (int32_t)n; }  // rows ascend: strict > keeps lowest
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int b = 0; b < MB; ++b) { wv_best[wave][b] = bv[b]; wi_best[wave][b] = bi[b]; }
  }
  __syncthreads();
  const int64_t nparts = gridDim.x;
  if (threadIdx.x < MB) {
    const int b = threadIdx.x;
    float v = wv_best[0][b];
    int32_t i = wi_best[0][b];
    for (int q = 1; q < 4; ++q) {
      const float v2 = wv_best[q][b];
      const int32_t i2 = wi_best[q][b];
      if (v2 > v || (v2 == v && i2 < i)) { v = v2; i = i2; }
    }
    pval[b * nparts + blockIdx.x] = v;
    pidx[b * nparts + blockIdx.x] = i;
  }
}

void launch_lm_vec(const bf16_t* x, int64_t x_stride, const bf16_t* w, int64_t V, int64_t K,
                   const bf16_t* norm_w, float eps, int64_t M, float* pval, int32_t* pidx,
                   int64_t* tok, int64_t* pos_inc, float* logits, hipStream_t s) {
  (void)K;  // the caller checked K == 2560
  const dim3 grid((unsigned)lm_vec_parts(V)), block(256);
  const size_t lds = (size_t)M * 5 * 64 * sizeof(uint4);
  if (M == 1)
    lm_vec_kernel<1><<<grid, block, lds, s>>>(x, x_stride, w, (int)V, norm_w, eps, pval, pidx,
                                              logits);
  else
    lm_vec_kernel<2><<<grid, block, lds, s>>>(x, x_stride, w, (int)V, norm_w, eps, pval, pidx,
                                              logits);
  launch_argmax_reduce(pval, pidx, lm_vec_parts(V), M, tok, pos_inc, s);
}
