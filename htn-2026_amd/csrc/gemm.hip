// MFMA decode / verify / prefill GEMM:  out[m, n] = epi( sum_k X[m, k] * W[n, k] )
// for any number of activation rows M (batched decode B >= 3, tree verification B*T rows,
// chunked prefill), with the same epilogues as the vector path plus a per-tile argmax for the
// LM head (gemv.py:61-116, fast.py:99-213, gemv.py:118-154).
//
// CDNA4 mapping (v_mfma_f32_16x16x32_bf16, wave64):
//  * a workgroup owns 16 weight rows (one MFMA N tile) and up to 64 activation rows (MT M tiles);
//    its NW waves split K into contiguous runs of 128-wide groups, summed in LDS at the end;
//  * MFMA s (s < 4) of group g contracts k = g*128 + 32 s .. +31: lane (q = lane / 16,
//    c = lane % 16) supplies k = 32 s + 8 q .. +7 of weight row n0 + c and of activation row
//    m0 + 16 mt + c, so one load instruction reads 64 contiguous bytes of each of 16 rows;
//  * each wave keeps its next D weight groups in flight (a ring refilled as groups are consumed)
//    and loads the next group's activation tiles one group ahead, so a workgroup has
//    D x NW x 4 KiB of weights outstanding instead of one group per wave;
//  * grid.x walks the M blocks fastest, so the workgroups that re-read one weight tile for
//    different M blocks run together and hit L2 / MALL instead of HBM.
// Accumulation is fp32; only the summation order differs from the reference.
#include "qd_launch.h"

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

__device__ __forceinline__ bf16x8_t as_bf8(uint4 v) { return __builtin_bit_cast(bf16x8_t, v); }

// Cross-wave reduction of the accumulators through LDS and the epilogue (store / residual /
// SwiGLU / per-tile argmax partials).
template <int MT, int EPI, int NW>
struct EpiLds {
  float red[NW][MT * 256];
  float red2[EPI == EPI_SWIGLU ? NW : 1][EPI == EPI_SWIGLU ? MT * 256 : 1];
  float tile[EPI == EPI_ARGMAX ? MT * 16 : 1][17];
};

template <int MT, int EPI, int NW>
__device__ __forceinline__ void gemm_epilogue(EpiLds<MT, EPI, NW>& sm, const f32x4_t (&acc)[MT],
                                              const f32x4_t* acc2, int64_t m0, int64_t n0, int M,
                                              int N, bf16_t* out, int64_t out_stride,
                                              const bf16_t* res, int64_t res_stride, float* pval,
                                              int32_t* pidx, float* logits) {
  constexpr bool SW = EPI == EPI_SWIGLU;
  auto& red = sm.red;
  auto& red2 = sm.red2;
  auto& tile = sm.tile;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  // D[i][j] of one 16x16 tile: lane holds rows i = 4 q + r (r < 4) of column j = c
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      red[wave][mt * 256 + lane * 4 + r] = acc[mt][r];
      if constexpr (SW) red2[wave][mt * 256 + lane * 4 + r] = acc2[mt][r];
    }
  __syncthreads();
  for (int e = threadIdx.x; e < MT * 256; e += NW * 64) {
    float v = red[0][e];
#pragma unroll
    for (int w2 = 1; w2 < NW; ++w2) v += red[w2][e];
    const int mt = e / 256, ln = (e % 256) / 4, r = e % 4;
    const int64_t m = m0 + mt * 16 + (ln >> 4) * 4 + r;
    const int64_t n = n0 + (ln & 15);
    if constexpr (EPI == EPI_ARGMAX) {
      const bool ok = m < M && n < N;
      if (ok && logits) logits[m * (int64_t)N + n] = v;
      tile[mt * 16 + (ln >> 4) * 4 + r][ln & 15] = ok ? rbf(v) : -INFINITY;
      continue;
    }
    if (m >= M || n >= N) continue;
    float y;
    if constexpr (EPI == EPI_RES) {
      y = bf2f(res[m * res_stride + n]) + rbf(v);
    } else if constexpr (SW) {
      float u = red2[0][e];
#pragma unroll
      for (int w2 = 1; w2 < NW; ++w2) u += red2[w2][e];
      y = silu_rbf(rbf(v)) * rbf(u);
    } else {
      y = v;
    }
    out[m * out_stride + n] = (bf16_t)f2bf(y);
  }
  if constexpr (EPI == EPI_ARGMAX) {
    __syncthreads();
    for (int i = threadIdx.x; i < MT * 16; i += NW * 64) {
      const int64_t m = m0 + i;
      if (m >= M) continue;
      float bv = -INFINITY;
      int32_t bi = 0x7FFFFFFF;
      for (int j = 0; j < 16; ++j) {
        const float v = tile[i][j];
        if (v > bv) { bv = v; bi = (int32_t)(n0 + j); }  // ascending n: strict > keeps lowest
      }
      pval[m * (int64_t)gridDim.y + blockIdx.y] = bv;
      pidx[m * (int64_t)gridDim.y + blockIdx.y] = bi;
    }
  }
}

// The main loop runs passes of G groups; within a pass the schedule is fully unrolled and every
// load sits in straight-line code (indices clamped into the wave's run, activation rows past M
// masked after the load), so the compiler's wait counts let the ring of D weight groups and the
// next group's activation tiles stay in flight while the current group's MFMAs run.  Only the
// MFMAs of groups past the wave's run are skipped (a wave-uniform branch with no loads in it).
template <int MT, int EPI, int NW, int G, int D>
__global__ __launch_bounds__(NW * 64) void gemm_kernel(
    const bf16_t* __restrict__ X, int64_t x_stride, int M, const bf16_t* __restrict__ W, int N,
    int K, bf16_t* out, int64_t out_stride, const bf16_t* res, int64_t res_stride, float* pval,
    int32_t* pidx, float* logits) {
  constexpr bool SW = EPI == EPI_SWIGLU;
  static_assert(D >= 1 && D <= G, "ring depth");
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int c = lane & 15, q = lane >> 4;
  const int64_t m0 = (int64_t)blockIdx.x * (MT * 16);
  const int64_t n0 = (int64_t)blockIdx.y * 16;
  const int64_t nrow = n0 + c < N ? n0 + c : N - 1;  // clamped rows are computed, never stored
  const uint4* wr = reinterpret_cast<const uint4*>(W + nrow * K);
  const uint4* wr2 = reinterpret_cast<const uint4*>(W + (nrow + (SW ? N : 0)) * K);
  const uint4* xr[MT];
  uint32_t xmask[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int64_t m = m0 + mt * 16 + c;
    xmask[mt] = m < M ? 0xFFFFFFFFu : 0u;
    xr[mt] = reinterpret_cast<const uint4*>(X + (m < M ? m : 0) * x_stride);
  }
  f32x4_t acc[MT], acc2[SW ? MT : 1];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  if constexpr (SW) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc2[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  // this wave's groups: a contiguous run [gbeg, gend) of 128-wide K groups
  const int ngroups = K / 128;
  const int per = (ngroups + NW - 1) / NW;
  const int gbeg = min(wave * per, ngroups);
  const int gend = min(gbeg + per, ngroups);
  uint4 wv[D][4], wv2[SW ? D : 1][4], xv[2][MT][4];
  for (int p0 = gbeg; p0 < gend; p0 += G) {
    const int n = min(G, gend - p0);
    // uint4 index of k = g*128 + 8 q (+ 32 s) for pass slot i, clamped into the run
    auto gcol = [&](int i) { return (int64_t)(p0 + (i < n ? i : n - 1)) * 16 + q; };
    auto load_w = [&](int slot, int i) {
      const int64_t c0 = gcol(i);
#pragma unroll
      for (int s = 0; s < 4; ++s) wv[slot][s] = ld_stream(wr + c0 + 4 * s);
      if constexpr (SW) {
#pragma unroll
        for (int s = 0; s < 4; ++s) wv2[slot][s] = ld_stream(wr2 + c0 + 4 * s);
      }
    };
    auto load_x = [&](int buf, int i) {
      const int64_t c0 = gcol(i);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          uint4 v = xr[mt][c0 + 4 * s];
          v.x &= xmask[mt]; v.y &= xmask[mt]; v.z &= xmask[mt]; v.w &= xmask[mt];
          xv[buf][mt][s] = v;
        }
    };
#pragma unroll
    for (int i = 0; i < D; ++i) load_w(i, i);
    load_x(0, 0);
#pragma unroll
    for (int i = 0; i < G; ++i) {
      if (i + 1 < G) load_x((i + 1) & 1, i + 1);
      if (i < n) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(xv[i & 1][mt][s]), as_bf8(wv[i % D][s]), acc[mt], 0, 0, 0);
            if constexpr (SW)
              acc2[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(xv[i & 1][mt][s]), as_bf8(wv2[i % D][s]), acc2[mt], 0, 0, 0);
          }
      }
      if (i + D < G) load_w(i % D, i + D);
    }
  }
  __shared__ EpiLds<MT, EPI, NW> esm;
  gemm_epilogue<MT, EPI, NW>(esm, acc, SW ? acc2 : nullptr, m0, n0, M, N, out, out_stride, res,
                             res_stride, pval, pidx, logits);
}

// ------------------------------------------------------------------ LDS-staged kernel (M <= 64)
// One 16-row weight tile (gate and up tiles for SwiGLU) x one block of MT*16 activation rows per
// workgroup of 8 waves, K in 512-wide chunks (K % 512 == 0).  Each chunk of every staged row
// (weight rows, then activation rows) is one 1 KiB-contiguous load instruction -- lane i loads
// 16-byte unit i -- written to LDS at unit i ^ (row & 15), so the MFMA fragment reads (16 rows x
// one 64-byte k slice) hit 16 distinct bank groups.  Wave w contracts k slices 2w and 2w + 1 of
// each chunk,
// and the waves' accumulators are summed in LDS at the end (gemm_epilogue).  NB chunks are in
// flight in registers (a ring refilled as each chunk is staged).  Weights stream from
// HBM in 1 KiB pieces and each activation row is read once per workgroup.
template <int MT, int EPI, int NB>
__global__ __launch_bounds__(512) void gemm_lds_kernel(
    const bf16_t* __restrict__ X, int64_t x_stride, int M, const bf16_t* __restrict__ W, int N,
    int K, bf16_t* out, int64_t out_stride, const bf16_t* res, int64_t res_stride, float* pval,
    int32_t* pidx, float* logits) {
  constexpr bool SW = EPI == EPI_SWIGLU;
  constexpr int NWV = 8;
  constexpr int WR = SW ? 32 : 16;               // staged weight rows
  constexpr int XR = MT * 16;                    // staged activation rows
  constexpr int R = WR + XR;
  static_assert(R % NWV == 0, "rows per wave");
  constexpr int LPW = R / NWV;                   // row-chunk loads per wave per chunk
  // R rows x 64 units of 16 B (512 k); after the last chunk the same LDS holds the epilogue's
  // cross-wave sums, so a workgroup needs only the staging bytes (two workgroups per CU with
  // the SwiGLU pair's 64 rows)
  constexpr int EPI_U4 = (int)((sizeof(EpiLds<MT, EPI, NWV>) + 15) / 16);
  __shared__ uint4 stage[R * 64 > EPI_U4 ? R * 64 : EPI_U4];
  EpiLds<MT, EPI, NWV>& esm = *reinterpret_cast<EpiLds<MT, EPI, NWV>*>(stage);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int c = lane & 15, q = lane >> 4;
  const int64_t m0 = (int64_t)blockIdx.x * XR;
  const int64_t n0 = (int64_t)blockIdx.y * 16;
  // source row of each of this wave's staged rows rr = wave + 8 j (clamped rows load valid data
  // whose results are never stored)
  const uint4* src[LPW];
  bool wrow[LPW];
#pragma unroll
  for (int j = 0; j < LPW; ++j) {
    const int rr = wave + NWV * j;
    if (rr < WR) {
      const int64_t nr = n0 + (rr & 15) < N ? n0 + (rr & 15) : N - 1;
      src[j] = reinterpret_cast<const uint4*>(W + (nr + (rr >= 16 ? N : 0)) * (int64_t)K);
      wrow[j] = true;
    } else {
      const int64_t mr = m0 + (rr - WR) < M ? m0 + (rr - WR) : M - 1;
      src[j] = reinterpret_cast<const uint4*>(X + mr * x_stride);
      wrow[j] = false;
    }
  }
  const int nchunks = K / 512;
  uint4 buf[NB][LPW];
  auto load = [&](int b, int kc) {
#pragma unroll
    for (int j = 0; j < LPW; ++j)
      buf[b][j] = wrow[j] ? ld_stream(src[j] + (int64_t)kc * 64 + lane) : src[j][(int64_t)kc * 64 + lane];
  };
  auto store = [&](int b) {
#pragma unroll
    for (int j = 0; j < LPW; ++j) {
      const int rr = wave + NWV * j;
      stage[rr * 64 + (lane ^ (rr & 15))] = buf[b][j];
    }
  };
  f32x4_t acc[MT], acc2[SW ? MT : 1];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  if constexpr (SW) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc2[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  auto compute = [&]() {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int u = (4 * (2 * wave + t) + q) ^ c;  // unit of k slice 2w + t, quarter q, row c
      const uint4 wf = stage[c * 64 + u];
      uint4 uf;
      if constexpr (SW) uf = stage[(16 + c) * 64 + u];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const uint4 xf = stage[(WR + 16 * mt + c) * 64 + u];
        acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(xf), as_bf8(wf), acc[mt], 0, 0, 0);
        if constexpr (SW)
          acc2[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(xf), as_bf8(uf), acc2[mt], 0, 0, 0);
      }
    }
  };
  // chunk k is staged from buf[k % NB]; chunk k + NB is then loaded into the same registers
  // (prefetches past the end re-load the last chunk: every load stays unconditional)
#pragma unroll
  for (int b = 0; b < NB; ++b) load(b, min(b, nchunks - 1));
  for (int kc = 0; kc < nchunks; kc += NB) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int k = kc + b;
      if (k < nchunks) {
        lds_barrier();                           // the previous chunk's fragments are read
        store(b);
        load(b, min(k + NB, nchunks - 1));
        lds_barrier();                           // this chunk is staged
        compute();
      }
    }
  }
  lds_barrier();                                 // every wave is done with the staged rows
  gemm_epilogue<MT, EPI, NWV>(esm, acc, SW ? acc2 : nullptr, m0, n0, M, N, out, out_stride, res,
                              res_stride, pval, pidx, logits);
}

// ------------------------------------------------------------------ streaming kernel (M <= 64)
// Weight-streaming MFMA GEMM for few activation rows (batched decode, small trees): the weights
// are read once and are the whole cost, so the design is about keeping every CU's share of the
// HBM stream going.  One workgroup per CU (grid = CU count; its LDS footprint keeps a second
// one off the CU), each owning a contiguous run of output units for the whole of K -- weight
// rows, or act rows (a gate row and its up row) for SwiGLU -- so every CU streams the same
// number of bytes and no split-K partials exist.
//  * Units are taken in passes of G 16-unit MFMA tiles; a step is one 512-wide K chunk of one
//    pass: the pass's weight rows (zeros past the run: padding is never read from HBM) and the
//    MT*16 activation rows (zeros past M) are staged in LDS, each row chunk one 1 KiB-contiguous
//    load instruction, written at unit i ^ (row & 15) (fragment reads hit 16 bank groups).
//  * NB steps are in flight in registers (a ring refilled as each step is staged); the ring
//    runs across pass boundaries, so the stream does not drain between passes.
//  * Output block (tile t, activation tile mt) belongs to one wave for the whole of K
//    (mt = wave % MT): no cross-wave reduction; the epilogue runs after a pass's last chunk.
// Accumulation is fp32 in k order within the chunk's 16 MFMAs; only the summation order
// differs from the reference.
// Used for the LM head (argmax epilogue, ~600 rows per workgroup).  For the projections
// (10-76 rows per workgroup at 256 CUs) re-staging the activation rows with every chunk costs
// more than the even split gains (measured at 32 rows: qkv 17.4 vs 13.7 us, gate/up 39.4 vs
// 30.4 us), so they stay on gemm_lds_kernel.
template <int MT, int EPI, int G>
constexpr int stream_nb() {
  constexpr int sr = (EPI == EPI_SWIGLU ? 2 : 1) * G * 16 + MT * 16;
  constexpr int lpw = sr / 8;
  return lpw <= 6 ? 4 : lpw <= 12 ? 3 : 2;
}

template <int MT, int EPI, int G, int NB>
__global__ __launch_bounds__(512) void gemm_stream_kernel(
    const bf16_t* __restrict__ X, int64_t x_stride, int M, const bf16_t* __restrict__ W, int N,
    int K, bf16_t* out, int64_t out_stride, const bf16_t* res, int64_t res_stride, float* pval,
    int32_t* pidx, float* logits) {
  constexpr bool SW = EPI == EPI_SWIGLU, AM = EPI == EPI_ARGMAX;
  constexpr int NWV = 8;
  constexpr int TU = G * 16;                    // units per pass
  constexpr int WR = SW ? 2 * TU : TU;          // staged weight rows (gate rows, then up rows)
  constexpr int XR = MT * 16;                   // staged activation rows
  constexpr int SR = WR + XR;
  static_assert(SR % NWV == 0 && NWV % MT == 0, "rows per wave");
  constexpr int LPW = SR / NWV;                 // row-chunk loads per wave per step
  constexpr int NBLK = G * MT;                  // output blocks per pass
  constexpr int BPW = (NBLK + NWV - 1) / NWV;   // blocks per wave
  constexpr int LDS_U4 = SR * 64 > 5248 ? SR * 64 : 5248;   // >= 82 KiB: one workgroup per CU
  __shared__ uint4 stage[LDS_U4];
  __shared__ float am_v[AM ? NWV : 1][AM ? XR : 1];
  __shared__ int32_t am_i[AM ? NWV : 1][AM ? XR : 1];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, c = lane & 15, q = lane >> 4;
  const int mt = wave % MT;                     // this wave's activation tile
  const int P = gridDim.x, wg = blockIdx.x;
  const int64_t u0 = (int64_t)N * wg / P, u1 = (int64_t)N * (wg + 1) / P;
  const int npass = (int)((u1 - u0 + TU - 1) / TU);
  const int nchunks = K / 512;
  const int S = npass * nchunks;                // steps (pass, chunk), chunk fastest
  uint4 buf[NB][LPW];
  // step s into ring slot b; a step past the end loads only activation rows (no HBM bytes)
  auto load = [&](int b, int s) {
    const int p = s / nchunks, kc = s - p * nchunks;
    const int64_t t0 = u0 + (int64_t)p * TU;
#pragma unroll
    for (int j = 0; j < LPW; ++j) {
      const int rr = wave + NWV * j;
      if (rr < WR) {
        const int u = rr % TU;
        const bool ok = s < S && t0 + u < u1;
        const int64_t row = (ok ? t0 + u : 0) + (rr >= TU ? N : 0);
        const uint4* src = reinterpret_cast<const uint4*>(W + row * K) + kc * 64 + lane;
        buf[b][j] = ok ? ld_stream(src) : make_uint4(0, 0, 0, 0);
      } else {
        const int m = rr - WR;
        const uint4 v = reinterpret_cast<const uint4*>(X + (int64_t)(m < M ? m : 0) * x_stride)[kc * 64 + lane];
        buf[b][j] = m < M ? v : make_uint4(0, 0, 0, 0);
      }
    }
  };
  auto store = [&](int b) {
#pragma unroll
    for (int j = 0; j < LPW; ++j) {
      const int rr = wave + NWV * j;
      stage[rr * 64 + (lane ^ (rr & 15))] = buf[b][j];
    }
  };
  f32x4_t acc[BPW], acc2[SW ? BPW : 1];
  auto zero = [&]() {
#pragma unroll
    for (int i = 0; i < BPW; ++i) {
      acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      if constexpr (SW) acc2[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
  };
  zero();
  auto compute = [&]() {
#pragma unroll
    for (int i = 0; i < BPW; ++i) {
      const int blk = wave + NWV * i;
      if (blk < NBLK) {
        const int t = blk / MT;
#pragma unroll
        for (int s = 0; s < 16; ++s) {          // k = 32 s + 8 q .. +7 of the chunk
          const int u = (4 * s + q) ^ c;
          const uint4 xf = stage[(WR + 16 * mt + c) * 64 + u];
          const uint4 wf = stage[(16 * t + c) * 64 + u];
          acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(xf), as_bf8(wf), acc[i], 0, 0, 0);
          if constexpr (SW) {
            const uint4 uf = stage[(TU + 16 * t + c) * 64 + u];
            acc2[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(xf), as_bf8(uf), acc2[i], 0, 0, 0);
          }
        }
      }
    }
  };
  // argmax state: lane (c, q) tracks rows m = 16 mt + 4 q + r over its columns
  float bv[4];
  int32_t bi[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) { bv[r] = -INFINITY; bi[r] = 0x7FFFFFFF; }
  // D of a block: lane (c, q) holds rows m = 16 mt + 4 q + r (r < 4) of unit column 16 t + c
  auto epilogue = [&](int p) {
    const int64_t t0 = u0 + (int64_t)p * TU;
#pragma unroll
    for (int i = 0; i < BPW; ++i) {
      const int blk = wave + NWV * i;
      if (blk < NBLK) {
        const int64_t n = t0 + 16 * (blk / MT) + c;
        if (n < u1) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int m = 16 * mt + 4 * q + r;
            if (m >= M) continue;
            const float v = acc[i][r];
            if constexpr (AM) {
              if (logits) logits[m * (int64_t)N + n] = v;
              const float vb = rbf(v);            // the reference's logits are bf16
              if (vb > bv[r]) { bv[r] = vb; bi[r] = (int32_t)n; }   // n ascends per lane
            } else {
              float y;
              if constexpr (EPI == EPI_RES) {
                y = bf2f(res[m * res_stride + n]) + rbf(v);
              } else if constexpr (SW) {
                y = silu_rbf(rbf(v)) * rbf(acc2[i][r]);
              } else {
                y = v;
              }
              out[m * out_stride + n] = (bf16_t)f2bf(y);
            }
          }
        }
      }
    }
    zero();
  };
#pragma unroll
  for (int b = 0; b < NB; ++b) load(b, b);
  for (int s0 = 0; s0 < S; s0 += NB) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int s = s0 + b;
      if (s < S) {
        lds_barrier();                           // the previous step's fragments are read
        store(b);
        load(b, s + NB);
        lds_barrier();                           // this step is staged
        compute();
        const int p = s / nchunks;
        if (s - p * nchunks == nchunks - 1) epilogue(p);
      }
    }
  }
  if constexpr (AM) {
    // best per row over the 16 columns of a lane group, then over the waves of this tile
#pragma unroll
    for (int r = 0; r < 4; ++r) {
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) {
        const float v2 = __shfl_xor(bv[r], off, 64);
        const int32_t i2 = __shfl_xor(bi[r], off, 64);
        if (v2 > bv[r] || (v2 == bv[r] && i2 < bi[r])) { bv[r] = v2; bi[r] = i2; }
      }
    }
    for (int e = lane; e < XR; e += 64) { am_v[wave][e] = -INFINITY; am_i[wave][e] = 0x7FFFFFFF; }
    __syncthreads();
    if (c == 0) {
#pragma unroll
      for (int r = 0; r < 4; ++r) { am_v[wave][16 * mt + 4 * q + r] = bv[r]; am_i[wave][16 * mt + 4 * q + r] = bi[r]; }
    }
    __syncthreads();
    for (int m = threadIdx.x; m < M && m < XR; m += NWV * 64) {
      float v = am_v[0][m];
      int32_t ix = am_i[0][m];
      for (int w2 = 1; w2 < NWV; ++w2) {
        const float v2 = am_v[w2][m];
        const int32_t i2 = am_i[w2][m];
        if (v2 > v || (v2 == v && i2 < ix)) { v = v2; ix = i2; }
      }
      pval[m * (int64_t)P + wg] = v;
      pidx[m * (int64_t)P + wg] = ix;
    }
  }
}

int64_t gemm_argmax_parts(int64_t N) { return (N + 15) / 16; }

// Waves per workgroup and groups per pass from the number of 128-wide K groups: K <= 2560 -> 4
// waves x 5 groups; K <= 5120 -> 8 x 5; otherwise 8 waves x 10 groups per pass.  Ring depth:
// the whole pass for one M tile (4 groups with the gate/up pair), 4 for two, 2 for four (whose
// activation buffers take the registers).
template <int MT, int EPI, int NW, int G>
static void gemm_launch(const bf16_t* x, int64_t xs, int64_t M, const bf16_t* w, int64_t N,
                        int64_t K, bf16_t* out, int64_t os, const bf16_t* res, int64_t rs,
                        float* pval, int32_t* pidx, float* logits, hipStream_t s) {
  constexpr bool SW = EPI == EPI_SWIGLU;
  constexpr int D0 = MT >= 4 ? 2 : MT == 2 ? 4 : (SW ? 4 : G);
  constexpr int D = D0 < G ? D0 : G;
  const dim3 grid((unsigned)((M + MT * 16 - 1) / (MT * 16)), (unsigned)((N + 15) / 16));
  gemm_kernel<MT, EPI, NW, G, D><<<grid, dim3(NW * 64), 0, s>>>(x, xs, (int)M, w, (int)N, (int)K,
                                                               out, os, res, rs, pval, pidx, logits);
}

template <int MT, int EPI>
static void gemm_go(const bf16_t* x, int64_t xs, int64_t M, const bf16_t* w, int64_t N, int64_t K,
                    bf16_t* out, int64_t os, const bf16_t* res, int64_t rs, float* pval,
                    int32_t* pidx, float* logits, hipStream_t s) {
  const int64_t ng = K / 128;
  if (ng <= 20)
    gemm_launch<MT, EPI, 4, 5>(x, xs, M, w, N, K, out, os, res, rs, pval, pidx, logits, s);
  else if (ng <= 40)
    gemm_launch<MT, EPI, 8, 5>(x, xs, M, w, N, K, out, os, res, rs, pval, pidx, logits, s);
  else
    gemm_launch<MT, EPI, 8, 10>(x, xs, M, w, N, K, out, os, res, rs, pval, pidx, logits, s);
}

#ifndef QD_GEMM_NB
#define QD_GEMM_NB 2
#endif
template <int MT, int EPI, int NB = QD_GEMM_NB>
static void gemm_lds_go(const bf16_t* x, int64_t xs, int64_t M, const bf16_t* w, int64_t N,
                        int64_t K, bf16_t* out, int64_t os, const bf16_t* res, int64_t rs,
                        float* pval, int32_t* pidx, float* logits, hipStream_t s) {
  const dim3 grid((unsigned)((M + MT * 16 - 1) / (MT * 16)), (unsigned)((N + 15) / 16));
  gemm_lds_kernel<MT, EPI, NB><<<grid, dim3(512), 0, s>>>(x, xs, (int)M, w, (int)N, (int)K, out,
                                                          os, res, rs, pval, pidx, logits);
}

// one workgroup per CU
static int stream_grid() {
  static int grid = -1;
  if (grid < 0) {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
      (void)hipGetLastError();
      cus = 0;
    }
    grid = cus;
  }
  return grid;
}

template <int MT, int EPI, int G>
static void stream_go(const bf16_t* x, int64_t xs, int64_t M, const bf16_t* w, int64_t N,
                      int64_t K, bf16_t* out, int64_t os, const bf16_t* res, int64_t rs,
                      float* pval, int32_t* pidx, float* logits, int P, hipStream_t s) {
  constexpr int NB = stream_nb<MT, EPI, G>();
  gemm_stream_kernel<MT, EPI, G, NB><<<dim3((unsigned)P), dim3(512), 0, s>>>(
      x, xs, (int)M, w, (int)N, (int)K, out, os, res, rs, pval, pidx, logits);
}

// Passes of G tiles from the units per workgroup: o / down (10 units at 256 CUs) one tile,
// qkv (24) two, gate/up (38 act rows) three gate + three up tiles (two at 64 rows, where the
// activation tiles take the LDS), the LM head (594) four per pass.
// The LM head: four 16-row tiles per pass (~600 rows per workgroup at 256 CUs).
template <int MT, int EPI>
static int64_t stream_mt(const bf16_t* x, int64_t xs, int64_t M, const bf16_t* w, int64_t N,
                         int64_t K, bf16_t* out, int64_t os, const bf16_t* res, int64_t rs,
                         float* pval, int32_t* pidx, float* logits, int P, hipStream_t s) {
  static_assert(EPI == EPI_ARGMAX, "the streaming kernel serves the LM head");
  stream_go<MT, EPI, 4>(x, xs, M, w, N, K, out, os, res, rs, pval, pidx, logits, P, s);
  return P;
}

template <int EPI>
static int64_t gemm_mt(const bf16_t* x, int64_t xs, int64_t M, const bf16_t* w, int64_t N,
                       int64_t K, bf16_t* out, int64_t os, const bf16_t* res, int64_t rs,
                       float* pval, int32_t* pidx, float* logits, float* part, int64_t part_floats,
                       hipStream_t s) {
  if (M >= GEMM_TILE_MIN_M && gemm_tile_ok(M, N, K, EPI, x, xs, w, out, os, res, rs))
    return launch_gemm_tile(x, xs, M, w, N, K, out, os, res, rs, EPI, pval, pidx, logits, part,
                            part_floats, s);
  const int P = stream_grid();
  const bool aligned = xs % 8 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(w) % 16 == 0;
  // the LM head: 3..32 rows on the skinny argmax kernel (activations resident in LDS per K
  // phase); 33..64 rows on the weight-streaming kernel (~600 rows per workgroup, so its per-chunk
  // activation re-reads stay small next to the weight rows); the projections: 3..32 rows on the
  // skinny kernel, 33..64 on the LDS-staged one
  if constexpr (EPI == EPI_ARGMAX) {
    if (M <= 32) {
      const int64_t parts = launch_lm_skinny(x, xs, M, w, N, K, pval, pidx, logits, s);
      if (parts > 0) return parts;
    }
    if (M <= 64 && K % 512 == 0 && aligned && P >= 1) {
      if (M <= 16) return stream_mt<1, EPI>(x, xs, M, w, N, K, out, os, res, rs, pval, pidx, logits, P, s);
      if (M <= 32) return stream_mt<2, EPI>(x, xs, M, w, N, K, out, os, res, rs, pval, pidx, logits, P, s);
      return stream_mt<4, EPI>(x, xs, M, w, N, K, out, os, res, rs, pval, pidx, logits, P, s);
    }
  }
  if constexpr (EPI != EPI_ARGMAX) {
    // 3..32 rows: the skinny kernel (one workgroup per CU, waves split K), unsplit here
    if (M <= 32 && launch_gemm_skinny(x, xs, M, w, N, K, EPI, 1, out, os, res, rs, nullptr, s))
      return 0;
  }
  if (M <= 64 && K % 512 == 0) {
    if (M <= 16) gemm_lds_go<1, EPI>(x, xs, M, w, N, K, out, os, res, rs, pval, pidx, logits, s);
    else gemm_lds_go<2, EPI>(x, xs, M, w, N, K, out, os, res, rs, pval, pidx, logits, s);
  } else if (M <= 16) {
    gemm_go<1, EPI>(x, xs, M, w, N, K, out, os, res, rs, pval, pidx, logits, s);
  } else if (M <= 32) {
    gemm_go<2, EPI>(x, xs, M, w, N, K, out, os, res, rs, pval, pidx, logits, s);
  } else {
    gemm_go<4, EPI>(x, xs, M, w, N, K, out, os, res, rs, pval, pidx, logits, s);
  }
  return EPI == EPI_ARGMAX ? gemm_argmax_parts(N) : 0;
}

int64_t launch_gemm(const bf16_t* x, int64_t x_stride, int64_t M, const bf16_t* w, int64_t N,
                    int64_t K, bf16_t* out, int64_t out_stride, const bf16_t* res,
                    int64_t res_stride, int epi, float* pval, int32_t* pidx, float* logits,
                    hipStream_t s, float* part, int64_t part_floats) {
  if (M <= 0) return 0;
#define QD_MT(E) \
  gemm_mt<E>(x, x_stride, M, w, N, K, out, out_stride, res, res_stride, pval, pidx, logits, part, \
             part_floats, s)
  switch (epi) {
    case EPI_RES: return QD_MT(EPI_RES);
    case EPI_SWIGLU: return QD_MT(EPI_SWIGLU);
    case EPI_ARGMAX: return QD_MT(EPI_ARGMAX);
    default: return QD_MT(EPI_NONE);
  }
#undef QD_MT
}
