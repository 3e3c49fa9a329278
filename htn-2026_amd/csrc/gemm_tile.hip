// LDS-tiled MFMA GEMM for many activation rows (tree verification B*T rows, prefill chunks):
//   out[m, n] = epi( sum_k X[m, k] * W[n, k] )
// with the epilogues of the decode GEMM (store / residual / SwiGLU / per-tile argmax for the LM
// head) -- the large-M counterpart of the reference's tensor-core GEMMs (gemv.py:61-116 with
// BLOCK_M >= 16, fast.py:161-213) and of its cuBLAS prefill (engine.py:550-592).
//
// CDNA4 mapping (v_mfma_f32_16x16x32_bf16, wave64, 160 KiB LDS per CU):
//  * a workgroup of 4 waves owns a 128 (weight rows) x 128 (activation rows) output tile; wave
//    (wn, wm) owns the 64 x 64 quarter (4 x 4 MFMA tiles, 64 fp32 accumulators per lane);
//  * K advances in stages of 64: both 128-row x 128-byte tiles are staged in LDS, each row as 8
//    16-byte units stored at unit ^ (row & 7), so the fragment reads (16 rows x one 16-byte unit)
//    and the staging writes (8 rows x 8 units per 8 lanes) hit distinct banks;
//  * two LDS buffers (64 KiB, two workgroups per CU) and a two-deep register ring: the global
//    loads of stage s + 2 are issued before stage s is contracted, stage s + 1 is written to the
//    other buffer after it, so one barrier per stage and two stages of loads in flight;
//  * A = weight rows, B = activation rows: the accumulator lane (c, q) holds output columns
//    n..n+3 (4 q + r) of row m (c), so every epilogue store is one 8-byte write;
//  * workgroup ids are remapped so the tiles that one XCD runs are consecutive in (M block
//    fastest, then N block): the M blocks that share a weight tile run on one XCD and meet in its
//    L2 instead of each XCD fetching the tile from HBM;
//  * when the tile grid is too small to fill the chip (few rows, narrow N), K is split over
//    workgroups; the fp32 partial tiles go to a caller-provided workspace and a second kernel
//    sums them in split order and applies the epilogue (deterministic).
// Requirements (checked by gemm_tile_ok): K % 64 == 0, N % 128 == 0 (SwiGLU: N % 64 == 0),
// 16-byte aligned X / W rows, 8-byte aligned output / residual rows.
#include "qd_launch.h"

namespace {

constexpr int TM = 128, TN = 128, TK = 64;
#ifndef QD_TILE_RING
#define QD_TILE_RING 2
#endif
// K stages of loads in flight per thread (even).  Measured on MI355X: 4 stages (250 VGPRs)
// took 8.18 ms per config-5 verify forward against 8.01 ms with 2 and left the 4 x 8192
// prefill unchanged -- the 256-row projections are not bound by load latency.
constexpr int TILE_RING = QD_TILE_RING;
static_assert(TILE_RING % 2 == 0, "the ring slots and the two LDS buffers advance together");
#ifndef QD_TILE_GROUP_M
#define QD_TILE_GROUP_M 8
#endif
constexpr int TILE_GROUP_M = QD_TILE_GROUP_M;
#ifndef QD_BIG_GROUP_M
#define QD_BIG_GROUP_M 4  // 256 x 256 tiles: 4 M blocks per group (8: 1-4 % slower at 32768 rows)
#endif
constexpr int BIG_GROUP_M = QD_BIG_GROUP_M;
#ifndef QD_TILE8
#define QD_TILE8 1        // 8-wave 128 x 128 tiles below the 256 x 256 kernel's row count
#endif
#ifndef QD_BIG_MIN_M
#define QD_BIG_MIN_M 1024
#endif
#ifndef QD_TILE_ROWS
#define QD_TILE_ROWS 1     // all-rows kernel at 65..256 rows
#endif
#ifndef QD_BIG_ARGMAX_MIN_M
#define QD_BIG_ARGMAX_MIN_M 129   // LM head rows from which the 256 x 256 argmax tile is used
#endif
#ifndef QD_BIG_EPIS
#define QD_BIG_EPIS 7     // epilogues (bit EPI_NONE, EPI_RES, EPI_SWIGLU) that take the big tile
#endif

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

__device__ __forceinline__ bf16x8_t as_bf8(uint4 v) { return __builtin_bit_cast(bf16x8_t, v); }

struct TileLds {
  uint4 w[2][TN * 8];
  uint4 x[2][TM * 8];
};

// one stage of one thread's staging units: 4 weight and 4 activation 16-byte units (named
// registers: arrays here end up in scratch or LDS)
struct Stage {
  uint4 w0, w1, w2, w3, x0, x1, x2, x3;
};
struct Src {
  const uint4 *W, *X;
  int64_t w0, w1, w2, w3, x0, x1, x2, x3;   // uint4 offsets of the thread's 4 + 4 rows
};
__device__ __forceinline__ void load_stage(Stage& st, const Src& s, int64_t kk) {
  st.w0 = ld_stream(s.W + s.w0 + kk);
  st.w1 = ld_stream(s.W + s.w1 + kk);
  st.w2 = ld_stream(s.W + s.w2 + kk);
  st.w3 = ld_stream(s.W + s.w3 + kk);
  st.x0 = s.X[s.x0 + kk];
  st.x1 = s.X[s.x1 + kk];
  st.x2 = s.X[s.x2 + kk];
  st.x3 = s.X[s.x3 + kk];
}
__device__ __forceinline__ void store_stage(const Stage& st, uint4* lw, uint4* lx) {
  lw[0] = st.w0;
  lw[256] = st.w1;
  lw[512] = st.w2;
  lw[768] = st.w3;
  lx[0] = st.x0;
  lx[256] = st.x1;
  lx[512] = st.x2;
  lx[768] = st.x3;
}

template <int EPI, bool SPLIT>
__global__ __launch_bounds__(256, 2) void gemm_tile_kernel(
    const bf16_t* __restrict__ X, int64_t x_stride, int M, const bf16_t* __restrict__ W, int N,
    int K, int mblocks, int nblocks, int ks_per, bf16_t* out, int64_t out_stride, const bf16_t* res,
    int64_t res_stride, float* pval, int32_t* pidx, float* logits, float* part) {
  __shared__ TileLds sm;
  __shared__ float amax_v[2][2][64];
  __shared__ int32_t amax_i[2][2][64];
  // XCD-aware remap: hardware workgroup h runs on XCD h % 8; give each XCD a contiguous run of
  // logical tiles
  const int total = gridDim.x, h = blockIdx.x;
  const int xq = total >> 3, xr = total & 7, xcd = h & 7, slot = h >> 3;
  const int L = xcd < xr ? xcd * (xq + 1) + slot : xr * (xq + 1) + (xcd - xr) * xq + slot;
  // within a K split, tiles go in groups of TILE_GROUP_M M blocks: M fastest inside a group,
  // then N, so the workgroups one XCD runs at a time cover a few M blocks x many N blocks and
  // both the weight tiles and the activation tiles they read are shared in that XCD's L2
  const int tiles = mblocks * nblocks;
  const int split = L / tiles;
  const int Lt = L - split * tiles;
  const int group = Lt / (TILE_GROUP_M * nblocks);
  const int first = group * TILE_GROUP_M;
  const int gm = min(TILE_GROUP_M, mblocks - first);
  const int rr = Lt - first * nblocks;
  const int mb = first + rr % gm;
  const int nb = rr / gm;

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int c = lane & 15, q = lane >> 4;
  const int wn = wave & 1, wm = wave >> 1;
  const int64_t m0 = (int64_t)mb * TM;
  const int ksteps = K / TK;
  const int kbeg = split * ks_per;
  const int kend = min(ksteps, kbeg + ks_per);

  // staging: thread tid moves units u = tid + 256 i (i < 4) of both tiles: row r0 + 32 i
  // (r0 = tid / 8), unit tid % 8.  Weight row of LDS row r0 + 32 i: nb*128 + r0 + 32 i, or for
  // SwiGLU (gate | up halves of W, 64 output columns per block) nb*64 + r0 + 32 (i / 2) plus N
  // for odd i (the up rows).
  const int r0 = tid >> 3, unit0 = tid & 7;
  const int Nrows = EPI == EPI_SWIGLU ? 2 * N : N;
  auto wrow_of = [&](int i) -> int64_t {
    const int64_t wr = EPI == EPI_SWIGLU
                           ? (int64_t)nb * 64 + r0 + 32 * (i >> 1) + ((i & 1) ? N : 0)
                           : (int64_t)nb * TN + r0 + 32 * i;
    return (wr < Nrows ? wr : Nrows - 1) * (K / 8) + unit0;          // in uint4 units
  };
  auto xrow_of = [&](int i) -> int64_t {
    const int64_t xm = m0 + r0 + 32 * i;
    return (xm < M ? xm : M - 1) * (x_stride / 8) + unit0;
  };
  const Src src{reinterpret_cast<const uint4*>(W), reinterpret_cast<const uint4*>(X),
                wrow_of(0), wrow_of(1), wrow_of(2), wrow_of(3),
                xrow_of(0), xrow_of(1), xrow_of(2), xrow_of(3)};
  uint4* lw0 = &sm.w[0][r0 * 8 + (unit0 ^ (r0 & 7))];              // + 256 i: rows + 32 i
  uint4* lx0 = &sm.x[0][r0 * 8 + (unit0 ^ (r0 & 7))];
  Stage st[TILE_RING];
// (the scheduling barrier keeps the loads at the head of the stage: left free, the scheduler
// moves them behind the contraction and shortens the prefetch distance)
#define QD_LOAD(SLOT, KS)                                          \
  {                                                                \
    load_stage(st[SLOT], src, ((KS) < kend ? (KS) : kend - 1) * 8);\
    __builtin_amdgcn_sched_barrier(0);                             \
  }
#define QD_STORE(SLOT, BUF) store_stage(st[SLOT], lw0 + (BUF) * (TN * 8), lx0 + (BUF) * (TM * 8))
  f32x4_t acc[4][4];
#pragma unroll
  for (int nt = 0; nt < 4; ++nt)
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) acc[nt][mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const int fa = (64 * wn + c) * 8, fb = (64 * wm + c) * 8;           // fragment rows (+ 128 t)
#define QD_COMPUTE(BUF)                                                                        \
  _Pragma("unroll") for (int s_ = 0; s_ < 2; ++s_) {                                           \
    const int u_ = (4 * s_ + q) ^ (c & 7);                                                     \
    uint4 a_[4], b_[4];                                                                        \
    _Pragma("unroll") for (int t = 0; t < 4; ++t) a_[t] = sm.w[BUF][fa + 128 * t + u_];        \
    _Pragma("unroll") for (int t = 0; t < 4; ++t) b_[t] = sm.x[BUF][fb + 128 * t + u_];        \
    _Pragma("unroll") for (int nt = 0; nt < 4; ++nt)                                           \
    _Pragma("unroll") for (int mt = 0; mt < 4; ++mt)                                           \
      acc[nt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(a_[nt]), as_bf8(b_[mt]),    \
                                                            acc[nt][mt], 0, 0, 0);             \
  }

  // Stage s sits in LDS buffer s & 1 while the loads of stages s + 1 .. s + TILE_RING are in
  // flight in the register ring (slot s % TILE_RING is refilled with stage s + TILE_RING once
  // stage s is in LDS).  Each stage: refill, contract, write stage s + 1 into the other buffer,
  // one barrier.  The loop body is TILE_RING stages with no exit between them (an exit there lets
  // the compiler sink loads to their use, behind the contraction they are meant to overlap);
  // the last partial round is guarded stage by stage.  Loads past the last stage are clamped.
#pragma unroll
  for (int r = 0; r < TILE_RING; ++r) QD_LOAD(r, kbeg + r);
  QD_STORE(0, 0);
  lds_barrier();
  int ks = kbeg;
  for (; ks + TILE_RING <= kend; ks += TILE_RING) {
#pragma unroll
    for (int r = 0; r < TILE_RING; ++r) {
      QD_LOAD(r, ks + r + TILE_RING);
      QD_COMPUTE(r & 1);
      QD_STORE((r + 1) % TILE_RING, (r + 1) & 1);
      lds_barrier();
    }
  }
#pragma unroll
  for (int r = 0; r < TILE_RING; ++r) {
    if (ks + r < kend) {
      QD_COMPUTE(r & 1);
      if (ks + r + 1 < kend) {
        QD_STORE((r + 1) % TILE_RING, (r + 1) & 1);
        lds_barrier();
      }
    }
  }
#undef QD_LOAD
#undef QD_STORE
#undef QD_COMPUTE

  // ---------------------------------------------------------------- epilogue
  // lane (c, q) of acc[nt][mt] holds rows 4 q + r (r < 4) of the weight tile = output columns
  // n .. n + 3, for activation row m = m0 + 64 wm + 16 mt + c
  if constexpr (SPLIT) {
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const int64_t m = m0 + 64 * wm + 16 * mt + c;
      if (m >= M) continue;
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const int64_t n = (int64_t)nb * TN + 64 * wn + 16 * nt + 4 * q;
        *reinterpret_cast<f32x4_t*>(part + ((int64_t)split * M + m) * N + n) = acc[nt][mt];
      }
    }
  } else if constexpr (EPI == EPI_ARGMAX) {
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const int64_t m = m0 + 64 * wm + 16 * mt + c;
      const bool ok = m < M;
      float bv = -INFINITY;
      int32_t bi = 0x7FFFFFFF;
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const int64_t n = (int64_t)nb * TN + 64 * wn + 16 * nt + 4 * q;
        if (ok && logits) *reinterpret_cast<f32x4_t*>(logits + m * (int64_t)N + n) = acc[nt][mt];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float v = rbf(acc[nt][mt][r]);
          if (v > bv) { bv = v; bi = (int32_t)(n + r); }   // ascending n within the lane
        }
      }
      // across the four q lanes of row c (interleaved column ranges): lowest index on ties
#pragma unroll
      for (int sh = 0; sh < 2; ++sh) {
        const float ov = sh ? lane_xor32(bv) : lane_xor16(bv);
        const int32_t oi = sh ? __builtin_bit_cast(int32_t, lane_xor32(__builtin_bit_cast(float, bi)))
                              : __builtin_bit_cast(int32_t, lane_xor16(__builtin_bit_cast(float, bi)));
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
      }
      if (q == 0) {
        amax_v[wm][wn][16 * mt + c] = bv;
        amax_i[wm][wn][16 * mt + c] = bi;
      }
    }
    lds_barrier();
    if (tid < 128) {
      const int wm2 = tid >> 6, r = tid & 63;
      const int64_t m = m0 + 64 * wm2 + r;
      if (m < M) {
        float bv = amax_v[wm2][0][r];
        int32_t bi = amax_i[wm2][0][r];
        const float ov = amax_v[wm2][1][r];
        const int32_t oi = amax_i[wm2][1][r];
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
        pval[m * (int64_t)nblocks + nb] = bv;
        pidx[m * (int64_t)nblocks + nb] = bi;
      }
    }
  } else {
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const int64_t m = m0 + 64 * wm + 16 * mt + c;
      if (m >= M) continue;
      if constexpr (EPI == EPI_SWIGLU) {
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          const int64_t n = (int64_t)nb * 64 + 32 * wn + 16 * nt + 4 * q;
          float y[4];
#pragma unroll
          for (int r = 0; r < 4; ++r)
            y[r] = silu_rbf(rbf(acc[nt][mt][r])) * rbf(acc[nt + 2][mt][r]);
          *reinterpret_cast<uint2*>(out + m * out_stride + n) =
              make_uint2(pack2(y[0], y[1]), pack2(y[2], y[3]));
        }
      } else {
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
          const int64_t n = (int64_t)nb * TN + 64 * wn + 16 * nt + 4 * q;
          float y[4];
          if constexpr (EPI == EPI_RES) {
            const uint2 rv = *reinterpret_cast<const uint2*>(res + m * res_stride + n);
            y[0] = bflo(rv.x) + rbf(acc[nt][mt][0]);
            y[1] = bfhi(rv.x) + rbf(acc[nt][mt][1]);
            y[2] = bflo(rv.y) + rbf(acc[nt][mt][2]);
            y[3] = bfhi(rv.y) + rbf(acc[nt][mt][3]);
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r) y[r] = acc[nt][mt][r];
          }
          *reinterpret_cast<uint2*>(out + m * out_stride + n) =
              make_uint2(pack2(y[0], y[1]), pack2(y[2], y[3]));
        }
      }
    }
  }
}

// ------------------------------------------------------------------ 128 x 128 tiles, 8 waves
// The same tile, K stages, LDS layout, remap and split-K as gemm_tile_kernel, with 8 waves per
// workgroup instead of 4: wave (wm, wn) owns activation rows 64 wm .. x weight rows 32 wn ..
// (4 x 2 MFMA tiles), so each SIMD holds two waves of one workgroup (four when two workgroups
// share a CU) to overlap one wave's loads and LDS traffic with another's MFMAs.  SwiGLU: a
// wave's 32 weight rows are 16 gate rows and the 16 up rows of the same outputs.
struct Stage8 {
  uint4 w0, w1, x0, x1;
};

template <int EPI, bool SPLIT>
__global__ __launch_bounds__(512, 2) void gemm_tile8_kernel(
    const bf16_t* __restrict__ X, int64_t x_stride, int M, const bf16_t* __restrict__ W, int N,
    int K, int mblocks, int nblocks, int ks_per, bf16_t* out, int64_t out_stride, const bf16_t* res,
    int64_t res_stride, float* part) {
  static_assert(EPI != EPI_ARGMAX, "the LM head keeps the 4-wave kernel");
  __shared__ TileLds sm;
  const int total = gridDim.x, h = blockIdx.x;
  const int xq = total >> 3, xr = total & 7, xcd = h & 7, slot = h >> 3;
  const int L = xcd < xr ? xcd * (xq + 1) + slot : xr * (xq + 1) + (xcd - xr) * xq + slot;
  const int tiles = mblocks * nblocks;
  const int split = L / tiles;
  const int Lt = L - split * tiles;
  const int group = Lt / (TILE_GROUP_M * nblocks);
  const int first = group * TILE_GROUP_M;
  const int gm = min(TILE_GROUP_M, mblocks - first);
  const int rr = Lt - first * nblocks;
  const int mb = first + rr % gm;
  const int nb = rr / gm;

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int c = lane & 15, q = lane >> 4;
  const int wn = wave & 3, wm = wave >> 2;
  const int64_t m0 = (int64_t)mb * TM;
  const int ksteps = K / TK;
  const int kbeg = split * ks_per;
  const int kend = min(ksteps, kbeg + ks_per);

  // staging: thread tid moves unit tid % 8 of LDS rows r0 + 64 i (r0 = tid / 8, i < 2) of both
  // tiles.  Weight row of LDS row R: nb*128 + R, or for SwiGLU nb*64 + 16 (R / 32) + R % 16,
  // plus N when (R / 16) is odd (the up rows)
  const int r0 = tid >> 3, unit0 = tid & 7;
  const int Nrows = EPI == EPI_SWIGLU ? 2 * N : N;
  auto wrow_of = [&](int i) -> int64_t {
    const int R = r0 + 64 * i;
    const int64_t wr = EPI == EPI_SWIGLU
                           ? (int64_t)nb * 64 + 16 * (R >> 5) + (R & 15) + (((R >> 4) & 1) ? N : 0)
                           : (int64_t)nb * TN + R;
    return (wr < Nrows ? wr : Nrows - 1) * (K / 8) + unit0;          // in uint4 units
  };
  auto xrow_of = [&](int i) -> int64_t {
    const int64_t xm = m0 + r0 + 64 * i;
    return (xm < M ? xm : M - 1) * (x_stride / 8) + unit0;
  };
  const uint4* W4 = reinterpret_cast<const uint4*>(W);
  const uint4* X4 = reinterpret_cast<const uint4*>(X);
  const int64_t wo0 = wrow_of(0), wo1 = wrow_of(1), xo0 = xrow_of(0), xo1 = xrow_of(1);
  uint4* lw0 = &sm.w[0][r0 * 8 + (unit0 ^ (r0 & 7))];              // + 512: rows + 64
  uint4* lx0 = &sm.x[0][r0 * 8 + (unit0 ^ (r0 & 7))];
  Stage8 st0, st1;
  auto load = [&](Stage8& st, int ks) {
    const int64_t kk = (int64_t)(ks < kend ? ks : kend - 1) * 8;
    st.w0 = ld_stream(W4 + wo0 + kk);
    st.w1 = ld_stream(W4 + wo1 + kk);
    st.x0 = X4[xo0 + kk];
    st.x1 = X4[xo1 + kk];
    __builtin_amdgcn_sched_barrier(0);
  };
  auto store = [&](const Stage8& st, int buf) {
    lw0[buf * (TN * 8)] = st.w0;
    lw0[buf * (TN * 8) + 512] = st.w1;
    lx0[buf * (TM * 8)] = st.x0;
    lx0[buf * (TM * 8) + 512] = st.x1;
  };
  f32x4_t acc[2][4];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt)
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) acc[nt][mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const int fa = (32 * wn + c) * 8, fb = (64 * wm + c) * 8;           // fragment rows (+ 128 t)
  auto compute = [&](int buf) {
#pragma unroll
    for (int s_ = 0; s_ < 2; ++s_) {
      const int u_ = (4 * s_ + q) ^ (c & 7);
      uint4 a_[2], b_[4];
#pragma unroll
      for (int t = 0; t < 2; ++t) a_[t] = sm.w[buf][fa + 128 * t + u_];
#pragma unroll
      for (int t = 0; t < 4; ++t) b_[t] = sm.x[buf][fb + 128 * t + u_];
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
          acc[nt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(a_[nt]), as_bf8(b_[mt]),
                                                                acc[nt][mt], 0, 0, 0);
    }
  };
  // as gemm_tile_kernel: stage s in LDS buffer s & 1, loads of stages s + 1, s + 2 in flight
  load(st0, kbeg);
  load(st1, kbeg + 1);
  store(st0, 0);
  lds_barrier();
  int ks = kbeg;
  for (; ks + 1 < kend; ks += 2) {
    load(st0, ks + 2);
    compute(0);
    store(st1, 1);
    lds_barrier();
    load(st1, ks + 3);
    compute(1);
    store(st0, 0);
    lds_barrier();
  }
  if (ks < kend) compute(0);

  // epilogue: lane (c, q) of acc[nt][mt] holds weight rows 4 q + r of tile nt = output columns
  // n .. n + 3 of activation row m = m0 + 64 wm + 16 mt + c
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    const int64_t m = m0 + 64 * wm + 16 * mt + c;
    if (m >= M) continue;
    if constexpr (SPLIT) {
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        const int64_t n = (int64_t)nb * TN + 32 * wn + 16 * nt + 4 * q;
        *reinterpret_cast<f32x4_t*>(part + ((int64_t)split * M + m) * N + n) = acc[nt][mt];
      }
    } else if constexpr (EPI == EPI_SWIGLU) {
      const int64_t n = (int64_t)nb * 64 + 16 * wn + 4 * q;
      float y[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) y[r] = silu_rbf(rbf(acc[0][mt][r])) * rbf(acc[1][mt][r]);
      *reinterpret_cast<uint2*>(out + m * out_stride + n) = make_uint2(pack2(y[0], y[1]), pack2(y[2], y[3]));
    } else {
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        const int64_t n = (int64_t)nb * TN + 32 * wn + 16 * nt + 4 * q;
        float y[4];
        if constexpr (EPI == EPI_RES) {
          const uint2 rv = *reinterpret_cast<const uint2*>(res + m * res_stride + n);
          y[0] = bflo(rv.x) + rbf(acc[nt][mt][0]);
          y[1] = bfhi(rv.x) + rbf(acc[nt][mt][1]);
          y[2] = bflo(rv.y) + rbf(acc[nt][mt][2]);
          y[3] = bfhi(rv.y) + rbf(acc[nt][mt][3]);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) y[r] = acc[nt][mt][r];
        }
        *reinterpret_cast<uint2*>(out + m * out_stride + n) = make_uint2(pack2(y[0], y[1]), pack2(y[2], y[3]));
      }
    }
  }
}

// Sum of the split partials in split order + epilogue (store / residual); one thread per four
// consecutive output columns.
template <int EPI>
__global__ __launch_bounds__(256) void gemm_split_reduce_kernel(const float* __restrict__ part,
                                                                int splits, int64_t M, int64_t N,
                                                                bf16_t* out, int64_t out_stride,
                                                                const bf16_t* res,
                                                                int64_t res_stride) {
  const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t n4 = N / 4;
  if (g >= M * n4) return;
  const int64_t m = g / n4, n = 4 * (g % n4);
  // partials summed in split order, loaded eight at a time before any of them is added
  constexpr int RB = 8;
  f32x4_t a = *reinterpret_cast<const f32x4_t*>(part + m * N + n);
  for (int z0 = 1; z0 < splits; z0 += RB) {
    f32x4_t v[RB];
#pragma unroll
    for (int i = 0; i < RB; ++i)
      v[i] = z0 + i < splits ? *reinterpret_cast<const f32x4_t*>(part + ((int64_t)(z0 + i) * M + m) * N + n)
                             : f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < RB; ++i)
      if (z0 + i < splits) a += v[i];
  }
  float y[4];
  if constexpr (EPI == EPI_RES) {
    const uint2 rv = *reinterpret_cast<const uint2*>(res + m * res_stride + n);
    y[0] = bflo(rv.x) + rbf(a[0]);
    y[1] = bfhi(rv.x) + rbf(a[1]);
    y[2] = bflo(rv.y) + rbf(a[2]);
    y[3] = bfhi(rv.y) + rbf(a[3]);
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r) y[r] = a[r];
  }
  *reinterpret_cast<uint2*>(out + m * out_stride + n) = make_uint2(pack2(y[0], y[1]), pack2(y[2], y[3]));
}

// ------------------------------------------------------------------ 256 x 256 tiles (prefill)
// At prefill row counts (thousands of activation rows) the 128 x 128 tile above moves every
// weight and activation byte through L1 once per 128 rows of the other operand (6.4 GB of
// L1->L2 reads per 4096-row gate/up launch, a third of them L2 misses even with the grouped
// tile order) and keeps the MFMA pipe 30 % busy.  This kernel doubles the tile both ways, halving
// the traffic per flop: a workgroup of 8 waves (two per SIMD) owns 256 weight rows x 256
// activation rows, wave (wm, wn) the 128 activation rows 128 wm .. x the 64 weight rows 64 wn ..
// (4 x 8 MFMA tiles, 128 fp32 accumulators per lane).  K advances in stages of 64 that go from
// global memory straight into LDS (global_load_lds_dwordx4: no staging registers, no LDS store
// instructions), two stage buffers of 64 KiB.  Each load instruction fetches whole 128-byte
// lines (8 rows x 128 bytes): with stages of 32 (16 rows x 64 bytes per instruction, half lines)
// the same kernel ran 6-10 % slower, and a timing copy whose loads all hit one L1 line ran 25-30
// % faster than either -- the cost is in the L1/L2 request stream, not in the LDS writes.  (With
// the loads staged through registers only one 64-deep stage fitted in flight, and a copy of that
// kernel without its MFMAs took 539 us of the full kernel's 714 us for a 6144-row gate/up.)
// SwiGLU: a wave's 64 weight rows are 32 gate rows and the 32 up rows of the same outputs.
constexpr int BT = 256;                      // weight rows and activation rows per workgroup
constexpr int BK = 64;                       // K per stage: 128 bytes of every row

// 8 waves (two per SIMD), two along the activation rows and four along the weight rows: wave
// (wm, wn) owns activation rows 128 wm .. and weight rows 64 wn .. (8 x 4 MFMA tiles, 128 fp32
// accumulators per lane).  SwiGLU: a wave's 64 weight rows are 32 gate rows and the 32 up rows
// of the same outputs.  Offsets are 32-bit (checked by the launcher).  (Four waves of 128 x 128,
// one per SIMD as in hipBLASLt's 256 x 256 tiles, need their 256 accumulators in the AGPRs; with
// the fragment double buffer below the compiler spilled 241 registers.)
constexpr int BIG_WAVES = 8;
template <int EPI>
__global__ __launch_bounds__(BIG_WAVES * 64, 1) void gemm_big_kernel(
    const bf16_t* __restrict__ X, int64_t x_stride, int M, const bf16_t* __restrict__ W, int N,
    int K, int mblocks, int nblocks, bf16_t* out, int64_t out_stride, const bf16_t* res,
    int64_t res_stride, float* pval, int32_t* pidx, float* logits) {
  constexpr int WAVES = BIG_WAVES;
  constexpr int WN = WAVES / 2;              // waves along the weight rows
  constexpr int NT = BT / WN / 16;           // MFMA tiles per wave along the weight rows
  constexpr int HALF = NT * 8;               // SwiGLU: gate rows per wave
  constexpr int ROWS = BT / WAVES;           // LDS rows of each tile a wave loads per stage
  constexpr int BLK = ROWS / 8;              // ... as 1 KiB blocks of 8 rows (one load each)
  static_assert(NT == 4 && BLK == 4, "the step below interleaves 4 x 2 loads with 4 x 8 MFMAs");
  // [stage buffer][weights, activations][row * 8 + position]: row r's 128 bytes hold its eight
  // 16-byte K units, unit u at position u ^ (r % 8), so that the 8 lanes of a fragment read
  // (rows c .. c + 7, one unit each) cover all 128 bytes of the banks
  __shared__ uint4 sm[2][2][BT * 8];
  const int total = gridDim.x, h = blockIdx.x;
  const int xq = total >> 3, xr = total & 7, xcd = h & 7, slot = h >> 3;
  const int L = xcd < xr ? xcd * (xq + 1) + slot : xr * (xq + 1) + (xcd - xr) * xq + slot;
  const int group = L / (BIG_GROUP_M * nblocks);
  const int first = group * BIG_GROUP_M;
  const int gm = min(BIG_GROUP_M, mblocks - first);
  const int rr = L - first * nblocks;
  const int mb = first + rr % gm;
  const int nb = rr / gm;

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int c = lane & 15, q = lane >> 4;
  const int wn = wave % WN, wm = wave / WN;
  const int64_t m0 = (int64_t)mb * BT;
  const int stages = K / BK;
  // weight row of LDS row r: plain nb*256 + r; SwiGLU: LDS rows [2 HALF j, 2 HALF j + HALF) are
  // the gate rows of outputs nb*128 + HALF j .., the next HALF the up rows (+ N) of the same outputs
  auto wrow = [&](int r) -> int64_t {
    if constexpr (EPI == EPI_SWIGLU) {
      return (int64_t)nb * 128 + HALF * (r / (2 * HALF)) + (r % HALF) + (((r / HALF) & 1) ? N : 0);
    } else if constexpr (EPI == EPI_ARGMAX) {
      const int64_t n = (int64_t)nb * BT + r;          // the last block may pass the vocabulary:
      return n < N ? n : N - 1;                        // reload a valid row, never ranked
    } else {
      return (int64_t)nb * BT + r;
    }
  };
  auto xrow = [&](int r) -> int64_t {
    const int64_t m = m0 + r;
    return m < M ? m : M - 1;
  };
  // loads: wave v fills LDS rows ROWS v .. of both tiles as BLK 1 KiB blocks of 8 rows; lane l
  // of a block writes position l % 8 of row l / 8 (row % 8 = l / 8), i.e. K unit (l % 8) ^ (l / 8)
  const int unit = (lane & 7) ^ (lane >> 3);
  uint32_t wof[BLK], xof[BLK];
#pragma unroll
  for (int j = 0; j < BLK; ++j) {
    const int r = ROWS * wave + 8 * j + (lane >> 3);
    wof[j] = (uint32_t)(wrow(r) * K * 2 + unit * 16);
    xof[j] = (uint32_t)(xrow(r) * x_stride * 2 + unit * 16);
  }
  const uint32_t lbase = __builtin_amdgcn_readfirstlane(lds_u32(&sm[0][0][0])) + wave * ROWS * 128;
  constexpr uint32_t XOFF = BT * 8 * 16, BUF = 2 * XOFF;   // activation tile, stage buffer (bytes)
  // load i (0..7) of stage st into buffer b: weights 0..3, activations 4..7
  auto load = [&](int st, int b, int i) {
    const char* base = reinterpret_cast<const char*>(i < BLK ? (const void*)W : (const void*)X) +
                       (size_t)st * (BK * 2);
    const int j = i % BLK;
    dma16(base, i < BLK ? wof[j] : xof[j], lbase + (uint32_t)b * BUF + (i < BLK ? 0u : XOFF) + 1024u * j);
  };
  f32x4_t acc[NT][8];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) acc[nt][mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // fragment of K half hf (units 4 hf .. 4 hf + 3) of a 16-row tile: lane (c, q) reads unit
  // 4 hf + q of row tile + c, at position (4 hf + q) ^ (c % 8); tiles are 16 rows = 128 uint4 apart
  const int pa0 = (64 * wn + c) * 8, pb0 = (128 * wm + c) * 8;
  const int u0 = q ^ (c & 7), u1 = (4 + q) ^ (c & 7);
  // fragments of one K half: NT weight tiles, 8 activation tiles (one 16-byte unit per lane each)
  struct Frag {
    uint4 a[NT], b[8];
  };
  // read fragment t (0..11: weight tiles 0..3, then activation tiles 0..7) of half hf of buffer b
  auto rd = [&](Frag& f, int b, int hf, int t) {
    const int u = hf ? u1 : u0;
    if (t < NT) f.a[t] = sm[b][0][pa0 + 128 * t + u];
    else f.b[t - NT] = sm[b][1][pb0 + 128 * (t - NT) + u];
  };
  // Sub-step j contracts K half j (stage j / 2) from registers while the fragments of half j + 1
  // are read, in four groups of (two loads, three fragment reads, eight MFMAs) so the load and
  // LDS instructions issue between MFMAs.  Stage s lives in buffer s % 2.  Odd sub-steps read the
  // next stage: they first wait for this wave's loads (all of them: stage s + 1 is the only one
  // in flight) and meet the other waves at a barrier, after which every wave's stage s + 1 has
  // landed and every wave has read stage s out of its buffer, which then takes stage s + 2 (the
  // loads of that sub-step).  One barrier per stage.
  auto sub = [&](int s, int hf, const Frag& cur, Frag& nxt) {
    const int b = s & 1;
    const bool ld = hf && s + 2 < stages, rdn = !hf || s + 1 < stages;
    const int rb = hf ? b ^ 1 : b;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      if (ld) {
        load(s + 2, b, 2 * g);
        load(s + 2, b, 2 * g + 1);
      }
      if (rdn) {
#pragma unroll
        for (int t = 3 * g; t < 3 * g + 3; ++t) rd(nxt, rb, hf ^ 1, t);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int mt = 2 * g; mt < 2 * g + 2; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
          acc[nt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(cur.a[nt]), as_bf8(cur.b[mt]),
                                                                acc[nt][mt], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
#pragma unroll
  for (int i = 0; i < 2 * BLK; ++i) load(0, 0, i);
  if (stages > 1) {
#pragma unroll
    for (int i = 0; i < 2 * BLK; ++i) load(1, 1, i);
    wait_vm<2 * BLK>();                        // stage 0 landed (stage 1 still in flight)
  } else {
    wait_vm<0>();
  }
  lds_barrier();
  Frag f0, f1;
#pragma unroll
  for (int t = 0; t < NT + 8; ++t) rd(f0, 0, 0, t);
  for (int s = 0; s < stages; ++s) {
    sub(s, 0, f0, f1);
    wait_vm<0>();
    lds_barrier();
    sub(s, 1, f1, f0);
  }

  // epilogue: lane (c, q) of acc[nt][mt] holds weight rows 4 q + r of tile nt = output columns
  // n .. n + 3 of activation row m = m0 + 128 wm + 16 mt + c
  if constexpr (EPI == EPI_ARGMAX) {
    // LM head: per activation row the maximum bf16 logit of the block's 256 vocabulary rows and
    // its lowest index (the lane's columns ascend with nt and r; lanes and waves hold interleaved
    // column ranges, so ties compare indices) -> pval / pidx[m][nb] for argmax_reduce_kernel
    __shared__ float amax_v[2][WN][128];
    __shared__ int32_t amax_i[2][WN][128];
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) {
      const int64_t m = m0 + 128 * wm + 16 * mt + c;
      float bv = -INFINITY;
      int32_t bi = 0x7FFFFFFF;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const int64_t n = (int64_t)nb * BT + NT * 16 * wn + 16 * nt + 4 * q;
        if (m < M && logits && n < N)
          *reinterpret_cast<f32x4_t*>(logits + m * (int64_t)N + n) = acc[nt][mt];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float v = rbf(acc[nt][mt][r]);
          if (n + r < N && v > bv) { bv = v; bi = (int32_t)(n + r); }
        }
      }
#pragma unroll
      for (int sh = 0; sh < 2; ++sh) {
        const float ov = sh ? lane_xor32(bv) : lane_xor16(bv);
        const int32_t oi = sh ? __builtin_bit_cast(int32_t, lane_xor32(__builtin_bit_cast(float, bi)))
                              : __builtin_bit_cast(int32_t, lane_xor16(__builtin_bit_cast(float, bi)));
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
      }
      if (q == 0) {
        amax_v[wm][wn][16 * mt + c] = bv;
        amax_i[wm][wn][16 * mt + c] = bi;
      }
    }
    lds_barrier();
    if (tid < 256) {
      const int wm2 = tid >> 7, r = tid & 127;
      const int64_t m = m0 + 128 * wm2 + r;
      if (m < M) {
        float bv = amax_v[wm2][0][r];
        int32_t bi = amax_i[wm2][0][r];
#pragma unroll
        for (int w = 1; w < WN; ++w) {
          const float ov = amax_v[wm2][w][r];
          const int32_t oi = amax_i[wm2][w][r];
          if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
        }
        pval[m * (int64_t)nblocks + nb] = bv;
        pidx[m * (int64_t)nblocks + nb] = bi;
      }
    }
    return;
  }
#pragma unroll
  for (int mt = 0; mt < 8; ++mt) {
    const int64_t m = m0 + 128 * wm + 16 * mt + c;
    if (m >= M) continue;
    if constexpr (EPI == EPI_SWIGLU) {
#pragma unroll
      for (int nt = 0; nt < NT / 2; ++nt) {
        const int64_t n = (int64_t)nb * 128 + HALF * wn + 16 * nt + 4 * q;
        float y[4];
#pragma unroll
        for (int r = 0; r < 4; ++r)
          y[r] = silu_rbf(rbf(acc[nt][mt][r])) * rbf(acc[nt + NT / 2][mt][r]);
        *reinterpret_cast<uint2*>(out + m * out_stride + n) = make_uint2(pack2(y[0], y[1]), pack2(y[2], y[3]));
      }
    } else {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const int64_t n = (int64_t)nb * BT + NT * 16 * wn + 16 * nt + 4 * q;
        float y[4];
        if constexpr (EPI == EPI_RES) {
          const uint2 rv = *reinterpret_cast<const uint2*>(res + m * res_stride + n);
          y[0] = bflo(rv.x) + rbf(acc[nt][mt][0]);
          y[1] = bfhi(rv.x) + rbf(acc[nt][mt][1]);
          y[2] = bflo(rv.y) + rbf(acc[nt][mt][2]);
          y[3] = bfhi(rv.y) + rbf(acc[nt][mt][3]);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) y[r] = acc[nt][mt][r];
        }
        *reinterpret_cast<uint2*>(out + m * out_stride + n) = make_uint2(pack2(y[0], y[1]), pack2(y[2], y[3]));
      }
    }
  }
}

// ------------------------------------------------------------------ all rows per workgroup (65..256)
// At a few hundred activation rows (a tree-verification forward: B x T = 256) a workgroup owns a
// block of weight rows for 128 MT of the activation rows (all of them, or one of two halves):
// 8 waves, wave w the 16 MT activation rows 16 MT w .. (NT x MT MFMA tiles; SwiGLU: NT gate
// tiles and the NT up tiles of the same outputs); K in stages of 64 that go from global memory
// straight into LDS (128-byte rows, unit u at u ^ (row & 7); the weight rows shared by the
// waves), RW_NBUF stage buffers, RW_NBUF - 1 stages in flight, one barrier per stage.  Every
// workgroup re-reads its activation rows' K range from L2, so the plan (rows_plan below) trades
// those re-reads against more K splits (fp32 partials for the consumer) or activation halves
// (each weight block read by two workgroups on one XCD, so the second read hits its L2).
// Measured on a config-5 verify (256 rows) against the 128 x 128 tiles: gate/up 58.6 -> 47.3 us,
// qkv 22.7 -> 20.3 us with the tiled kernel's split counts; stages of 32 in 7-8 buffers (twice
// the bytes in flight, twice the barriers) were slower (8.16 against 7.19 ms per verify).
constexpr int RW_MAXM = 256;                // activation rows per workgroup at most (8 waves x 32)
// Stage buffers: three (two stages in flight).  Four or five, which the LDS holds for every
// instantiation here, measured slower on a config-5 verify (6.56 / 6.60 against 6.51 ms): the
// loop's DMA, LDS reads and MFMAs each take about as long as the whole loop (timing copies),
// so deeper prefetch only adds LDS traffic.
#ifndef QD_RW_NBUF_MAX
#define QD_RW_NBUF_MAX 3
#endif
constexpr int RW_LDS_BYTES = 160 * 1024;
// stage buffers for `rows` staged rows (128 bytes each): as many as fit the CU's LDS, 3..max
__host__ __device__ constexpr int rw_nbuf(int rows) {
  return RW_LDS_BYTES / (rows * 128) > QD_RW_NBUF_MAX ? QD_RW_NBUF_MAX : RW_LDS_BYTES / (rows * 128);
}

template <int EPI, bool SPLIT, int NT, int MT>
__global__ __launch_bounds__(512, 1) void gemm_rows_kernel(
    const bf16_t* __restrict__ X, int64_t x_stride, int M, const bf16_t* __restrict__ W, int N,
    int K, int rows_per_wg, int S, int ks_per, int mh, bf16_t* out, int64_t out_stride,
    const bf16_t* res, int64_t res_stride, float* part) {
  constexpr bool SW = EPI == EPI_SWIGLU;
  constexpr int WT = SW ? 2 * NT : NT;       // weight tiles (gate tiles, then up tiles)
  constexpr int WR = 16 * WT;                // staged weight rows
  constexpr int RM = 128 * MT;               // staged activation rows
  constexpr int ROWS = WR + RM;              // staged rows per stage (weights, then activations)
  constexpr int NBLK = ROWS / 8;             // 1 KiB load blocks per stage (8 rows x 128 bytes)
  constexpr int PER = (NBLK + 7) / 8;        // loads per wave per stage (at most)
  constexpr int RW_NBUF = rw_nbuf(ROWS);
  static_assert(RW_NBUF >= 3 && RW_NBUF * ROWS * 128 <= RW_LDS_BYTES, "stage buffers");
  __shared__ uint4 sm[RW_NBUF][ROWS * 8];
  // workgroup -> (weight block, K split, activation half): the halves of one weight block are
  // workgroups g and g + 8 (dispatch puts workgroup g on XCD g % 8), so they share an L2
  const int nb = (N + rows_per_wg - 1) / rows_per_wg;
  int blkid = blockIdx.x, mb = 0;
  if (mh > 1) {
    const int slot = blockIdx.x >> 3;
    mb = slot % mh;
    blkid = (slot / mh) * 8 + (blockIdx.x & 7);
    if (blkid >= nb * S) return;             // the grid's padding to whole groups of 8
  }
  const int rb = blkid / S, split = blkid - rb * S;
  const int m0 = mb * RM;
  const int n0 = rb * rows_per_wg;
  const int nrows = min(rows_per_wg, N - n0);
  const int ksteps = K / TK;
  const int kbeg = split * ks_per, kend = min(ksteps, kbeg + ks_per);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: load bases in SGPRs
  const int c = lane & 15, q = lane >> 4;
  // LDS row r < WR: weight row n0 + r (SwiGLU: gate rows, then up rows + N); r >= WR: activation
  // row m0 + r - WR; rows past the block / past M reload a valid row (never stored)
  auto grow_off = [&](int r) -> uint32_t {
    if (r < WR) {
      int wr = SW ? (r % (16 * NT)) : r;
      wr = min(wr, nrows - 1);
      const int64_t row = (int64_t)n0 + wr + ((SW && r >= 16 * NT) ? N : 0);
      return (uint32_t)(row * K * 2);
    }
    const int xm = min(m0 + r - WR, M - 1);
    return (uint32_t)((int64_t)xm * x_stride * 2);
  };
  // wave w loads blocks w, w + 8, ... < NBLK (PER of them, or PER - 1 where NBLK is not a
  // multiple of 8: repeating blocks to even the waves out cost 10-12 % more load requests, the
  // stream this loop is bound by); lane l of a block: row l / 8, position l % 8, K unit
  // (l % 8) ^ (row % 8)
  static_assert(PER >= 2, "PER - 1 loads for the short waves");
  const bool full = wave + 8 * (PER - 1) < NBLK;   // uniform per wave
  uint32_t voff[PER];
  int blk[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    blk[j] = (wave + 8 * j) % NBLK;
    const int r = blk[j] * 8 + (lane >> 3);
    voff[j] = grow_off(r) + (uint32_t)(((lane & 7) ^ ((lane >> 3) & 7)) * 16);
  }
  const uint32_t lbase = __builtin_amdgcn_readfirstlane(lds_u32(&sm[0][0]));
  // loads j0 .. j1 - 1 of this wave's PER (or PER - 1) for stage ks into buffer buf
  auto issue = [&](int ks, int buf, int j0 = 0, int j1 = 1 << 30) {
    const char* wb = reinterpret_cast<const char*>(W) + (size_t)ks * (TK * 2);
    const char* xb = reinterpret_cast<const char*>(X) + (size_t)ks * (TK * 2);
    const uint32_t l = lbase + (uint32_t)buf * (ROWS * 128);
#pragma unroll
    for (int j = 0; j < PER; ++j)
      if (j >= j0 && j < j1 && (j < PER - 1 || full))
        dma16(blk[j] * 8 < WR ? wb : xb, voff[j], l + (uint32_t)blk[j] * 1024);
  };
  f32x4_t acc[WT][MT];
#pragma unroll
  for (int t = 0; t < WT; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const bool active = m0 + 16 * MT * wave < M;   // uniform per wave
  // contract the stage in buffer buf as two halves of K = 32, each preceded by half of the loads
  // of stage ks_next (< 0: none) into buf_next: issued between the MFMAs rather than all ahead of
  // them, the verify took 6.39 instead of 6.51 ms
  auto compute = [&](int buf, int ks_next, int buf_next) {
    const uint4* b0 = sm[buf];
#pragma unroll
    for (int s_ = 0; s_ < 2; ++s_) {
      if (ks_next >= 0) issue(ks_next, buf_next, s_ ? PER / 2 : 0, s_ ? PER : PER / 2);
      __builtin_amdgcn_sched_barrier(0);
      const int u_ = (4 * s_ + q) ^ (c & 7);
      uint4 a_[WT], b_[MT];
#pragma unroll
      for (int t = 0; t < WT; ++t) a_[t] = b0[(16 * t + c) * 8 + u_];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) b_[mt] = b0[(WR + 16 * MT * wave + 16 * mt + c) * 8 + u_];
#pragma unroll
      for (int t = 0; t < WT; ++t)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          acc[t][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(a_[t]), as_bf8(b_[mt]),
                                                               acc[t][mt], 0, 0, 0);
    }
  };
  // stage kbeg + i in buffer i % RW_NBUF; at the top of step i this wave's loads of stage i have
  // landed once at most min(RW_NBUF - 2, stages after it) stages of its loads (PER or PER - 1 a
  // stage) are outstanding; after the barrier every wave's have, and every wave is done with
  // stage i - 1, whose buffer then takes stage i + RW_NBUF - 1
  constexpr int P = RW_NBUF - 1;
  const int nst = kend - kbeg;
#pragma unroll
  for (int i = 0; i < P; ++i)
    if (i < nst) issue(kbeg + i, i);
  int buf = 0;
  for (int i = 0; i < nst; ++i) {
    if (full) wait_stages<PER, P - 1>(nst - 1 - i);
    else wait_stages<PER - 1, P - 1>(nst - 1 - i);
    lds_barrier();
    const int kn = i + P < nst ? kbeg + i + P : -1, bn = buf + P < RW_NBUF ? buf + P : buf + P - RW_NBUF;
    if (active) compute(buf, kn, bn);
    else if (kn >= 0) issue(kn, bn);
    buf = buf + 1 < RW_NBUF ? buf + 1 : 0;
  }

  // epilogue: lane (c, q) of acc[t][mt] holds weight rows 4 q + r of tile t = output columns
  // n .. n + 3 of activation row m = m0 + 16 MT wave + 16 mt + c
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int64_t m = m0 + 16 * MT * wave + 16 * mt + c;
    if (m >= M) continue;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int u = 16 * t + 4 * q;          // output column offset in the block
      if (u >= nrows) continue;
      const int64_t n = (int64_t)n0 + u;
      if constexpr (SPLIT) {
        *reinterpret_cast<f32x4_t*>(part + ((int64_t)split * M + m) * N + n) = acc[t][mt];
      } else {
        float y[4];
        if constexpr (SW) {
#pragma unroll
          for (int r = 0; r < 4; ++r) y[r] = silu_rbf(rbf(acc[t][mt][r])) * rbf(acc[NT + t][mt][r]);
        } else if constexpr (EPI == EPI_RES) {
          const uint2 rv = *reinterpret_cast<const uint2*>(res + m * res_stride + n);
          y[0] = bflo(rv.x) + rbf(acc[t][mt][0]);
          y[1] = bfhi(rv.x) + rbf(acc[t][mt][1]);
          y[2] = bflo(rv.y) + rbf(acc[t][mt][2]);
          y[3] = bfhi(rv.y) + rbf(acc[t][mt][3]);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) y[r] = acc[t][mt][r];
        }
        *reinterpret_cast<uint2*>(out + m * out_stride + n) = make_uint2(pack2(y[0], y[1]), pack2(y[2], y[3]));
      }
    }
  }
}

int64_t tile_nblocks(int64_t N, int epi) { return epi == EPI_SWIGLU ? N / 64 : N / TN; }

}  // namespace

bool gemm_tile_ok(int64_t M, int64_t N, int64_t K, int epi, const void* x, int64_t x_stride,
                  const void* w, const void* out, int64_t out_stride, const void* res,
                  int64_t res_stride) {
  if (M <= 0 || K % TK != 0 || K < 2 * TK) return false;
  if (epi == EPI_SWIGLU ? N % 64 != 0 : N % TN != 0) return false;
  if (x_stride % 8 || reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(w) % 16)
    return false;
  if (epi != EPI_ARGMAX && (out_stride % 4 || reinterpret_cast<uintptr_t>(out) % 8)) return false;
  if (epi == EPI_RES && (res_stride % 4 || reinterpret_cast<uintptr_t>(res) % 8)) return false;
  return M * (int64_t)(N / 16) < (1ll << 40) && (M + TM - 1) / TM * tile_nblocks(N, epi) < (1ll << 30);
}

static int64_t tile_cus() {
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

// K splits: only the store / residual epilogues split, when the tile grid leaves CUs idle; as
// many as keep the grid within one workgroup per CU (a grid a little past that puts two on some
// CUs, which then set the kernel's time: measured at 256 rows, 288 / 280-workgroup grids 9.09 ms
// per verify forward, the same GEMMs split to 192 / 240 workgroups 8.15 ms, to 480 8.72 ms), and
// at least 4 stages per split
int gemm_tile_splits(int64_t M, int64_t N, int64_t K, int epi) {
  if (epi != EPI_NONE && epi != EPI_RES) return 1;
  const int64_t tiles = (M + TM - 1) / TM * tile_nblocks(N, epi);
  if (tiles >= 160) return 1;
  int64_t sp = tile_cus() / tiles;
  const int64_t maxsp = (K / TK) / 4;
  if (sp > maxsp) sp = maxsp;
  return sp < 1 ? 1 : (int)sp;
}

// The all-rows kernel's plan for M <= 256 rows.  One round of workgroups; each workgroup moves
// (through its CU's L1 -> L2 request stream, which bounds this kernel) its weight rows' and its
// activation rows' K range, and with K splits writes fp32 partials that the consumer reads
// back.  The plan minimises that per-workgroup traffic over the K split count S (store /
// residual epilogues, when the caller takes partials), the activation halves (1 or 2) and the
// block height (a multiple of 4 rows, at most RW_NT_MAX MFMA tiles, the skinny GEMM's rule for
// the resulting workgroup count):
//   2 (K / S) (activation rows + weight rows) + [S > 1] 4 (activation rows x block rows
//   + S M N / CUs).
// On a config-5 verify (256 rows, 256 CUs) that picks two activation halves for every
// projection: qkv 96-row blocks in 2 K splits, o and down 124-row blocks in 6, gate/up 76 + 76
// rows (SwiGLU, no split); the four launches went from 105.9 to 98.7 us per layer (one half per
// workgroup for gate/up only: 6.86 against 6.63 ms per verify).
struct RowsPlan {
  int rows = 0, nt = 0, mt = 0, mh = 0, splits = 0, ks_per = 0;
};
constexpr int RW_NT_MAX = 8, RW_NT_MAX_SW = 5;

static int rows_nt_round(int nt, bool sw) {   // the instantiated block heights (MFMA tiles)
  if (sw) return nt < 2 ? 2 : nt;                              // 2..5
  if (nt <= 4) return nt;                                      // 1..4
  return nt <= 6 ? 6 : 8;
}

static bool rows_plan(int64_t M, int64_t N, int64_t K, int epi, bool can_split, RowsPlan& best) {
  best = RowsPlan();
  if (!QD_TILE_ROWS || M > RW_MAXM || epi == EPI_ARGMAX) return false;
  const bool sw = epi == EPI_SWIGLU;
  if ((sw ? 2 * N : N) * K * 2 >= (1ll << 32)) return false;
  const int64_t cus = tile_cus(), ksteps = K / TK;
  // the K split count stays the tiled kernel's (more splits measured slower at 256 rows: qkv in
  // 5 splits 20.2 -> 19.4 us, down in 12 splits 25.5 -> 24.0 us, but their consumers, which
  // read every split's partials, 8.8 -> 12.0 and 5.3 -> 7.7 us)
  const int64_t smax = can_split && !sw ? gemm_tile_splits(M, N, K, epi) : 1;
  double best_cost = 0;
  for (int mt = 1; mt <= 2; ++mt) {
    const int64_t rm = 128 * mt, mh = (M + rm - 1) / rm;
    if (mh > 2 || (mt == 2 && M <= 128)) continue;
    for (int64_t S0 = smax; S0 <= smax; ++S0) {
      const int64_t ks_per = (ksteps + S0 - 1) / S0, S = (ksteps + ks_per - 1) / ks_per;
      const int64_t per = cus / (S * mh);                      // weight blocks in one round
      if (per < 1) break;
      const int64_t rows = ((N + per - 1) / per + 3) / 4 * 4;
      const int nt = rows_nt_round((int)((rows + 15) / 16), sw);
      const int ntmax = sw ? RW_NT_MAX_SW : S > 1 ? RW_NT_MAX : 4;   // instantiated heights
      if (nt > ntmax || 16 * nt < rows) continue;
      const int64_t wgs = (N + rows - 1) / rows * S * mh;
      if (wgs > cus) continue;
      const double act = (double)(M < rm ? M : rm), wrows = (double)rows * (sw ? 2 : 1);
      double cost = 2.0 * ks_per * TK * (act + wrows);
      if (S > 1) cost += 4.0 * act * rows + 4.0 * S * M * N / cus;
      if (best.splits == 0 || cost < best_cost) {
        best_cost = cost;
        best.rows = (int)rows; best.nt = nt; best.mt = mt; best.mh = (int)mh;
        best.splits = (int)S; best.ks_per = (int)ks_per;
      }
    }
  }
  return best.splits > 0;
}

// The block height (MFMA tiles) of the instantiation launch_rows picks for a plan: SwiGLU 2..5,
// split-K 1..4, 6, 8, unsplit store / residual 1..4 (rows_plan's rounding and limits keep
// 16 x this >= the plan's rows).
static int rows_inst_nt(int nt, int epi, bool split) {
  if (epi == EPI_SWIGLU) return nt <= 2 ? 2 : nt >= 5 ? 5 : nt;
  if (split) return nt <= 1 ? 1 : nt <= 4 ? nt : nt <= 6 ? 6 : 8;
  return nt <= 1 ? 1 : nt >= 4 ? 4 : nt;
}

// What the launchers run on the all-rows kernel for (M, N, K, epi) with `part_floats` floats of
// split-partial room (0: none).  Returns -1 when the kernel does not take the shape (the tiled
// kernels do), 0 when it does but the caller only takes split partials (gemm_tile_partials) and
// no split fits, 1 with the plan to launch: split when the plan splits and the partials fit,
// else the unsplit plan.
static int rows_launch_plan(int64_t M, int64_t N, int64_t K, int epi, bool partials_only,
                            int64_t part_floats, RowsPlan& P) {
  if (M < GEMM_TILE_MIN_M || !rows_plan(M, N, K, epi, true, P)) return -1;
  const bool room = part_floats >= (int64_t)P.splits * M * N;
  if (partials_only) return P.splits > 1 && room ? 1 : 0;
  if (P.splits > 1 && !room) rows_plan(M, N, K, epi, false, P);   // no room for partials: S = 1
  return P.splits > 0 ? 1 : -1;
}

template <int EPI, bool SPLIT>
static void launch_rows(const RowsPlan& P, const bf16_t* x, int64_t xs, int M, const bf16_t* w,
                        int N, int K, bf16_t* out, int64_t os, const bf16_t* res, int64_t rs,
                        float* part, hipStream_t s) {
  const int nblk = (N + P.rows - 1) / P.rows * P.splits;
  const int ng = P.mh > 1 ? (nblk + 7) / 8 * 8 * P.mh : nblk;
  const dim3 g((unsigned)ng), b(512);
#define QD_RW(NT, MT)                                                                           \
  gemm_rows_kernel<EPI, SPLIT, NT, MT><<<g, b, 0, s>>>(x, xs, M, w, N, K, P.rows, P.splits,       \
                                                       P.ks_per, P.mh, out, os, res, rs, part)
#define QD_RW_MT(NT) \
  do { if (P.mt == 1) QD_RW(NT, 1); else QD_RW(NT, 2); } while (0)
  const int nt = rows_inst_nt(P.nt, EPI, SPLIT);
  if constexpr (EPI == EPI_SWIGLU) {
    switch (nt) {
      case 2: QD_RW_MT(2); break;
      case 3: QD_RW_MT(3); break;
      case 4: QD_RW_MT(4); break;
      default: QD_RW_MT(5); break;
    }
  } else if constexpr (SPLIT) {
    switch (nt) {
      case 1: QD_RW_MT(1); break;
      case 2: QD_RW_MT(2); break;
      case 3: QD_RW_MT(3); break;
      case 4: QD_RW_MT(4); break;
      case 6: QD_RW_MT(6); break;
      default: QD_RW_MT(8); break;
    }
  } else {
    switch (nt) {
      case 1: QD_RW_MT(1); break;
      case 2: QD_RW_MT(2); break;
      case 3: QD_RW_MT(3); break;
      default: QD_RW_MT(4); break;
    }
  }
#undef QD_RW_MT
#undef QD_RW
}

int gemm_rows_query(int64_t M, int64_t N, int64_t K, int epi, bool partials_only,
                    int64_t part_floats, int64_t* out) {
  RowsPlan P;
  const int rp = rows_launch_plan(M, N, K, epi, partials_only, part_floats, P);
  if (rp != 1) return rp;
  const bool split = P.splits > 1;
  const int nt = rows_inst_nt(P.nt, split ? EPI_NONE : epi, split);
  const int64_t nblk = (N + P.rows - 1) / P.rows * P.splits;
  const int wt = (!split && epi == EPI_SWIGLU) ? 2 * nt : nt;
  out[0] = P.rows;
  out[1] = nt;
  out[2] = P.mt;
  out[3] = P.mh;
  out[4] = P.splits;
  out[5] = P.ks_per;
  out[6] = P.mh > 1 ? (nblk + 7) / 8 * 8 * P.mh : nblk;             // grid (launch_rows)
  out[7] = (int64_t)rw_nbuf(16 * wt + 128 * P.mt) * (16 * wt + 128 * P.mt) * 128;   // static LDS bytes
  return 1;
}

int64_t gemm_tile_ws_floats(int64_t M, int64_t N, int64_t K, int epi) {
  RowsPlan P;
  const int sp = rows_plan(M, N, K, epi, true, P) ? P.splits : gemm_tile_splits(M, N, K, epi);
  return sp > 1 ? (int64_t)sp * M * N : 0;
}

int gemm_tile_partials(const bf16_t* x, int64_t xs, int64_t M, const bf16_t* w, int64_t N,
                       int64_t K, float* part, int64_t part_floats, hipStream_t s) {
  if (M < GEMM_TILE_MIN_M || !part ||
      !gemm_tile_ok(M, N, K, EPI_NONE, x, xs, w, part, N, nullptr, 0))
    return 0;
  RowsPlan P;
  const int rp = rows_launch_plan(M, N, K, EPI_NONE, true, part_floats, P);
  if (rp == 0) return 0;
  if (rp == 1) {
    launch_rows<EPI_NONE, true>(P, x, xs, (int)M, w, (int)N, (int)K, nullptr, 0, nullptr, 0,
                                part, s);
    return P.splits;
  }
  int splits = gemm_tile_splits(M, N, K, EPI_NONE);
  if (splits <= 1 || part_floats < (int64_t)splits * M * N) return 0;
  const int ksteps = (int)(K / TK);
  const int ks_per = (ksteps + splits - 1) / splits;
  splits = (ksteps + ks_per - 1) / ks_per;              // no empty split
  const int64_t mblocks = (M + TM - 1) / TM, nblocks = tile_nblocks(N, EPI_NONE);
  if (QD_TILE8)
    gemm_tile8_kernel<EPI_NONE, true><<<dim3((unsigned)(mblocks * nblocks * splits)), dim3(512), 0, s>>>(
        x, xs, (int)M, w, (int)N, (int)K, (int)mblocks, (int)nblocks, ks_per, nullptr, 0, nullptr,
        0, part);
  else
    gemm_tile_kernel<EPI_NONE, true><<<dim3((unsigned)(mblocks * nblocks * splits)), dim3(256), 0, s>>>(
        x, xs, (int)M, w, (int)N, (int)K, (int)mblocks, (int)nblocks, ks_per, nullptr, 0, nullptr,
        0, nullptr, nullptr, nullptr, part);
  return splits;
}

// Returns the number of argmax partials per row written (EPI_ARGMAX), else 0.
int64_t launch_gemm_tile(const bf16_t* x, int64_t xs, int64_t M, const bf16_t* w, int64_t N,
                         int64_t K, bf16_t* out, int64_t os, const bf16_t* res, int64_t rs, int epi,
                         float* pval, int32_t* pidx, float* logits, float* part,
                         int64_t part_floats, hipStream_t s) {
  if (epi != EPI_ARGMAX && ((QD_BIG_EPIS >> epi) & 1) && M >= QD_BIG_MIN_M &&
      (epi == EPI_SWIGLU ? N % 128 == 0 : N % BT == 0) &&
      (epi == EPI_SWIGLU ? 2 * N : N) * K * 2 < (1ll << 32) && M * xs * 2 < (1ll << 32)) {
    const int64_t mbl = (M + BT - 1) / BT, nbl = epi == EPI_SWIGLU ? N / 128 : N / BT;
    const dim3 g((unsigned)(mbl * nbl)), b(BIG_WAVES * 64);
#define QD_BIG(E) \
  gemm_big_kernel<E><<<g, b, 0, s>>>(x, xs, (int)M, w, (int)N, (int)K, (int)mbl, (int)nbl, out, os, res, rs, \
                                     nullptr, nullptr, nullptr)
    if (epi == EPI_RES) QD_BIG(EPI_RES);
    else if (epi == EPI_SWIGLU) QD_BIG(EPI_SWIGLU);
    else QD_BIG(EPI_NONE);
#undef QD_BIG
    return 0;
  }
  if (epi == EPI_ARGMAX && M >= QD_BIG_ARGMAX_MIN_M && N % 4 == 0 && N >= BT &&
      N * K * 2 < (1ll << 32) && M * xs * 2 < (1ll << 32)) {
    // LM head over many rows (a tree verification's 256): 256 x 256 tiles read every weight
    // byte once per 256 activation rows, half the L2 traffic of the 128 x 128 tiles
    const int64_t mbl = (M + BT - 1) / BT, nbl = (N + BT - 1) / BT;
    gemm_big_kernel<EPI_ARGMAX><<<dim3((unsigned)(mbl * nbl)), dim3(BIG_WAVES * 64), 0, s>>>(
        x, xs, (int)M, w, (int)N, (int)K, (int)mbl, (int)nbl, nullptr, 0, nullptr, 0, pval, pidx,
        logits);
    return nbl;
  }
  RowsPlan P;
  if (epi != EPI_ARGMAX && rows_launch_plan(M, N, K, epi, false, part ? part_floats : 0, P) == 1) {
    if (P.splits > 1) {
      launch_rows<EPI_NONE, true>(P, x, xs, (int)M, w, (int)N, (int)K, nullptr, 0, nullptr, 0,
                                  part, s);
      const int64_t thr = M * (N / 4);
      const dim3 rg((unsigned)((thr + 255) / 256)), rb(256);
      if (epi == EPI_RES)
        gemm_split_reduce_kernel<EPI_RES><<<rg, rb, 0, s>>>(part, P.splits, M, N, out, os, res, rs);
      else
        gemm_split_reduce_kernel<EPI_NONE><<<rg, rb, 0, s>>>(part, P.splits, M, N, out, os, res, rs);
      return 0;
    }
    if (epi == EPI_RES)
      launch_rows<EPI_RES, false>(P, x, xs, (int)M, w, (int)N, (int)K, out, os, res, rs, part, s);
    else if (epi == EPI_SWIGLU)
      launch_rows<EPI_SWIGLU, false>(P, x, xs, (int)M, w, (int)N, (int)K, out, os, res, rs, part, s);
    else
      launch_rows<EPI_NONE, false>(P, x, xs, (int)M, w, (int)N, (int)K, out, os, res, rs, part, s);
    return 0;
  }
  const int64_t mblocks = (M + TM - 1) / TM, nblocks = tile_nblocks(N, epi);
  int splits = gemm_tile_splits(M, N, K, epi);
  if (splits > 1 && (!part || part_floats < (int64_t)splits * M * N)) splits = 1;
  const int ksteps = (int)(K / TK);
  const int ks_per = (ksteps + splits - 1) / splits;
  splits = (ksteps + ks_per - 1) / ks_per;              // no empty split
  const dim3 grid((unsigned)(mblocks * nblocks * splits)), block(256);
  const int Mi = (int)M, Ni = (int)N, Ki = (int)K, mbi = (int)mblocks, nbi = (int)nblocks;
#define QD_TILE(E, SP)                                                                           \
  do {                                                                                           \
    if (QD_TILE8 && E != EPI_ARGMAX)                                                             \
      gemm_tile8_kernel<E == EPI_ARGMAX ? EPI_NONE : E, SP><<<grid, dim3(512), 0, s>>>(          \
          x, xs, Mi, w, Ni, Ki, mbi, nbi, ks_per, out, os, res, rs, part);                       \
    else                                                                                         \
      gemm_tile_kernel<E, SP><<<grid, block, 0, s>>>(x, xs, Mi, w, Ni, Ki, mbi, nbi, ks_per, out, \
                                                     os, res, rs, pval, pidx, logits, part);     \
  } while (0)
  if (splits > 1) {
    if (epi == EPI_RES) QD_TILE(EPI_RES, true);
    else QD_TILE(EPI_NONE, true);
    const int64_t thr = M * (N / 4);
    const dim3 rg((unsigned)((thr + 255) / 256));
    if (epi == EPI_RES)
      gemm_split_reduce_kernel<EPI_RES><<<rg, block, 0, s>>>(part, splits, M, N, out, os, res, rs);
    else
      gemm_split_reduce_kernel<EPI_NONE><<<rg, block, 0, s>>>(part, splits, M, N, out, os, res, rs);
    return 0;
  }
  switch (epi) {
    case EPI_RES: QD_TILE(EPI_RES, false); break;
    case EPI_SWIGLU: QD_TILE(EPI_SWIGLU, false); break;
    case EPI_ARGMAX: QD_TILE(EPI_ARGMAX, false); return nblocks;
    default: QD_TILE(EPI_NONE, false); break;
  }
#undef QD_TILE
  return 0;
}
