// The skinny GEMM's workgroup body (gemm_skinny.hip's skinny_gemm_kernel): see gemm_skinny.hip
// for the design.
#pragma once

#include "qd_launch.h"

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

__device__ __forceinline__ bf16x8_t as_bf8(uint4 v) { return __builtin_bit_cast(bf16x8_t, v); }

#ifndef QD_SK_DEPTH_SMALL
#define QD_SK_DEPTH_SMALL 3
#endif
#ifndef QD_SK_DEPTH_MID
#define QD_SK_DEPTH_MID 2
#endif
#ifndef QD_SK_DEPTH_LARGE
#define QD_SK_DEPTH_LARGE 2
#endif

constexpr int SK_WAVES = 8;
constexpr int SK_KC = 64;   // k per chunk: 128 bytes of a row, 8 units of 16 bytes
constexpr int SK_RSRC_WORD3 = 0x00020000;   // buffer resource dword 3: raw 32-bit data, no swizzle
constexpr int SK_NT = 2;                    // cache policy of the weight loads: non-temporal

// LDS position of 16-byte unit u of staged row r: rows of 128 bytes; the swizzle makes the 16
// lanes of a fragment read (rows c = 0..15, one unit) cover 16 distinct bank groups
__device__ __forceinline__ int sk_slot(int r, int u) { return r * 8 + (u ^ ((r >> 1) & 7)); }

template <int MT, int NT, int EPI>
struct SkinnyShape {
  static constexpr bool SW = EPI == EPI_SWIGLU;
  static constexpr int WT = SW ? 2 * NT : NT;   // staged weight tiles (gate tiles, then up tiles)
  static constexpr int WR = WT * 16;            // staged weight rows
  static constexpr int XR = MT * 16;            // staged activation rows
  static constexpr int LW = WR / 8, LX = XR / 8, L = LW + LX;   // load instructions per chunk
  static constexpr int STAGE_U4 = SK_WAVES * (WR + XR) * 8;      // wave tiles
  static constexpr int RED_U4 = SK_WAVES * WT * MT * 64;         // cross-wave sums
  static constexpr int LDS_U4 = STAGE_U4 > RED_U4 ? STAGE_U4 : RED_U4;
};

// One workgroup's block g (row block g / S, K range g % S) of the GEMM, with lds (LDS_U4 16-byte
// units) as its staging and reduction space.
// register ring depth: chunks in flight per wave, within the register budget (no spills at 32
// rows)
template <int MT, int NT, int EPI>
constexpr int skinny_depth() {
  constexpr int L = SkinnyShape<MT, NT, EPI>::L;
  return L <= 8 ? QD_SK_DEPTH_SMALL : L <= 12 ? QD_SK_DEPTH_MID : QD_SK_DEPTH_LARGE;
}

template <int MT, int NT, int EPI, bool PART, int D>
__device__ __forceinline__ void skinny_block(uint4* lds, const bf16_t* __restrict__ X, int64_t xs,
                                             int M, const bf16_t* __restrict__ W, int N, int K,
                                             int rows_per_wg, int S, int g, bf16_t* out,
                                             int64_t os, const bf16_t* res, int64_t rs,
                                             float* part) {
  using SH = SkinnyShape<MT, NT, EPI>;
  constexpr bool SW = SH::SW;
  constexpr int WT = SH::WT, WR = SH::WR, L = SH::L, LW = SH::LW;
  const int tid = (int)threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int rb = g / S, ks = g - rb * S;
  const int64_t n0 = (int64_t)rb * rows_per_wg;
  const int nrows = (int)(N - n0 < rows_per_wg ? N - n0 : rows_per_wg);   // > 0 by the grid
  // this workgroup's K range (in chunks), then this wave's run of it
  const int KC = K / SK_KC;
  const int c0 = (int)((int64_t)KC * ks / S), c1 = (int)((int64_t)KC * (ks + 1) / S);
  const int wc0 = c0 + (c1 - c0) * wave / SK_WAVES;
  const int wc1 = c0 + (c1 - c0) * (wave + 1) / SK_WAVES;
  // Loads are buffer loads.  The range check of a raw buffer covers the per-lane offset only
  // (not the wave-uniform scalar offset), so each slot's lane offset holds the row (slot i:
  // staged rows 8i .. 8i+7, lane l takes row 8i + (l >> 3), unit l & 7) and the chunk offset
  // is the scalar one; the resources' extents (this block's rows; the M activation rows) make
  // rows past them read as zeros and never touch memory outside the operands.
  const int lr = lane >> 3, lu = lane & 7;
  const uint32_t wbytes = (uint32_t)nrows * (uint32_t)K * 2u;
  const __amdgpu_buffer_rsrc_t rg = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(W + n0 * (int64_t)K), (short)0, (int)wbytes, SK_RSRC_WORD3);
  const __amdgpu_buffer_rsrc_t ru = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(W + (n0 + (SW ? N : 0)) * (int64_t)K), (short)0, (int)wbytes, SK_RSRC_WORD3);
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
      (void*)X, (short)0, (int)((uint32_t)M * (uint32_t)xs * 2u), SK_RSRC_WORD3);
  uint32_t vofs[L];
#pragma unroll
  for (int i = 0; i < L; ++i) {
    if (i < LW) {
      const int ii = (SW && i >= LW / 2) ? i - LW / 2 : i;   // up-tile slots restart at row 0
      vofs[i] = ((uint32_t)(8 * ii + lr) * (uint32_t)K + 8u * lu) * 2u;
    } else {
      vofs[i] = ((uint32_t)(8 * (i - LW) + lr) * (uint32_t)xs + 8u * lu) * 2u;
    }
  }
  uint4* tile = lds + wave * ((WR + SH::XR) * 8);
  uint4 buf[D][L];
  auto load = [&](int b, int c) {
    if (c >= wc1) return;                        // past the wave's run: nothing to prefetch
    const uint32_t so = (uint32_t)c * (SK_KC * 2);
#pragma unroll
    for (int i = 0; i < L; ++i) {
      const bool up = SW && i < LW && i >= LW / 2;
      const u32x4_t v = i < LW ? __builtin_amdgcn_raw_buffer_load_b128(up ? ru : rg, vofs[i], so, SK_NT)
                               : __builtin_amdgcn_raw_buffer_load_b128(rx, vofs[i], so, 0);
      buf[b][i] = make_uint4(v.x, v.y, v.z, v.w);
    }
  };
  f32x4_t acc[WT][MT];
#pragma unroll
  for (int t = 0; t < WT; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const int c = lane & 15, q = lane >> 4;
  auto contract = [&]() {
#pragma unroll
    for (int s = 0; s < 2; ++s) {                // the chunk's two 32-wide k steps
      uint4 a[WT], b[MT];
#pragma unroll
      for (int t = 0; t < WT; ++t) a[t] = tile[sk_slot(16 * t + c, 4 * s + q)];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) b[mt] = tile[sk_slot(WR + 16 * mt + c, 4 * s + q)];
#pragma unroll
      for (int t = 0; t < WT; ++t)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          acc[t][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(a[t]), as_bf8(b[mt]),
                                                               acc[t][mt], 0, 0, 0);
    }
  };
  // chunk wc0 + j sits in ring slot j % D; its slot is refilled with chunk + D as soon as it is
  // written to the tile, so D - 1 chunks stay in flight while one is contracted
#pragma unroll
  for (int b = 0; b < D; ++b) load(b, wc0 + b);
  for (int cc = wc0; cc < wc1; cc += D) {
#pragma unroll
    for (int b = 0; b < D; ++b) {
      if (cc + b < wc1) {
#pragma unroll
        for (int i = 0; i < L; ++i) tile[sk_slot(8 * i + lr, lu)] = buf[b][i];
        load(b, cc + b + D);
        contract();
      }
    }
  }
  // cross-wave sums (wave order) and the epilogue
  __syncthreads();                               // every wave is done with its tile
  f32x4_t* red = reinterpret_cast<f32x4_t*>(lds);
#pragma unroll
  for (int t = 0; t < WT; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) red[((wave * WT + t) * MT + mt) * 64 + lane] = acc[t][mt];
  __syncthreads();
  constexpr int GROUPS = NT * MT * 64;           // (output tile, activation tile, lane)
  for (int gi = tid; gi < GROUPS; gi += 512) {
    const int t = gi / (MT * 64), mt = (gi / 64) % MT, ln = gi & 63;
    const int m = 16 * mt + (ln & 15);
    const int unit = 16 * t + 4 * (ln >> 4);     // 4 consecutive output columns
    if (m >= M || unit >= nrows) continue;
    f32x4_t v = red[(t * MT + mt) * 64 + ln];
#pragma unroll
    for (int w = 1; w < SK_WAVES; ++w) v += red[((w * WT + t) * MT + mt) * 64 + ln];
    const int64_t n = n0 + unit;
    if constexpr (PART) {
      *reinterpret_cast<f32x4_t*>(part + ((int64_t)ks * M + m) * N + n) = v;
    } else {
      float y[4];
      if constexpr (SW) {
        f32x4_t u = red[((NT + t) * MT + mt) * 64 + ln];
#pragma unroll
        for (int w = 1; w < SK_WAVES; ++w) u += red[((w * WT + NT + t) * MT + mt) * 64 + ln];
#pragma unroll
        for (int r = 0; r < 4; ++r) y[r] = silu_rbf(rbf(v[r])) * rbf(u[r]);
      } else if constexpr (EPI == EPI_RES) {
        const uint2 rv = *reinterpret_cast<const uint2*>(res + m * rs + n);
        y[0] = bflo(rv.x) + rbf(v[0]);
        y[1] = bfhi(rv.x) + rbf(v[1]);
        y[2] = bflo(rv.y) + rbf(v[2]);
        y[3] = bfhi(rv.y) + rbf(v[3]);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) y[r] = v[r];
      }
      *reinterpret_cast<uint2*>(out + m * os + n) = make_uint2(pack2(y[0], y[1]), pack2(y[2], y[3]));
    }
  }
}
