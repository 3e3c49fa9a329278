// Skinny MFMA GEMM for batched decode (M <= 32 activation rows, the B >= 3 decode step):
//   out[m, n] = epi( sum_k X[m, k] * W[n, k] )          (S == 1)
//   part[ks][m][n] = sum over the ks-th K range            (S > 1: split-K partials)
// (the reference's tensor-core decode GEMM, gemv.py:61-116 / fast.py:99-213 with BLOCK_M >= 16).
//
// At 32 rows every weight byte is used 32 times and read once: the kernel is a weight stream,
// and what bounds it is how many bytes each CU keeps in flight.  Design (gfx950, wave64):
//  * one 512-thread workgroup per CU (grid = row blocks x K ranges = the CU count), each owning a
//    contiguous block of rows_per_wg weight rows (gate / up row pairs for SwiGLU) and one of S
//    K ranges, so every CU streams the same bytes in one round;
//  * the 8 waves split the workgroup's K range into contiguous runs of 64-wide chunks and work
//    independently: a wave loads a chunk of its weight rows and of the activation rows straight
//    into registers (8 rows x 128 contiguous bytes per load instruction), keeps the next D - 1
//    chunks in flight behind it, writes the chunk to a wave-private LDS tile (16-byte units
//    XOR-swizzled so the fragment reads hit 16 distinct bank groups) and contracts it on
//    v_mfma_f32_16x16x32_bf16 (A = weight rows, B = activation rows).  No workgroup barrier
//    until the end: a wave's LDS writes and reads are ordered within the wave;
//  * the 8 waves' accumulators are summed through LDS once, in wave order, and the epilogue
//    stores bf16 (plain / residual / SwiGLU) or fp32 partials, 4 consecutive columns per lane.
// Accumulation is fp32; only the summation order differs from the reference.
#include "qd_launch.h"

namespace {

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

template <int MT, int NT, int EPI, bool PART, int D>
__global__ __launch_bounds__(512, 1) void skinny_gemm_kernel(
    const bf16_t* __restrict__ X, int64_t xs, int M, const bf16_t* __restrict__ W, int N, int K,
    int rows_per_wg, int S, bf16_t* out, int64_t os, const bf16_t* res, int64_t rs,
    float* part) {
  using SH = SkinnyShape<MT, NT, EPI>;
  constexpr bool SW = SH::SW;
  constexpr int WT = SH::WT, WR = SH::WR, L = SH::L, LW = SH::LW;
  __shared__ uint4 lds[SH::LDS_U4];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int g = blockIdx.x;
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
  for (int gi = threadIdx.x; gi < GROUPS; gi += 512) {
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
        for (int r = 0; r < 4; ++r) y[r] = rbf(silu_f(rbf(v[r]))) * rbf(u[r]);
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

// ------------------------------------------------------------------ LM head + argmax (M <= 32)
// The tied LM head at batched decode: 151936 vocab rows x K, argmax per activation row
// (gemv.py:118-154, fast.py:380-465).  One 512-thread workgroup per CU owns ~600 contiguous
// vocab rows; wave w owns TPW consecutive 16-row tiles of them for the whole of K, so no
// cross-wave sums exist.  The activation rows of one K phase (KP wide) sit in LDS for all
// waves (reloaded between phases behind two barriers); each step streams one 64-wide chunk
// of all the wave's tiles through a 2-deep register ring into its private LDS tile and
// contracts it against the resident activations.  The ring runs across phase boundaries, so
// the weight stream does not drain while the activations are swapped.  Epilogue: bf16 logits
// (the reference's logits are bf16), max with the lowest vocab index on ties per activation
// row, per-workgroup partials for argmax_reduce_kernel.
constexpr int SKA_KP = 640;

template <int MT, int TPW>
__global__ __launch_bounds__(512, 1) void skinny_argmax_kernel(
    const bf16_t* __restrict__ X, int64_t xs, int M, const bf16_t* __restrict__ W, int N, int K,
    int rows_per_wg, float* pval, int32_t* pidx, float* logits) {
  constexpr int XR = MT * 16;
  constexpr int XU = SKA_KP / 8;                     // 16-byte units per activation row (phase)
  constexpr int LW = 2 * TPW;                        // load slots per step: 8 rows each
  constexpr int D = 2;
  __shared__ uint4 xl[XR * XU];
  __shared__ uint4 wtile[SK_WAVES][TPW * 16 * 8];
  __shared__ float am_v[SK_WAVES][XR];
  __shared__ int32_t am_i[SK_WAVES][XR];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, c = lane & 15, q = lane >> 4;
  const int wg = blockIdx.x, P = gridDim.x;
  const int64_t n0 = (int64_t)wg * rows_per_wg;
  const int nrows = (int)(N - n0 < rows_per_wg ? N - n0 : rows_per_wg);
  const int TW = (nrows + 15) / 16;
  const int t0 = TW * wave / SK_WAVES, ntw = TW * (wave + 1) / SK_WAVES - t0;   // <= TPW
  const int CPP = SKA_KP / SK_KC;                    // chunks per phase
  const int S = (K / SKA_KP) * CPP;                  // steps: every chunk of K
  const int lr = lane >> 3, lu = lane & 7;
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(W + n0 * (int64_t)K), (short)0, (int)((uint32_t)nrows * (uint32_t)K * 2u),
      SK_RSRC_WORD3);
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
      (void*)X, (short)0, (int)((uint32_t)M * (uint32_t)xs * 2u), SK_RSRC_WORD3);
  // slot i of a step: rows 16 t0 + 8 i + (lane >> 3) of the block (range-checked lane offset)
  uint32_t vofs[LW];
#pragma unroll
  for (int i = 0; i < LW; ++i)
    vofs[i] = ((uint32_t)(16 * t0 + 8 * i + lr) * (uint32_t)K + 8u * lu) * 2u;
  uint4 buf[D][LW];
  auto load = [&](int b, int st) {
    if (st >= S) return;
    const uint32_t so = (uint32_t)st * (SK_KC * 2);  // chunk st of K
#pragma unroll
    for (int i = 0; i < LW; ++i) {
      if (i / 2 < ntw) {
        const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rw, vofs[i], so, SK_NT);
        buf[b][i] = make_uint4(v.x, v.y, v.z, v.w);
      }
    }
  };
  // Phase p's activation rows are loaded into registers one phase ahead (right after the
  // previous swap): loads retire in issue order, so waiting for loads issued at the swap itself
  // would also wait for the whole weight ring behind them.
  constexpr int XPT = (XR * XU + 511) / 512;         // 16-byte units per thread
  uint4 xa[XPT];
  auto load_acts = [&](int p) {
    if (p * SKA_KP >= K) return;
#pragma unroll
    for (int j = 0; j < XPT; ++j) {
      const int e = threadIdx.x + 512 * j;
      if (e < XR * XU) {
        const int r = e / XU, u = e - r * XU;
        const uint32_t off = ((uint32_t)r * (uint32_t)xs + (uint32_t)(p * SKA_KP + 8 * u)) * 2u;
        const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0);
        xa[j] = make_uint4(v.x, v.y, v.z, v.w);
      }
    }
  };
  auto store_acts = [&]() {
#pragma unroll
    for (int j = 0; j < XPT; ++j) {
      const int e = threadIdx.x + 512 * j;
      if (e < XR * XU) {
        const int r = e / XU, u = e - r * XU;
        xl[r * XU + (u ^ (r & 15))] = xa[j];
      }
    }
  };
  f32x4_t acc[TPW][MT];
#pragma unroll
  for (int j = 0; j < TPW; ++j)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[j][mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  uint4* tile = wtile[wave];
  load_acts(0);
#pragma unroll
  for (int b = 0; b < D; ++b) load(b, b);
  for (int s0 = 0; s0 < S; s0 += D) {
#pragma unroll
    for (int b = 0; b < D; ++b) {
      const int st = s0 + b;
      if (st < S) {
        const int cc = st % CPP;
        if (cc == 0) {                               // a new phase: swap the activations
          lds_barrier();                             // every wave is done with the last phase
          store_acts();
          lds_barrier();
          load_acts(st / CPP + 1);                   // the next phase's, one phase ahead
        }
#pragma unroll
        for (int i = 0; i < LW; ++i)
          if (i / 2 < ntw) tile[sk_slot(8 * i + lr, lu)] = buf[b][i];
        load(b, st + D);
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          uint4 bx[MT];
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const int r = 16 * mt + c, u = cc * 8 + 4 * s + q;
            bx[mt] = xl[r * XU + (u ^ (r & 15))];
          }
#pragma unroll
          for (int j = 0; j < TPW; ++j) {
            if (j < ntw) {
              const uint4 a = tile[sk_slot(16 * j + c, 4 * s + q)];
#pragma unroll
              for (int mt = 0; mt < MT; ++mt)
                acc[j][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf8(a), as_bf8(bx[mt]),
                                                                     acc[j][mt], 0, 0, 0);
            }
          }
        }
      }
    }
  }
  // argmax: lane (c, q) of acc[j][mt] holds vocab rows n = 16 (t0 + j) + 4 q + r of the block
  // for activation row m = 16 mt + c; n ascends over (j, r), so strict > keeps the lowest index
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = 16 * mt + c;
    float bv = -INFINITY;
    int32_t bi = 0x7FFFFFFF;
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
      if (j < ntw) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int unit = 16 * (t0 + j) + 4 * q + r;
          if (unit < nrows && m < M) {
            const int64_t n = n0 + unit;
            if (logits) logits[m * (int64_t)N + n] = acc[j][mt][r];
            const float v = rbf(acc[j][mt][r]);
            if (v > bv) { bv = v; bi = (int32_t)n; }
          }
        }
      }
    }
#pragma unroll
    for (int sh = 0; sh < 2; ++sh) {                 // the four q lanes of row c
      const float ov = sh ? lane_xor32(bv) : lane_xor16(bv);
      const int32_t oi = __builtin_bit_cast(int32_t, sh ? lane_xor32(__builtin_bit_cast(float, bi))
                                                        : lane_xor16(__builtin_bit_cast(float, bi)));
      if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
    if (q == 0) { am_v[wave][m] = bv; am_i[wave][m] = bi; }
  }
  __syncthreads();
  for (int m = threadIdx.x; m < M; m += 512) {
    float v = am_v[0][m];
    int32_t ix = am_i[0][m];
    for (int w = 1; w < SK_WAVES; ++w) {
      const float v2 = am_v[w][m];
      const int32_t i2 = am_i[w][m];
      if (v2 > v || (v2 == v && i2 < ix)) { v = v2; ix = i2; }
    }
    pval[m * (int64_t)P + wg] = v;
    pidx[m * (int64_t)P + wg] = ix;
  }
}

int skinny_cus() {
  static int cus = -1;
  if (cus < 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
      (void)hipGetLastError();
      n = 0;
    }
    cus = n;
  }
  return cus;
}

// rows per workgroup for N output units over (CU count / S) row blocks: a multiple of 4 (the
// epilogue's column groups)
int64_t skinny_rows(int64_t N, int S) {
  const int P = skinny_cus();
  const int64_t rb = P / S > 0 ? P / S : 1;
  const int64_t r = (N + rb - 1) / rb;
  return (r + 3) / 4 * 4;
}

template <int MT, int NT, int EPI, bool PART>
void skinny_go(const bf16_t* x, int64_t xs, int M, const bf16_t* w, int N, int K, int rows, int S,
               bf16_t* out, int64_t os, const bf16_t* res, int64_t rs, float* part, hipStream_t s) {
  constexpr int L = SkinnyShape<MT, NT, EPI>::L;
  // ring depth: chunks in flight per wave, within the register budget (no spills at 32 rows)
  constexpr int D = L <= 8 ? QD_SK_DEPTH_SMALL : L <= 12 ? QD_SK_DEPTH_MID : QD_SK_DEPTH_LARGE;
  const int rb = (int)((N + rows - 1) / rows);
  skinny_gemm_kernel<MT, NT, EPI, PART, D><<<dim3((unsigned)(rb * S)), dim3(512), 0, s>>>(
      x, xs, M, w, N, K, rows, S, out, os, res, rs, part);
}

template <int MT, int EPI, bool PART>
bool skinny_nt(const bf16_t* x, int64_t xs, int M, const bf16_t* w, int N, int K, int rows, int S,
               bf16_t* out, int64_t os, const bf16_t* res, int64_t rs, float* part, hipStream_t s) {
  const int nt = (rows + 15) / 16;
  switch (nt) {
    case 1: skinny_go<MT, 1, EPI, PART>(x, xs, M, w, N, K, rows, S, out, os, res, rs, part, s); return true;
    case 2: skinny_go<MT, 2, EPI, PART>(x, xs, M, w, N, K, rows, S, out, os, res, rs, part, s); return true;
    case 3: skinny_go<MT, 3, EPI, PART>(x, xs, M, w, N, K, rows, S, out, os, res, rs, part, s); return true;
    case 4:
      if constexpr (EPI != EPI_SWIGLU) {
        skinny_go<MT, 4, EPI, PART>(x, xs, M, w, N, K, rows, S, out, os, res, rs, part, s);
        return true;
      }
      return false;
    default: return false;
  }
}

}  // namespace

bool skinny_ok(int64_t M, int64_t N, int64_t K, int epi, int S, const void* x, int64_t xs,
               const void* w, int64_t os) {
  if (M < 1 || M > 32 || S < 1 || skinny_cus() < S) return false;
  if (epi != EPI_NONE && epi != EPI_RES && epi != EPI_SWIGLU) return false;
  if (K % SK_KC || N % 4 || N >= (1 << 30) || K >= (1 << 30)) return false;
  if (K / SK_KC < S) return false;
  if (xs % 8 || reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(w) % 16) return false;
  if (os % 4) return false;
  const int64_t rows = skinny_rows(N, S);
  return (rows + 15) / 16 <= (epi == EPI_SWIGLU ? 3 : 4);
}

int64_t skinny_part_floats(int64_t M, int64_t N, int S) { return S > 1 ? (int64_t)S * M * N : 0; }

// part == nullptr: the epilogue writes out (S must be 1); part != nullptr: fp32 partials
// part[S][M][N] for the caller to sum (epi, out and res unused; S >= 1).  Returns false, with
// nothing launched, when the shape is not supported or a destination is missing.
bool launch_gemm_skinny(const bf16_t* x, int64_t xs, int64_t M, const bf16_t* w, int64_t N,
                        int64_t K, int epi, int S, bf16_t* out, int64_t os, const bf16_t* res,
                        int64_t rs, float* part, hipStream_t s) {
  const bool partials = part != nullptr;
  if (!partials && (S != 1 || !out || (epi == EPI_RES && !res))) return false;
  if (!x || !w) return false;
  if (!skinny_ok(M, N, K, partials ? EPI_NONE : epi, S, x, xs, w, partials ? N : os)) return false;
  const int rows = (int)skinny_rows(N, S);
  const int Mi = (int)M, Ni = (int)N, Ki = (int)K;
#define QD_SK(MT, E, P) skinny_nt<MT, E, P>(x, xs, Mi, w, Ni, Ki, rows, S, out, os, res, rs, part, s)
  if (partials) return M <= 16 ? QD_SK(1, EPI_NONE, true) : QD_SK(2, EPI_NONE, true);
  switch (epi) {
    case EPI_RES: return M <= 16 ? QD_SK(1, EPI_RES, false) : QD_SK(2, EPI_RES, false);
    case EPI_SWIGLU: return M <= 16 ? QD_SK(1, EPI_SWIGLU, false) : QD_SK(2, EPI_SWIGLU, false);
    default: return M <= 16 ? QD_SK(1, EPI_NONE, false) : QD_SK(2, EPI_NONE, false);
  }
#undef QD_SK
}

// LM head + argmax partials at <= 32 rows: writes P = CU-count partials per row (pval / pidx
// [M, P]) and returns P, or 0 when the shape is not supported (nothing launched).
int64_t launch_lm_skinny(const bf16_t* x, int64_t xs, int64_t M, const bf16_t* w, int64_t N,
                         int64_t K, float* pval, int32_t* pidx, float* logits, hipStream_t s) {
  const int P = skinny_cus();
  if (M < 1 || M > 32 || P < 1 || P > 1024 || K % SKA_KP || N >= (1 << 30) || K >= (1 << 30))
    return 0;   // (the LM workspace holds at most 1024 partials per row beyond V / 16)
  if (xs % 8 || reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(w) % 16) return 0;
  if (!x || !w || !pval || !pidx) return 0;
  const int64_t rows = (N + P - 1) / P;
  const int64_t blocks = (N + rows - 1) / rows;               // every block holds rows
  const int tpw = (int)(((rows + 15) / 16 + SK_WAVES - 1) / SK_WAVES);
  const dim3 grid((unsigned)blocks), block(512);
  const int Mi = (int)M, Ni = (int)N, Ki = (int)K, Ri = (int)rows;
#define QD_SKA(MT, T) skinny_argmax_kernel<MT, T><<<grid, block, 0, s>>>(x, xs, Mi, w, Ni, Ki, Ri, pval, pidx, logits)
  if (M <= 16) {
    switch (tpw) {
      case 4: QD_SKA(1, 4); break;
      case 5: QD_SKA(1, 5); break;
      case 6: QD_SKA(1, 6); break;
      default: return 0;
    }
  } else {
    switch (tpw) {
      case 4: QD_SKA(2, 4); break;
      case 5: QD_SKA(2, 5); break;
      case 6: QD_SKA(2, 6); break;
      default: return 0;
    }
  }
#undef QD_SKA
  return blocks;
}
