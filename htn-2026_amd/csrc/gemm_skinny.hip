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
#include "skinny_core.h"

namespace {

// the GEMM of skinny_block, one workgroup per block
template <int MT, int NT, int EPI, bool PART, int D>
__global__ __launch_bounds__(512, 1) void skinny_gemm_kernel(
    const bf16_t* __restrict__ X, int64_t xs, int M, const bf16_t* __restrict__ W, int N, int K,
    int rows_per_wg, int S, bf16_t* out, int64_t os, const bf16_t* res, int64_t rs,
    float* part) {
  __shared__ uint4 lds[SkinnyShape<MT, NT, EPI>::LDS_U4];
  skinny_block<MT, NT, EPI, PART, D>(lds, X, xs, M, W, N, K, rows_per_wg, S, (int)blockIdx.x, out,
                                     os, res, rs, part);
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

template <int MT, int NT, int EPI, bool PART>
void skinny_go(const bf16_t* x, int64_t xs, int M, const bf16_t* w, int N, int K, int rows, int S,
               bf16_t* out, int64_t os, const bf16_t* res, int64_t rs, float* part, hipStream_t s) {
  constexpr int D = skinny_depth<MT, NT, EPI>();
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
