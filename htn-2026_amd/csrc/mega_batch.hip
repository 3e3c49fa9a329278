// Persistent batched decode step (17 <= B <= 32 sequences): the 36 layers of qd_decode_step's
// skinny-GEMM step -- per layer RMSNorm, qkv (K split 2), attention (one key split), o (K split
// 4), RMSNorm, gate/up + SwiGLU, down (K split 4) -- and the final RMSNorm, in ONE launch of one
// workgroup per CU (the batched counterpart of mega.hip; engine/kernels/mega.py:1-15 is the
// reference's persistent tier).  The step's embedding (+ RoPE row) launch runs before it and
// the LM head after it, as in qd_decode_step.
//
// Why: the per-launch B = 32 step is 256 launches of 4-45 us, and each launch boundary costs
// a drain, a ramp-up and the next kernel's first load latency (~5 us per projection beyond its
// weight stream).  Here each workgroup runs the phases in order; a GEMM phase issues its
// weight loads (which never depend on the input) before it waits for its activation rows, so
// the weight stream of a phase overlaps the hand-off of the previous one.
//
// Every phase is the per-launch kernel's workgroup body (skinny_core.h, attn_mfma.h) run for
// the same block index, so the arithmetic and its order are the same bit for bit:
//  * GEMM phases: workgroup g runs block g of the per-launch grid (row block g / S, K range
//    g % S), its activation rows read from hand-off words and its partials / outputs written as
//    hand-off words;
//  * attention: workgroup g < 8 B runs the (KV head g % 8, sequence g / 8) unit, waiting for
//    its qkv partials;
//  * RMSNorm: workgroup m < B normalises row m as the 256 threads of part_add_rmsnorm_kernel /
//    add_rmsnorm_kernel do (same chunking, same reduction order), with the residual row in
//    plain memory (only workgroup m ever touches row m in the launch).
// Hand-off words (handoff.h) live in two copies that alternate with the parity of the epoch
// word: a launch writes its copy, each word once, and zeroes the other copy, every workgroup its
// share, layer by layer; at the end every workgroup posts a done word and workgroup 0, having
// seen all of them (so every workgroup has read the epoch), advances the epoch.  Waits are
// bounded (handoff.h); a failed wait leaves error 1, an out-of-cache position error 2.
// Every workgroup is resident at once (grid = CU count >= 256, one 512-thread workgroup per CU,
// checked against the occupancy API on the host), phases only wait on earlier phases, and
// every workgroup runs every phase, so every wait is eventually satisfied.
#include "qd_launch.h"

#include "attn_mfma.h"
#include "handoff.h"
#include "norm_row.h"
#include "skinny_core.h"

namespace {

constexpr int MB_NT = 512;
// model shape of this kernel (Qwen3-4B); the host checks the weights against it
constexpr int H = 2560, INTER = 9728, HQ = 32, HKV = 8, HD = 128;
constexpr int NQKV = (HQ + 2 * HKV) * HD;   // 6144
constexpr int QD = HQ * HD;                 // 4096
constexpr int SQ = 2, SO = 4, SD = 4;       // K splits of qkv, o and down, as qd_decode_step's
constexpr int MIN_WG = 256;                 // workgroups: >= every phase's block count

// GEMM phases: 32-row tiles (MT 2) of 3 16-row weight tiles (NT 3): the plans at 256 CUs
constexpr int D_NONE = skinny_depth<2, 3, EPI_NONE>();
constexpr int D_SWIGLU = skinny_depth<2, 3, EPI_SWIGLU>();

// hand-off words of one layer: every region a multiple of 4 words (16-byte aligned)
struct MbLayout {
  int64_t xn1, qkv, att, op, xn2, act, dp, per_layer;
};

__host__ __device__ inline MbLayout mb_layout(int B) {
  MbLayout a;
  a.xn1 = 0;                                   // RMSNorm(x; ln1), bf16 pairs [B][H / 2]
  a.qkv = a.xn1 + (int64_t)B * H / 2;          // qkv partials, fp32 [SQ][B][NQKV]
  a.att = a.qkv + (int64_t)SQ * B * NQKV;      // attention rows, bf16 pairs [B][QD / 2]
  a.op = a.att + (int64_t)B * QD / 2;          // o partials, fp32 [SO][B][H]
  a.xn2 = a.op + (int64_t)SO * B * H;          // RMSNorm(x; ln2)
  a.act = a.xn2 + (int64_t)B * H / 2;          // SwiGLU output, bf16 pairs [B][INTER / 2]
  a.dp = a.act + (int64_t)B * INTER / 2;       // down partials, fp32 [SD][B][H]
  a.per_layer = a.dp + (int64_t)SD * B * H;
  return a;
}

struct MbParams {
  const bf16_t *w_qkv, *w_o, *w_gu, *w_down, *ln1, *ln2, *q_norm, *k_norm, *final_norm;
  const bf16_t* rope;      // the step's RoPE row: cos [128], sin [128]
  bf16_t *k_cache, *v_cache;
  const int64_t* pos;
  bf16_t* x;               // residual rows [B][H]
  bf16_t* xn_out;          // final RMSNorm rows [B][H], for the LM head
  uint32_t* ctl;           // [0] epoch, [1] error
  uint32_t* ll;            // two copies of `region` hand-off words
  int64_t region, cap, chunk;
  int B, L, rows_qkv, rows_o, rows_gu, rows_down;
  int blk_qkv, blk_o, blk_gu, blk_down;     // each GEMM's blocks (per-launch grid)
  float eps;
};

union MbSmem {
  uint4 sk[SkinnyShape<2, 3, EPI_SWIGLU>::LDS_U4];   // the largest skinny phase (gate/up)
  DecodeMfmaLds attn;
  float red[MB_NT / 64];
};
static_assert(SkinnyShape<2, 3, EPI_NONE>::LDS_U4 <= SkinnyShape<2, 3, EPI_SWIGLU>::LDS_U4,
              "LDS of the plain GEMM phases");

__global__ __launch_bounds__(MB_NT, 1) void mega_batch_kernel(MbParams p) {
  __shared__ MbSmem sm;
  const int wg = blockIdx.x, P = gridDim.x, B = p.B;
  uint32_t* err = p.ctl + 1;
  const uint32_t epoch = __hip_atomic_load(p.ctl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  uint32_t* ll = p.ll + (int64_t)(epoch & 1u) * p.region;          // this launch's words
  uint32_t* nxt = p.ll + (int64_t)((epoch & 1u) ^ 1u) * p.region;   // the next launch's
  const int64_t pos = p.pos[0];
  if (pos < 0 || pos >= p.cap) {   // uniform over the grid: nothing is written, nobody waits
    if (wg == 0 && threadIdx.x == 0)
      __hip_atomic_store(err, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  const MbLayout ly = mb_layout(B);
  const int64_t layer_kv = (int64_t)B * HKV * p.cap * HD;
  const float scale = 1.0f / sqrtf((float)HD);
  for (int l = 0; l < p.L; ++l) {
    uint32_t* LL = ll + (int64_t)l * ly.per_layer;
    // x' = x + the previous layer's down partials; xn1 = RMSNorm(x'; ln1)
    if (wg < B) {
      if (l == 0)
        norm_row<0, true, H>(nullptr, B, wg, p.x, p.ln1, LL + ly.xn1, p.eps, sm.red, err);
      else
        norm_row<SD, true, H>(LL - ly.per_layer + ly.dp, B, wg, p.x, p.ln1 + (int64_t)l * H,
                              LL + ly.xn1, p.eps, sm.red, err);
    }
    // qkv partials
    if (wg < p.blk_qkv)
      skinny_block<2, 3, EPI_NONE, true, D_NONE, true>(
        sm.sk, reinterpret_cast<const bf16_t*>(LL + ly.xn1), H, B, p.w_qkv + (int64_t)l * NQKV * H,
        NQKV, H, p.rows_qkv, SQ, wg, nullptr, 0, nullptr, 0, reinterpret_cast<float*>(LL + ly.qkv),
        err);
    lds_barrier();
    // attention unit (KV head wg % 8, sequence wg / 8)
    if (wg < HKV * B)
      decode_attn_mfma_block<true, true, SQ>(
          sm.attn, 0, wg % HKV, wg / HKV, 1, B, nullptr, 0, p.q_norm + (int64_t)l * HD,
          p.k_norm + (int64_t)l * HD, p.rope, p.rope + HD, p.pos, p.k_cache + l * layer_kv,
          p.v_cache + l * layer_kv, HQ, HKV, p.cap, p.chunk, p.eps, scale, nullptr, nullptr,
          reinterpret_cast<bf16_t*>(LL + ly.att), reinterpret_cast<const float*>(LL + ly.qkv), SQ,
          err);
    lds_barrier();
    // o partials
    if (wg < p.blk_o)
      skinny_block<2, 3, EPI_NONE, true, D_NONE, true>(
        sm.sk, reinterpret_cast<const bf16_t*>(LL + ly.att), QD, B, p.w_o + (int64_t)l * H * QD, H,
        QD, p.rows_o, SO, wg, nullptr, 0, nullptr, 0, reinterpret_cast<float*>(LL + ly.op), err);
    lds_barrier();
    // x'' = x' + o partials; xn2 = RMSNorm(x''; ln2)
    if (wg < B)
      norm_row<SO, true, H>(LL + ly.op, B, wg, p.x, p.ln2 + (int64_t)l * H, LL + ly.xn2, p.eps,
                            sm.red, err);
    // act = SwiGLU(xn2 . Wgate^T, xn2 . Wup^T)
    if (wg < p.blk_gu)
      skinny_block<2, 3, EPI_SWIGLU, false, D_SWIGLU, true>(
          sm.sk, reinterpret_cast<const bf16_t*>(LL + ly.xn2), H, B,
          p.w_gu + (int64_t)l * 2 * INTER * H, INTER, H, p.rows_gu, 1, wg,
          reinterpret_cast<bf16_t*>(LL + ly.act), INTER, nullptr, 0, nullptr, err);
    lds_barrier();
    // down partials
    if (wg < p.blk_down)
      skinny_block<2, 3, EPI_NONE, true, D_NONE, true>(
        sm.sk, reinterpret_cast<const bf16_t*>(LL + ly.act), INTER, B,
        p.w_down + (int64_t)l * H * INTER, H, INTER, p.rows_down, SD, wg, nullptr, 0, nullptr, 0,
        reinterpret_cast<float*>(LL + ly.dp), err);
    lds_barrier();
    hw_clear<MB_NT>(nxt + (int64_t)l * ly.per_layer, ly.per_layer, wg, P);
  }
  // final RMSNorm of x + the last down partials, for the LM head launch
  if (wg < B)
    norm_row<SD, false, H>(ll + (int64_t)(p.L - 1) * ly.per_layer + ly.dp, B, wg, p.x,
                           p.final_norm, p.xn_out, p.eps, sm.red, err);
  // done words; workgroup 0 advances the epoch once every workgroup has posted its word
  uint32_t* done = ll + (int64_t)p.L * ly.per_layer;
  if (threadIdx.x == 0) {
    hw_put(done + wg, 1u);
    __hip_atomic_store(nxt + (int64_t)p.L * ly.per_layer + wg, 0u, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
  if (wg == 0) {
    for (int q = threadIdx.x; q < P; q += MB_NT) (void)hw_wait(hw_raw(done + q), done + q, err);
    __syncthreads();
    if (threadIdx.x == 0)
      __hip_atomic_store(p.ctl, epoch + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// words of one copy of the hand-off area (a multiple of 64: each copy 256-byte aligned)
int64_t mb_region_words(int L, int B, int grid) {
  return ((int64_t)L * mb_layout(B).per_layer + grid + 63) / 64 * 64;
}

}  // namespace

// ------------------------------------------------------------------ host side
int mega_batch_grid() {
  static int grid = -1;
  if (grid < 0) {
    int dev = 0, cus = 0, occ = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, mega_batch_kernel, MB_NT, 0) !=
            hipSuccess) {
      (void)hipGetLastError();
      grid = 0;
    } else {
      grid = (occ >= 1 && cus >= MIN_WG) ? cus : 0;
    }
  }
  return grid;
}

// The shapes this kernel runs: Qwen3-4B, 17..32 sequences, every GEMM plan of 3 weight tiles
// per workgroup (the skinny step's plans on this device) and one key split of attention.
bool mega_batch_ok(int hidden, int inter, int hq, int hkv, int head_dim, int64_t B, int64_t cap) {
  if (hidden != H || inter != INTER || hq != HQ || hkv != HKV || head_dim != HD) return false;
  if (B < 17 || B > 32 || mega_batch_grid() <= 0) return false;
  const int64_t rows[4] = {skinny_rows(NQKV, SQ), skinny_rows(H, SO), skinny_rows(INTER, 1),
                           skinny_rows(H, SD)};
  for (int64_t r : rows)
    if ((r + 15) / 16 != 3) return false;
  if (cap > 0 && decode_attn_splits(B, HKV, cap) != 1) return false;
  return true;
}

int64_t mega_batch_ll_bytes(int L, int64_t B) {
  const int grid = mega_batch_grid();
  return grid > 0 ? 2 * mb_region_words(L, (int)B, grid) * 4 : 0;
}

hipError_t launch_mega_batch(const MegaBatchLaunch& m, hipStream_t s) {
  const int grid = mega_batch_grid();
  if (grid <= 0) return hipErrorInvalidConfiguration;
  MbParams p;
  p.w_qkv = m.w_qkv; p.w_o = m.w_o; p.w_gu = m.w_gu; p.w_down = m.w_down; p.ln1 = m.ln1;
  p.ln2 = m.ln2; p.q_norm = m.q_norm; p.k_norm = m.k_norm; p.final_norm = m.final_norm;
  p.rope = m.rope; p.k_cache = m.k_cache; p.v_cache = m.v_cache; p.pos = m.pos; p.x = m.x;
  p.xn_out = m.xn_out; p.ctl = m.ctl; p.ll = m.ll; p.cap = m.cap; p.B = (int)m.B; p.L = m.L;
  p.eps = m.eps;
  p.chunk = decode_attn_chunk(m.cap, 1);
  p.region = mb_region_words(m.L, p.B, grid);
  p.rows_qkv = (int)skinny_rows(NQKV, SQ);
  p.rows_o = (int)skinny_rows(H, SO);
  p.rows_gu = (int)skinny_rows(INTER, 1);
  p.rows_down = (int)skinny_rows(H, SD);
  p.blk_qkv = (NQKV + p.rows_qkv - 1) / p.rows_qkv * SQ;
  p.blk_o = (H + p.rows_o - 1) / p.rows_o * SO;
  p.blk_gu = (INTER + p.rows_gu - 1) / p.rows_gu;
  p.blk_down = (H + p.rows_down - 1) / p.rows_down * SD;
  if (p.blk_qkv > grid || p.blk_o > grid || p.blk_gu > grid || p.blk_down > grid || HKV * p.B > grid)
    return hipErrorInvalidConfiguration;
  mega_batch_kernel<<<dim3((unsigned)grid), dim3(MB_NT), 0, s>>>(p);
  return hipGetLastError();
}
