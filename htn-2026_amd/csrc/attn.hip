// GQA attention over a contiguous bf16 KV cache [B, Hkv, cap, 128] (one layer), 4 query heads
// per KV head, head_dim 128.
//
// decode_attn  one new token per sequence at the device position pos[0] (fast.py:217-342,
//              decode_attn.py:26-119): q-RMSNorm + RoPE of the group's 4 q heads, the split that
//              owns `pos` normalises + ropes the new K, writes K/V into the cache and attends the
//              new key from LDS; every split runs an online softmax over its cached keys
//              [start, min(end, pos)) and writes (m, l, acc); a second launch merges (LSE).
// block_attn   T query tokens per sequence (tree verification / chunked prefill, tree.py:72-142):
//              keys < base[b] are visible to every token, block slot base + j is visible to
//              token t iff bit j of anc[b, t] (tree) or j <= t (causal chunk).
//
// Numerics (decode_attn.py:7-11): fp32 scores q.k * 128^-1/2, fp32 online softmax, P rounded
// to bf16 before P.V, fp32 accumulate, split merge by log-sum-exp, / l in fp32, bf16 out.
//
// Work mapping: a wave is 4 groups of 16 lanes; a group handles KPG consecutive keys per
// iteration and lane i of the group owns dims [8i, 8i+8) -- one 16-byte load per key row for K
// and for V, so a group reads a 256-byte K row and a 256-byte V row contiguously.
#include "qd_launch.h"

#include "attn_core.h"
#include "attn_mfma.h"

// ROPE_ROW: cos_t / sin_t point at this step's RoPE row (written by the embedding kernel), so
// no prologue load waits for pos; otherwise they are [cap, 128] tables indexed by pos.
template <int NW, bool ROPE_ROW>
__global__ __launch_bounds__(NW * 64) void decode_attn_kernel(
    const bf16_t* __restrict__ qkv, int64_t qkv_stride, const bf16_t* __restrict__ qn,
    const bf16_t* __restrict__ kn, const bf16_t* __restrict__ cos_t,
    const bf16_t* __restrict__ sin_t, const int64_t* __restrict__ pos_ptr, bf16_t* k_cache,
    bf16_t* v_cache, int Hq, int Hkv, int64_t cap, int64_t chunk, float eps, float scale,
    float* ws_acc, float* ws_ml, bf16_t* out) {
  __shared__ DecodeAttnLds<NW> sm;
  const int split = blockIdx.x, kvh = blockIdx.y;
  const int64_t b = blockIdx.z;
  const int splits = gridDim.x;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const bf16_t* row = qkv + b * qkv_stride;
  // every prologue load is issued before pos is known: this wave's head row, its norm weights
  // and (ROPE_ROW) the RoPE row; all waves run the same straight-line loads
  auto fetch = [&](HeadVals& hv) -> int64_t {
    const bf16_t* qsrc = row + attn_q_elem(wave, kvh);
    const bf16_t* ksrc = row + attn_kv_elem<NW>(wave, kvh, Hq, Hkv);
    hv.q1 = qsrc[lane]; hv.q2 = qsrc[lane + 64];
    hv.k1 = ksrc[lane]; hv.k2 = ksrc[lane + 64];
    hv.qw1 = bf2f(qn[lane]); hv.qw2 = bf2f(qn[lane + 64]);
    hv.kw1 = bf2f(kn[lane]); hv.kw2 = bf2f(kn[lane + 64]);
    if constexpr (ROPE_ROW) {
      hv.c1 = bf2f(cos_t[lane]); hv.c2 = bf2f(cos_t[lane + 64]);
      hv.s1 = bf2f(sin_t[lane]); hv.s2 = bf2f(sin_t[lane + 64]);
    }
    const int64_t pos = pos_ptr[0];
    if constexpr (!ROPE_ROW) {
      const int64_t pr = (pos >= 0 && pos < cap ? pos : 0) * 128;   // a valid row either way
      hv.c1 = bf2f(cos_t[pr + lane]); hv.c2 = bf2f(cos_t[pr + lane + 64]);
      hv.s1 = bf2f(sin_t[pr + lane]); hv.s2 = bf2f(sin_t[pr + lane + 64]);
    }
    return pos;
  };
  const int64_t qrow0 = b * Hq + kvh * GRP;
  auto final_out = [&](int h, int d, float y0, float y1) {
    *reinterpret_cast<uint32_t*>(out + (qrow0 + h) * 128 + d) = pack2(y0, y1);
  };
  auto partial_out = [&](int h, int d, float A0, float A1, float M, float L) {
    const int64_t idx = (qrow0 + h) * splits + split;
    *reinterpret_cast<float2*>(ws_acc + idx * 128 + d) = make_float2(A0, A1);
    if ((threadIdx.x & 63) == 0) *reinterpret_cast<float2*>(ws_ml + idx * 2) = make_float2(M, L);
  };
  decode_attn_unit<NW>(sm, fetch, final_out, partial_out, k_cache, v_cache,
                       ((b * Hkv + kvh) * cap) * 128, cap, (int64_t)split * chunk, chunk,
                       splits == 1, eps, scale);
}

// One wave per (token row, head): log-sum-exp merge of the split partials -> bf16 out
// [rows, Hq*128] (decode_attn.py:74-86, tree.py:130-142).  A separate launch: the kernel
// boundary is the only cross-workgroup synchronisation, so no workgroup fences or waits.
// Lanes read the splits' (m, l) in parallel; each lane then owns 2 of the 128 dims.
constexpr int MERGE_MAX_SPLITS = 1024;

__global__ __launch_bounds__(64) void attn_merge_kernel(const float* __restrict__ ws_acc,
                                                         const float* __restrict__ ws_ml,
                                                         int splits, bf16_t* __restrict__ out) {
  const int64_t r = blockIdx.x;  // (b*T + t)*Hq + h
  const int lane = threadIdx.x;
  const float2* ml = reinterpret_cast<const float2*>(ws_ml) + r * splits;
  const float2* acc = reinterpret_cast<const float2*>(ws_acc + r * splits * 128) + lane;
  const float2 y = merge_splits(
      splits, [&](int sp) { return ml[sp]; },
      [&](int first, int n, float2 (&a)[MERGE_BATCH]) {
#pragma unroll
        for (int q = 0; q < MERGE_BATCH; ++q)
          a[q] = q < n ? acc[(int64_t)(first + q) * 64] : make_float2(0.f, 0.f);
      });
  *reinterpret_cast<uint32_t*>(out + r * 128 + lane * 2) = pack2(y.x, y.y);
}

// Split policy: ATTN_NW waves per workgroup take ATTN_TILE keys per iteration.  Splits of at
// most ATTN_SPLIT_KEYS keys; while (batch x KV heads x splits) < 128 workgroups, more splits
// (whole tiles) up to ~1 workgroup per CU.  Chosen from a sweep on MI355X of {4, 8} waves x
// splits at B = 1 (cap 768), 4 (cap 8512) and 32 (cap 2176).
constexpr int64_t ATTN_TILE = ATTN_NW * 16;
constexpr int64_t ATTN_SPLIT_KEYS = 4096;

int64_t decode_attn_splits(int64_t B, int Hkv, int64_t cap) {
  const int64_t pairs = B * Hkv;
  int64_t sp = (cap + ATTN_SPLIT_KEYS - 1) / ATTN_SPLIT_KEYS;     // bound the keys per split
  const int64_t fill = (256 + pairs - 1) / pairs;                  // ~1 workgroup per CU
  const int64_t max_sp = (cap + ATTN_TILE - 1) / ATTN_TILE;
  if (pairs * sp < 128 && sp < fill) sp = fill < max_sp ? fill : max_sp;
  if (sp < 1) sp = 1;
  const int64_t chunk = decode_attn_chunk(cap, sp);
  return (cap + chunk - 1) / chunk;
}

int64_t decode_attn_chunk(int64_t cap, int64_t splits) {
  int64_t chunk = (cap + splits - 1) / splits;
  return (chunk + ATTN_TILE - 1) / ATTN_TILE * ATTN_TILE;
}

static void launch_decode_attn_mfma(const bf16_t* qkv, int64_t qkv_stride, const bf16_t* qn,
                                    const bf16_t* kn, const bf16_t* cos_t, const bf16_t* sin_t,
                                    const int64_t* pos, bf16_t* k_cache, bf16_t* v_cache,
                                    int64_t B, int Hq, int Hkv, int64_t cap, int64_t splits,
                                    int64_t chunk, float eps, float* ws_acc, float* ws_ml,
                                    bf16_t* out, bool rope_row, hipStream_t s,
                                    const float* part = nullptr, int part_S = 0);

void launch_decode_attn(const bf16_t* qkv, int64_t qkv_stride, const bf16_t* qn, const bf16_t* kn,
                        const bf16_t* cos_t, const bf16_t* sin_t, const int64_t* pos,
                        bf16_t* k_cache, bf16_t* v_cache, int64_t B, int Hq, int Hkv, int64_t cap,
                        int64_t splits, float eps, float* ws_acc, float* ws_ml, bf16_t* out,
                        bool rope_row, hipStream_t s) {
  const int64_t chunk = decode_attn_chunk(cap, splits);
  const dim3 grid((unsigned)splits, (unsigned)Hkv, (unsigned)B), block(ATTN_NW * 64);
  if (B >= 2)
    launch_decode_attn_mfma(qkv, qkv_stride, qn, kn, cos_t, sin_t, pos, k_cache, v_cache, B, Hq,
                            Hkv, cap, splits, chunk, eps, ws_acc, ws_ml, out, rope_row, s);
  else if (rope_row)
    decode_attn_kernel<ATTN_NW, true><<<grid, block, 0, s>>>(
        qkv, qkv_stride, qn, kn, cos_t, sin_t, pos, k_cache, v_cache, Hq, Hkv, cap, chunk, eps,
        1.0f / sqrtf(128.0f), ws_acc, ws_ml, out);
  else
    decode_attn_kernel<ATTN_NW, false><<<grid, block, 0, s>>>(
        qkv, qkv_stride, qn, kn, cos_t, sin_t, pos, k_cache, v_cache, Hq, Hkv, cap, chunk, eps,
        1.0f / sqrtf(128.0f), ws_acc, ws_ml, out);
  if (splits > 1)
    attn_merge_kernel<<<dim3((unsigned)(B * Hq)), dim3(64), 0, s>>>(ws_acc, ws_ml, (int)splits, out);
}

// ------------------------------------------------------------------ block (tree / causal chunk)
constexpr int64_t BLOCK_CHUNK = 512;

// Block attention for T query tokens per sequence (tree verification with ancestor masks, causal
// prefill chunks): query token t of sequence b sees every cached key < base[b] and block key
// base[b] + j iff bit j of anc[b*T + t] (tree.py:72-195, engine.py:445-461) or j <= t (causal).
// v_mfma_f32_16x16x32_bf16.  Workgroup = (key split of `chunk` keys, KV head, block of
// BA_TQ = 64 query tokens of one sequence), 8 waves: wave w handles query head kvh*4 + (w & 3)
// for the block's tokens 32 (w >> 2) .. + 31 (two 16-row tiles), so every staged K/V tile
// serves 64 tokens x 4 heads.  Keys go in tiles of BA_KT = 64:
//  * S' = K . Q^T: A = K tile rows (LDS, 16-byte units XOR-swizzled by key), B = the lane's query
//    row (registers); lane (c, q) ends up holding the scores of its query row c against keys
//    16 h + 4q .. 16 h + 4q + 3 of the tile, h = 0..3;
//  * softmax in log2 units: s' = (q.k) * 128^-1/2 * log2(e) (the scale folded into one fma with
//    the subtraction of the row's reference maximum m), p = 2^(s' - m) on v_exp_f32, P rounded
//    to bf16.  m moves only when a tile's maximum exceeds it by more than BA_TAU, so p <= 2^TAU
//    and the rescale of O and l by 2^(m_old - m_new) runs only when some row's maximum jumped
//    (the first visible tile, rarely after); the row max / sum across the four q lanes of a row
//    go through permlane swaps;
//  * O^T += V^T . P^T per 32-key half: A = V^T fragments, B = the lane's 8 probabilities, taken
//    in that same key order (a permutation of the contraction index shared by both operands), so
//    O^T's lane (c, q) holds dims 16 dt + 4q..+3 of row c and the per-row rescale needs no
//    cross-lane traffic.  V is staged key-major like K (one 16-byte store per thread and key) and
//    read transposed with gfx950's ds_read_b64_tr_b16: within a 16-lane group, lane j = 4a + b
//    receives element b of the 8-byte pieces that lanes a, a + 4, a + 8, a + 12 address, so lane
//    i addressing dims 16 dt + 4 (i % 4) .. + 3 of key 4q + i / 4 makes lane c receive
//    V[4q + r][16 dt + c], r = 0..3 (measured on MI355X with an in-bounds layout probe);
//  * pipeline: three LDS tile buffers; in the step of tile i a wave contracts S' of tile i + 1
//    (its MFMAs independent of the softmax of tile i, which the compiler interleaves with them),
//    runs the softmax and O update of tile i, and the workgroup stages tile i + 2 from registers
//    loaded two steps earlier (thread i moves K and V unit i % 16 of keys i / 16 and i / 16 + 32);
//    one barrier per tile.
// Numerics against the math path: every p is one bf16 rounding of a probability scaled by at
// most 2^TAU, and the running rescale is exact up to fp32 rounding, as in any online softmax.
// Writes (m, l, acc) partials per (query row, head, split) -- m in natural-log units, as
// attn_merge_kernel expects; ws_acc[idx * 128 + d], ws_ml[idx * 2], idx = ((b*T + t)*Hq + h)*splits
// + split -- or, with one split, the normalised bf16 rows.
constexpr int BA_TQ = 64;
constexpr int BA_KT = 64;
#ifndef QD_BA_NBUF
#define QD_BA_NBUF 4
#endif
constexpr int BA_NBUF = QD_BA_NBUF;   // LDS tile buffers (BA_NBUF - 3 tiles in flight beyond the next)
#ifndef QD_BA_TAU
#define QD_BA_TAU 8.0f
#endif
constexpr float BA_TAU = QD_BA_TAU;
constexpr float BA_LN2 = 0.69314718055994531f;

struct BlockAttnLds {
  uint4 k[BA_NBUF][BA_KT * 16];
  uint4 v[BA_NBUF][BA_KT * 16];
};

__global__ __launch_bounds__(512) void block_attn_mfma_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k_cache,
    const bf16_t* __restrict__ v_cache, const int64_t* __restrict__ base_ptr,
    const uint64_t* __restrict__ anc, int64_t T, int Hq, int Hkv, int64_t cap, int64_t chunk,
    float scale_log2, float* ws_acc, float* ws_ml, bf16_t* __restrict__ out) {
  typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
  typedef __attribute__((ext_vector_type(4))) float f32x4_t;
  __shared__ BlockAttnLds sm;
  const int split = blockIdx.x, kvh = blockIdx.y;
  const int splits = gridDim.x;
  const int64_t QB = (T + BA_TQ - 1) / BA_TQ;
  const int64_t b = blockIdx.z / QB;
  // query blocks in descending order: under a causal mask the later blocks hold the most keys,
  // and starting them first leaves the short ones for the end of the launch
  const int64_t tb = (QB - 1 - blockIdx.z % QB) * BA_TQ;    // the workgroup's first token
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int head = wave & 3;
  const int64_t t0 = tb + 32 * (wave >> 2);                 // this wave's first token
  const int c = lane & 15, q4 = lane >> 4;
  const int64_t base = base_ptr[b];
  // query rows of this lane: token t0 + 16 rt + c, head kvh * 4 + head
  uint4 qf[2][4];
  uint64_t mask[2];
  int64_t tok[2];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    tok[rt] = t0 + 16 * rt + c;
    const int64_t tt = tok[rt] < T ? tok[rt] : T - 1;
    const uint4* qr = reinterpret_cast<const uint4*>(q + ((b * T + tt) * Hq + kvh * GRP + head) * 128);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) qf[rt][kk] = qr[4 * kk + q4];
    mask[rt] = anc ? anc[b * T + tt] : 0;
  }
  const int64_t start = (int64_t)split * chunk;
  int64_t kend = start + chunk;
  if (kend > base + T) kend = base + T;
  if (!anc && kend > base + tb + BA_TQ) kend = base + tb + BA_TQ;   // causal: later keys unseen
  if (kend > cap) kend = cap;
  const int ntiles = kend > start ? (int)((kend - start + BA_KT - 1) / BA_KT) : 0;
  const int64_t head_off = ((b * Hkv + kvh) * cap) * 128;
  const uint4* kb = reinterpret_cast<const uint4*>(k_cache + head_off);
  const uint4* vb = reinterpret_cast<const uint4*>(v_cache + head_off);
  // o[rt][dt]: O^T dims 16 dt + 4 q4 .. + 3 of the lane's row c; lsum[rt]: the fp32 sum of the
  // lane's probabilities of that row (its four q lanes hold disjoint keys)
  float m[2] = {M_FLOOR, M_FLOOR}, lsum[2] = {0.f, 0.f};
  f32x4_t o[2][8];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[rt][dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // Staging by DMA (global_load_lds_dwordx4, no registers): wave w moves the 1 KiB blocks 2w
  // and 2w + 1 of a tile's K and of its V (block j = keys 4j .. 4j + 3); lane l of block j lands
  // in LDS slot 64 j + l = unit (l & 15) of key 4 j + (l >> 4) as stored, i.e. logical unit
  // (l & 15) ^ (key & 15) (the XOR swizzle the fragment reads undo).  Keys past the cache
  // reload its last row (valid, never used).  Key indices and byte offsets within a head are
  // 32-bit: cap is at most 1024 splits x BLOCK_CHUNK keys (checked by the entry points), 134 MB
  // of K per head.
  const int dk0 = 8 * wave + (lane >> 4), dk1 = dk0 + 4;
  const uint32_t du0 = (uint32_t)((lane & 15) ^ (dk0 & 15)) * 16u;
  const uint32_t du1 = (uint32_t)((lane & 15) ^ (dk1 & 15)) * 16u;
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_u32(&sm.k[0][0])) + (uint32_t)wave * 2048u;
  constexpr uint32_t TILE_B = BA_KT * 16 * 16;                  // bytes of one K (V) tile
  constexpr uint32_t V_OFF = BA_NBUF * TILE_B;                  // sm.v after sm.k
  const int start32 = (int)start, last = (int)cap - 1;
  // the tile's K blocks (half 0), its V blocks (half 1), or both (-1)
  auto issue = [&](int it, int buf, int half = -1) {
    const int ts = start32 + BA_KT * it;
    const uint32_t oa = (uint32_t)min(ts + dk0, last) * 256u + du0;
    const uint32_t ob = (uint32_t)min(ts + dk1, last) * 256u + du1;
    const uint32_t l = lds0 + (uint32_t)buf * TILE_B;
    if (half != 1) {
      dma16(kb, oa, l);
      dma16(kb, ob, l + 1024u);
    }
    if (half != 0) {
      dma16(vb, oa, l + V_OFF);
      dma16(vb, ob, l + V_OFF + 1024u);
    }
  };
  // S' of the tile in `buf` for both row tiles: sc[rt][h] = keys 16 h + 4 q4 .. + 3, row c
  auto scores = [&](int buf, f32x4_t (&sc)[2][4]) {
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int h = 0; h < 4; ++h) sc[rt][h] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const int key = 16 * h + c;                            // key & 15 == c
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const uint4 kf = sm.k[buf][key * 16 + ((4 * kk + q4) ^ c)];
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
          sc[rt][h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bf16x8_t, kf), __builtin_bit_cast(bf16x8_t, qf[rt][kk]),
              sc[rt][h], 0, 0, 0);
      }
    }
  };
  // invisible keys of a tile that touches the block or the range end -> -inf, from one 64-bit
  // visibility word per row (bit i = tile key j0 + i): the tile's cached keys (below base), the
  // block keys the row sees (its ancestor bits, or for a causal chunk the keys up to itself),
  // cut at kend
  auto mask_tile = [&](int64_t j0, f32x4_t (&sc)[2][4]) {
    const int jrel0 = (int)(j0 - base);                       // block index of key j0 (may be < 0)
    const int lim = (int)(kend - j0);                         // keys of the tile below kend
    const uint64_t limbits = lim >= 64 ? ~0ull : lim <= 0 ? 0ull : (1ull << lim) - 1;
    const uint64_t cached = jrel0 >= 0 ? 0ull : jrel0 <= -64 ? ~0ull : (1ull << -jrel0) - 1;
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      uint64_t blk;
      if (anc) {
        blk = jrel0 >= 64 ? 0ull : jrel0 >= 0 ? mask[rt] >> jrel0
                                   : jrel0 <= -64 ? 0ull : mask[rt] << -jrel0;
      } else {
        const int64_t n = tok[rt] - jrel0 + 1;                // block keys jrel0 .. tok visible
        blk = n <= 0 ? 0ull : n >= 64 ? ~0ull : (1ull << n) - 1;
      }
      const uint64_t vis = (cached | blk) & limbits;
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const uint32_t nib = (uint32_t)(vis >> (16 * h + 4 * q4)) & 15u;
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (!((nib >> r) & 1u)) sc[rt][h][r] = NEG_INF;
      }
    }
  };
  // softmax of a tile's scores: rescale O / l if a row's maximum jumped, then the tile's
  // probabilities as bf16 MFMA B fragments pf (keys 8 j .. 8 j + 7 of the lane's order)
  auto softmax = [&](const f32x4_t (&sc)[2][4], uint4 (&pf)[2][2]) {
    float mx[2];
    bool need[2];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      float x[4];
#pragma unroll
      for (int h = 0; h < 4; ++h)
        x[h] = fmaxf(fmaxf(sc[rt][h][0], sc[rt][h][1]), fmaxf(sc[rt][h][2], sc[rt][h][3]));
      float y = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
      y = fmaxf(y, lane_xor16(y));
      y = fmaxf(y, lane_xor32(y));
      mx[rt] = y * scale_log2;                                // = max of the scaled scores
      need[rt] = mx[rt] > m[rt] + BA_TAU;
    }
    if (__ballot(need[0] || need[1]) != 0) {                 // wave-uniform
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        const float mn = need[rt] ? mx[rt] : m[rt];
        const float a = __builtin_amdgcn_exp2f(m[rt] - mn);  // 1 for rows that keep m
        m[rt] = mn;
        lsum[rt] *= a;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) o[rt][dt] *= a;
      }
    }
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      float p[16];
#pragma unroll
      for (int h = 0; h < 4; ++h)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          p[4 * h + r] = __builtin_amdgcn_exp2f(fmaf(sc[rt][h][r], scale_log2, -m[rt]));
      float t[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) t[e] = p[e] + p[e + 8];
#pragma unroll
      for (int e = 0; e < 4; ++e) t[e] += t[e + 4];
      lsum[rt] += (t[0] + t[2]) + (t[1] + t[3]);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        pf[rt][j] = make_uint4(pack2(p[8 * j + 0], p[8 * j + 1]), pack2(p[8 * j + 2], p[8 * j + 3]),
                               pack2(p[8 * j + 4], p[8 * j + 5]), pack2(p[8 * j + 6], p[8 * j + 7]));
    }
  };
  // this lane's transposed-read address for V dims 16 dt + 4 (c % 4) .. + 3 of key 16 h + 4 q4 +
  // c / 4: 16-byte unit 2 dt + (c / 2) % 2, half c % 2
  auto vt_addr = [&](int buf, int dt, int h) -> const void* {
    const int key = 16 * h + 4 * q4 + (c >> 2);
    const int u = 2 * dt + ((c >> 1) & 1);
    return reinterpret_cast<const char*>(&sm.v[buf][key * 16 + (u ^ (key & 15))]) + 8 * (c & 1);
  };
  // O^T += V^T . P^T from the tile in `buf`, per 32-key half j: keys 32 j + 4 q4 .. + 3 and
  // 32 j + 16 + 4 q4 .. + 3
  auto pv = [&](int buf, const uint4 (&pf)[2][2]) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const uint2 lo = lds_read_tr16(vt_addr(buf, dt, 2 * j));
        const uint2 hi = lds_read_tr16(vt_addr(buf, dt, 2 * j + 1));
        const uint4 vf = make_uint4(lo.x, lo.y, hi.x, hi.y);
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
          o[rt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bf16x8_t, vf), __builtin_bit_cast(bf16x8_t, pf[rt][j]),
              o[rt][dt], 0, 0, 0);
      }
    }
  };
  // Tile it sits in buffer it % BA_NBUF.  Step it issues the DMA of tile it + BA_NBUF - 2 into the
  // buffer of tile it - 2 (last read in step it - 1, before its barrier), does its share of the
  // contraction, then waits for its own DMA of tile it + 1 (the loads of the tiles after it may
  // stay in flight) and meets the other waves at the barrier, after which tile it + 1 is
  // visible.  Tiles past ntiles are loaded (valid cache rows) but never consumed.
  // Waves w and w + 4 share a SIMD.  Waves 0-3 run step it as O += P(it-1) V(it-1), S'(it),
  // softmax(it) -- MFMA, then VALU -- and waves 4-7 half a step behind as softmax(it-1),
  // O += P(it-1) V(it-1), S'(it) -- VALU, then MFMA -- so that on every SIMD one wave's MFMAs can
  // run beside the other's softmax.  Each wave still applies its tiles in order.
  constexpr int AHEAD = BA_NBUF - 2;
#pragma unroll
  for (int i = 0; i < AHEAD; ++i) issue(i, i);
  wait_vm<4 * (AHEAD - 1)>();
  lds_barrier();
  const bool lead = wave < 4;                                // wave-uniform
  f32x4_t sc[2][4];
  uint4 pf[2][2];
  // a tile is visible to every row of the workgroup when it ends below kend and below base --
  // or, in a causal chunk, below the workgroup's first token (every row sees the block keys
  // before it)
  const int64_t open_end = anc ? base : base + tb;
  auto whole = [&](int it) {
    const int64_t j0 = start + (int64_t)BA_KT * it;
    return j0 + BA_KT <= open_end && j0 + BA_KT <= kend;
  };
  // A causal chunk issues a step's V loads after its first phase (the P V update, or for waves
  // 4-7 softmax + P V) instead of with the K loads: 2596 -> 2548 us per 4 x 8192 layer (two
  // traced runs each); with ancestor masks (a verify) that measured slower (54.5 -> 55.4 us), so
  // there all four go first.
  const bool late_v = anc == nullptr;                        // uniform
  int buf = 0, bprev = BA_NBUF - 1;                          // tiles it and it - 1
  for (int it = 0; it < ntiles; ++it) {
    const int bl = bprev == 0 ? BA_NBUF - 1 : bprev - 1;     // tile it - 2's buffer
    issue(it + AHEAD, bl, late_v ? 0 : -1);
    if (lead) {
      if (it > 0) pv(bprev, pf);
      if (late_v) issue(it + AHEAD, bl, 1);
      scores(buf, sc);
      if (!whole(it)) mask_tile(start + (int64_t)BA_KT * it, sc);
      softmax(sc, pf);
    } else {
      if (it > 0) {
        if (!whole(it - 1)) mask_tile(start + (int64_t)BA_KT * (it - 1), sc);
        softmax(sc, pf);
        pv(bprev, pf);
      }
      if (late_v) issue(it + AHEAD, bl, 1);
      scores(buf, sc);
    }
    wait_vm<4 * (AHEAD - 1)>();
    lds_barrier();
    bprev = buf;
    buf = buf == BA_NBUF - 1 ? 0 : buf + 1;
  }
  if (ntiles > 0) {                                          // the last tile's O update
    if (!lead) {
      if (!whole(ntiles - 1)) mask_tile(start + (int64_t)BA_KT * (ntiles - 1), sc);
      softmax(sc, pf);
    }
    pv(bprev, pf);
  }
  wait_vm<0>();                                              // no DMA outlives the workgroup
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    float l = lsum[rt];
    l += lane_xor16(l);
    l += lane_xor32(l);
    if (tok[rt] >= T) continue;
    const int64_t idx = ((b * T + tok[rt]) * Hq + kvh * GRP + head) * splits + split;
    if (splits == 1) {
      // one key split: the row is complete here (attn_merge_kernel over one split computes
      // the same acc * (1 / l))
      const float inv = 1.0f / l;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const f32x4_t a = o[rt][dt];
        *reinterpret_cast<uint2*>(out + idx * 128 + 16 * dt + 4 * q4) =
            make_uint2(pack2(a[0] * inv, a[1] * inv), pack2(a[2] * inv, a[3] * inv));
      }
      continue;
    }
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
      *reinterpret_cast<f32x4_t*>(ws_acc + idx * 128 + 16 * dt + 4 * q4) = o[rt][dt];
    if (q4 == 0) { ws_ml[idx * 2] = m[rt] * BA_LN2; ws_ml[idx * 2 + 1] = l; }
  }
}

// the most splits (BLOCK_CHUNK keys each) a launch may use: what the workspace is sized for
// ------------------------------------------------------------------ decode attention on MFMA (B >= 2)
// The decode unit (decode_attn_unit: same prologue, same numerics) with its two contractions on
// v_mfma_f32_16x16x32_bf16.  Workgroup = (key split, KV head, sequence), 8 waves.  After the
// prologue (q / k RMSNorm + RoPE, the new token's K/V written to the cache by the split that
// owns pos), wave w takes tiles w, w + 8, ... of 32 keys of the split's range, the new token
// included: it stages each tile key-major in its own LDS region (one 1 KiB-contiguous
// non-temporal load per 4 keys, 16-byte units XOR-swizzled by key; the new token's row from
// LDS) and contracts it as the block kernel does, with the group's 4 query heads as columns
// 0..3 of the 16-column B operand: S' = K . Q^T, online softmax per column, O^T += V^T . P^T
// with transposed V reads.  The waves' (m, l, O) are then combined in LDS (over the staging
// region) and written exactly as the unit writes them (normalised output, or split partials
// for attn_merge_kernel).  Measured at B = 32 (256 workgroups, ~2112 keys each): the VALU unit
// takes 51.9 us per layer (VALU busy 77 % of its cycles); this kernel with 4 waves and plain
// loads 51.0 us (the same whether one or two tiles are in flight per wave), with 8 waves
// ~49.7 us, with the K/V loads non-temporal 45.0 us.  Agrees with decode_attn_kernel up to fp32
// summation order; B = 1 keeps decode_attn_kernel, whose arithmetic the persistent step shares
// bit for bit.
template <bool ROPE_ROW>
__global__ __launch_bounds__(DM_NW * 64) void decode_attn_mfma_kernel(
    const bf16_t* __restrict__ qkv, int64_t qkv_stride, const bf16_t* __restrict__ qn,
    const bf16_t* __restrict__ kn, const bf16_t* __restrict__ cos_t,
    const bf16_t* __restrict__ sin_t, const int64_t* __restrict__ pos_ptr, bf16_t* k_cache,
    bf16_t* v_cache, int Hq, int Hkv, int64_t cap, int64_t chunk, float eps, float scale,
    float* ws_acc, float* ws_ml, bf16_t* out, const float* __restrict__ part, int part_S) {
  __shared__ DecodeMfmaLds sm;
  decode_attn_mfma_block<ROPE_ROW>(sm, (int)blockIdx.x, (int)blockIdx.y, (int64_t)blockIdx.z,
                                   (int)gridDim.x, (int64_t)gridDim.z, qkv, qkv_stride, qn, kn,
                                   cos_t, sin_t, pos_ptr, k_cache, v_cache, Hq, Hkv, cap, chunk, eps,
                                   scale, ws_acc, ws_ml, out, part, part_S);
}

static void launch_decode_attn_mfma(const bf16_t* qkv, int64_t qkv_stride, const bf16_t* qn,
                                    const bf16_t* kn, const bf16_t* cos_t, const bf16_t* sin_t,
                                    const int64_t* pos, bf16_t* k_cache, bf16_t* v_cache,
                                    int64_t B, int Hq, int Hkv, int64_t cap, int64_t splits,
                                    int64_t chunk, float eps, float* ws_acc, float* ws_ml,
                                    bf16_t* out, bool rope_row, hipStream_t s,
                                    const float* part, int part_S) {
  const dim3 grid((unsigned)splits, (unsigned)Hkv, (unsigned)B), block(DM_NW * 64);
  const float scale = 1.0f / sqrtf(128.0f);
  if (rope_row)
    decode_attn_mfma_kernel<true><<<grid, block, 0, s>>>(qkv, qkv_stride, qn, kn, cos_t, sin_t,
                                                         pos, k_cache, v_cache, Hq, Hkv, cap,
                                                         chunk, eps, scale, ws_acc, ws_ml, out,
                                                         part, part_S);
  else
    decode_attn_mfma_kernel<false><<<grid, block, 0, s>>>(qkv, qkv_stride, qn, kn, cos_t, sin_t,
                                                          pos, k_cache, v_cache, Hq, Hkv, cap,
                                                          chunk, eps, scale, ws_acc, ws_ml, out,
                                                          part, part_S);
}

void launch_decode_attn_part(const float* part, int part_S, const bf16_t* qn, const bf16_t* kn,
                             const bf16_t* cos_t, const bf16_t* sin_t, const int64_t* pos,
                             bf16_t* k_cache, bf16_t* v_cache, int64_t B, int Hq, int Hkv,
                             int64_t cap, int64_t splits, float eps, float* ws_acc, float* ws_ml,
                             bf16_t* out, bool rope_row, hipStream_t s) {
  const int64_t chunk = decode_attn_chunk(cap, splits);
  launch_decode_attn_mfma(nullptr, 0, qn, kn, cos_t, sin_t, pos, k_cache, v_cache, B, Hq, Hkv,
                          cap, splits, chunk, eps, ws_acc, ws_ml, out, rope_row, s, part, part_S);
  if (splits > 1)
    attn_merge_kernel<<<dim3((unsigned)(B * Hq)), dim3(64), 0, s>>>(ws_acc, ws_ml, (int)splits, out);
}

int64_t block_attn_splits(int64_t cap) { return (cap + BLOCK_CHUNK - 1) / BLOCK_CHUNK; }

// Key splits are only there to fill the chip when few query blocks exist (a tree verification:
// B blocks per KV head).  Every extra split writes and re-reads a full set of fp32 partials for
// every query row, and the kernel runs one 8-wave workgroup per CU (its registers), so the
// launch uses as many splits as fit in ONE round of workgroups over the CUs (at least one), each
// covering a whole number of 32-key tiles.  Measured on MI355X (config 5): 17 splits of 512
// keys (544 workgroups, a 1/8-full third round) 10.44 ms per verify forward, 16 splits 9.66 ms,
// 8 splits 9.08 ms; the 4 x 8192 prefill 0.69 -> 0.59 s with one split instead of 17.
static int64_t block_attn_cus() {
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

int64_t block_attn_launch_splits(int64_t B, int64_t T, int Hkv, int64_t cap) {
  const int64_t QB = (T + BA_TQ - 1) / BA_TQ;
  const int64_t blocks = (int64_t)Hkv * B * QB;
  int64_t use = block_attn_cus() / (blocks > 0 ? blocks : 1);
  const int64_t most = block_attn_splits(cap);
  if (use > most) use = most;
  if (use < 1) use = 1;
  int64_t chunk = (cap + use - 1) / use;
  chunk = (chunk + 31) / 32 * 32;
  return (cap + chunk - 1) / chunk;                     // no empty trailing split
}

int64_t block_attn_partial_rows(int64_t B, int64_t T, int Hq, int Hkv, int64_t cap) {
  // the split count is constant over the T of one query-block count and the rows grow with T,
  // so the largest need of each query-block count sits at its largest T
  int64_t most = 0;
  const int64_t QB = (T + BA_TQ - 1) / BA_TQ;
  for (int64_t qb = 1; qb <= QB; ++qb) {
    const int64_t t = qb * BA_TQ < T ? qb * BA_TQ : T;
    const int64_t use = block_attn_launch_splits(B, t, Hkv, cap);
    const int64_t rows = use > 1 ? B * t * Hq * use : 0;
    if (rows > most) most = rows;
  }
  return most;
}

void launch_block_attn(const bf16_t* q, const bf16_t* k_cache, const bf16_t* v_cache,
                       const int64_t* base, const uint64_t* anc, int64_t B, int64_t T, int Hq,
                       int Hkv, int64_t cap, float* ws_acc, float* ws_ml, bf16_t* out,
                       hipStream_t s) {
  if (B * T <= 0) return;
  const int64_t QB = (T + BA_TQ - 1) / BA_TQ;
  const int64_t use = block_attn_launch_splits(B, T, Hkv, cap);
  const int64_t chunk = ((cap + use - 1) / use + 31) / 32 * 32;
  block_attn_mfma_kernel<<<dim3((unsigned)use, (unsigned)Hkv, (unsigned)(B * QB)), dim3(512), 0,
                           s>>>(q, k_cache, v_cache, base, anc, T, Hq, Hkv, cap, chunk,
                                (1.0f / sqrtf(128.0f)) * 1.44269504088896341f, ws_acc, ws_ml,
                                out);
  if (use > 1)      // one split writes its rows itself
    attn_merge_kernel<<<dim3((unsigned)(B * T * Hq)), dim3(64), 0, s>>>(ws_acc, ws_ml, (int)use,
                                                                        out);
}
