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
// serves 64 tokens x 4 heads.  Keys go in tiles of 32:
//  * S' = K . Q^T: A = K tile rows (LDS, 16-byte units XOR-swizzled by key), B = the lane's query
//    row (registers); lane (c, q) ends up holding the scores of its query row c against keys
//    4q..4q+3 and 16+4q..16+4q+3 of the tile;
//  * online softmax per query row in fp32 (the row max / sum across the four q lanes through
//    permlane swaps), P rounded to bf16;
//  * O^T += V^T . P^T: A = V^T fragments, B = the lane's 8 probabilities, taken in that same key
//    order (a permutation of the contraction index shared by both operands), so O^T's lane (c, q)
//    holds dims 16 dt + 4q..+3 of row c and the per-row rescale needs no cross-lane traffic.  V is
//    staged key-major like K (one 16-byte store per thread) and read transposed with gfx950's
//    ds_read_b64_tr_b16: within a 16-lane group, lane j = 4a + b receives element b of the
//    8-byte pieces that lanes a, a + 4, a + 8, a + 12 address, so lane i addressing dims
//    16 dt + 4 (i % 4) .. + 3 of key 4q + i / 4 makes lane c receive V[4q + r][16 dt + c],
//    r = 0..3 (measured on MI355X with an in-bounds layout probe);
//  * staging: thread i moves K and V unit i % 16 of key i / 16 of a tile; the next three tiles'
//    loads are in flight (a register ring) while a tile is staged and contracted.
// Writes (m, l, acc) partials per (query row, head, split) -- ws_acc[idx * 128 + d], ws_ml[idx * 2],
// idx = ((b*T + t)*Hq + h)*splits + split -- which attn_merge_kernel merges.
constexpr int BA_TQ = 64;


__global__ __launch_bounds__(512) void block_attn_mfma_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k_cache,
    const bf16_t* __restrict__ v_cache, const int64_t* __restrict__ base_ptr,
    const uint64_t* __restrict__ anc, int64_t T, int Hq, int Hkv, int64_t cap, int64_t chunk,
    float scale, float* ws_acc, float* ws_ml, bf16_t* __restrict__ out) {
  typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
  typedef __attribute__((ext_vector_type(4))) float f32x4_t;
  __shared__ uint4 ks[32 * 16];
  __shared__ uint4 vs[32 * 16];
  const int split = blockIdx.x, kvh = blockIdx.y;
  const int splits = gridDim.x;
  const int64_t QB = (T + BA_TQ - 1) / BA_TQ;
  const int64_t b = blockIdx.z / QB;
  const int64_t tb = (blockIdx.z % QB) * BA_TQ;             // the workgroup's first token
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
  const int ntiles = kend > start ? (int)((kend - start + 31) / 32) : 0;
  const int64_t head_off = ((b * Hkv + kvh) * cap) * 128;
  const uint4* kb = reinterpret_cast<const uint4*>(k_cache + head_off);
  const uint4* vb = reinterpret_cast<const uint4*>(v_cache + head_off);
  float m[2] = {M_FLOOR, M_FLOOR}, lsum[2] = {0.f, 0.f};
  f32x4_t o[2][8];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[rt][dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const int skey = tid >> 4, su = tid & 15;
  // load tile `it` (clamped into the cache: tiles past the range reload valid keys, unused)
#define BA_LD(IT, KX, VX)                                                      \
  {                                                                            \
    const int64_t jn_ = start + 32 * (int64_t)(IT) + skey;                     \
    const int64_t j_ = jn_ < cap ? jn_ : cap - 1;                              \
    KX = kb[j_ * 16 + su];                                                     \
    VX = vb[j_ * 16 + su];                                                     \
  }
  auto stage = [&](const uint4& kx, const uint4& vx) {
    ks[skey * 16 + (su ^ (skey & 15))] = kx;
    vs[skey * 16 + (su ^ (skey & 15))] = vx;
  };
  // this lane's transposed-read address for V dims 16 dt + 4 (c % 4) .. + 3 of key 16 h2 + 4 q4 +
  // c / 4: 16-byte unit 2 dt + (c / 2) % 2, half c % 2
  auto vt_addr = [&](int dt, int h2) -> const void* {
    const int key = 16 * h2 + 4 * q4 + (c >> 2);
    const int u = 2 * dt + ((c >> 1) & 1);
    return reinterpret_cast<const char*>(&vs[key * 16 + (u ^ (key & 15))]) + 8 * (c & 1);
  };
  auto contract = [&](int64_t j0) {
    // S' = K . Q^T for both key halves and both row tiles
    f32x4_t sc[2][2];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) sc[rt][h2] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      const int key = 16 * h2 + c;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const uint4 kf = ks[key * 16 + ((4 * kk + q4) ^ c)];
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
          sc[rt][h2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bf16x8_t, kf), __builtin_bit_cast(bf16x8_t, qf[rt][kk]),
              sc[rt][h2], 0, 0, 0);
      }
    }
    // online softmax of both row tiles; P packed in the key order {4q4..+3, 16+4q4..+3}
    uint4 pf[2];
    float alpha[2];
    // a tile of cached keys only (below base and kend) is visible to every row: no per-score
    // test (the common case: all of the context but the block's own split)
    const bool whole = j0 + 32 <= base && j0 + 32 <= kend;   // uniform over the workgroup
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      float sv[8];
      if (whole) {
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
          for (int r = 0; r < 4; ++r) sv[4 * h2 + r] = sc[rt][h2][r] * scale;
      } else {
        // key j = j0 + 16 h2 + 4 q4 + r, as offsets from the tile start and from base
        const int jrel0 = (int)(j0 - base);                   // may be negative
        const int lim = (int)(kend - j0);                     // keys of the tile below kend
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int o = 16 * h2 + 4 * q4 + r;
            const int jb = jrel0 + o;                         // block index (< 0: cached key)
            bool vis = o < lim;
            if (jb >= 0)
              vis = vis && (anc ? jb < 64 && ((mask[rt] >> (jb & 63)) & 1ull) != 0
                                : (int64_t)jb <= tok[rt]);
            sv[4 * h2 + r] = vis ? sc[rt][h2][r] * scale : NEG_INF;
          }
      }
      float mx = sv[0];
#pragma unroll
      for (int e = 1; e < 8; ++e) mx = fmaxf(mx, sv[e]);
      mx = fmaxf(mx, lane_xor16(mx));
      mx = fmaxf(mx, lane_xor32(mx));
      const float mn = fmaxf(m[rt], mx);
      alpha[rt] = __expf(m[rt] - mn);
      m[rt] = mn;
      float p[8], ps = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) { p[e] = __expf(sv[e] - mn); ps += p[e]; }
      lsum[rt] = lsum[rt] * alpha[rt] + ps;
      pf[rt] = make_uint4(pack2(p[0], p[1]), pack2(p[2], p[3]), pack2(p[4], p[5]), pack2(p[6], p[7]));
    }
    // rescale O only if some row's running max moved (alpha == 1 exactly otherwise, and
    // x * 1 == x: skipping it changes no bit); wave-uniform
    if (__ballot(alpha[0] != 1.f || alpha[1] != 1.f) != 0) {
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) o[rt][dt] *= alpha[rt];
    }
    // O^T += V^T . P^T: V^T fragment of dims 16 dt + c, keys 4q4..+3 and 16+4q4..+3
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const uint2 lo = lds_read_tr16(vt_addr(dt, 0));
      const uint2 hi = lds_read_tr16(vt_addr(dt, 1));
      const uint4 vf = make_uint4(lo.x, lo.y, hi.x, hi.y);
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
        o[rt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            __builtin_bit_cast(bf16x8_t, vf), __builtin_bit_cast(bf16x8_t, pf[rt]), o[rt][dt], 0,
            0, 0);
    }
  };
  // Tile `it` is staged from ring slot it % 3 and the slot is then refilled with tile it + 3.
  // The loop body is three tiles with no exit between them (an exit there lets the compiler
  // sink a refill behind the contraction it should overlap); the last 0..2 tiles follow it.
  uint4 k0, v0, k1, v1, k2, v2;
  BA_LD(0, k0, v0);
  BA_LD(1, k1, v1);
  BA_LD(2, k2, v2);
  int it = 0;
  for (; it + 2 < ntiles; it += 3) {
    lds_barrier();                                     // the previous tile is consumed
    stage(k0, v0);
    lds_barrier();                                     // the tile is staged
    BA_LD(it + 3, k0, v0);
    contract(start + 32 * (int64_t)it);
    lds_barrier();
    stage(k1, v1);
    lds_barrier();
    BA_LD(it + 4, k1, v1);
    contract(start + 32 * (int64_t)(it + 1));
    lds_barrier();
    stage(k2, v2);
    lds_barrier();
    BA_LD(it + 5, k2, v2);
    contract(start + 32 * (int64_t)(it + 2));
  }
  if (it < ntiles) {
    lds_barrier();
    stage(k0, v0);
    lds_barrier();
    contract(start + 32 * (int64_t)it);
  }
  if (it + 1 < ntiles) {
    lds_barrier();
    stage(k1, v1);
    lds_barrier();
    contract(start + 32 * (int64_t)(it + 1));
  }
#undef BA_LD
  // per-row totals: the four q lanes of a row hold disjoint key subsets of l
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    float l = lsum[rt];
    l += lane_xor16(l);
    l += lane_xor32(l);
    if (tok[rt] >= T) continue;
    const int64_t idx = ((b * T + tok[rt]) * Hq + kvh * GRP + head) * splits + split;
    if (splits == 1) {
      // one key split: the row is complete here.  attn_merge_kernel over one split computes
      // acc * (1 / l) (its weight exp(m - m) = 1 and sum l are exact), so this store is
      // bit-identical to the partials + merge it replaces
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
    if (q4 == 0) { ws_ml[idx * 2] = m[rt]; ws_ml[idx * 2 + 1] = l; }
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

void launch_block_attn(const bf16_t* q, const bf16_t* k_cache, const bf16_t* v_cache,
                       const int64_t* base, const uint64_t* anc, int64_t B, int64_t T, int Hq,
                       int Hkv, int64_t cap, int64_t splits, float* ws_acc, float* ws_ml,
                       bf16_t* out, hipStream_t s) {
  if (B * T <= 0) return;
  const int64_t QB = (T + BA_TQ - 1) / BA_TQ;
  const int64_t blocks = (int64_t)Hkv * B * QB;
  int64_t use = block_attn_cus() / blocks;
  if (use > splits) use = splits;
  if (use < 1) use = 1;
  int64_t chunk = (cap + use - 1) / use;
  chunk = (chunk + 31) / 32 * 32;
  use = (cap + chunk - 1) / chunk;                      // no empty trailing split
  block_attn_mfma_kernel<<<dim3((unsigned)use, (unsigned)Hkv, (unsigned)(B * QB)), dim3(512), 0,
                           s>>>(q, k_cache, v_cache, base, anc, T, Hq, Hkv, cap, chunk,
                                1.0f / sqrtf(128.0f), ws_acc, ws_ml, out);
  if (use > 1)      // one split writes its rows itself
    attn_merge_kernel<<<dim3((unsigned)(B * T * Hq)), dim3(64), 0, s>>>(ws_acc, ws_ml, (int)use,
                                                                        out);
}
