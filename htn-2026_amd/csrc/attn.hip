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

namespace {
constexpr int GRP = 4;   // query heads per KV head
constexpr int KPG = 4;   // keys per group per iteration
constexpr float NEG_INF = -INFINITY;
// Running maxima start at a finite floor: an invisible key scores -inf, so exp(s - m) is exactly
// 0 without a branch, and exp(m_old - m_new) is 0 for an empty state -- no inf - inf anywhere.
constexpr float M_FLOOR = -1e30f;

struct SoftmaxState {
  float m[GRP], l[GRP], acc[GRP][8];
};

__device__ __forceinline__ void state_init(SoftmaxState& st) {
#pragma unroll
  for (int h = 0; h < GRP; ++h) {
    st.m[h] = M_FLOOR;
    st.l[h] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) st.acc[h][e] = 0.f;
  }
}

// s[kk][h] are scores (NEG_INF when invisible); v[kk] are the lane's 8 dims of each V row.
__device__ __forceinline__ void state_update(SoftmaxState& st, const float (&s)[KPG][GRP],
                                             const float (&v)[KPG][8]) {
#pragma unroll
  for (int h = 0; h < GRP; ++h) {
    float mx = s[0][h];
#pragma unroll
    for (int kk = 1; kk < KPG; ++kk) mx = fmaxf(mx, s[kk][h]);
    const float mn = fmaxf(st.m[h], mx);
    const float alpha = __expf(st.m[h] - mn);
    float psum = 0.f, pv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) pv[e] = 0.f;
#pragma unroll
    for (int kk = 0; kk < KPG; ++kk) {
      const float p = __expf(s[kk][h] - mn);
      psum += p;
      const float pb = rbf(p);
#pragma unroll
      for (int e = 0; e < 8; ++e) pv[e] = fmaf(pb, v[kk][e], pv[e]);
    }
    st.l[h] = st.l[h] * alpha + psum;
#pragma unroll
    for (int e = 0; e < 8; ++e) st.acc[h][e] = fmaf(st.acc[h][e], alpha, pv[e]);
    st.m[h] = mn;
  }
}

// merge the state of lane ^ off into this lane's (all lanes active)
__device__ __forceinline__ void state_merge_xor(SoftmaxState& st, int off) {
#pragma unroll
  for (int h = 0; h < GRP; ++h) {
    const float m2 = __shfl_xor(st.m[h], off, 64);
    const float l2 = __shfl_xor(st.l[h], off, 64);
    const float mn = fmaxf(st.m[h], m2);
    const float a1 = __expf(st.m[h] - mn);
    const float a2 = __expf(m2 - mn);
    st.l[h] = st.l[h] * a1 + l2 * a2;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float o = __shfl_xor(st.acc[h][e], off, 64);
      st.acc[h][e] = st.acc[h][e] * a1 + o * a2;
    }
    st.m[h] = mn;
  }
}

__device__ __forceinline__ void unpack8(uint4 u, float* f) {
  f[0] = bflo(u.x); f[1] = bfhi(u.x); f[2] = bflo(u.y); f[3] = bfhi(u.y);
  f[4] = bflo(u.z); f[5] = bfhi(u.z); f[6] = bflo(u.w); f[7] = bfhi(u.w);
}

// scores of KPG keys for the GRP heads: each 16-lane group reduces its partial dots
__device__ __forceinline__ void group_scores(const float (&qv)[GRP][8], const float (&k)[KPG][8],
                                             const bool (&ok)[KPG], float scale,
                                             float (&s)[KPG][GRP]) {
#pragma unroll
  for (int kk = 0; kk < KPG; ++kk)
#pragma unroll
    for (int h = 0; h < GRP; ++h) {
      float d = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) d = fmaf(qv[h][e], k[kk][e], d);
      d = row16_sum(d) * scale;
      s[kk][h] = ok[kk] ? d : NEG_INF;
    }
}

// RMSNorm (128) + RoPE of one head held as lane dims (lane, lane + 64); returns rounded floats
__device__ __forceinline__ void norm_rope_head(const bf16_t* src, const bf16_t* wn,
                                               const bf16_t* cos_row, const bf16_t* sin_row,
                                               float eps, float& o1, float& o2) {
  const int lane = threadIdx.x & 63;
  const float x1 = bf2f(src[lane]), x2 = bf2f(src[lane + 64]);
  const float r = rstd_of(wave_sum(x1 * x1 + x2 * x2), 128, eps);
  const float y1 = norm_elem(x1, r, bf2f(wn[lane])), y2 = norm_elem(x2, r, bf2f(wn[lane + 64]));
  const float c1 = bf2f(cos_row[lane]), c2 = bf2f(cos_row[lane + 64]);
  const float s1 = bf2f(sin_row[lane]), s2 = bf2f(sin_row[lane + 64]);
  o1 = rbf(rbf(y1 * c1) + rbf(-y2 * s1));
  o2 = rbf(rbf(y2 * c2) + rbf(y1 * s2));
}
}  // namespace

// ------------------------------------------------------------------ decode
// q held as packed bf16 (it is bf16-rounded after RoPE, so the packing is exact): scores use
// v_dot2_f32_bf16 directly on the raw K rows.
__device__ __forceinline__ void group_scores_packed(const uint4 (&qp)[GRP], const uint4 (&kx)[KPG],
                                                    const bool (&ok)[KPG], float scale,
                                                    float (&s)[KPG][GRP]) {
#pragma unroll
  for (int kk = 0; kk < KPG; ++kk)
#pragma unroll
    for (int h = 0; h < GRP; ++h) {
      const float d = row16_sum(dot8(qp[h], kx[kk], 0.f)) * scale;
      s[kk][h] = ok[kk] ? d : NEG_INF;
    }
}

// RMSNorm (128) + RoPE of one head from values already in registers (lane dims l, l + 64)
__device__ __forceinline__ void norm_rope_vals(float x1, float x2, float w1, float w2, float c1,
                                               float c2, float s1, float s2, float eps, float& o1,
                                               float& o2) {
  const float r = rstd_of(wave_sum(x1 * x1 + x2 * x2), 128, eps);
  const float y1 = norm_elem(x1, r, w1), y2 = norm_elem(x2, r, w2);
  o1 = rbf(rbf(y1 * c1) + rbf(-y2 * s1));
  o2 = rbf(rbf(y2 * c2) + rbf(y1 * s2));
}

// ROPE_ROW: cos_t / sin_t point at this step's RoPE row (written by the embedding kernel), so
// no prologue load waits for pos; otherwise they are [cap, 128] tables indexed by pos.
template <int NW, bool ROPE_ROW>
__global__ __launch_bounds__(NW * 64) void decode_attn_kernel(
    const bf16_t* __restrict__ qkv, int64_t qkv_stride, const bf16_t* __restrict__ qn,
    const bf16_t* __restrict__ kn, const bf16_t* __restrict__ cos_t,
    const bf16_t* __restrict__ sin_t, const int64_t* __restrict__ pos_ptr, bf16_t* k_cache,
    bf16_t* v_cache, int Hq, int Hkv, int64_t cap, int64_t chunk, float eps, float scale,
    float* ws_acc, float* ws_ml, bf16_t* out) {
  __shared__ uint32_t qs[GRP][64];        // packed bf16 pairs (d, d+1)
  __shared__ uint32_t kns[64];
  __shared__ float vnew[128];
  __shared__ float wm[NW][GRP], wl[NW][GRP];
  __shared__ float wacc[NW][GRP][128];
  const int split = blockIdx.x, kvh = blockIdx.y;
  const int64_t b = blockIdx.z;
  const int splits = gridDim.x;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, i = lane & 15;
  const int64_t start = (int64_t)split * chunk;
  const int64_t head_off = ((b * Hkv + kvh) * cap) * 128;
  const uint4* kb = reinterpret_cast<const uint4*>(k_cache + head_off);
  const uint4* vb = reinterpret_cast<const uint4*>(v_cache + head_off);
  // ---- every prologue load is issued before pos is known: the first key tile (addresses
  // clamped into the cache; validity applied later), this wave's q / k / v head values, the
  // norm weights and (ROPE_ROW) the RoPE row
  constexpr int TILE = NW * GRP * KPG;    // keys per workgroup iteration
  uint4 kx[KPG], vx[KPG];
  int64_t j0 = start + (int64_t)wave * GRP * KPG;
#pragma unroll
  for (int kk = 0; kk < KPG; ++kk) {
    const int64_t j = j0 + g * KPG + kk;
    const int64_t jj = j < cap ? j : cap - 1;
    kx[kk] = kb[jj * 16 + i];
    vx[kk] = vb[jj * 16 + i];
  }
  const bf16_t* row = qkv + b * qkv_stride;
  const int kw = NW > GRP ? GRP : 0, vw = NW > GRP + 1 ? GRP + 1 : 1;  // waves doing the new K / V
  float qx1 = 0.f, qx2 = 0.f, qw1 = 0.f, qw2 = 0.f, kx1 = 0.f, kx2 = 0.f, kw1 = 0.f, kw2 = 0.f;
  bf16_t v1 = 0, v2 = 0;
  if (wave < GRP) {
    const bf16_t* src = row + (int64_t)(kvh * GRP + wave) * 128;
    qx1 = bf2f(src[lane]); qx2 = bf2f(src[lane + 64]);
    qw1 = bf2f(qn[lane]); qw2 = bf2f(qn[lane + 64]);
  }
  if (wave == kw) {
    const bf16_t* src = row + (int64_t)(Hq + kvh) * 128;
    kx1 = bf2f(src[lane]); kx2 = bf2f(src[lane + 64]);
    kw1 = bf2f(kn[lane]); kw2 = bf2f(kn[lane + 64]);
  }
  if (wave == vw) {
    const bf16_t* src = row + (int64_t)(Hq + Hkv + kvh) * 128;
    v1 = src[lane]; v2 = src[lane + 64];
  }
  float c1 = 0.f, c2 = 0.f, s1 = 0.f, s2 = 0.f;
  if constexpr (ROPE_ROW) {
    c1 = bf2f(cos_t[lane]); c2 = bf2f(cos_t[lane + 64]);
    s1 = bf2f(sin_t[lane]); s2 = bf2f(sin_t[lane + 64]);
  }
  const int64_t pos = pos_ptr[0];
  if (pos < 0 || pos >= cap) return;  // uniform over the grid: no slot to write
  if constexpr (!ROPE_ROW) {
    c1 = bf2f(cos_t[pos * 128 + lane]); c2 = bf2f(cos_t[pos * 128 + lane + 64]);
    s1 = bf2f(sin_t[pos * 128 + lane]); s2 = bf2f(sin_t[pos * 128 + lane + 64]);
  }
  const int64_t kend = min(start + chunk, pos);  // cached keys only; `pos` is the new token
  bool ok[KPG];
#pragma unroll
  for (int kk = 0; kk < KPG; ++kk) ok[kk] = j0 + g * KPG + kk < kend;
  if (wave < GRP) {
    float o1, o2;
    norm_rope_vals(qx1, qx2, qw1, qw2, c1, c2, s1, s2, eps, o1, o2);
    // lane l holds dims l and l + 64; repack as bf16 pairs through LDS
    reinterpret_cast<bf16_t*>(qs[wave])[lane] = (bf16_t)f2bf(o1);
    reinterpret_cast<bf16_t*>(qs[wave])[lane + 64] = (bf16_t)f2bf(o2);
  }
  const bool owns = pos >= start && pos < start + chunk;
  if (owns && wave == kw) {
    float o1, o2;
    norm_rope_vals(kx1, kx2, kw1, kw2, c1, c2, s1, s2, eps, o1, o2);
    const bf16_t k1 = (bf16_t)f2bf(o1), k2 = (bf16_t)f2bf(o2);
    k_cache[head_off + pos * 128 + lane] = k1;
    k_cache[head_off + pos * 128 + lane + 64] = k2;
    reinterpret_cast<bf16_t*>(kns)[lane] = k1;
    reinterpret_cast<bf16_t*>(kns)[lane + 64] = k2;
  }
  if (owns && wave == vw) {
    v_cache[head_off + pos * 128 + lane] = v1;
    v_cache[head_off + pos * 128 + lane + 64] = v2;
    vnew[lane] = bf2f(v1);
    vnew[lane + 64] = bf2f(v2);
  }
  lds_barrier();
  uint4 qp[GRP];
#pragma unroll
  for (int h = 0; h < GRP; ++h) qp[h] = reinterpret_cast<const uint4*>(qs[h])[i];
  SoftmaxState st;
  state_init(st);
  while (j0 < kend) {
    const int64_t jn = j0 + TILE;
    uint4 kn_[KPG], vn_[KPG];
    if (jn < kend) {                        // prefetch the next tile (wave-uniform branch)
#pragma unroll
      for (int kk = 0; kk < KPG; ++kk) {
        const int64_t j = jn + g * KPG + kk;
        const int64_t jj = j < cap ? j : cap - 1;
        kn_[kk] = kb[jj * 16 + i];
        vn_[kk] = vb[jj * 16 + i];
      }
    }
    float s[KPG][GRP], vf[KPG][8];
    group_scores_packed(qp, kx, ok, scale, s);
#pragma unroll
    for (int kk = 0; kk < KPG; ++kk) unpack8(vx[kk], vf[kk]);
    state_update(st, s, vf);
    j0 = jn;
    if (j0 < kend) {
#pragma unroll
      for (int kk = 0; kk < KPG; ++kk) {
        kx[kk] = kn_[kk];
        vx[kk] = vn_[kk];
        ok[kk] = j0 + g * KPG + kk < kend;
      }
    }
  }
  if (owns && wave == 0 && g == 0) {  // the new key, attended from LDS (lanes 0..15)
    float s[KPG][GRP], vf[KPG][8];
    uint4 kk4[KPG];
    bool ok1[KPG];
#pragma unroll
    for (int kk = 0; kk < KPG; ++kk) {
      ok1[kk] = kk == 0;
      kk4[kk] = reinterpret_cast<const uint4*>(kns)[i];
#pragma unroll
      for (int e = 0; e < 8; ++e) vf[kk][e] = vnew[8 * i + e];
    }
    group_scores_packed(qp, kk4, ok1, scale, s);
    state_update(st, s, vf);
  }
  state_merge_xor(st, 16);
  state_merge_xor(st, 32);
  if (lane < 16) {
#pragma unroll
    for (int h = 0; h < GRP; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) wacc[wave][h][8 * i + e] = st.acc[h][e];
  }
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < GRP; ++h) { wm[wave][h] = st.m[h]; wl[wave][h] = st.l[h]; }
  }
  lds_barrier();
  if (tid >= 256) return;                 // 4 waves combine: one per head, 2 dims per lane
  const int h = tid >> 6, d = (tid & 63) * 2;
  float M = wm[0][h];
  for (int w = 1; w < NW; ++w) M = fmaxf(M, wm[w][h]);
  float L = 0.f, A0 = 0.f, A1 = 0.f;
  for (int w = 0; w < NW; ++w) {
    const float a = __expf(wm[w][h] - M);
    L += a * wl[w][h];
    A0 += a * wacc[w][h][d];
    A1 += a * wacc[w][h][d + 1];
  }
  if (splits == 1) {                      // the whole key range is here: write the output
    const float inv = 1.0f / L;
    *reinterpret_cast<uint32_t*>(out + (b * Hq + kvh * GRP + h) * 128 + d) = pack2(A0 * inv, A1 * inv);
    return;
  }
  const int64_t idx = ((b * Hq + kvh * GRP + h) * splits + split);
  *reinterpret_cast<float2*>(ws_acc + idx * 128 + d) = make_float2(A0, A1);
  if ((tid & 63) == 0) *reinterpret_cast<float2*>(ws_ml + idx * 2) = make_float2(M, L);
}

// One wave per (token row, head): log-sum-exp merge of the split partials -> bf16 out
// [rows, Hq*128] (decode_attn.py:74-86, tree.py:130-142).  A separate launch: the kernel
// boundary is the only cross-workgroup synchronisation, so no workgroup fences or waits.
// Lanes read the splits' (m, l) in parallel; each lane then owns 2 of the 128 dims.
constexpr int MERGE_MAX_SPLITS = 1024;
constexpr int MERGE_BATCH = 16;   // partial rows loaded per pass (all in flight together)

__global__ __launch_bounds__(64) void attn_merge_kernel(const float* __restrict__ ws_acc,
                                                         const float* __restrict__ ws_ml,
                                                         int splits, bf16_t* __restrict__ out) {
  const int64_t r = blockIdx.x;  // (b*T + t)*Hq + h
  const int lane = threadIdx.x;
  const float2* ml = reinterpret_cast<const float2*>(ws_ml) + r * splits;
  const float2* acc = reinterpret_cast<const float2*>(ws_acc + r * splits * 128) + lane;
  float n0 = 0.f, n1 = 0.f, den = 0.f, M = M_FLOOR;
  for (int base = 0; base < splits; base += 64) {
    // this pass: up to 64 splits' (m, l), one per lane, and their acc rows in batches
    const int sp = base + lane;
    const float2 v = sp < splits ? ml[sp] : make_float2(M_FLOOR, 0.f);
    const float Mp = wave_max(v.x);
    const float Mn = fmaxf(M, Mp);
    const float scale_old = __expf(M - Mn);
    n0 *= scale_old; n1 *= scale_old; den *= scale_old;
    M = Mn;
    const float w = __expf(v.x - M);
    den += wave_sum(w * v.y);
    const int cnt = splits - base < 64 ? splits - base : 64;
    for (int s0 = 0; s0 < cnt; s0 += MERGE_BATCH) {
      float2 a[MERGE_BATCH];
#pragma unroll
      for (int q = 0; q < MERGE_BATCH; ++q)
        a[q] = s0 + q < cnt ? acc[(int64_t)(base + s0 + q) * 64] : make_float2(0.f, 0.f);
#pragma unroll
      for (int q = 0; q < MERGE_BATCH; ++q) {
        const float wq = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), (s0 + q) & 63));
        if (s0 + q < cnt) { n0 = fmaf(wq, a[q].x, n0); n1 = fmaf(wq, a[q].y, n1); }
      }
    }
  }
  const float inv = 1.0f / den;
  *reinterpret_cast<uint32_t*>(out + r * 128 + lane * 2) = pack2(n0 * inv, n1 * inv);
}

// Split policy: 16 waves per workgroup take 256 keys per iteration.  One split (no merge launch)
// while a split has at most ATTN_SPLIT_KEYS keys and the batch alone fills half the CUs;
// otherwise enough splits of at most ATTN_SPLIT_KEYS keys for ~2 workgroups per CU.
#ifndef QD_ATTN_NW
#define QD_ATTN_NW 8
#endif
constexpr int ATTN_NW = QD_ATTN_NW;
constexpr int64_t ATTN_TILE = ATTN_NW * 16;
constexpr int64_t ATTN_SPLIT_KEYS = 1024;

int64_t decode_attn_splits(int64_t B, int Hkv, int64_t cap) {
  const int64_t pairs = B * Hkv;
  int64_t sp = (cap + ATTN_SPLIT_KEYS - 1) / ATTN_SPLIT_KEYS;     // bound the keys per split
  const int64_t fill = (512 + pairs - 1) / pairs;                  // ~2 workgroups per CU
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

void launch_decode_attn(const bf16_t* qkv, int64_t qkv_stride, const bf16_t* qn, const bf16_t* kn,
                        const bf16_t* cos_t, const bf16_t* sin_t, const int64_t* pos,
                        bf16_t* k_cache, bf16_t* v_cache, int64_t B, int Hq, int Hkv, int64_t cap,
                        int64_t splits, float eps, float* ws_acc, float* ws_ml, bf16_t* out,
                        bool rope_row, hipStream_t s) {
  const int64_t chunk = decode_attn_chunk(cap, splits);
  const dim3 grid((unsigned)splits, (unsigned)Hkv, (unsigned)B), block(ATTN_NW * 64);
  if (rope_row)
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

__global__ __launch_bounds__(256) void block_attn_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k_cache,
    const bf16_t* __restrict__ v_cache, const int64_t* __restrict__ base_ptr,
    const uint64_t* __restrict__ anc, int64_t T, int Hq, int Hkv, int64_t cap, float scale,
    float* ws_acc, float* ws_ml) {
  const int split = blockIdx.x, kvh = blockIdx.y;
  const int splits = gridDim.x;
  const int64_t TQ = (T + 3) / 4;
  const int64_t b = blockIdx.z / TQ;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t t = (blockIdx.z % TQ) * 4 + wave;
  if (t >= T) return;  // no barrier below: waves are independent
  const int g = lane >> 4, i = lane & 15;
  const int64_t base = base_ptr[b];
  const uint64_t mask = anc ? anc[b * T + t] : 0;
  float qv[GRP][8];
  const uint4* qr = reinterpret_cast<const uint4*>(q + ((b * T + t) * Hq + kvh * GRP) * 128);
#pragma unroll
  for (int h = 0; h < GRP; ++h) unpack8(qr[h * 16 + i], qv[h]);
  SoftmaxState st;
  state_init(st);
  const int64_t start = (int64_t)split * BLOCK_CHUNK;
  int64_t kend = start + BLOCK_CHUNK;
  if (kend > base + T) kend = base + T;
  if (kend > cap) kend = cap;
  const int64_t head_off = ((b * Hkv + kvh) * cap) * 128;
  const uint4* kb = reinterpret_cast<const uint4*>(k_cache + head_off);
  const uint4* vb = reinterpret_cast<const uint4*>(v_cache + head_off);
  for (int64_t j0 = start; j0 < kend; j0 += GRP * KPG) {
    float kf[KPG][8], vf[KPG][8], s[KPG][GRP];
    bool ok[KPG];
#pragma unroll
    for (int kk = 0; kk < KPG; ++kk) {
      const int64_t j = j0 + g * KPG + kk;
      bool vis = j < kend;
      if (vis && j >= base) {
        const int64_t jb = j - base;
        vis = anc ? ((mask >> jb) & 1ull) != 0 : jb <= t;
      }
      ok[kk] = vis;
      const int64_t jj = j < kend ? j : start;
      unpack8(kb[jj * 16 + i], kf[kk]);
      unpack8(vb[jj * 16 + i], vf[kk]);
    }
    group_scores(qv, kf, ok, scale, s);
    state_update(st, s, vf);
  }
  state_merge_xor(st, 16);
  state_merge_xor(st, 32);
  if (lane < 16) {
#pragma unroll
    for (int h = 0; h < GRP; ++h) {
      const int64_t idx = (((b * T + t) * Hq + kvh * GRP + h) * splits + split);
#pragma unroll
      for (int e = 0; e < 8; ++e) ws_acc[idx * 128 + 8 * i + e] = st.acc[h][e];
      if (i == 0) { ws_ml[idx * 2] = st.m[h]; ws_ml[idx * 2 + 1] = st.l[h]; }
    }
  }
}

int64_t block_attn_splits(int64_t cap) { return (cap + BLOCK_CHUNK - 1) / BLOCK_CHUNK; }

void launch_block_attn(const bf16_t* q, const bf16_t* k_cache, const bf16_t* v_cache,
                       const int64_t* base, const uint64_t* anc, int64_t B, int64_t T, int Hq,
                       int Hkv, int64_t cap, int64_t splits, float* ws_acc, float* ws_ml,
                       bf16_t* out, hipStream_t s) {
  if (B * T <= 0) return;
  const int64_t TQ = (T + 3) / 4;
  block_attn_kernel<<<dim3((unsigned)splits, (unsigned)Hkv, (unsigned)(B * TQ)), dim3(256), 0, s>>>(
      q, k_cache, v_cache, base, anc, T, Hq, Hkv, cap, 1.0f / sqrtf(128.0f), ws_acc, ws_ml);
  attn_merge_kernel<<<dim3((unsigned)(B * T * Hq)), dim3(64), 0, s>>>(ws_acc, ws_ml, (int)splits,
                                                                      out);
}
