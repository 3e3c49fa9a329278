// Decode-attention building blocks shared by the per-launch kernels (attn.hip) and the
// persistent step kernel (mega.hip): both run exactly this arithmetic, so their results agree
// bit for bit.  Numerics (decode_attn.py:7-11): fp32 scores q.k * 128^-1/2, fp32 online
// softmax, P rounded to bf16 before P.V, fp32 accumulate, split merge by log-sum-exp, / l in
// fp32, bf16 out.
//
// Work mapping: a wave is 4 groups of 16 lanes; a group handles KPG consecutive keys per
// iteration and lane i of the group owns dims [8i, 8i+8) -- one 16-byte load per key row for K
// and for V, so a group reads a 256-byte K row and a 256-byte V row contiguously.
#pragma once
#include "qd_common.h"

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

// merge the state of lane ^ off (off = 16 or 32) into this lane's (all lanes active)
__device__ __forceinline__ void state_merge_xor(SoftmaxState& st, int off) {
#pragma unroll
  for (int h = 0; h < GRP; ++h) {
    const float m2 = off == 16 ? lane_xor16(st.m[h]) : lane_xor32(st.m[h]);
    const float l2 = off == 16 ? lane_xor16(st.l[h]) : lane_xor32(st.l[h]);
    const float mn = fmaxf(st.m[h], m2);
    const float a1 = __expf(st.m[h] - mn);
    const float a2 = __expf(m2 - mn);
    st.l[h] = st.l[h] * a1 + l2 * a2;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float o = off == 16 ? lane_xor16(st.acc[h][e]) : lane_xor32(st.acc[h][e]);
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
  const float r = rstd_of(wave_sum(sq_pair(x1, x2)), 128, eps);
  const float y1 = norm_elem(x1, r, bf2f(wn[lane])), y2 = norm_elem(x2, r, bf2f(wn[lane + 64]));
  const float c1 = bf2f(cos_row[lane]), c2 = bf2f(cos_row[lane + 64]);
  const float s1 = bf2f(sin_row[lane]), s2 = bf2f(sin_row[lane + 64]);
  o1 = rbf(rbf(y1 * c1) + rbf(-y2 * s1));
  o2 = rbf(rbf(y2 * c2) + rbf(y1 * s2));
}
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
  const float r = rstd_of(wave_sum(sq_pair(x1, x2)), 128, eps);
  const float y1 = norm_elem(x1, r, w1), y2 = norm_elem(x2, r, w2);
  o1 = rbf(rbf(y1 * c1) + rbf(-y2 * s1));
  o2 = rbf(rbf(y2 * c2) + rbf(y1 * s2));
}

// One wave's inputs to a decode-attention unit (lane holds dims lane and lane + 64): the raw
// bf16 values of q head kvh * GRP + (wave % GRP) and of the new token's k (v for wave vw), the
// q_norm / k_norm weights and the RoPE values.  Every wave of a unit loads a full set from valid
// addresses in straight-line code (no wave-divergent branch around a load) and uses what its
// role needs.
struct HeadVals {
  uint32_t q1 = 0, q2 = 0, k1 = 0, k2 = 0;   // raw bf16 bits (k1/k2 hold v on wave vw)
  float qw1 = 0.f, qw2 = 0.f, kw1 = 0.f, kw2 = 0.f;
  float c1 = 0.f, c2 = 0.f, s1 = 0.f, s2 = 0.f;
};

template <int NW>
struct DecodeAttnLds {
  uint32_t qs[GRP][64];        // packed bf16 pairs (d, d+1)
  uint32_t kns[64];
  float vnew[128];
  float wm[NW][GRP], wl[NW][GRP];
  float wacc[NW][GRP][128];
};

template <int NW>
__device__ __forceinline__ constexpr int attn_k_wave() { return NW > GRP ? GRP : 0; }
template <int NW>
__device__ __forceinline__ constexpr int attn_v_wave() { return NW > GRP + 1 ? GRP + 1 : 1; }

// Element offsets, within a packed qkv row ([Hq | Hkv | Hkv] heads of 128), of the q head and
// of the k (or, for wave vw, v) head that `wave` reads for KV head kvh.  Pure arithmetic.
__device__ __forceinline__ int64_t attn_q_elem(int wave, int kvh) {
  return (int64_t)(kvh * GRP + (wave & (GRP - 1))) * 128;
}
template <int NW>
__device__ __forceinline__ int64_t attn_kv_elem(int wave, int kvh, int Hq, int Hkv) {
  return (int64_t)(Hq + (wave == attn_v_wave<NW>() ? Hkv : 0) + kvh) * 128;
}

// One (sequence, KV head, key split) unit over keys [start, start + chunk) of one layer's cache
// (head_off = element offset of this sequence's KV head).  Order of work: the first key tile is
// loaded, then fetch(hv) loads this wave's head values and returns pos (so a caller can issue
// every load before pos is known); a pos outside [0, cap) ends the unit.  The split owning pos
// normalises + ropes the new K, writes K/V slot pos and attends the new key from LDS.  Result:
// final(h, d, y0, y1) with the normalised output dims d, d+1 of head h when `whole` (the unit
// covers every key), else partial(h, d, A0, A1, M, L) with the unnormalised accumulators and
// the (max, sum) pair.  The last step runs on waves 0..3 only (threads 0..255, one head each).
// In a workgroup of more than NW waves, the waves past NW do no work but run the unit's
// barriers (fetch must return pos for them too).
template <int NW, class Fetch, class Final, class Partial>
__device__ __forceinline__ void decode_attn_unit(DecodeAttnLds<NW>& sm, const Fetch& fetch,
                                                 const Final& final_out,
                                                 const Partial& partial_out, bf16_t* k_cache,
                                                 bf16_t* v_cache, int64_t head_off, int64_t cap,
                                                 int64_t start, int64_t chunk, bool whole,
                                                 float eps, float scale) {
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, i = lane & 15;
  const bool act = wave < NW;             // waves past NW only take part in the barriers
  const uint4* kb = reinterpret_cast<const uint4*>(k_cache + head_off);
  const uint4* vb = reinterpret_cast<const uint4*>(v_cache + head_off);
  constexpr int TILE = NW * GRP * KPG;    // keys per workgroup iteration
  constexpr int kw = attn_k_wave<NW>(), vw = attn_v_wave<NW>();
  uint4 kx[KPG], vx[KPG];
  int64_t j0 = start + (int64_t)wave * GRP * KPG;
  if (act) {
#pragma unroll
    for (int kk = 0; kk < KPG; ++kk) {
      const int64_t j = j0 + g * KPG + kk;
      const int64_t jj = j < cap ? j : cap - 1;
      kx[kk] = kb[jj * 16 + i];
      vx[kk] = vb[jj * 16 + i];
    }
  }
  HeadVals hv;
  const int64_t pos = fetch(hv);          // every wave: fetch loads nothing for waves past NW
  if (pos < 0 || pos >= cap) return;  // uniform over the unit: no slot to write
  const int64_t kend = min(start + chunk, pos);  // cached keys only; `pos` is the new token
  bool ok[KPG];
#pragma unroll
  for (int kk = 0; kk < KPG; ++kk) ok[kk] = j0 + g * KPG + kk < kend;
  if (wave < GRP) {
    float o1, o2;
    norm_rope_vals(bf2f(hv.q1), bf2f(hv.q2), hv.qw1, hv.qw2, hv.c1, hv.c2, hv.s1, hv.s2, eps, o1,
                   o2);
    // lane l holds dims l and l + 64; repack as bf16 pairs through LDS
    reinterpret_cast<bf16_t*>(sm.qs[wave])[lane] = (bf16_t)f2bf(o1);
    reinterpret_cast<bf16_t*>(sm.qs[wave])[lane + 64] = (bf16_t)f2bf(o2);
  }
  const bool owns = pos >= start && pos < start + chunk;
  if (owns && wave == kw) {
    float o1, o2;
    norm_rope_vals(bf2f(hv.k1), bf2f(hv.k2), hv.kw1, hv.kw2, hv.c1, hv.c2, hv.s1, hv.s2, eps, o1,
                   o2);
    const bf16_t k1 = (bf16_t)f2bf(o1), k2 = (bf16_t)f2bf(o2);
    k_cache[head_off + pos * 128 + lane] = k1;
    k_cache[head_off + pos * 128 + lane + 64] = k2;
    reinterpret_cast<bf16_t*>(sm.kns)[lane] = k1;
    reinterpret_cast<bf16_t*>(sm.kns)[lane + 64] = k2;
  }
  if (owns && wave == vw) {
    v_cache[head_off + pos * 128 + lane] = (bf16_t)hv.k1;
    v_cache[head_off + pos * 128 + lane + 64] = (bf16_t)hv.k2;
    sm.vnew[lane] = bf2f(hv.k1);
    sm.vnew[lane + 64] = bf2f(hv.k2);
  }
  lds_barrier();
  if (act) {
  uint4 qp[GRP];
#pragma unroll
  for (int h = 0; h < GRP; ++h) qp[h] = reinterpret_cast<const uint4*>(sm.qs[h])[i];
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
      kk4[kk] = reinterpret_cast<const uint4*>(sm.kns)[i];
#pragma unroll
      for (int e = 0; e < 8; ++e) vf[kk][e] = sm.vnew[8 * i + e];
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
      for (int e = 0; e < 8; ++e) sm.wacc[wave][h][8 * i + e] = st.acc[h][e];
  }
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < GRP; ++h) { sm.wm[wave][h] = st.m[h]; sm.wl[wave][h] = st.l[h]; }
  }
  }  // act
  lds_barrier();
  if (tid >= 256) return;                 // 4 waves combine: one per head, 2 dims per lane
  const int h = tid >> 6, d = (tid & 63) * 2;
  float M = sm.wm[0][h];
  for (int w = 1; w < NW; ++w) M = fmaxf(M, sm.wm[w][h]);
  float L = 0.f, A0 = 0.f, A1 = 0.f;
  for (int w = 0; w < NW; ++w) {
    const float a = __expf(sm.wm[w][h] - M);
    L += a * sm.wl[w][h];
    A0 += a * sm.wacc[w][h][d];
    A1 += a * sm.wacc[w][h][d + 1];
  }
  if (whole) {                            // the whole key range is here: normalise
    const float inv = 1.0f / L;
    final_out(h, d, A0 * inv, A1 * inv);
  } else {
    partial_out(h, d, A0, A1, M, L);
  }
}

// Log-sum-exp merge of one head's split partials by one wave (lane owns dims 2 lane, 2 lane + 1).
// ml(sp) returns split sp's (m, l); acc_batch(first, n, a) fills a[q] (q < n) with split
// first + q's (acc[2 lane], acc[2 lane + 1]), issuing every load of the batch before using any.
// Returns the normalised pair.
constexpr int MERGE_BATCH = 16;   // partial rows loaded per pass (all in flight together)

template <class Ml, class AccBatch>
__device__ __forceinline__ float2 merge_splits(int splits, const Ml& ml, const AccBatch& acc_batch) {
  const int lane = threadIdx.x & 63;
  float n0 = 0.f, n1 = 0.f, den = 0.f, M = M_FLOOR;
  for (int base = 0; base < splits; base += 64) {
    // this pass: up to 64 splits' (m, l), one per lane, and their acc rows in batches
    const int sp = base + lane;
    const float2 v = sp < splits ? ml(sp) : make_float2(M_FLOOR, 0.f);
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
      acc_batch(base + s0, cnt - s0 < MERGE_BATCH ? cnt - s0 : MERGE_BATCH, a);
#pragma unroll
      for (int q = 0; q < MERGE_BATCH; ++q) {
        const float wq = __builtin_bit_cast(
            float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), (s0 + q) & 63));
        if (s0 + q < cnt) { n0 = fmaf(wq, a[q].x, n0); n1 = fmaf(wq, a[q].y, n1); }
      }
    }
  }
  const float inv = 1.0f / den;
  return make_float2(n0 * inv, n1 * inv);
}
