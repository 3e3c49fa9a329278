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

struct SoftmaxState {
  float m[GRP], l[GRP], acc[GRP][8];
};

__device__ __forceinline__ void state_init(SoftmaxState& st) {
#pragma unroll
  for (int h = 0; h < GRP; ++h) {
    st.m[h] = NEG_INF;
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
    if (mn == NEG_INF) continue;  // nothing visible yet
    const float alpha = st.m[h] == NEG_INF ? 0.f : expf(st.m[h] - mn);
    float psum = 0.f, pv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) pv[e] = 0.f;
#pragma unroll
    for (int kk = 0; kk < KPG; ++kk) {
      const float p = s[kk][h] == NEG_INF ? 0.f : expf(s[kk][h] - mn);
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
    const float a1 = st.m[h] == NEG_INF ? 0.f : expf(st.m[h] - mn);
    const float a2 = m2 == NEG_INF ? 0.f : expf(m2 - mn);
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
__global__ __launch_bounds__(256) void decode_attn_kernel(
    const bf16_t* __restrict__ qkv, int64_t qkv_stride, const bf16_t* __restrict__ qn,
    const bf16_t* __restrict__ kn, const bf16_t* __restrict__ cos_t,
    const bf16_t* __restrict__ sin_t, const int64_t* __restrict__ pos_ptr, bf16_t* k_cache,
    bf16_t* v_cache, int Hq, int Hkv, int64_t cap, int64_t chunk, float eps, float scale,
    float* ws_acc, float* ws_ml) {
  __shared__ float qs[GRP][128];
  __shared__ float knew[128], vnew[128];
  __shared__ float wm[4][GRP], wl[4][GRP];
  __shared__ float wacc[4][GRP][128];
  const int split = blockIdx.x, kvh = blockIdx.y;
  const int64_t b = blockIdx.z;
  const int splits = gridDim.x;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int64_t pos = pos_ptr[0];
  if (pos < 0 || pos >= cap) return;  // uniform over the grid: no slot to write
  const bf16_t* row = qkv + b * qkv_stride;
  const bf16_t* cos_row = cos_t + pos * 128;
  const bf16_t* sin_row = sin_t + pos * 128;
  {
    float o1, o2;
    norm_rope_head(row + (int64_t)(kvh * GRP + wave) * 128, qn, cos_row, sin_row, eps, o1, o2);
    qs[wave][lane] = o1;
    qs[wave][lane + 64] = o2;
  }
  const int64_t start = (int64_t)split * chunk;
  const bool owns = pos >= start && pos < start + chunk;
  const int64_t head_off = ((b * Hkv + kvh) * cap) * 128;
  if (owns && wave == 0) {
    float o1, o2;
    norm_rope_head(row + (int64_t)(Hq + kvh) * 128, kn, cos_row, sin_row, eps, o1, o2);
    k_cache[head_off + pos * 128 + lane] = (bf16_t)f2bf(o1);
    k_cache[head_off + pos * 128 + lane + 64] = (bf16_t)f2bf(o2);
    knew[lane] = o1;
    knew[lane + 64] = o2;
  }
  if (owns && wave == 1) {
    const bf16_t* src = row + (int64_t)(Hq + Hkv + kvh) * 128;
    const bf16_t v1 = src[lane], v2 = src[lane + 64];
    v_cache[head_off + pos * 128 + lane] = v1;
    v_cache[head_off + pos * 128 + lane + 64] = v2;
    vnew[lane] = bf2f(v1);
    vnew[lane + 64] = bf2f(v2);
  }
  __syncthreads();

  const int g = lane >> 4, i = lane & 15;
  float qv[GRP][8];
#pragma unroll
  for (int h = 0; h < GRP; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) qv[h][e] = qs[h][8 * i + e];
  SoftmaxState st;
  state_init(st);
  const int64_t kend = min(start + chunk, pos);  // cached keys only; `pos` is the new token
  const uint4* kb = reinterpret_cast<const uint4*>(k_cache + head_off);
  const uint4* vb = reinterpret_cast<const uint4*>(v_cache + head_off);
  for (int64_t j0 = start + (int64_t)wave * GRP * KPG; j0 < kend; j0 += 16 * KPG) {
    float kf[KPG][8], vf[KPG][8], s[KPG][GRP];
    bool ok[KPG];
#pragma unroll
    for (int kk = 0; kk < KPG; ++kk) {
      const int64_t j = j0 + g * KPG + kk;
      ok[kk] = j < kend;
      const int64_t jj = ok[kk] ? j : start;
      unpack8(kb[jj * 16 + i], kf[kk]);
      unpack8(vb[jj * 16 + i], vf[kk]);
    }
    group_scores(qv, kf, ok, scale, s);
    state_update(st, s, vf);
  }
  if (owns && wave == 0 && g == 0) {  // the new key, attended from LDS (lanes 0..15)
    float s[KPG][GRP], vf[KPG][8], kf[KPG][8];
    bool ok[KPG];
#pragma unroll
    for (int kk = 0; kk < KPG; ++kk) {
      ok[kk] = kk == 0;
#pragma unroll
      for (int e = 0; e < 8; ++e) { kf[kk][e] = knew[8 * i + e]; vf[kk][e] = vnew[8 * i + e]; }
    }
    group_scores(qv, kf, ok, scale, s);
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
  __syncthreads();
  {
    const int h = tid >> 6, d = (tid & 63) * 2;
    float M = wm[0][h];
    for (int w = 1; w < 4; ++w) M = fmaxf(M, wm[w][h]);
    float L = 0.f, A0 = 0.f, A1 = 0.f;
    for (int w = 0; w < 4; ++w) {
      const float a = wm[w][h] == NEG_INF ? 0.f : expf(wm[w][h] - M);
      L += a * wl[w][h];
      A0 += a * wacc[w][h][d];
      A1 += a * wacc[w][h][d + 1];
    }
    const int64_t idx = ((b * Hq + kvh * GRP + h) * splits + split);
    ws_acc[idx * 128 + d] = A0;
    ws_acc[idx * 128 + d + 1] = A1;
    if ((tid & 63) == 0) { ws_ml[idx * 2] = M; ws_ml[idx * 2 + 1] = L; }
  }
}

// One wave per (token row, head): log-sum-exp merge of the split partials -> bf16 out
// [rows, Hq*128] (decode_attn.py:74-86, tree.py:130-142).  A separate launch: the kernel
// boundary is the only cross-workgroup synchronisation, so no workgroup fences or waits.
__global__ __launch_bounds__(64) void attn_merge_kernel(const float* __restrict__ ws_acc,
                                                         const float* __restrict__ ws_ml,
                                                         int splits, bf16_t* __restrict__ out) {
  const int64_t r = blockIdx.x;  // (b*T + t)*Hq + h
  const int d = threadIdx.x * 2;
  float M = NEG_INF;
  for (int sp = 0; sp < splits; ++sp) M = fmaxf(M, ws_ml[(r * splits + sp) * 2]);
  float n0 = 0.f, n1 = 0.f, den = 0.f;
  for (int sp = 0; sp < splits; ++sp) {
    const float ms = ws_ml[(r * splits + sp) * 2];
    if (ms == NEG_INF) continue;
    const float a = expf(ms - M);
    den += a * ws_ml[(r * splits + sp) * 2 + 1];
    n0 += a * ws_acc[(r * splits + sp) * 128 + d];
    n1 += a * ws_acc[(r * splits + sp) * 128 + d + 1];
  }
  out[r * 128 + d] = (bf16_t)f2bf(n0 / den);
  out[r * 128 + d + 1] = (bf16_t)f2bf(n1 / den);
}

int64_t decode_attn_splits(int64_t B, int Hkv, int64_t cap) {
  const int64_t want = (1024 + B * Hkv - 1) / (B * Hkv);  // ~4 workgroups per CU
  const int64_t max_splits = (cap + 63) / 64;
  int64_t sp = want < 1 ? 1 : want;
  if (sp > max_splits) sp = max_splits;
  const int64_t chunk = decode_attn_chunk(cap, sp);
  return (cap + chunk - 1) / chunk;
}

int64_t decode_attn_chunk(int64_t cap, int64_t splits) {
  int64_t chunk = (cap + splits - 1) / splits;
  return (chunk + 63) / 64 * 64;
}

void launch_decode_attn(const bf16_t* qkv, int64_t qkv_stride, const bf16_t* qn, const bf16_t* kn,
                        const bf16_t* cos_t, const bf16_t* sin_t, const int64_t* pos,
                        bf16_t* k_cache, bf16_t* v_cache, int64_t B, int Hq, int Hkv, int64_t cap,
                        int64_t splits, float eps, float* ws_acc, float* ws_ml, bf16_t* out,
                        hipStream_t s) {
  const int64_t chunk = decode_attn_chunk(cap, splits);
  decode_attn_kernel<<<dim3((unsigned)splits, (unsigned)Hkv, (unsigned)B), dim3(256), 0, s>>>(
      qkv, qkv_stride, qn, kn, cos_t, sin_t, pos, k_cache, v_cache, Hq, Hkv, cap, chunk, eps,
      1.0f / sqrtf(128.0f), ws_acc, ws_ml);
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
