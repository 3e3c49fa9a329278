// The MFMA decode-attention workgroup (attn.hip's decode_attn_mfma_kernel): see attn.hip for
// the design.
#pragma once

#include "attn_core.h"

typedef short ba_v4i16_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) ba_v4i16_t ba_lds_v4i16_t;
// four bf16 of the transposed 16-lane read at p (LDS), as two packed 32-bit words
__device__ __forceinline__ uint2 lds_read_tr16(const void* p) {
  const ba_v4i16_t r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((ba_lds_v4i16_t*)p);
  return __builtin_bit_cast(uint2, r);
}

constexpr int DM_NW = 8;

struct DecodeMfmaLds {
  union {
    struct {
      uint4 ks[DM_NW][32 * 16];   // each wave's staged K tile (32 keys x 16 units)
      uint4 vs[DM_NW][32 * 16];
    } t;
    float wacc[DM_NW][GRP][128];  // after every wave's last tile: the waves' O
  } u;
  uint32_t qs[GRP][64];        // normalised q of the group's heads, packed bf16 pairs
  uint32_t kns[64], vns[64];   // the new token's K (normalised) and V rows
  float wm[DM_NW][GRP], wl[DM_NW][GRP];
};

// Workgroup (split, kvh, b) of the launch below, nb sequences, with sm as its LDS.
template <bool ROPE_ROW>
__device__ __forceinline__ void decode_attn_mfma_block(
    DecodeMfmaLds& sm, int split, int kvh, int64_t b, int splits, int64_t nb,
    const bf16_t* __restrict__ qkv, int64_t qkv_stride, const bf16_t* __restrict__ qn,
    const bf16_t* __restrict__ kn, const bf16_t* __restrict__ cos_t,
    const bf16_t* __restrict__ sin_t, const int64_t* __restrict__ pos_ptr, bf16_t* k_cache,
    bf16_t* v_cache, int Hq, int Hkv, int64_t cap, int64_t chunk, float eps, float scale,
    float* ws_acc, float* ws_ml, bf16_t* out, const float* __restrict__ part, int part_S) {
  typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
  typedef __attribute__((ext_vector_type(4))) float f32x4_t;
  // 16-byte units as a native vector: copies of HIP's uint4 struct are memcpys, which keep the
  // staging arrays out of registers
  typedef unsigned int u4v __attribute__((ext_vector_type(4)));
  const int tid = (int)threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int c = lane & 15, q4 = lane >> 4;
  const int64_t head_off = ((b * Hkv + kvh) * cap) * 128;
  const u4v* kb = reinterpret_cast<const u4v*>(k_cache + head_off);
  const u4v* vb = reinterpret_cast<const u4v*>(v_cache + head_off);
  const int64_t start = (int64_t)split * chunk;
  // staging: lane moves 16-byte unit c of keys q4 + 4 j (j < 8) of a tile; keys at or past lim
  // reload row lim - 1 (a valid row, never attended as such)
  // one tile in flight per wave (registers), refilled as soon as the tile is staged
  u4v kx[8], vx[8];
#define DM_LD(KX, VX, J0, LIM)                                                 \
  _Pragma("unroll") for (int dm_j_ = 0; dm_j_ < 8; ++dm_j_) {                  \
    const int64_t dm_key_ = (J0) + q4 + 4 * dm_j_;                             \
    const int64_t dm_row_ = dm_key_ < (LIM) ? dm_key_ : (LIM) - 1;             \
    const int64_t dm_r_ = dm_row_ > 0 ? dm_row_ : 0;                           \
    KX[dm_j_] = __builtin_nontemporal_load(kb + dm_r_ * 16 + c);               \
    VX[dm_j_] = __builtin_nontemporal_load(vb + dm_r_ * 16 + c);               \
  }
  DM_LD(kx, vx, start + 32 * wave, cap);   // the wave's first tile, before pos is known
  // prologue loads: q head kvh * 4 + wave (waves 0..3; the others load it too and drop it);
  // wave 0 the new k, wave 1 the new v
  const int64_t eq = (int64_t)(kvh * GRP + (wave & (GRP - 1))) * 128;
  const int64_t ek = (int64_t)(Hq + (wave == 1 ? Hkv : 0) + kvh) * 128;
  uint32_t q1, q2, k1, k2;
  if (part) {
    // the qkv projection's split-K partials part[S][B][W]: each value is their sum in split
    // order rounded to bf16, the bits the projection's own epilogue stores when unsplit over
    // the same order
    const int64_t W = (int64_t)(Hq + 2 * Hkv) * 128;
    const float* p0 = part + b * W;
    float aq1 = p0[eq + lane], aq2 = p0[eq + lane + 64];
    float ak1 = p0[ek + lane], ak2 = p0[ek + lane + 64];
    for (int sp = 1; sp < part_S; ++sp) {
      const float* ps = part + ((int64_t)sp * nb + b) * W;
      aq1 += ps[eq + lane]; aq2 += ps[eq + lane + 64];
      ak1 += ps[ek + lane]; ak2 += ps[ek + lane + 64];
    }
    q1 = f2bf(aq1); q2 = f2bf(aq2); k1 = f2bf(ak1); k2 = f2bf(ak2);
  } else {
    const bf16_t* row = qkv + b * qkv_stride;
    q1 = row[eq + lane]; q2 = row[eq + lane + 64];
    k1 = row[ek + lane]; k2 = row[ek + lane + 64];
  }
  const float qw1 = bf2f(qn[lane]), qw2 = bf2f(qn[lane + 64]);
  const float kw1 = bf2f(kn[lane]), kw2 = bf2f(kn[lane + 64]);
  float c1, c2, s1, s2;
  if constexpr (ROPE_ROW) {
    c1 = bf2f(cos_t[lane]); c2 = bf2f(cos_t[lane + 64]);
    s1 = bf2f(sin_t[lane]); s2 = bf2f(sin_t[lane + 64]);
  }
  const int64_t pos = pos_ptr[0];
  if constexpr (!ROPE_ROW) {
    const int64_t pr = (pos >= 0 && pos < cap ? pos : 0) * 128;
    c1 = bf2f(cos_t[pr + lane]); c2 = bf2f(cos_t[pr + lane + 64]);
    s1 = bf2f(sin_t[pr + lane]); s2 = bf2f(sin_t[pr + lane + 64]);
  }
  if (pos < 0 || pos >= cap) return;   // uniform over the grid: no slot to write
  const bool owns = pos >= start && pos < start + chunk;
  const int64_t kend = owns ? pos + 1 : (start + chunk < pos ? start + chunk : pos);
  if (wave < GRP) {
    float o1, o2;
    norm_rope_vals(bf2f(q1), bf2f(q2), qw1, qw2, c1, c2, s1, s2, eps, o1, o2);
    reinterpret_cast<bf16_t*>(sm.qs[wave])[lane] = (bf16_t)f2bf(o1);
    reinterpret_cast<bf16_t*>(sm.qs[wave])[lane + 64] = (bf16_t)f2bf(o2);
  }
  if (owns && wave == 0) {
    float o1, o2;
    norm_rope_vals(bf2f(k1), bf2f(k2), kw1, kw2, c1, c2, s1, s2, eps, o1, o2);
    const bf16_t n1 = (bf16_t)f2bf(o1), n2 = (bf16_t)f2bf(o2);
    k_cache[head_off + pos * 128 + lane] = n1;
    k_cache[head_off + pos * 128 + lane + 64] = n2;
    reinterpret_cast<bf16_t*>(sm.kns)[lane] = n1;
    reinterpret_cast<bf16_t*>(sm.kns)[lane + 64] = n2;
  }
  if (owns && wave == 1) {
    v_cache[head_off + pos * 128 + lane] = (bf16_t)k1;
    v_cache[head_off + pos * 128 + lane + 64] = (bf16_t)k2;
    reinterpret_cast<bf16_t*>(sm.vns)[lane] = (bf16_t)k1;
    reinterpret_cast<bf16_t*>(sm.vns)[lane + 64] = (bf16_t)k2;
  }
  lds_barrier();
  // B operand: column c < 4 is query head kvh * 4 + c (dims 32 kk + 8 q4 .. + 7); the other
  // columns are zero
  u4v qf[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk)
    qf[kk] = c < GRP ? reinterpret_cast<const u4v*>(sm.qs[c & (GRP - 1)])[4 * kk + q4]
                     : u4v{0u, 0u, 0u, 0u};
  u4v* ks = reinterpret_cast<u4v*>(sm.u.t.ks[wave]);
  u4v* vs = reinterpret_cast<u4v*>(sm.u.t.vs[wave]);
  // transposed-read address of V dims 16 dt + 4 (c % 4) .. + 3 of key 16 h2 + 4 q4 + c / 4
  auto vt_addr = [&](int dt, int h2) -> const void* {
    const int key = 16 * h2 + 4 * q4 + (c >> 2);
    const int u = 2 * dt + ((c >> 1) & 1);
    return reinterpret_cast<const char*>(&vs[key * 16 + (u ^ (key & 15))]) + 8 * (c & 1);
  };
  // the new token's unit c of K and V, written over its row by the tile that holds pos
  const u4v knew = reinterpret_cast<const u4v*>(sm.kns)[c];
  const u4v vnew = reinterpret_cast<const u4v*>(sm.vns)[c];
  float m = M_FLOOR, lsum = 0.f;
  f32x4_t o[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) o[dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const int ntiles = kend > start ? (int)((kend - start + 31) / 32) : 0;
  // stage tile j0 from (kx_, vx_) into this wave's LDS region; the new token's row from LDS
  auto stage = [&](const u4v (&kx_)[8], const u4v (&vx_)[8], int64_t j0) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int key = q4 + 4 * j;
      ks[key * 16 + (c ^ (key & 15))] = kx_[j];
      vs[key * 16 + (c ^ (key & 15))] = vx_[j];
    }
    const int64_t pk = pos - j0;                       // LDS keeps a wave's stores in order:
    if (pk >= 0 && pk < 32 && q4 == 0) {               // this one wins
      ks[pk * 16 + (c ^ (pk & 15))] = knew;
      vs[pk * 16 + (c ^ (pk & 15))] = vnew;
    }
  };
  // contract the staged tile at j0 into (m, lsum, o).  The region is this wave's alone and LDS
  // serves a wave's accesses in order; the fences keep the compiler from moving fragment reads
  // above the staging stores, or the next staging above these reads.
  auto contract = [&](int64_t j0) {
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    f32x4_t sc[2] = {f32x4_t{0.f, 0.f, 0.f, 0.f}, f32x4_t{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      const int key = 16 * h2 + c;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const u4v kf = ks[key * 16 + ((4 * kk + q4) ^ c)];
        sc[h2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kf),
                                                        __builtin_bit_cast(bf16x8_t, qf[kk]),
                                                        sc[h2], 0, 0, 0);
      }
    }
    // lane (c, q4): scores of column c against keys 16 h2 + 4 q4 + r of the tile
    const int lim = kend - j0 < 32 ? (int)(kend - j0) : 32;
    float sv[8];
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        sv[4 * h2 + r] = 16 * h2 + 4 * q4 + r < lim ? sc[h2][r] * scale : NEG_INF;
    float mx = sv[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) mx = fmaxf(mx, sv[e]);
    mx = fmaxf(mx, lane_xor16(mx));
    mx = fmaxf(mx, lane_xor32(mx));
    const float mn = fmaxf(m, mx);
    const float alpha = __expf(m - mn);
    m = mn;
    float p[8], ps = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) { p[e] = __expf(sv[e] - mn); ps += p[e]; }
    lsum = lsum * alpha + ps;
    const uint4 pf = make_uint4(pack2(p[0], p[1]), pack2(p[2], p[3]), pack2(p[4], p[5]), pack2(p[6], p[7]));
    if (__ballot(alpha != 1.f) != 0) {               // x * 1 == x: skipping changes no bit
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) o[dt] *= alpha;
    }
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const uint2 lo = lds_read_tr16(vt_addr(dt, 0));
      const uint2 hi = lds_read_tr16(vt_addr(dt, 1));
      const uint4 vf = make_uint4(lo.x, lo.y, hi.x, hi.y);
      o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, vf),
                                                     __builtin_bit_cast(bf16x8_t, pf), o[dt], 0, 0, 0);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  };
  for (int t = wave; t < ntiles; t += DM_NW) {
    const int64_t j0 = start + 32 * (int64_t)t;
    stage(kx, vx, j0);
    DM_LD(kx, vx, j0 + 32 * DM_NW, kend);   // the wave's next tile
    contract(j0);
  }
#undef DM_LD
  // column totals (the four q4 lanes of a column hold disjoint keys), then the waves' states
  float l = lsum;
  l += lane_xor16(l);
  l += lane_xor32(l);
  lds_barrier();                          // every wave is done with the staging region
  if (c < GRP) {
    if (q4 == 0) { sm.wm[wave][c] = m; sm.wl[wave][c] = l; }
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) sm.u.wacc[wave][c][16 * dt + 4 * q4 + r] = o[dt][r];
  }
  lds_barrier();
  if (tid >= GRP * 64) return;            // one head per wave for the combine
  // as decode_attn_unit: one head per wave, dims d, d + 1 per lane
  const int h = tid >> 6, d = (tid & 63) * 2;
  float M = sm.wm[0][h];
  for (int w = 1; w < DM_NW; ++w) M = fmaxf(M, sm.wm[w][h]);
  float L = 0.f, A0 = 0.f, A1 = 0.f;
  for (int w = 0; w < DM_NW; ++w) {
    const float a = __expf(sm.wm[w][h] - M);
    L += a * sm.wl[w][h];
    A0 += a * sm.u.wacc[w][h][d];
    A1 += a * sm.u.wacc[w][h][d + 1];
  }
  const int64_t qrow = b * Hq + kvh * GRP + h;
  if (splits == 1) {
    const float inv = 1.0f / L;
    *reinterpret_cast<uint32_t*>(out + qrow * 128 + d) = pack2(A0 * inv, A1 * inv);
  } else {
    const int64_t idx = qrow * splits + split;
    *reinterpret_cast<float2*>(ws_acc + idx * 128 + d) = make_float2(A0, A1);
    if ((tid & 63) == 0) *reinterpret_cast<float2*>(ws_ml + idx * 2) = make_float2(M, L);
  }
}
