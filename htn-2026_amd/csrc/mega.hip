// Persistent decode step for one sequence (B = 1): the whole greedy step -- per layer qkv,
// attention (+ split merge), o + residual, gate/up + SwiGLU, down + residual, then the final
// norm, LM head and argmax, pos += 1 -- in ONE launch of one workgroup per CU
// (engine/kernels/mega.py:1-15 is the reference's persistent tier; arithmetic as its T5 units,
// fast.py).
//
// Why: a B = 1 step is ~216 dependent launches of 2-20 us each; every launch boundary costs a
// drain, a cache write-back and a ramp-up.  Here each workgroup runs the step's phases in
// order and, before it waits for a phase's input, issues the loads of that phase's weight rows
// (which never depend on the input), so HBM keeps streaming weights across phase boundaries.
//
// Cross-workgroup hand-off without fences: every produced value travels in 32-bit words (two
// bf16, or one fp32 / index) written with agent-scope relaxed atomic stores and read with
// agent-scope relaxed atomic loads, mostly two words per load (single-copy atomic per word,
// coherent across the XCDs' L2s).  A word holds its payload inverted (~payload), so 0 means
// "not written yet": a consumer waits until every word it loaded is nonzero.  The one payload
// whose inverse is 0, 0xFFFFFFFF (two bf16 NaNs, or an fp32 NaN), is stored as 0xFFFFFFFE, still
// NaN.  The hand-off area has two copies that alternate with the parity of the epoch (a word in
// the workspace, read by every workgroup at the start and advanced by workgroup 0 at the very
// end, after every other workgroup has delivered its LM-head partial, which depends on
// everything it read): a launch writes the copy of its parity, each word once, and zeroes the
// other copy for the next launch, every workgroup its share, layer by layer.  Against a word of
// {payload, 32-bit tag}, consumers load half the bytes.
// Waits are bounded: after HW_SPIN_LIMIT polls, or once any wait has failed, a wait sets the
// error word and returns; the launch then completes with garbage instead of hanging, and the
// host reads the error word (qd_mega_ctl_offset) after the first replay.  The workspace starts
// zero-filled, and must be zero-filled again before a launch with another split plan (another
// cap), which moves the words.
//
// Every workgroup is resident at once (grid = CU count, one 512-thread workgroup per CU,
// checked against the occupancy API on the host), phases only wait on earlier phases, and
// every workgroup runs every phase, so every wait is eventually satisfied.
//
// Results are bit-identical to qd_decode_step at B = 1: the GEMV rows use the same per-wave
// dot order and wave reduction, the RMSNorm statistics the same virtual thread partition
// (512 threads for the qkv / gate-up prologues, 256 for the final norm), and attention the same
// units (attn_core.h) with the same split plan.
#include "qd_launch.h"

#include "attn_core.h"
#include "handoff.h"

namespace {

constexpr int MG_NW = 8;                 // waves per workgroup
constexpr int MG_NT = MG_NW * 64;

// model shape of this kernel (Qwen3-4B); the host checks the weights against it
constexpr int H = 2560, INTER = 9728, HQ = 32, HKV = 8, HD = 128;
constexpr int NQKV = (HQ + 2 * HKV) * HD;     // 6144
constexpr int MIN_WG = 256;                   // rows per wave below assume >= 256 workgroups

// Hand-off words of one layer (32-bit words): the layer's input residual comes from the previous
// layer's OUT (layer 0 reads the embedding row directly); offsets are even (8-byte aligned)
struct Layout {
  int64_t qkv, att, mid, act, out, part, ml, per_layer, lm;
};

__host__ __device__ inline Layout ll_layout(int L, int64_t splits) {
  Layout a;
  a.qkv = 0;
  a.att = a.qkv + NQKV / 2;
  a.mid = a.att + HQ * HD / 2;
  a.act = a.mid + H / 2;
  a.out = a.act + INTER / 2;
  a.part = a.out + H / 2;
  a.ml = a.part + (splits > 1 ? HQ * splits * HD : 0);
  a.per_layer = a.ml + (splits > 1 ? HQ * splits * 2 : 0);
  a.lm = (int64_t)L * a.per_layer;
  return a;
}

struct MegaParams {
  const bf16_t *embed, *lm_head, *final_norm, *w_qkv, *w_o, *w_gu, *w_down, *ln1, *ln2, *q_norm, *k_norm;
  const bf16_t *cos, *sin;
  bf16_t *k_cache, *v_cache;
  int64_t *tok, *pos;
  bf16_t* x_out;       // final residual [H] (plain stores, for inspection)
  uint32_t* ctl;       // [0] epoch, [1] error
  uint32_t* ll;        // two copies of `region` hand-off words
  int64_t cap, chunk, vocab, region;
  int L, splits;
  float eps;
};

// zero this workgroup's share of words [0, n)
__device__ __forceinline__ void hw_clear(uint32_t* dst, int64_t n, int wg, int P) {
  ::hw_clear<MG_NT>(dst, n, wg, P);
}

// words [0, n) of src -> dst (LDS); n even, src 8-byte aligned, n / 2 <= WPT * MG_NT; two words
// per load, WPT loads per thread, all issued before any wait
template <int WPT>
__device__ __forceinline__ void ll_fetch_lds(const uint32_t* src, int n, uint32_t* err,
                                             uint32_t* dst) {
  const uint64_t* s2 = reinterpret_cast<const uint64_t*>(src);
  uint64_t* d2 = reinterpret_cast<uint64_t*>(dst);
  const int np = n / 2;
  uint64_t v[WPT];
#pragma unroll
  for (int j = 0; j < WPT; ++j) {
    const int idx = threadIdx.x + j * MG_NT;
    v[j] = idx < np ? hw_raw(s2 + idx) : 0;
  }
  // A pair still unwritten here was most likely written while the loads were in flight, and so
  // were the thread's other unwritten pairs: once the first one has arrived, re-issue all of
  // them together (one round trip) instead of polling them one after the other.
  if (WPT > 1 && threadIdx.x < np && !hw_ready(v[0])) {
    v[0] = hw_spin(s2 + threadIdx.x, err);
#pragma unroll
    for (int j = 1; j < WPT; ++j) {
      const int idx = threadIdx.x + j * MG_NT;
      if (idx < np && !hw_ready(v[j])) v[j] = hw_raw(s2 + idx);
    }
  }
#pragma unroll
  for (int j = 0; j < WPT; ++j) {
    const int idx = threadIdx.x + j * MG_NT;
    if (idx < np) d2[idx] = hw_wait(v[j], s2 + idx, err);
  }
}

// ------------------------------------------------------------------ GEMV pieces
// lane l reads the 16-byte chunks l, l + 64, ... of a row (as gemv_kernel)
template <int KCH>
__device__ __forceinline__ void mg_load_row(const bf16_t* __restrict__ w, int64_t n, uint4* dst) {
  const uint4* wr = reinterpret_cast<const uint4*>(w + n * (int64_t)(KCH * 512));
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < KCH; ++j) dst[j] = ld_stream(wr + lane + 64 * j);
}

template <int KCH>
__device__ __forceinline__ float mg_dot(const uint4* wv, const uint4* xs) {
  const int lane = threadIdx.x & 63;
  float a = 0.f;
#pragma unroll
  for (int j = 0; j < KCH; ++j) a = dot8(wv[j], xs[lane + 64 * j], a);
  return wave_sum(a);
}

// The thread's chunk of an RMSNorm weight vector (chunk threadIdx.x of KCH * 64), loaded when
// a phase starts so that the norm after the input's hand-off does not wait on it.
template <int KCH>
__device__ __forceinline__ uint4 mg_norm_w(const bf16_t* __restrict__ norm_w) {
  static_assert(KCH * 64 <= MG_NT, "one chunk per thread");
  const int tid = threadIdx.x;
  return tid < KCH * 64 ? reinterpret_cast<const uint4*>(norm_w)[tid] : make_uint4(0, 0, 0, 0);
}

// RMSNorm of the raw row in xs (in place), statistics over VNT virtual threads exactly as a
// VNT-thread workgroup of gemv_kernel / lm_vec_kernel computes them (VNT in {256, 512}); nw is
// the thread's weight chunk (mg_norm_w).
template <int KCH, int VNT>
__device__ __forceinline__ void mg_norm(uint4* xs, uint4 nw, float eps, float* red) {
  constexpr int NCH = KCH * 64;
  static_assert(VNT == 256 || VNT == 512, "virtual thread count");
  const int tid = threadIdx.x;
  float ss = 0.f;
  if (tid < VNT)
    for (int c = tid; c < NCH; c += VNT) ss += sumsq8(xs[c]);
  ss = wave_sum(ss);
  if ((tid & 63) == 0 && tid < VNT) red[tid >> 6] = ss;
  lds_barrier();
  float tot = 0.f;
  for (int q = 0; q < VNT / 64; ++q) tot += red[q];
  const float rstd = rstd_of(tot, KCH * 512, eps);
  if (tid < NCH) xs[tid] = norm8(xs[tid], nw, rstd);
  lds_barrier();
}

__device__ __forceinline__ void part_range(int64_t n, int p, int P, int64_t& a, int64_t& b) {
  a = n * p / P;
  b = n * (p + 1) / P;
}

// o-projection rows of workgroup wg.  With at least 107 workgroups that run no attention unit
// and no split merge, those take all of the rows (at most 24 each): an attention workgroup
// issues its o / gate-up weight loads only after its unit, so o rows there would put its late
// weight stream on the critical path of the MID hand-off.  Otherwise all workgroups share them.
__device__ __forceinline__ void o_rows(const MegaParams& p, int wg, int P, int64_t& a, int64_t& b) {
  const int units = HKV * p.splits;
  const int nmerge = p.splits > 1 ? HQ : 0;
  const int nfree = P - units - nmerge;
  if (nfree >= 107) {
    const int f = wg - units;
    if (f >= 0 && f < nfree) {
      part_range(H / 2, f, nfree, a, b);
    } else {
      a = b = 0;
    }
  } else {
    part_range(H / 2, wg, P, a, b);
  }
}

struct Smem {
  uint4 xs[INTER / 8];             // the phase's input row (bf16), up to 9728 values
  float red[16];
  uint16_t obuf[64];               // the workgroup's outputs of the phase, in row order
  float rown[32];                  // residual values of the workgroup's o / down rows
  float best_v[MG_NW];
  int32_t best_i[MG_NW];
  DecodeAttnLds<ATTN_NW> attn;
};

// the workgroup's outputs obuf[0, nrows) -> hand-off words [w0, w0 + nrows / 2) of dst
__device__ __forceinline__ void put_pairs(Smem& sm, uint32_t* dst, int64_t w0, int nrows) {
  const int t = threadIdx.x;
  if (t < nrows / 2)
    hw_put(dst + w0 + t, (uint32_t)sm.obuf[2 * t] | ((uint32_t)sm.obuf[2 * t + 1] << 16));
}

// ------------------------------------------------------------------ phases
// The phases take their thread index from hw_tid() (threadIdx.x through an empty asm), so the
// compiler recomputes the lane offsets derived from it in each phase instead of keeping them
// live across the layer loop: no VGPR spills (252 VGPRs, no scratch; with threadIdx.x here 16
// VGPRs went to scratch and the step was 0.25 % slower).  The GEMV helpers above keep
// threadIdx.x: their offsets are hoisted out of the row loops, and an opaque index there costs
// 3 % of the step.
// qkv = RMSNorm(x; ln1) . Wqkv^T   (rows wave, wave + 8, wave + 16 of the workgroup's 24)
__device__ void phase_qkv(const MegaParams& p, Smem& sm, int l, int wg, int P, uint32_t* ll,
                          int64_t tok) {
  const int wave = hw_tid() >> 6;
  const Layout ly = ll_layout(p.L, p.splits);
  uint32_t* LL = ll + (int64_t)l * ly.per_layer;
  int64_t a, b;
  part_range(NQKV / 2, wg, P, a, b);
  const int64_t r0 = 2 * a;
  const int nr = (int)(2 * (b - a));
  const bf16_t* W = p.w_qkv + (int64_t)l * NQKV * H;
  uint4 w[3][5];
#pragma unroll
  for (int rr = 0; rr < 3; ++rr)
    if (wave + rr * MG_NW < nr) mg_load_row<5>(W, r0 + wave + rr * MG_NW, w[rr]);
  const uint4 nw = mg_norm_w<5>(p.ln1 + (int64_t)l * H);
  uint32_t* xs32 = reinterpret_cast<uint32_t*>(sm.xs);
  if (l == 0) {                    // the embedding row (an id outside the vocab reads zeros)
    const bool ok = tok >= 0 && tok < p.vocab;
    const uint4* src = reinterpret_cast<const uint4*>(p.embed + (ok ? tok : 0) * H);
    for (int c = hw_tid(); c < H / 8; c += MG_NT) sm.xs[c] = ok ? src[c] : make_uint4(0, 0, 0, 0);
  } else {
    const uint32_t* prev = ll + (int64_t)(l - 1) * ly.per_layer + ly.out;
    ll_fetch_lds<2>(prev, H / 2, p.ctl + 1, xs32);
  }
  lds_barrier();
  {                                // residual values of this workgroup's o rows
    int64_t oa, ob;
    o_rows(p, wg, P, oa, ob);
    const int t = hw_tid();
    if (t < 2 * (ob - oa)) sm.rown[t] = bf2f(reinterpret_cast<const bf16_t*>(sm.xs)[2 * oa + t]);
  }
  mg_norm<5, 512>(sm.xs, nw, p.eps, sm.red);
#pragma unroll
  for (int rr = 0; rr < 3; ++rr) {
    const int k = wave + rr * MG_NW;
    if (k < nr) {
      const float acc = mg_dot<5>(w[rr], sm.xs);
      if ((hw_tid() & 63) == 0) sm.obuf[k] = (uint16_t)f2bf(acc);
    }
  }
  lds_barrier();
  put_pairs(sm, LL + ly.qkv, a, nr);
}

// one decode-attention unit (KV head, split) of layer l
__device__ void phase_attn_unit(const MegaParams& p, Smem& sm, int l, int unit, uint32_t* ll,
                                int64_t pos) {
  const int wave = hw_tid() >> 6, lane = hw_tid() & 63;
  const Layout ly = ll_layout(p.L, p.splits);
  uint32_t* LL = ll + (int64_t)l * ly.per_layer;
  const int kvh = unit / p.splits, split = unit % p.splits;
  const int64_t layer_kv = (int64_t)HKV * p.cap * HD;
  uint32_t* err = p.ctl + 1;
  const uint32_t* qkv = LL + ly.qkv;
  auto fetch = [&](HeadVals& hv) -> int64_t {
    // element e of the packed qkv row lives in word e / 2, half e & 1; the unit's waves read
    // their q and k (v) rows in straight-line code, the other waves nothing
    if (wave < ATTN_NW) {
      const int64_t eq = attn_q_elem(wave, kvh), ek = attn_kv_elem<ATTN_NW>(wave, kvh, HQ, HKV);
      const uint32_t* wq1 = qkv + ((eq + lane) >> 1);
      const uint32_t* wq2 = qkv + ((eq + lane + 64) >> 1);
      const uint32_t* wk1 = qkv + ((ek + lane) >> 1);
      const uint32_t* wk2 = qkv + ((ek + lane + 64) >> 1);
      const uint32_t rq1 = hw_raw(wq1), rq2 = hw_raw(wq2), rk1 = hw_raw(wk1), rk2 = hw_raw(wk2);
      const bf16_t* qn = p.q_norm + (int64_t)l * HD;
      const bf16_t* kn = p.k_norm + (int64_t)l * HD;
      hv.qw1 = bf2f(qn[lane]); hv.qw2 = bf2f(qn[lane + 64]);
      hv.kw1 = bf2f(kn[lane]); hv.kw2 = bf2f(kn[lane + 64]);
      hv.c1 = bf2f(p.cos[pos * HD + lane]); hv.c2 = bf2f(p.cos[pos * HD + lane + 64]);
      hv.s1 = bf2f(p.sin[pos * HD + lane]); hv.s2 = bf2f(p.sin[pos * HD + lane + 64]);
      const uint32_t sh = (lane & 1) * 16;
      hv.q1 = (hw_wait(rq1, wq1, err) >> sh) & 0xFFFF;
      hv.q2 = (hw_wait(rq2, wq2, err) >> sh) & 0xFFFF;
      hv.k1 = (hw_wait(rk1, wk1, err) >> sh) & 0xFFFF;
      hv.k2 = (hw_wait(rk2, wk2, err) >> sh) & 0xFFFF;
    }
    return pos;
  };
  auto final_out = [&](int h, int d, float y0, float y1) {
    hw_put(LL + ly.att + ((int64_t)(kvh * GRP + h) * HD + d) / 2, pack2(y0, y1));
  };
  auto partial_out = [&](int h, int d, float A0, float A1, float M, float Lsum) {
    const int64_t idx = (int64_t)(kvh * GRP + h) * p.splits + split;
    hw_put2(LL + ly.part + idx * HD + d, __float_as_uint(A0), __float_as_uint(A1));
    if ((hw_tid() & 63) == 0)
      hw_put2(LL + ly.ml + idx * 2, __float_as_uint(M), __float_as_uint(Lsum));
  };
  decode_attn_unit<ATTN_NW>(sm.attn, fetch, final_out, partial_out,
                          p.k_cache + (int64_t)l * layer_kv, p.v_cache + (int64_t)l * layer_kv,
                          (int64_t)kvh * p.cap * HD, p.cap, (int64_t)split * p.chunk, p.chunk,
                          p.splits == 1, p.eps, 1.0f / sqrtf((float)HD));
}

// LSE merge of q head hq's split partials (one wave) -> ATT words of the head
__device__ void phase_merge(const MegaParams& p, int l, int hq, uint32_t* ll) {
  const int lane = hw_tid() & 63;
  const Layout ly = ll_layout(p.L, p.splits);
  uint32_t* LL = ll + (int64_t)l * ly.per_layer;
  uint32_t* err = p.ctl + 1;
  const int S = p.splits;
  // (M, sum) of split sp, and the two accumulator values of this lane: one 8-byte pair each
  const uint64_t* ml = reinterpret_cast<const uint64_t*>(LL + ly.ml + (int64_t)hq * S * 2);
  const uint64_t* acc =
      reinterpret_cast<const uint64_t*>(LL + ly.part + (int64_t)hq * S * HD + 2 * lane);
  auto f2 = [](uint64_t v) {
    return make_float2(__uint_as_float((uint32_t)v), __uint_as_float((uint32_t)(v >> 32)));
  };
  const float2 y = merge_splits(
      S,
      [&](int sp) { return f2(hw_wait(hw_raw(ml + sp), ml + sp, err)); },
      [&](int first, int n, float2 (&a)[MERGE_BATCH]) {
        uint64_t r[MERGE_BATCH];
#pragma unroll
        for (int q = 0; q < MERGE_BATCH; ++q)
          if (q < n) r[q] = hw_raw(acc + (int64_t)(first + q) * (HD / 2));
#pragma unroll
        for (int q = 0; q < MERGE_BATCH; ++q)
          a[q] = q < n ? f2(hw_wait(r[q], acc + (int64_t)(first + q) * (HD / 2), err))
                       : make_float2(0.f, 0.f);
      });
  hw_put(LL + ly.att + (int64_t)hq * (HD / 2) + lane, pack2(y.x, y.y));
}

// mid = x + bf16(attn . Wo^T)   (the workgroup's o rows, o_rows: row wave + 8 rr), then
// act = bf16(silu(bf16(g))) * bf16(u), g / u = RMSNorm(mid; ln2) . Wgate / Wup^T (act rows
// wave + 8 rr of the workgroup's 38).  The first two act rows' gate/up weights are loaded
// together with the o rows, before the attention output is awaited, so they stream during the
// attention hand-offs; the third after the o rows are consumed, so it streams during the MID
// hand-off; later act rows refill the 3-slot ring as rows are consumed.  A workgroup without o
// rows skips the attention output and goes straight to the MID wait.
__device__ void phase_o_gu(const MegaParams& p, Smem& sm, int l, int wg, int P, uint32_t* ll) {
  const int wave = hw_tid() >> 6;
  const Layout ly = ll_layout(p.L, p.splits);
  uint32_t* LL = ll + (int64_t)l * ly.per_layer;
  int64_t a, b;
  o_rows(p, wg, P, a, b);
  const int64_t r0 = 2 * a;
  const int nr = (int)(2 * (b - a));
  int64_t ga, gb;
  part_range(INTER / 2, wg, P, ga, gb);
  const int64_t g0 = 2 * ga;
  const int ng = (int)(2 * (gb - ga));
  const bf16_t* W = p.w_o + (int64_t)l * H * (HQ * HD);
  const bf16_t* WG = p.w_gu + (int64_t)l * 2 * INTER * H;
  constexpr int RW = 5;            // act rows per wave (<= 38 per workgroup)
  uint4 w[3][8], g[3][5], u[3][5];  // o rows; a 3-slot ring of act rows (gate, up)
  auto load_gu = [&](int slot, int rr) {
    const int k = wave + rr * MG_NW;
    if (k < ng) {
      mg_load_row<5>(WG, g0 + k, g[slot]);
      mg_load_row<5>(WG, g0 + k + INTER, u[slot]);
    }
  };
#pragma unroll
  for (int rr = 0; rr < 3; ++rr)
    if (wave + rr * MG_NW < nr) mg_load_row<8>(W, r0 + wave + rr * MG_NW, w[rr]);
  load_gu(0, 0);
  load_gu(1, 1);
  if (nr > 0) {                    // uniform over the workgroup
    ll_fetch_lds<2>(LL + ly.att, HQ * HD / 2, p.ctl + 1, reinterpret_cast<uint32_t*>(sm.xs));
    lds_barrier();
#pragma unroll
    for (int rr = 0; rr < 3; ++rr) {
      const int k = wave + rr * MG_NW;
      if (k < nr) {
        const float acc = mg_dot<8>(w[rr], sm.xs);
        if ((hw_tid() & 63) == 0) sm.obuf[k] = (uint16_t)f2bf(sm.rown[k] + rbf(acc));
      }
    }
    lds_barrier();
    put_pairs(sm, LL + ly.mid, a, nr);
  }
  load_gu(2, 2);                   // streams during the MID hand-off
  const uint4 nw = mg_norm_w<5>(p.ln2 + (int64_t)l * H);
  // ---- gate/up + SwiGLU
  ll_fetch_lds<2>(LL + ly.mid, H / 2, p.ctl + 1, reinterpret_cast<uint32_t*>(sm.xs));
  lds_barrier();
  {                                // residual values of this workgroup's down rows
    int64_t da, db;
    part_range(H / 2, wg, P, da, db);
    const int t = hw_tid();
    if (t < 2 * (db - da))
      sm.rown[t] = bf2f(reinterpret_cast<const bf16_t*>(sm.xs)[2 * da + t]);
  }
  mg_norm<5, 512>(sm.xs, nw, p.eps, sm.red);
#pragma unroll
  for (int rr = 0; rr < RW; ++rr) {
    const int k = wave + rr * MG_NW;
    if (k < ng) {
      const float ag = mg_dot<5>(g[rr % 3], sm.xs);
      const float au = mg_dot<5>(u[rr % 3], sm.xs);
      if (rr + 3 < RW) load_gu(rr % 3, rr + 3);
      if ((hw_tid() & 63) == 0) sm.obuf[k] = (uint16_t)f2bf(silu_rbf(rbf(ag)) * rbf(au));
    }
  }
  lds_barrier();
  put_pairs(sm, LL + ly.act, ga, ng);
}

// out = mid + bf16(act . Wdown^T)   (10 rows as phase_o); with the weights in flight, the
// workgroup zeroes its share of layer l's words in the other copy (nxt)
__device__ void phase_down(const MegaParams& p, Smem& sm, int l, int wg, int P, uint32_t* ll,
                           uint32_t* nxt) {
  const int wave = hw_tid() >> 6;
  const Layout ly = ll_layout(p.L, p.splits);
  uint32_t* LL = ll + (int64_t)l * ly.per_layer;
  int64_t a, b;
  part_range(H / 2, wg, P, a, b);
  const int64_t r0 = 2 * a;
  const int nr = (int)(2 * (b - a));
  const bf16_t* W = p.w_down + (int64_t)l * H * INTER;
  uint4 w[2][19];
#pragma unroll
  for (int rr = 0; rr < 2; ++rr)
    if (wave + rr * MG_NW < nr) mg_load_row<19>(W, r0 + wave + rr * MG_NW, w[rr]);
  hw_clear(nxt + (int64_t)l * ly.per_layer, ly.per_layer, wg, P);
  ll_fetch_lds<5>(LL + ly.act, INTER / 2, p.ctl + 1, reinterpret_cast<uint32_t*>(sm.xs));
  lds_barrier();
#pragma unroll
  for (int rr = 0; rr < 2; ++rr) {
    const int k = wave + rr * MG_NW;
    if (k < nr) {
      const float acc = mg_dot<19>(w[rr], sm.xs);
      if ((hw_tid() & 63) == 0) sm.obuf[k] = (uint16_t)f2bf(sm.rown[k] + rbf(acc));
    }
  }
  lds_barrier();
  put_pairs(sm, LL + ly.out, a, nr);
  if (l == p.L - 1 && hw_tid() < nr) p.x_out[r0 + hw_tid()] = sm.obuf[hw_tid()];
}

// final RMSNorm + LM head over the workgroup's vocab rows: best (bf16 logit, lowest index)
// -> 2 hand-off words (and the same two words of the other copy zeroed); four rows in flight
// per wave
__device__ void phase_lm(const MegaParams& p, Smem& sm, int wg, int P, uint32_t* ll,
                         uint32_t* nxt) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const Layout ly = ll_layout(p.L, p.splits);
  int64_t r0, r1;
  part_range(p.vocab, wg, P, r0, r1);
  const int nr = (int)(r1 - r0);
  uint4 buf[4][5];
#pragma unroll
  for (int s = 0; s < 4; ++s)
    if (wave + s * MG_NW < nr) mg_load_row<5>(p.lm_head, r0 + wave + s * MG_NW, buf[s]);
  const uint4 nw = mg_norm_w<5>(p.final_norm);
  const uint32_t* last = ll + (int64_t)(p.L - 1) * ly.per_layer + ly.out;
  ll_fetch_lds<2>(last, H / 2, p.ctl + 1, reinterpret_cast<uint32_t*>(sm.xs));
  lds_barrier();
  mg_norm<5, 256>(sm.xs, nw, p.eps, sm.red);
  float bv = -INFINITY;
  int32_t bi = 0x7FFFFFFF;
  for (int k0 = wave; k0 < nr; k0 += 4 * MG_NW) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int k = k0 + s * MG_NW;
      if (k < nr) {
        const float v = rbf(mg_dot<5>(buf[s], sm.xs));   // the reference's logits are bf16
        const int kn = k + 4 * MG_NW;
        if (kn < nr) mg_load_row<5>(p.lm_head, r0 + kn, buf[s]);
        if (v > bv) { bv = v; bi = (int32_t)(r0 + k); }  // rows ascend per wave: strict >
      }
    }
  }
  if (lane == 0) { sm.best_v[wave] = bv; sm.best_i[wave] = bi; }
  lds_barrier();
  if (threadIdx.x == 0) {
    float v = sm.best_v[0];
    int32_t i = sm.best_i[0];
    for (int q = 1; q < MG_NW; ++q) {
      const float v2 = sm.best_v[q];
      const int32_t i2 = sm.best_i[q];
      if (v2 > v || (v2 == v && i2 < i)) { v = v2; i = i2; }
    }
    hw_put2(ll + ly.lm + 2 * wg, __float_as_uint(v), (uint32_t)i);
    __hip_atomic_store(reinterpret_cast<uint64_t*>(nxt + ly.lm + 2 * wg), (uint64_t)0,
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// workgroup 0: global (max, lowest index) over the partials -> tok; pos += 1; epoch += 1
__device__ void phase_final(const MegaParams& p, Smem& sm, int P, uint32_t* ll, uint32_t epoch,
                            int64_t pos) {
  const Layout ly = ll_layout(p.L, p.splits);
  const uint64_t* lm = reinterpret_cast<const uint64_t*>(ll + ly.lm);
  uint32_t* err = p.ctl + 1;
  float bv = -INFINITY;
  int32_t bi = 0x7FFFFFFF;
  for (int q = threadIdx.x; q < P; q += MG_NT) {
    const uint64_t r = hw_wait(hw_raw(lm + q), lm + q, err);
    const float v = __uint_as_float((uint32_t)r);
    const int32_t i = (int32_t)(uint32_t)(r >> 32);
    if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
  }
  // wave argmax, then across waves
  for (int off = 32; off > 0; off >>= 1) {
    const float v2 = __shfl_xor(bv, off, 64);
    const int32_t i2 = __shfl_xor(bi, off, 64);
    if (v2 > bv || (v2 == bv && i2 < bi)) { bv = v2; bi = i2; }
  }
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  lds_barrier();                   // best_v / best_i were read by phase_lm's thread 0
  if (lane == 0) { sm.best_v[wave] = bv; sm.best_i[wave] = bi; }
  lds_barrier();
  if (threadIdx.x == 0) {
    float v = sm.best_v[0];
    int32_t i = sm.best_i[0];
    for (int q = 1; q < MG_NW; ++q) {
      const float v2 = sm.best_v[q];
      const int32_t i2 = sm.best_i[q];
      if (v2 > v || (v2 == v && i2 < i)) { v = v2; i = i2; }
    }
    p.tok[0] = i == 0x7FFFFFFF ? 0 : (int64_t)i;
    p.pos[0] = pos + 1;
    __hip_atomic_store(p.ctl, epoch + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

__global__ __launch_bounds__(MG_NT) void mega_step_kernel(MegaParams p) {
  __shared__ Smem sm;
  const int wg = blockIdx.x, P = gridDim.x;
  const int wave = threadIdx.x >> 6;
  const uint32_t epoch = __hip_atomic_load(p.ctl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  uint32_t* ll = p.ll + (int64_t)(epoch & 1u) * p.region;          // this launch's words
  uint32_t* nxt = p.ll + (int64_t)((epoch & 1u) ^ 1u) * p.region;   // the next launch's
  const int64_t pos = p.pos[0];
  const int64_t tok = p.tok[0];
  if (pos < 0 || pos >= p.cap) {   // uniform over the grid: nothing is written, nobody waits
    if (wg == 0 && threadIdx.x == 0)
      __hip_atomic_store(p.ctl + 1, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  const int units = HKV * p.splits;
  const int merge0 = P - HQ;       // workgroups merge0 .. P-1 merge one q head each
  for (int l = 0; l < p.L; ++l) {
    phase_qkv(p, sm, l, wg, P, ll, tok);
    for (int u = wg; u < units; u += P) phase_attn_unit(p, sm, l, u, ll, pos);
    if (p.splits > 1 && wg >= merge0 && wave == 0) phase_merge(p, l, wg - merge0, ll);
    phase_o_gu(p, sm, l, wg, P, ll);
    phase_down(p, sm, l, wg, P, ll, nxt);
  }
  phase_lm(p, sm, wg, P, ll, nxt);
  if (wg == 0) phase_final(p, sm, P, ll, epoch, pos);
}

}  // namespace

// ------------------------------------------------------------------ host side
int mega_grid() {
  static int grid = -1;
  if (grid < 0) {
    int dev = 0, cus = 0, occ = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, mega_step_kernel, MG_NT, 0) !=
            hipSuccess) {
      (void)hipGetLastError();
      grid = 0;
    } else {
      grid = (occ >= 1 && cus >= MIN_WG && cus >= HQ) ? cus : 0;
    }
  }
  return grid;
}

bool mega_shape_ok(int hidden, int inter, int hq, int hkv, int head_dim) {
  return hidden == H && inter == INTER && hq == HQ && hkv == HKV && head_dim == HD;
}

// words of one copy of the hand-off area (a multiple of 64: each copy 256-byte aligned)
static int64_t ll_region_words(int L, int64_t splits, int grid) {
  const Layout ly = ll_layout(L, splits);
  return (ly.lm + 2 * (int64_t)grid + 63) / 64 * 64;
}

int64_t mega_ll_bytes(int L, int64_t splits, int grid) {
  return 2 * ll_region_words(L, splits, grid) * 4;
}

int64_t mega_splits(int64_t cap) { return decode_attn_splits(1, HKV, cap); }

hipError_t launch_mega_step(const MegaLaunch& m, hipStream_t s) {
  MegaParams p;
  p.embed = m.embed; p.lm_head = m.lm_head; p.final_norm = m.final_norm; p.w_qkv = m.w_qkv; p.w_o = m.w_o;
  p.w_gu = m.w_gu; p.w_down = m.w_down; p.ln1 = m.ln1; p.ln2 = m.ln2; p.q_norm = m.q_norm;
  p.k_norm = m.k_norm; p.cos = m.cos; p.sin = m.sin; p.k_cache = m.k_cache;
  p.v_cache = m.v_cache; p.tok = m.tok; p.pos = m.pos; p.x_out = m.x_out; p.ctl = m.ctl;
  p.ll = m.ll; p.cap = m.cap; p.vocab = m.vocab; p.L = m.L; p.eps = m.eps;
  p.splits = (int)mega_splits(m.cap);
  p.chunk = decode_attn_chunk(m.cap, p.splits);
  const int grid = mega_grid();
  if (grid <= 0) return hipErrorInvalidConfiguration;
  p.region = ll_region_words(m.L, p.splits, grid);
  mega_step_kernel<<<dim3((unsigned)grid), dim3(MG_NT), 0, s>>>(p);
  return hipGetLastError();
}
