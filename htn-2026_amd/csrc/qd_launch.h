// Internal host-side launchers shared between the kernel translation units and the step
// sequencer.  Every launcher validates nothing (the extern "C" entry points in qd_api.cpp and
// the step sequencer validate shapes once) and only enqueues on `s`.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qd_common.h"

enum { EPI_NONE = 0, EPI_RES = 1, EPI_SWIGLU = 2, EPI_ARGMAX = 3 };
enum { POS_T = 0, POS_SHARED = 1, POS_ROW = 2, POS_TREE = 3, POS_CHUNK = 4 };

// elementwise.hip
void launch_embed(const int64_t* ids, const bf16_t* table, bf16_t* out, int64_t n, int64_t vocab,
                  int64_t hidden, int64_t out_stride, hipStream_t s);
// embedding gather that also copies this step's RoPE row (cos[pos], sin[pos]) to rope_out[256]
void launch_embed_rope(const int64_t* ids, const bf16_t* table, bf16_t* out, int64_t n,
                       int64_t vocab, int64_t hidden, int64_t out_stride, const bf16_t* cos_t,
                       const bf16_t* sin_t, const int64_t* pos, int64_t cap, bf16_t* rope_out,
                       hipStream_t s);
void launch_add_rmsnorm(const bf16_t* x, const bf16_t* res, const bf16_t* w, bf16_t* res_out,
                        bf16_t* y, int64_t rows, int64_t hidden, int64_t in_stride, int64_t y_stride,
                        float eps, hipStream_t s);
// split-K partials [S][rows][hidden] fp32 + residual (in/out) + RMSNorm
void launch_part_add_rmsnorm(const float* part, int S, int64_t rows, bf16_t* res, const bf16_t* w,
                             bf16_t* y, int64_t hidden, float eps, hipStream_t s);
void launch_qk_norm_rope(const bf16_t* qkv, int64_t qkv_stride, const bf16_t* qn, const bf16_t* kn,
                         const bf16_t* cos_t, const bf16_t* sin_t, int64_t table_len,
                         const int64_t* pos, const int64_t* depth, int mode, bf16_t* q_out,
                         bf16_t* k_cache, bf16_t* v_cache, int64_t B, int64_t T, int Hq, int Hkv,
                         int64_t cap, float eps, hipStream_t s);
// the same with the qkv rows given as split-K partials part[S][B*T][(Hq + 2 Hkv) * 128] fp32
void launch_qk_norm_rope_part(const float* part, int S, const bf16_t* qn, const bf16_t* kn,
                              const bf16_t* cos_t, const bf16_t* sin_t, int64_t table_len,
                              const int64_t* pos, const int64_t* depth, int mode, bf16_t* q_out,
                              bf16_t* k_cache, bf16_t* v_cache, int64_t B, int64_t T, int Hq,
                              int Hkv, int64_t cap, float eps, hipStream_t s);
void launch_swiglu(const bf16_t* gu, int64_t gu_stride, bf16_t* out, int64_t out_stride,
                   int64_t rows, int64_t inter, hipStream_t s);
void launch_kv_compact(bf16_t* k_all, bf16_t* v_all, int64_t L, int64_t B, int Hkv, int64_t cap,
                       const int64_t* base, const int32_t* src, const int32_t* cnt, int64_t T,
                       hipStream_t s);
void launch_synth(bf16_t* out, int64_t count, uint64_t seed, uint64_t stream, uint64_t start,
                  float scale, hipStream_t s);
void launch_fill(bf16_t* out, int64_t count, uint16_t value, hipStream_t s);
void launch_read_probe(const void* buf, int64_t bytes, int grid, uint32_t* sink, hipStream_t s);
void launch_argmax_reduce(const float* pval, const int32_t* pidx, int64_t nparts, int64_t M,
                          int64_t* tok, int64_t* pos_inc, hipStream_t s);

// gemv.hip (vector path, 1..2 rows)
int gemv_supported(int64_t M, int64_t K);
void launch_gemv(const bf16_t* x, int64_t x_stride, const bf16_t* w, int64_t N, int64_t K,
                 bf16_t* out, int64_t out_stride, const bf16_t* res, int64_t res_stride,
                 const bf16_t* norm_w, float eps, int epi, int64_t M, hipStream_t s);
int64_t lm_vec_parts(int64_t V);
void launch_lm_vec(const bf16_t* x, int64_t x_stride, const bf16_t* w, int64_t V, int64_t K,
                   const bf16_t* norm_w, float eps, int64_t M, float* pval, int32_t* pidx,
                   int64_t* tok, int64_t* pos_inc, float* logits, hipStream_t s);

// gemm.hip (MFMA path, any M).  launch_gemm returns the argmax partials written per row
// (EPI_ARGMAX; at most gemm_argmax_parts(N)), else 0.  `part` (optional, part_floats floats) is
// the split-K workspace of the tiled kernel (gemm_tile_ws_floats); without it K is not split.
int64_t gemm_argmax_parts(int64_t N);
int64_t launch_gemm(const bf16_t* x, int64_t x_stride, int64_t M, const bf16_t* w, int64_t N,
                    int64_t K, bf16_t* out, int64_t out_stride, const bf16_t* res,
                    int64_t res_stride, int epi, float* pval, int32_t* pidx, float* logits,
                    hipStream_t s, float* part = nullptr, int64_t part_floats = 0);
// gemm_skinny.hip (batched decode, M <= 32: one workgroup per CU, waves split K).  part == NULL:
// the epilogue writes out (S == 1); else fp32 split-K partials part[S][M][N] for the caller to
// sum.  Returns false (nothing launched) for an unsupported shape or a missing destination.
bool skinny_ok(int64_t M, int64_t N, int64_t K, int epi, int S, const void* x, int64_t xs,
               const void* w, int64_t os);
int64_t skinny_part_floats(int64_t M, int64_t N, int S);
// LM head + argmax partials at <= 32 rows: returns the partials written per row (one per
// workgroup, at most the CU count), or 0 when the shape is not supported (nothing launched)
int64_t launch_lm_skinny(const bf16_t* x, int64_t xs, int64_t M, const bf16_t* w, int64_t N,
                         int64_t K, float* pval, int32_t* pidx, float* logits, hipStream_t s);
bool launch_gemm_skinny(const bf16_t* x, int64_t xs, int64_t M, const bf16_t* w, int64_t N,
                        int64_t K, int epi, int S, bf16_t* out, int64_t os, const bf16_t* res,
                        int64_t rs, float* part, hipStream_t s);
// gemm_tile.hip (LDS-tiled MFMA GEMM for M > 64).  gemm_tile_partials: when the tile grid
// would split K, launch only the split kernel (fp32 partials part[S][M][N], no reduce) and
// return S; otherwise launch nothing and return 0.
int gemm_tile_partials(const bf16_t* x, int64_t xs, int64_t M, const bf16_t* w, int64_t N,
                       int64_t K, float* part, int64_t part_floats, hipStream_t s);
bool gemm_tile_ok(int64_t M, int64_t N, int64_t K, int epi, const void* x, int64_t x_stride,
                  const void* w, const void* out, int64_t out_stride, const void* res,
                  int64_t res_stride);
int gemm_tile_splits(int64_t M, int64_t N, int64_t K, int epi);
// The all-rows kernel's launch for a shape (qd_gemm_rows_plan): -1 / 0 / 1 as rows_launch_plan;
// with 1, out[8] = rows per workgroup, instantiated block height (MFMA tiles), activation
// tiles per wave, activation halves, K splits, K steps per split, grid, static LDS bytes.
int gemm_rows_query(int64_t M, int64_t N, int64_t K, int epi, bool partials_only,
                    int64_t part_floats, int64_t* out);
int64_t gemm_tile_ws_floats(int64_t M, int64_t N, int64_t K, int epi);
int64_t launch_gemm_tile(const bf16_t* x, int64_t xs, int64_t M, const bf16_t* w, int64_t N,
                         int64_t K, bf16_t* out, int64_t os, const bf16_t* res, int64_t rs, int epi,
                         float* pval, int32_t* pidx, float* logits, float* part,
                         int64_t part_floats, hipStream_t s);
// rows from which the tiled kernel takes over
constexpr int64_t GEMM_TILE_MIN_M = 65;

// attn.hip
// waves per decode-attention unit (4 query heads x 16 keys per wave per iteration)
#ifndef QD_ATTN_NW
#define QD_ATTN_NW 4
#endif
constexpr int ATTN_NW = QD_ATTN_NW;
int64_t decode_attn_splits(int64_t B, int Hkv, int64_t cap);

int skinny_cus();                                   // the CU count (0 if unknown)
int64_t skinny_rows(int64_t N, int S);              // weight rows per skinny workgroup
// persistent B = 1 decode step (mega.hip)
struct MegaLaunch {
  const bf16_t *embed, *lm_head, *final_norm, *w_qkv, *w_o, *w_gu, *w_down, *ln1, *ln2, *q_norm, *k_norm;
  const bf16_t *cos, *sin;
  bf16_t *k_cache, *v_cache;
  int64_t *tok, *pos;
  bf16_t* x_out;
  uint32_t* ctl;        // [0] epoch, [1] error; zero before the first launch
  uint32_t* ll;         // mega_ll_bytes, zero before the first launch with this split plan
  int64_t cap, vocab;
  int L;
  float eps;
};
int mega_grid();                                   // workgroups per launch; 0 = unsupported device
bool mega_shape_ok(int hidden, int inter, int hq, int hkv, int head_dim);
int64_t mega_ll_bytes(int L, int64_t splits, int grid);
int64_t mega_splits(int64_t cap);
hipError_t launch_mega_step(const MegaLaunch& m, hipStream_t s);
int64_t decode_attn_chunk(int64_t cap, int64_t splits);
void launch_decode_attn(const bf16_t* qkv, int64_t qkv_stride, const bf16_t* qn, const bf16_t* kn,
                        const bf16_t* cos_t, const bf16_t* sin_t, const int64_t* pos,
                        bf16_t* k_cache, bf16_t* v_cache, int64_t B, int Hq, int Hkv, int64_t cap,
                        int64_t splits, float eps, float* ws_acc, float* ws_ml, bf16_t* out,
                        bool rope_row, hipStream_t s);
// B >= 2 decode attention whose q / k / v come from the qkv projection's split-K partials
// part[part_S][B][(Hq + 2 Hkv) * 128] (fp32, summed in split order and rounded to bf16)
void launch_decode_attn_part(const float* part, int part_S, const bf16_t* qn, const bf16_t* kn,
                             const bf16_t* cos_t, const bf16_t* sin_t, const int64_t* pos,
                             bf16_t* k_cache, bf16_t* v_cache, int64_t B, int Hq, int Hkv,
                             int64_t cap, int64_t splits, float eps, float* ws_acc, float* ws_ml,
                             bf16_t* out, bool rope_row, hipStream_t s);
// Block attention (tree verification, causal prefill chunks).  Keys split into at most
// block_attn_splits(cap) ranges; a launch of B x T query rows uses block_attn_launch_splits(),
// as many as fit one round of workgroups over the CUs.  With more than one split it writes
// fp32 partials (128 + 2 floats per query-head row and split) and merges them;
// block_attn_partial_rows() is the number of partial rows any launch with T' <= T needs
// (0 when all of them run one split and write their output directly).
int64_t block_attn_splits(int64_t cap);
int64_t block_attn_launch_splits(int64_t B, int64_t T, int Hkv, int64_t cap);
int64_t block_attn_partial_rows(int64_t B, int64_t T, int Hq, int Hkv, int64_t cap);
void launch_block_attn(const bf16_t* q, const bf16_t* k_cache, const bf16_t* v_cache,
                       const int64_t* base, const uint64_t* anc, int64_t B, int64_t T, int Hq,
                       int Hkv, int64_t cap, float* ws_acc, float* ws_ml, bf16_t* out,
                       hipStream_t s);
