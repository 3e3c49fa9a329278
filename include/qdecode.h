/* qdecode -- MI355X-native (gfx950) Qwen3 greedy-decode kernels behind a plain C ABI.
 *
 * The reference (Yokanater/htn-2026) is a Python engine whose GPU code is Triton; its own
 * kernel wrappers (the .py files under engine/kernels/) take caller-owned torch tensors.  This library is the
 * drop-in for that layer: every entry point takes raw device pointers, int64 sizes and a
 * hipStream_t (passed as void*), allocates nothing, never synchronises the host, and is
 * therefore capturable into a hipGraph.  Tensors are row-major and contiguous unless a
 * stride argument says otherwise; bf16 values are passed as uint16_t bit patterns.
 *
 * Return value: 0 on success; QD_EARG (-1) for an invalid shape/pointer/size argument;
 * QD_EWS (-2) when a workspace is too small; otherwise the hipError_t of the failed launch.
 * No C++ exception crosses this boundary.
 *
 * Workspaces are caller-owned device buffers of at least the size the matching
 * *_workspace_bytes function returns.  They hold split partials that each call writes before
 * it reads them, so they need no initialisation.  Calls that share one workspace must not run
 * concurrently (each call is ordered on its stream).
 */
#ifndef QDECODE_H
#define QDECODE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QD_EARG (-1)
#define QD_EWS (-2)
#define QD_ESTATE (-3)

/* epilogues of qd_linear (engine/kernels/gemv.py:1-9, EPI_* at gemv.py:21) */
#define QD_EPI_NONE 0   /* out = bf16(acc)                                              */
#define QD_EPI_RES 1    /* out = bf16(res + bf16(acc)); res may alias out                */
#define QD_EPI_SWIGLU 2 /* out = bf16(bf16(silu(bf16(acc_gate))) * bf16(acc_up)), rows n
                           of W are gate, rows n + N are up (w_gu packing engine.py:271-272) */

/* position modes of qd_qk_norm_rope (engine/kernels/fused.py:34 POS_MODE, tree.py:26-35) */
#define QD_POS_T 0      /* position = t                                     */
#define QD_POS_SHARED 1 /* position = pos[0] + t                            */
#define QD_POS_ROW 2    /* position = pos[b] + t                            */
#define QD_POS_TREE 3   /* RoPE at pos[b] + depth[b*T+t], cache slot pos[b] + t */

const char *qd_version(void);

/* Embedding gather: out[i, :] = table[ids[i], :] (bit copy).
 * Replaces F.embedding on the decode path (engine/engine.py:338,603) and the gather half of
 * embed_ss (engine/kernels/fast.py:53-76).  ids outside [0, vocab) give a zero row. */
int qd_embed_gather(const int64_t *ids, const uint16_t *table, uint16_t *out, int64_t n_ids,
                    int64_t vocab, int64_t hidden, int64_t out_stride, void *stream);

/* Residual add + RMSNorm per row: res_out = bf16(x + residual) (x may be NULL: no add,
 * res_out ignored), y = bf16(bf16(r * rsqrt(mean(r^2) + eps)) * w).
 * Replaces rms_norm_rows (engine/kernels/rmsnorm.py:15-53) plus the residual add of the
 * decoder layer (EPI_RES, gemv.py:50-51).  res_out may alias residual. */
int qd_add_rmsnorm(const uint16_t *x, const uint16_t *residual, const uint16_t *w,
                   uint16_t *res_out, uint16_t *y, int64_t rows, int64_t hidden,
                   int64_t in_stride, int64_t y_stride, float eps, void *stream);

/* Per-head q/k RMSNorm + RoPE and the K/V cache write for B*T token rows of a packed qkv
 * [B*T, (Hq + 2 Hkv) * 128].  q_out is [B, T, Hq, 128]; k_cache/v_cache are one layer,
 * [B, Hkv, cap, 128]; cos/sin are [table_len, 128] bf16; batch <= 65535.
 * Replaces qk_norm_rope_cache (engine/kernels/fused.py:84-98) and tree_qk (tree.py:198-204). */
int qd_qk_norm_rope(const uint16_t *qkv, int64_t qkv_stride, const uint16_t *q_norm_w,
                    const uint16_t *k_norm_w, const uint16_t *cos, const uint16_t *sin,
                    int64_t table_len, const int64_t *pos, const int64_t *depth, int32_t mode,
                    uint16_t *q_out, uint16_t *k_cache, uint16_t *v_cache, int64_t batch,
                    int64_t T, int64_t n_q_heads, int64_t n_kv_heads, int64_t cap, float eps,
                    void *stream);

/* SwiGLU of a packed [rows, 2*inter] (gate | up): out = bf16(bf16(silu(g)) * u).
 * Replaces silu_mul (engine/kernels/fused.py:101-120). */
int qd_swiglu(const uint16_t *gu, int64_t gu_stride, uint16_t *out, int64_t out_stride,
              int64_t rows, int64_t inter, void *stream);

/* Decode projection out[m, n] = epi(sum_k xin[m, k] W[n, k]) for m < rows, n < n_out, fp32
 * accumulate; xin = RMSNorm(x; norm_w) when norm_w != NULL.  rows <= 2 run the vector-ALU
 * GEMV, more rows the MFMA kernels.  Workspace: rows*k*2 bytes for the normalised activations
 * when norm_w != NULL (required), then the split-K partials of the tiled kernel (optional: with
 * less than qd_linear_workspace_bytes, K is not split).
 * Replaces Gemv (engine/kernels/gemv.py:161-234) and FastGemm (fast.py:161-213); the split-K
 * partials play the role of the caller-owned partial buffers of gemv.py:189-208. */
int64_t qd_linear_workspace_bytes(int64_t rows, int64_t n_out, int64_t k, int32_t has_norm);
int qd_linear(const uint16_t *x, int64_t x_stride, const uint16_t *w, int64_t n_out, int64_t k,
              uint16_t *out, int64_t out_stride, int64_t rows, const uint16_t *norm_w, float eps,
              int32_t epilogue, const uint16_t *res, int64_t res_stride, void *workspace,
              int64_t workspace_bytes, void *stream);

/* LM head + greedy argmax: tok[m] = argmax_n bf16(RMSNorm(x[m]; norm_w) . W[n]) with the
 * lowest index on exact ties; pos_inc (may be NULL) is incremented once.  logits (may be
 * NULL) receives the fp32 logits before bf16 rounding, [rows, vocab].
 * Replaces LmHeadArgmax (engine/kernels/gemv.py:237-287) and FastLmHead (fast.py:439-465). */
int64_t qd_lm_head_workspace_bytes(int64_t rows, int64_t vocab, int64_t k);
int qd_lm_head_argmax(const uint16_t *x, int64_t x_stride, const uint16_t *w, int64_t vocab,
                      int64_t k, int64_t rows, const uint16_t *norm_w, float eps, int64_t *tok,
                      int64_t *pos_inc, float *logits, void *workspace, int64_t workspace_bytes,
                      void *stream);

/* Fused decode attention for one new token per sequence at device position pos[0]:
 * q/k RMSNorm + RoPE from the packed qkv rows, K/V written to slot pos, split-K GQA flash
 * decode over keys [0, pos], merge by the last split.  out is [batch, Hq, 128].
 * Replaces FastAttention (engine/kernels/fast.py:353-376) and, with the K/V write,
 * qk_norm_rope_cache + DecodeAttention (fused.py:84-98, decode_attn.py:89-119). */
int64_t qd_decode_attn_workspace_bytes(int64_t batch, int64_t n_q_heads, int64_t n_kv_heads,
                                       int64_t cap);
int qd_decode_attn(const uint16_t *qkv, int64_t qkv_stride, const uint16_t *q_norm_w,
                   const uint16_t *k_norm_w, const uint16_t *cos, const uint16_t *sin,
                   const int64_t *pos, uint16_t *k_cache, uint16_t *v_cache, int64_t batch,
                   int64_t n_q_heads, int64_t n_kv_heads, int64_t cap, float eps, uint16_t *out,
                   void *workspace, int64_t workspace_bytes, void *stream);

/* Block attention for T query tokens per sequence (q [B, T, Hq, 128], already normed and
 * rotated): keys < base[b] are visible to every token; block slot base[b] + j is visible to
 * token t iff bit j of anc[b*T + t] (anc != NULL, T <= 64) or j <= t (anc == NULL, causal).
 * out is [B, T, Hq, 128].  Replaces TreeAttention (engine/kernels/tree.py:166-195). */
int64_t qd_block_attn_workspace_bytes(int64_t batch, int64_t T, int64_t n_q_heads, int64_t cap);
int qd_block_attn(const uint16_t *q, const uint16_t *k_cache, const uint16_t *v_cache,
                  const int64_t *base, const uint64_t *anc, int64_t batch, int64_t T,
                  int64_t n_q_heads, int64_t n_kv_heads, int64_t cap, uint16_t *out,
                  void *workspace, int64_t workspace_bytes, void *stream);

/* KV compaction of accepted tree paths over all layers of k_all/v_all [L, B, Hkv, cap, 128]:
 * for 1 <= k < cnt[b]: slot base[b] + k <- slot base[b] + src[b*T + k].
 * Replaces compact (engine/kernels/tree.py:207-211). */
int qd_kv_compact(uint16_t *k_all, uint16_t *v_all, int64_t n_layers, int64_t batch,
                  int64_t n_kv_heads, int64_t cap, const int64_t *base, const int32_t *src,
                  const int32_t *cnt, int64_t T, void *stream);

/* Synthetic benchmark weights (no reference counterpart; the benchmark configs ask for
 * seeded random-init weights): out[j] = bf16 of the counter-based generator value at
 * element start + j of (seed, stream), scaled by `scale`. */
int qd_synth_bf16(uint16_t *out, int64_t count, uint64_t seed, uint64_t stream, uint64_t start,
                  float scale, void *stream_);
int qd_fill_bf16(uint16_t *out, int64_t count, uint16_t value, void *stream);

/* Read-stream probe (no reference counterpart; the benchmark's measuring stick): reads `bytes`
 * (a multiple of 16, buf 16-byte aligned) with non-temporal 16-byte loads from `grid`
 * workgroups of 256 threads and writes nothing (sink is never written for real data).  Timed
 * over the same bytes as a kernel, it gives the read rate one launch of that size can reach. */
int qd_read_probe(const void *buf, int64_t bytes, int32_t grid, uint32_t *sink, void *stream);

/* ------------------------------------------------------------------ whole steps */
/* Stacked, packed weights as the reference lays them out (engine/engine.py:250-282). */
typedef struct {
  int32_t n_layers, hidden, inter, vocab, n_q_heads, n_kv_heads, head_dim;
  float eps;
  const uint16_t *embed;      /* [vocab, hidden]; also the tied lm_head */
  const uint16_t *final_norm; /* [hidden] */
  const uint16_t *w_qkv;      /* [L, (Hq + 2 Hkv) * 128, hidden] = q | k | v */
  const uint16_t *w_o;        /* [L, hidden, Hq * 128] */
  const uint16_t *w_gu;       /* [L, 2 * inter, hidden] = gate | up */
  const uint16_t *w_down;     /* [L, hidden, inter] */
  const uint16_t *ln1;        /* [L, hidden] input_layernorm */
  const uint16_t *ln2;        /* [L, hidden] post_attention_layernorm */
  const uint16_t *q_norm;     /* [L, 128] */
  const uint16_t *k_norm;     /* [L, 128] */
  const uint16_t *lm_head;    /* [vocab, hidden] untied output projection, or NULL: the LM head
                                 reads embed (tie_word_embeddings, engine.py:246-247) */
} qd_weights;

/* One greedy decode step for `batch` sequences at the shared device position pos[0]. */
typedef struct {
  int32_t batch;
  int64_t cap;              /* KV capacity (slots) */
  uint16_t *k_cache;        /* [L, batch, Hkv, cap, 128] */
  uint16_t *v_cache;
  const uint16_t *cos;      /* [cap, 128] */
  const uint16_t *sin;
  int64_t *tok;             /* [batch] in: this step's token, out: the next greedy token */
  int64_t *pos;             /* [1] in: this token's position; incremented by the step */
  uint16_t *x;              /* [batch, hidden] residual stream */
  uint16_t *qkv;            /* [batch, (Hq + 2 Hkv) * 128] */
  uint16_t *attn;           /* [batch, Hq * 128] */
  uint16_t *act;            /* [batch, inter] */
  void *workspace;          /* qd_decode_workspace_bytes, zero-filled once */
  int64_t workspace_bytes;
} qd_decode_state;

/* Replaces the T5 decode step (engine/engine.py:463-477): embed, per layer qkv / attention /
 * o + residual / gate-up + SwiGLU / down + residual, final norm + LM head + argmax, pos += 1. */
int64_t qd_decode_workspace_bytes(const qd_weights *w, int64_t batch, int64_t cap);
int qd_decode_step(const qd_weights *w, const qd_decode_state *st, void *stream);

/* qd_decode_step without a caller workspace.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under hipGraph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  The step's split partials live in a file-scope device array
 * of QD_NOALLOC_SCRATCH_BYTES per GPU (held until the process ends); st->workspace and
 * st->workspace_bytes are ignored.  Same kernels and results as qd_decode_step (bit-identical).
 * Returns QD_ESCRATCH, before touching the device, when qd_decode_workspace_bytes(w, batch, cap)
 * exceeds the array (at Qwen3-4B's shape batch 32 fits up to cap 106496, batch 64 up to 40960).
 * A first call under hipGraph capture (relaxed mode) resolves the array's address there and
 * is supported.
 * The stream must belong to the current device.  Every call on one GPU shares that GPU's
 * array, whose contents the next call overwrites: calls that overlap on one GPU
 * (different streams, or host threads) race and must be serialised by the caller.  Allocates
 * nothing (no hipMalloc / hipFree, no allocating library call). */
#define QD_ESCRATCH (-4)
#define QD_NOALLOC_SCRATCH_BYTES (16 * 1024 * 1024)
int qd_decode_step_noalloc(const qd_weights *w, const qd_decode_state *st, void *stream);

/* The same step (batch == 1) as ONE persistent launch of one workgroup per CU that hands
 * activations between phases through hand-off words in the workspace instead of launch
 * boundaries.
 * Replaces the T6 tier (engine/kernels/mega.py:1-15, MegaStep; used at engine/engine.py:596-597).
 * Bit-identical to qd_decode_step at batch 1 (tokens, K/V, st->x = final residual; st->qkv,
 * st->attn and st->act are not written).  Needs a workspace of qd_mega_workspace_bytes (which
 * also covers qd_decode_step's), zero-filled before the first step and again before a step
 * with a different cap (the hand-off words move with the attention split plan); the 32-bit word at
 * byte qd_mega_ctl_offset of it is the step epoch and the next one the error word: 0 = ok,
 * 1 = a hand-off wait expired (the step's results are invalid), 2 = pos outside [0, cap)
 * (nothing written).  The error word stays set until the caller clears it.
 * qd_mega_supported is 1 when this device and model shape can run it (batch 1, Qwen3-4B
 * layer shape, >= 256 CUs); otherwise the entry points return QD_EARG / 0 / -1. */
int qd_mega_supported(const qd_weights *w, int64_t batch);
int64_t qd_mega_workspace_bytes(const qd_weights *w, int64_t batch, int64_t cap);
int64_t qd_mega_ctl_offset(const qd_weights *w, int64_t batch, int64_t cap);
int qd_mega_step(const qd_weights *w, const qd_decode_state *st, void *stream);

#define QD_LM_ALL 0
#define QD_LM_LAST 1
#define QD_LM_NONE 2

/* One forward of T tokens per sequence through all layers (tree verification, or a causal
 * chunk of the prompt), writing their K/V and the greedy token after each row. */
typedef struct {
  int32_t batch, T;
  int32_t causal;           /* 1: token t sees block slots <= t (prefill chunk); 0: anc mask */
  int32_t lm_mode;          /* QD_LM_ALL: every row (out_tok [batch*T]); QD_LM_LAST: token T-1
                               of each row (out_tok [batch]); QD_LM_NONE: K/V only */
  int64_t cap;
  uint16_t *k_cache, *v_cache;   /* [L, batch, Hkv, cap, 128] */
  const uint16_t *cos, *sin;     /* [cap, 128] */
  const int64_t *tokens;         /* [batch * T] */
  const int64_t *base;           /* [batch]: first block slot (= RoPE base) */
  const int64_t *depth;          /* [batch * T] tree depth (RoPE at base + depth); causal: NULL */
  const uint64_t *anc;           /* [batch * T] ancestor-or-self masks; causal: NULL */
  const int64_t *c_base;         /* optional KV compaction before the forward (NULL: none) */
  const int32_t *c_src;          /* [batch * T] */
  const int32_t *c_cnt;          /* [batch] */
  int64_t *out_tok;              /* see lm_mode (may be NULL with QD_LM_NONE) */
  uint16_t *x;                   /* [batch * T, hidden] */
  uint16_t *xn;                  /* [batch * T, hidden] */
  uint16_t *qkv;                 /* [batch * T, (Hq + 2 Hkv) * 128] */
  uint16_t *q;                   /* [batch * T, Hq * 128] */
  uint16_t *attn;                /* [batch * T, Hq * 128] */
  uint16_t *act;                 /* [batch * T, inter] */
  void *workspace;
  int64_t workspace_bytes;
} qd_block_state;

/* Replaces _verify_tree (engine/engine.py:445-461) and, as a causal chunk, the prompt
 * forward of _prefill (engine/engine.py:550-592).
 * Workspace: qd_block_workspace_bytes_lm() is what a step with this lm_mode and any T' <= T
 * needs (the LM head's partials for batch * T rows with QD_LM_ALL, for batch rows otherwise;
 * attention split partials only where the launch splits the keys, which does not grow with
 * cap; the projections' split-K partials); qd_block_workspace_bytes() is the QD_LM_ALL size,
 * enough for every mode.  Both depend on the current device's CU count (256 assumed when no
 * device is visible). */
int64_t qd_block_workspace_bytes(const qd_weights *w, int64_t batch, int64_t T, int64_t cap);
int64_t qd_block_workspace_bytes_lm(const qd_weights *w, int64_t batch, int64_t T, int64_t cap,
                                    int32_t lm_mode);
int qd_block_step(const qd_weights *w, const qd_block_state *st, void *stream);

/* Host-only plan query of the all-rows projection kernel (65..256 activation rows, the
 * tree-verification GEMMs): what qd_linear / qd_block_step launch for an M x K by N x K
 * product with epilogue `epi` (QD_EPI_NONE / RES / SWIGLU) and `part_floats` floats of room for
 * fp32 split-K partials (partials_only != 0: the block step's partial-summing consumers, which
 * launch nothing unless the plan splits).  Returns -1 when another kernel serves the shape, 0
 * when partials_only finds no split, 1 with out[8] = {rows per workgroup, block height in MFMA
 * tiles, activation tiles per wave, activation halves, K splits, K steps per split, grid, static
 * LDS bytes}; QD_EARG for bad arguments.  No reference counterpart: the CPU tests use it to
 * check every plan's grid coverage and store bounds without a GPU. */
int qd_gemm_rows_plan(int64_t M, int64_t N, int64_t K, int32_t epi, int64_t part_floats,
                      int32_t partials_only, int64_t *out);

/* hipGraph capture of whatever is enqueued on `stream` between begin and end (replaces the
 * torch.cuda.CUDAGraph capture of the decode step, engine/engine.py:685-713). */
int qd_graph_begin(void *stream);
int qd_graph_end(void *stream, void **exec_out);
int qd_graph_launch(void *exec, void *stream);
int qd_graph_destroy(void *exec);

#ifdef __cplusplus
}
#endif
#endif /* QDECODE_H */
