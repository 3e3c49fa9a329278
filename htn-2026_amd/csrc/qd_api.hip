// extern "C" entry points (include/qdecode.h): argument validation, workspace layout and the
// whole-step launch sequences.  Kernels live in elementwise.hip, gemv.hip, gemm.hip, attn.hip.
#include "../../include/qdecode.h"

#include <string.h>

#include <mutex>

#include "qd_launch.h"

namespace {

inline hipStream_t S(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline int launched() { return qd_err(hipGetLastError()); }

inline int64_t align256(int64_t v) { return (v + 255) / 256 * 256; }

// Carves consecutive 256-byte-aligned regions out of a workspace.
struct Carver {
  char* base;
  int64_t off = 0;
  explicit Carver(void* p) : base(static_cast<char*>(p)) {}
  template <typename T>
  T* take(int64_t count) {
    T* p = base ? reinterpret_cast<T*>(base + off) : nullptr;
    off += align256(count * (int64_t)sizeof(T));
    return p;
  }
};

// Every workspace region is fully written before it is read within one call: workspaces need
// no initialisation and may be reused with other shapes.
struct AttnWs {
  float* acc;
  float* ml;
};
AttnWs carve_decode_attn(Carver& c, int64_t B, int64_t Hq, int64_t Hkv, int64_t splits) {
  (void)Hkv;
  AttnWs a;
  a.acc = c.take<float>(B * Hq * splits * 128);
  a.ml = c.take<float>(B * Hq * splits * 2);
  return a;
}

struct LmWs {
  float* val;
  int32_t* idx;
  bf16_t* xn;
  int64_t parts;
};
LmWs carve_lm(Carver& c, int64_t rows, int64_t V, int64_t K) {
  LmWs l;
  const bool vec = gemv_supported(rows, K) && K == 2560;
  l.parts = vec ? lm_vec_parts(V) : gemm_argmax_parts(V);
  // room for the partials of whichever LM-head kernel serves these rows: the vector path, the
  // 16-row tiles, or one per workgroup of the skinny kernel (at most min(V, CU count))
  int64_t cap_parts = gemm_argmax_parts(V);
  if (lm_vec_parts(V) > cap_parts) cap_parts = lm_vec_parts(V);
  if ((V < 1024 ? V : 1024) > cap_parts) cap_parts = V < 1024 ? V : 1024;
  l.val = c.take<float>(rows * cap_parts);
  l.idx = c.take<int32_t>(rows * cap_parts);
  l.xn = vec ? nullptr : c.take<bf16_t>(rows * K);
  return l;
}

// LM head + argmax over `rows` rows of x (row stride x_stride)
int lm_head(const bf16_t* x, int64_t x_stride, const bf16_t* w, int64_t V, int64_t K,
            int64_t rows, const bf16_t* norm_w, float eps, int64_t* tok, int64_t* pos_inc,
            float* logits, const LmWs& l, hipStream_t s) {
  if (gemv_supported(rows, K) && K == 2560) {
    launch_lm_vec(x, x_stride, w, V, K, norm_w, eps, rows, l.val, l.idx, tok, pos_inc, logits, s);
  } else {
    launch_add_rmsnorm(nullptr, x, norm_w, nullptr, l.xn, rows, K, x_stride, K, eps, s);
    const int64_t parts = launch_gemm(l.xn, K, rows, w, V, K, nullptr, 0, nullptr, 0, EPI_ARGMAX,
                                      l.val, l.idx, logits, s);
    launch_argmax_reduce(l.val, l.idx, parts, rows, tok, pos_inc, s);
  }
  return launched();
}

// LM head + argmax over `rows` already-normalised rows of xn (row stride xs; the MFMA path)
int lm_head_normed_strided(const bf16_t* xn, int64_t xs, const bf16_t* w, int64_t V, int64_t K,
                           int64_t rows, int64_t* tok, const LmWs& l, hipStream_t s,
                           int64_t* pos_inc = nullptr) {
  const int64_t parts = launch_gemm(xn, xs, rows, w, V, K, nullptr, 0, nullptr, 0, EPI_ARGMAX,
                                    l.val, l.idx, nullptr, s);
  launch_argmax_reduce(l.val, l.idx, parts, rows, tok, pos_inc, s);
  return launched();
}
int lm_head_normed(const bf16_t* xn, const bf16_t* w, int64_t V, int64_t K, int64_t rows,
                   int64_t* tok, int64_t* pos_inc, const LmWs& l, hipStream_t s) {
  return lm_head_normed_strided(xn, K, w, V, K, rows, tok, l, s, pos_inc);
}

bool weights_ok(const qd_weights* w) {
  if (!w || !w->embed || !w->final_norm || !w->w_qkv || !w->w_o || !w->w_gu || !w->w_down ||
      !w->ln1 || !w->ln2 || !w->q_norm || !w->k_norm)
    return false;
  if (w->n_layers <= 0 || w->head_dim != 128 || w->n_kv_heads <= 0 ||
      w->n_q_heads != 4 * w->n_kv_heads || w->vocab <= 0)
    return false;
  if (w->hidden % 128 || w->inter % 128 || (w->n_q_heads * 128) % 128) return false;
  return true;
}

// Batched decode (3..32 rows) on the skinny kernel: K splits of the qkv, o and down projections
// (fewer activation bytes re-read per workgroup; the qkv partials are summed by the attention
// prologue, the o / down partials by the following residual-add + RMSNorm launch); gate/up runs
// unsplit (its SwiGLU epilogue needs whole sums).  Measured per projection at 32 rows on MI355X.
#ifndef QD_SK_SPLIT_QKV
#define QD_SK_SPLIT_QKV 2
#endif
#ifndef QD_SK_SPLIT_O
#define QD_SK_SPLIT_O 4
#endif
#ifndef QD_SK_SPLIT_DOWN
#define QD_SK_SPLIT_DOWN 4
#endif
constexpr int SK_SPLIT_QKV = QD_SK_SPLIT_QKV, SK_SPLIT_O = QD_SK_SPLIT_O,
              SK_SPLIT_DOWN = QD_SK_SPLIT_DOWN;

// Whether a B-row step runs the skinny path: shapes only (the workspace size depends on it), and
// with a state, also the alignment of the step's own buffers (checked before anything launches)
bool skinny_step_ok(const qd_weights* w, int64_t B, const qd_decode_state* st = nullptr) {
  if (B < 3 || B > 32) return false;
  const int64_t H = w->hidden, I = w->inter, QD = (int64_t)w->n_q_heads * 128;
  const int64_t NQKV = (int64_t)(w->n_q_heads + 2 * w->n_kv_heads) * 128;
  const void* a = reinterpret_cast<const void*>(256);    // workspace regions: 256-aligned
  const void* attn = st ? st->attn : a;
  const void* act = st ? st->act : a;
  return skinny_ok(B, NQKV, H, EPI_NONE, SK_SPLIT_QKV, a, H, st ? w->w_qkv : a, NQKV) &&
         skinny_ok(B, H, QD, EPI_NONE, SK_SPLIT_O, attn, QD, st ? w->w_o : a, H) &&
         skinny_ok(B, I, H, EPI_SWIGLU, 1, a, H, st ? w->w_gu : a, I) &&
         skinny_ok(B, H, I, EPI_NONE, SK_SPLIT_DOWN, act, I, st ? w->w_down : a, H) &&
         (!st || (reinterpret_cast<uintptr_t>(st->qkv) % 8 == 0 &&
                  reinterpret_cast<uintptr_t>(st->act) % 8 == 0));
}

inline int64_t qkv_width(const qd_weights* w) { return (int64_t)(w->n_q_heads + 2 * w->n_kv_heads) * 128; }

// one partials buffer, reused: each projection's partials are consumed before the next
// projection writes its own
int64_t skinny_step_part_floats(const qd_weights* w, int64_t B) {
  const int S = SK_SPLIT_O > SK_SPLIT_DOWN ? SK_SPLIT_O : SK_SPLIT_DOWN;
  const int64_t od = skinny_part_floats(B, w->hidden, S);
  const int64_t q = skinny_part_floats(B, qkv_width(w), SK_SPLIT_QKV);
  return od > q ? od : q;
}

// the LM head's weight: the untied output projection when given, else the tied embedding
inline const bf16_t* lm_weight(const qd_weights* w) { return w->lm_head ? w->lm_head : w->embed; }


}  // namespace

extern "C" {

const char* qd_version(void) { return "qdecode 0.1 gfx950"; }

int qd_embed_gather(const int64_t* ids, const uint16_t* table, uint16_t* out, int64_t n_ids,
                    int64_t vocab, int64_t hidden, int64_t out_stride, void* stream) {
  if (n_ids < 0 || vocab <= 0 || hidden <= 0 || hidden % 8 || out_stride < hidden || out_stride % 8)
    return QD_EARG;
  if (n_ids == 0) return QD_OK;
  if (!ids || !table || !out) return QD_EARG;
  launch_embed(ids, table, out, n_ids, vocab, hidden, out_stride, S(stream));
  return launched();
}

int qd_add_rmsnorm(const uint16_t* x, const uint16_t* residual, const uint16_t* w,
                   uint16_t* res_out, uint16_t* y, int64_t rows, int64_t hidden, int64_t in_stride,
                   int64_t y_stride, float eps, void* stream) {
  if (rows < 0 || hidden <= 0 || hidden % 8 || in_stride < hidden || in_stride % 8 ||
      y_stride < hidden || y_stride % 8 || !(eps >= 0.f))
    return QD_EARG;
  if (rows == 0) return QD_OK;
  if (!residual || !w || !y || (x && !res_out)) return QD_EARG;
  launch_add_rmsnorm(x, residual, w, res_out, y, rows, hidden, in_stride, y_stride, eps, S(stream));
  return launched();
}

int qd_qk_norm_rope(const uint16_t* qkv, int64_t qkv_stride, const uint16_t* q_norm_w,
                    const uint16_t* k_norm_w, const uint16_t* cos, const uint16_t* sin,
                    int64_t table_len, const int64_t* pos, const int64_t* depth, int32_t mode,
                    uint16_t* q_out, uint16_t* k_cache, uint16_t* v_cache, int64_t batch,
                    int64_t T, int64_t n_q_heads, int64_t n_kv_heads, int64_t cap, float eps,
                    void* stream) {
  if (batch < 0 || T < 0 || n_q_heads <= 0 || n_kv_heads <= 0 || cap <= 0 || table_len <= 0)
    return QD_EARG;
  if (batch > 65535) return QD_EARG;           // one grid row per sequence
  if (qkv_stride < (n_q_heads + 2 * n_kv_heads) * 128) return QD_EARG;
  if (mode < QD_POS_T || mode > QD_POS_TREE) return QD_EARG;
  if (batch * T == 0) return QD_OK;
  if (!qkv || !q_norm_w || !k_norm_w || !cos || !sin || !q_out || !k_cache || !v_cache)
    return QD_EARG;
  if (mode != QD_POS_T && !pos) return QD_EARG;
  if (mode == QD_POS_TREE && !depth) return QD_EARG;
  launch_qk_norm_rope(qkv, qkv_stride, q_norm_w, k_norm_w, cos, sin, table_len, pos, depth, mode,
                      q_out, k_cache, v_cache, batch, T, (int)n_q_heads, (int)n_kv_heads, cap, eps,
                      S(stream));
  return launched();
}

int qd_swiglu(const uint16_t* gu, int64_t gu_stride, uint16_t* out, int64_t out_stride,
              int64_t rows, int64_t inter, void* stream) {
  if (rows < 0 || inter <= 0 || inter % 8 || gu_stride < 2 * inter || gu_stride % 8 ||
      out_stride < inter || out_stride % 8)
    return QD_EARG;
  if (rows == 0) return QD_OK;
  if (!gu || !out) return QD_EARG;
  launch_swiglu(gu, gu_stride, out, out_stride, rows, inter, S(stream));
  return launched();
}

int64_t qd_linear_workspace_bytes(int64_t rows, int64_t n_out, int64_t k, int32_t has_norm) {
  if (rows <= 0 || n_out <= 0 || k <= 0) return 0;
  if (gemv_supported(rows, k)) return 0;
  const int64_t xn = has_norm ? align256(rows * k * 2) : 0;
  return xn + align256(gemm_tile_ws_floats(rows, n_out, k, QD_EPI_RES) * 4);
}

int qd_linear(const uint16_t* x, int64_t x_stride, const uint16_t* w, int64_t n_out, int64_t k,
              uint16_t* out, int64_t out_stride, int64_t rows, const uint16_t* norm_w, float eps,
              int32_t epilogue, const uint16_t* res, int64_t res_stride, void* workspace,
              int64_t workspace_bytes, void* stream) {
  if (rows < 0 || n_out <= 0 || k <= 0 || k % 128 || x_stride < k || x_stride % 8) return QD_EARG;
  if (epilogue < QD_EPI_NONE || epilogue > QD_EPI_SWIGLU) return QD_EARG;
  if (rows == 0) return QD_OK;
  if (!x || !w || !out) return QD_EARG;
  if (epilogue == QD_EPI_RES && !res) return QD_EARG;
  hipStream_t s = S(stream);
  if (gemv_supported(rows, k)) {
    launch_gemv(x, x_stride, w, n_out, k, out, out_stride, res, res_stride, norm_w, eps, epilogue,
                rows, s);
    return launched();
  }
  const bf16_t* xin = x;
  int64_t xin_stride = x_stride;
  if (norm_w) {
    const int64_t need = align256(rows * k * 2);
    if (!workspace || workspace_bytes < need) return QD_EWS;
    bf16_t* xn = static_cast<bf16_t*>(workspace);
    launch_add_rmsnorm(nullptr, x, norm_w, nullptr, xn, rows, k, x_stride, k, eps, s);
    xin = xn;
    xin_stride = k;
  }
  // the rest of the workspace (if any) takes split-K partials; with too little, K is not split
  const int64_t used = norm_w ? align256(rows * k * 2) : 0;
  float* part = workspace && workspace_bytes > used
                    ? reinterpret_cast<float*>(static_cast<char*>(workspace) + used) : nullptr;
  const int64_t part_floats = part ? (workspace_bytes - used) / 4 : 0;
  launch_gemm(xin, xin_stride, rows, w, n_out, k, out, out_stride, res, res_stride, epilogue,
              nullptr, nullptr, nullptr, s, part, part_floats);
  return launched();
}

int64_t qd_lm_head_workspace_bytes(int64_t rows, int64_t vocab, int64_t k) {
  if (rows <= 0 || vocab <= 0 || k <= 0) return 0;
  Carver c(nullptr);
  carve_lm(c, rows, vocab, k);
  return c.off;
}

int qd_lm_head_argmax(const uint16_t* x, int64_t x_stride, const uint16_t* w, int64_t vocab,
                      int64_t k, int64_t rows, const uint16_t* norm_w, float eps, int64_t* tok,
                      int64_t* pos_inc, float* logits, void* workspace, int64_t workspace_bytes,
                      void* stream) {
  if (rows < 0 || vocab <= 0 || vocab >= 0x7FFFFFFF || k <= 0 || k % 128 || x_stride < k ||
      x_stride % 8)
    return QD_EARG;
  if (rows == 0) return QD_OK;
  if (!x || !w || !norm_w || !tok) return QD_EARG;
  if (!workspace || workspace_bytes < qd_lm_head_workspace_bytes(rows, vocab, k)) return QD_EWS;
  Carver c(workspace);
  LmWs l = carve_lm(c, rows, vocab, k);
  return lm_head(x, x_stride, w, vocab, k, rows, norm_w, eps, tok, pos_inc, logits, l, S(stream));
}

int64_t qd_decode_attn_workspace_bytes(int64_t batch, int64_t n_q_heads, int64_t n_kv_heads,
                                       int64_t cap) {
  if (batch <= 0 || n_kv_heads <= 0 || cap <= 0) return 0;
  Carver c(nullptr);
  carve_decode_attn(c, batch, n_q_heads, n_kv_heads, decode_attn_splits(batch, (int)n_kv_heads, cap));
  return c.off;
}

int qd_decode_attn(const uint16_t* qkv, int64_t qkv_stride, const uint16_t* q_norm_w,
                   const uint16_t* k_norm_w, const uint16_t* cos, const uint16_t* sin,
                   const int64_t* pos, uint16_t* k_cache, uint16_t* v_cache, int64_t batch,
                   int64_t n_q_heads, int64_t n_kv_heads, int64_t cap, float eps, uint16_t* out,
                   void* workspace, int64_t workspace_bytes, void* stream) {
  if (batch < 0 || n_kv_heads <= 0 || n_q_heads != 4 * n_kv_heads || cap <= 0 ||
      qkv_stride < (n_q_heads + 2 * n_kv_heads) * 128)
    return QD_EARG;
  if (batch == 0) return QD_OK;
  if (!qkv || !q_norm_w || !k_norm_w || !cos || !sin || !pos || !k_cache || !v_cache || !out)
    return QD_EARG;
  if (!workspace || workspace_bytes < qd_decode_attn_workspace_bytes(batch, n_q_heads, n_kv_heads, cap))
    return QD_EWS;
  const int64_t splits = decode_attn_splits(batch, (int)n_kv_heads, cap);
  Carver c(workspace);
  AttnWs a = carve_decode_attn(c, batch, n_q_heads, n_kv_heads, splits);
  launch_decode_attn(qkv, qkv_stride, q_norm_w, k_norm_w, cos, sin, pos, k_cache, v_cache, batch,
                     (int)n_q_heads, (int)n_kv_heads, cap, splits, eps, a.acc, a.ml,
                     out, false, S(stream));
  return launched();
}

int64_t qd_block_attn_workspace_bytes(int64_t batch, int64_t T, int64_t n_q_heads, int64_t cap) {
  if (batch <= 0 || T <= 0 || cap <= 0 || n_q_heads < 4) return 0;
  const int64_t rows = block_attn_partial_rows(batch, T, (int)n_q_heads, (int)(n_q_heads / 4), cap);
  return align256(rows * 128 * 4) + align256(rows * 2 * 4);
}

int qd_block_attn(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                  const int64_t* base, const uint64_t* anc, int64_t batch, int64_t T,
                  int64_t n_q_heads, int64_t n_kv_heads, int64_t cap, uint16_t* out,
                  void* workspace, int64_t workspace_bytes, void* stream) {
  if (batch < 0 || T < 0 || n_kv_heads <= 0 || n_q_heads != 4 * n_kv_heads || cap <= 0) return QD_EARG;
  if (anc && T > 64) return QD_EARG;
  if (block_attn_splits(cap) > 1024) return QD_EARG;  // the merge holds <= 1024 split weights
  if (batch * T == 0) return QD_OK;
  if (!q || !k_cache || !v_cache || !base || !out) return QD_EARG;
  if (!workspace || workspace_bytes < qd_block_attn_workspace_bytes(batch, T, n_q_heads, cap))
    return QD_EWS;
  Carver c(workspace);
  const int64_t rows = block_attn_partial_rows(batch, T, (int)n_q_heads, (int)n_kv_heads, cap);
  float* acc = c.take<float>(rows * 128);
  float* ml = c.take<float>(rows * 2);
  launch_block_attn(q, k_cache, v_cache, base, anc, batch, T, (int)n_q_heads, (int)n_kv_heads, cap,
                    acc, ml, out, S(stream));
  return launched();
}

int qd_kv_compact(uint16_t* k_all, uint16_t* v_all, int64_t n_layers, int64_t batch,
                  int64_t n_kv_heads, int64_t cap, const int64_t* base, const int32_t* src,
                  const int32_t* cnt, int64_t T, void* stream) {
  if (n_layers < 0 || batch < 0 || n_kv_heads <= 0 || cap <= 0 || T <= 0) return QD_EARG;
  if (n_layers * batch == 0) return QD_OK;
  if (!k_all || !v_all || !base || !src || !cnt) return QD_EARG;
  launch_kv_compact(k_all, v_all, n_layers, batch, (int)n_kv_heads, cap, base, src, cnt, T, S(stream));
  return launched();
}

int qd_synth_bf16(uint16_t* out, int64_t count, uint64_t seed, uint64_t stream, uint64_t start,
                  float scale, void* stream_) {
  if (count < 0 || seed > 0xFFFFFFFFull || stream > 0xFFFFFFFFull) return QD_EARG;
  if (count == 0) return QD_OK;
  if (!out || (reinterpret_cast<uintptr_t>(out) & 15)) return QD_EARG;
  launch_synth(out, count, seed, stream, start, scale, S(stream_));
  return launched();
}

int qd_fill_bf16(uint16_t* out, int64_t count, uint16_t value, void* stream) {
  if (count < 0) return QD_EARG;
  if (count == 0) return QD_OK;
  if (!out) return QD_EARG;
  launch_fill(out, count, value, S(stream));
  return launched();
}

int qd_read_probe(const void* buf, int64_t bytes, int32_t grid, uint32_t* sink, void* stream) {
  if (bytes < 0 || (bytes & 15) || grid < 1 || grid > 65536 || !sink) return QD_EARG;
  if (bytes == 0) return QD_OK;
  if (!buf || (reinterpret_cast<uintptr_t>(buf) & 15)) return QD_EARG;
  launch_read_probe(buf, bytes, grid, sink, S(stream));
  return launched();
}

// ------------------------------------------------------------------ decode step
int64_t qd_decode_workspace_bytes(const qd_weights* w, int64_t batch, int64_t cap) {
  if (!w || batch <= 0 || cap <= 0) return 0;
  Carver c(nullptr);
  carve_decode_attn(c, batch, w->n_q_heads, w->n_kv_heads, decode_attn_splits(batch, w->n_kv_heads, cap));
  carve_lm(c, batch, w->vocab, w->hidden);
  c.take<bf16_t>(batch * (int64_t)w->hidden);  // normalised activations (MFMA path)
  c.take<bf16_t>(256);                         // this step's RoPE row
  if (skinny_step_ok(w, batch)) c.take<float>(skinny_step_part_floats(w, batch));
  return c.off;
}

int qd_decode_step(const qd_weights* w, const qd_decode_state* st, void* stream) {
  if (!weights_ok(w) || !st) return QD_EARG;
  const int64_t B = st->batch, cap = st->cap, H = w->hidden, I = w->inter, V = w->vocab;
  const int Hq = w->n_q_heads, Hkv = w->n_kv_heads;
  if (B <= 0 || cap <= 0 || !st->k_cache || !st->v_cache || !st->cos || !st->sin || !st->tok ||
      !st->pos || !st->x || !st->qkv || !st->attn || !st->act)
    return QD_EARG;
  if (!st->workspace || st->workspace_bytes < qd_decode_workspace_bytes(w, B, cap)) return QD_EWS;
  hipStream_t s = S(stream);
  const int64_t splits = decode_attn_splits(B, Hkv, cap);
  Carver c(st->workspace);
  AttnWs aw = carve_decode_attn(c, B, Hq, Hkv, splits);
  LmWs lw = carve_lm(c, B, V, H);
  bf16_t* xn = c.take<bf16_t>(B * H);
  bf16_t* rope_row = c.take<bf16_t>(256);
  const int64_t NQKV = qkv_width(w), QD = (int64_t)Hq * 128;
  const int64_t layer_kv = B * Hkv * cap * 128;
  const bool vec_h = gemv_supported(B, H), vec_q = gemv_supported(B, QD), vec_i = gemv_supported(B, I);

  launch_embed_rope(st->tok, w->embed, st->x, B, V, H, H, st->cos, st->sin, st->pos, cap, rope_row, s);
  if (skinny_step_ok(w, B)) {
    if (!skinny_step_ok(w, B, st)) return QD_EARG;       // misaligned step buffers
    // 3..32 rows: skinny GEMMs; the o / down K-split partials are folded into the residual by
    // the next RMSNorm launch (r' = bf16(x + bf16(sum of partials)), the EPI_RES rounding)
    float* part = c.take<float>(skinny_step_part_floats(w, B));
    launch_add_rmsnorm(nullptr, st->x, w->ln1, nullptr, xn, B, H, H, H, w->eps, s);
    for (int64_t l = 0; l < w->n_layers; ++l) {
      if (l > 0)
        launch_part_add_rmsnorm(part, SK_SPLIT_DOWN, B, st->x, w->ln1 + l * H, xn, H, w->eps, s);
      if (SK_SPLIT_QKV > 1) {
        launch_gemm_skinny(xn, H, B, w->w_qkv + l * NQKV * H, NQKV, H, EPI_NONE, SK_SPLIT_QKV,
                           nullptr, 0, nullptr, 0, part, s);
        launch_decode_attn_part(part, SK_SPLIT_QKV, w->q_norm + l * 128, w->k_norm + l * 128,
                                rope_row, rope_row + 128, st->pos, st->k_cache + l * layer_kv,
                                st->v_cache + l * layer_kv, B, Hq, Hkv, cap, splits, w->eps,
                                aw.acc, aw.ml, st->attn, true, s);
      } else {
        launch_gemm_skinny(xn, H, B, w->w_qkv + l * NQKV * H, NQKV, H, EPI_NONE, 1, st->qkv,
                           NQKV, nullptr, 0, nullptr, s);
        launch_decode_attn(st->qkv, NQKV, w->q_norm + l * 128, w->k_norm + l * 128, rope_row,
                           rope_row + 128, st->pos, st->k_cache + l * layer_kv,
                           st->v_cache + l * layer_kv, B, Hq, Hkv, cap, splits, w->eps, aw.acc,
                           aw.ml, st->attn, true, s);
      }
      launch_gemm_skinny(st->attn, QD, B, w->w_o + l * H * QD, H, QD, EPI_NONE, SK_SPLIT_O,
                         nullptr, 0, nullptr, 0, part, s);
      launch_part_add_rmsnorm(part, SK_SPLIT_O, B, st->x, w->ln2 + l * H, xn, H, w->eps, s);
      launch_gemm_skinny(xn, H, B, w->w_gu + l * 2 * I * H, I, H, EPI_SWIGLU, 1, st->act, I,
                         nullptr, 0, nullptr, s);
      launch_gemm_skinny(st->act, I, B, w->w_down + l * H * I, H, I, EPI_NONE, SK_SPLIT_DOWN,
                         nullptr, 0, nullptr, 0, part, s);
    }
    launch_part_add_rmsnorm(part, SK_SPLIT_DOWN, B, st->x, w->final_norm, lw.xn, H, w->eps, s);
    return lm_head_normed(lw.xn, lm_weight(w), V, H, B, st->tok, st->pos, lw, s);
  }
  for (int64_t l = 0; l < w->n_layers; ++l) {
    const bf16_t* wqkv = w->w_qkv + l * NQKV * H;
    const bf16_t* wo = w->w_o + l * H * QD;
    const bf16_t* wgu = w->w_gu + l * 2 * I * H;
    const bf16_t* wd = w->w_down + l * H * I;
    const bf16_t* ln1 = w->ln1 + l * H;
    const bf16_t* ln2 = w->ln2 + l * H;
    // qkv = RMSNorm(x; ln1) . Wqkv
    if (vec_h) {
      launch_gemv(st->x, H, wqkv, NQKV, H, st->qkv, NQKV, nullptr, 0, ln1, w->eps, EPI_NONE, B, s);
    } else {
      launch_add_rmsnorm(nullptr, st->x, ln1, nullptr, xn, B, H, H, H, w->eps, s);
      launch_gemm(xn, H, B, wqkv, NQKV, H, st->qkv, NQKV, nullptr, 0, EPI_NONE, nullptr, nullptr, nullptr, s);
    }
    // attention (q/k norm + RoPE + KV write + split-K + merge)
    launch_decode_attn(st->qkv, NQKV, w->q_norm + l * 128, w->k_norm + l * 128, rope_row,
                       rope_row + 128, st->pos, st->k_cache + l * layer_kv,
                       st->v_cache + l * layer_kv, B, Hq, Hkv, cap, splits, w->eps, aw.acc, aw.ml,
                       st->attn, true, s);
    // x = x + attn . Wo
    if (vec_q)
      launch_gemv(st->attn, QD, wo, H, QD, st->x, H, st->x, H, nullptr, 0.f, EPI_RES, B, s);
    else
      launch_gemm(st->attn, QD, B, wo, H, QD, st->x, H, st->x, H, EPI_RES, nullptr, nullptr, nullptr, s);
    // act = SwiGLU(RMSNorm(x; ln2) . Wgu)
    if (vec_h) {
      launch_gemv(st->x, H, wgu, I, H, st->act, I, nullptr, 0, ln2, w->eps, EPI_SWIGLU, B, s);
    } else {
      launch_add_rmsnorm(nullptr, st->x, ln2, nullptr, xn, B, H, H, H, w->eps, s);
      launch_gemm(xn, H, B, wgu, I, H, st->act, I, nullptr, 0, EPI_SWIGLU, nullptr, nullptr, nullptr, s);
    }
    // x = x + act . Wdown
    if (vec_i)
      launch_gemv(st->act, I, wd, H, I, st->x, H, st->x, H, nullptr, 0.f, EPI_RES, B, s);
    else
      launch_gemm(st->act, I, B, wd, H, I, st->x, H, st->x, H, EPI_RES, nullptr, nullptr, nullptr, s);
  }
  return lm_head(st->x, H, lm_weight(w), V, H, B, w->final_norm, w->eps, st->tok, st->pos, nullptr, lw, s);
}

}  // extern "C"

// ------------------------------------------------------------------ decode step, no allocation
// The split partials of qd_decode_step_noalloc.  In host code `scratch` names a host-side
// stand-in, not device memory: only the address hipGetSymbolAddress returns (per device) may
// reach a kernel or a copy.  qd_decode_step's workspace is written before it is read within a
// step, so the array needs no clearing between calls.
static __device__ __align__(256) unsigned char scratch[QD_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices] = {};   // device address of `scratch` per device, once resolved

// Device address of `scratch` on the current device, resolved once per device (the module's
// copy of the array is per device, at its own address).
int scratch_on_current_device(hipStream_t stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return qd_err(e);
  if (dev < 0 || dev >= kMaxDevices) return QD_EARG;
  if (stream) {
    hipDevice_t sdev = -1;
    e = hipStreamGetDevice(stream, &sdev);
    if (e != hipSuccess) return qd_err(e);
    if (sdev != dev) return QD_EARG;   // the array resolved here would belong to another GPU
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return e != hipSuccess ? qd_err(e) : QD_ESTATE;
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return QD_OK;
}
}  // namespace

extern "C" {

int qd_decode_step_noalloc(const qd_weights* w, const qd_decode_state* st, void* stream) {
  if (!weights_ok(w) || !st || st->batch <= 0 || st->cap <= 0) return QD_EARG;
  const int64_t need = qd_decode_workspace_bytes(w, st->batch, st->cap);
  if (need <= 0) return QD_EARG;
  if (need > (int64_t)QD_NOALLOC_SCRATCH_BYTES) return QD_ESCRATCH;
  void* ptr = nullptr;
  const int rc = scratch_on_current_device(S(stream), &ptr);
  if (rc != QD_OK) return rc;
  qd_decode_state s2 = *st;
  s2.workspace = ptr;
  s2.workspace_bytes = QD_NOALLOC_SCRATCH_BYTES;
  return qd_decode_step(w, &s2, stream);
}


// ------------------------------------------------------------------ persistent decode step
// Workspace: qd_decode_step's region, then (256-byte aligned) the control block {epoch, error}
// and the hand-off words of the persistent kernel.
static int64_t mega_ctl_off(const qd_weights* w, int64_t batch, int64_t cap) {
  return (qd_decode_workspace_bytes(w, batch, cap) + 255) / 256 * 256;
}

static bool mega_ok(const qd_weights* w, int64_t batch) {
  return w && batch == 1 && w->hidden % 512 == 0 &&
         mega_shape_ok(w->hidden, w->inter, w->n_q_heads, w->n_kv_heads, w->head_dim) &&
         mega_grid() > 0;
}

int qd_mega_supported(const qd_weights* w, int64_t batch) {
  return weights_ok(w) && mega_ok(w, batch) ? 1 : 0;
}

int64_t qd_mega_workspace_bytes(const qd_weights* w, int64_t batch, int64_t cap) {
  if (!weights_ok(w) || cap <= 0 || !mega_ok(w, batch)) return 0;
  return mega_ctl_off(w, batch, cap) + 256 + mega_ll_bytes(w->n_layers, mega_splits(cap), mega_grid());
}

int64_t qd_mega_ctl_offset(const qd_weights* w, int64_t batch, int64_t cap) {
  if (!weights_ok(w) || cap <= 0 || !mega_ok(w, batch)) return -1;
  return mega_ctl_off(w, batch, cap);
}

int qd_mega_step(const qd_weights* w, const qd_decode_state* st, void* stream) {
  if (!weights_ok(w) || !st || !mega_ok(w, st->batch)) return QD_EARG;
  if (st->cap <= 0 || !st->k_cache || !st->v_cache || !st->cos || !st->sin || !st->tok ||
      !st->pos || !st->x)
    return QD_EARG;
  const int64_t need = qd_mega_workspace_bytes(w, st->batch, st->cap);
  if (!st->workspace || need <= 0 || st->workspace_bytes < need) return QD_EWS;
  char* ws = static_cast<char*>(st->workspace);
  const int64_t off = mega_ctl_off(w, st->batch, st->cap);
  MegaLaunch m;
  m.embed = w->embed; m.lm_head = lm_weight(w); m.final_norm = w->final_norm; m.w_qkv = w->w_qkv; m.w_o = w->w_o;
  m.w_gu = w->w_gu; m.w_down = w->w_down; m.ln1 = w->ln1; m.ln2 = w->ln2;
  m.q_norm = w->q_norm; m.k_norm = w->k_norm; m.cos = st->cos; m.sin = st->sin;
  m.k_cache = st->k_cache; m.v_cache = st->v_cache; m.tok = st->tok; m.pos = st->pos;
  m.x_out = st->x; m.ctl = reinterpret_cast<uint32_t*>(ws + off);
  m.ll = reinterpret_cast<uint32_t*>(ws + off + 256);
  m.cap = st->cap; m.vocab = w->vocab; m.L = w->n_layers; m.eps = w->eps;
  const hipError_t e = launch_mega_step(m, S(stream));
  return e == hipSuccess ? QD_OK : (int)e;
}

// ------------------------------------------------------------------ block (tree / prefill chunk)
// split-K partials of the block step's projections (the largest of qkv, o, down)
static int64_t block_part_floats(const qd_weights* w, int64_t M) {
  const int64_t H = w->hidden, QD = (int64_t)w->n_q_heads * 128;
  int64_t f = gemm_tile_ws_floats(M, qkv_width(w), H, EPI_NONE);
  const int64_t o = gemm_tile_ws_floats(M, H, QD, EPI_RES);
  const int64_t d = gemm_tile_ws_floats(M, H, w->inter, EPI_RES);
  if (o > f) f = o;
  if (d > f) f = d;
  return f;
}

int64_t qd_block_workspace_bytes_lm(const qd_weights* w, int64_t batch, int64_t T, int64_t cap,
                                    int32_t lm_mode) {
  if (!w || batch <= 0 || T <= 0 || cap <= 0 || lm_mode < QD_LM_ALL || lm_mode > QD_LM_NONE)
    return 0;
  // LM-head region first: partials for every row (QD_LM_ALL) or the last row per sequence
  Carver c(nullptr);
  carve_lm(c, lm_mode == QD_LM_ALL ? batch * T : batch, w->vocab, w->hidden);
  // attention split partials only for the row counts whose launches split the keys (a tree
  // verification; a prefill chunk of >= 1024 rows runs one split and needs none)
  const int64_t rows = block_attn_partial_rows(batch, T, w->n_q_heads, w->n_kv_heads, cap);
  c.take<float>(rows * 128);
  c.take<float>(rows * 2);
  c.take<float>(block_part_floats(w, batch * T));
  return c.off;
}

int64_t qd_block_workspace_bytes(const qd_weights* w, int64_t batch, int64_t T, int64_t cap) {
  return qd_block_workspace_bytes_lm(w, batch, T, cap, QD_LM_ALL);   // enough for every mode
}

int qd_block_step(const qd_weights* w, const qd_block_state* st, void* stream) {
  if (!weights_ok(w) || !st) return QD_EARG;
  const int64_t B = st->batch, T = st->T, cap = st->cap, H = w->hidden, I = w->inter, V = w->vocab;
  const int Hq = w->n_q_heads, Hkv = w->n_kv_heads;
  if (B <= 0 || T <= 0 || cap <= 0 || !st->k_cache || !st->v_cache || !st->cos || !st->sin ||
      !st->tokens || !st->base || !st->x || !st->xn || !st->qkv || !st->q || !st->attn ||
      !st->act || st->lm_mode < QD_LM_ALL || st->lm_mode > QD_LM_NONE ||
      (st->lm_mode != QD_LM_NONE && !st->out_tok))
    return QD_EARG;
  if (!st->causal && (!st->anc || !st->depth || T > 64)) return QD_EARG;
  if (block_attn_splits(cap) > 1024) return QD_EARG;
  if (!st->workspace || st->workspace_bytes < qd_block_workspace_bytes_lm(w, B, T, cap, st->lm_mode))
    return QD_EWS;
  hipStream_t s = S(stream);
  const int64_t M = B * T;
  Carver c(st->workspace);
  const int64_t lm_rows = st->lm_mode == QD_LM_ALL ? M : B;
  LmWs lw = carve_lm(c, lm_rows, V, H);
  const int64_t arows = block_attn_partial_rows(B, T, Hq, Hkv, cap);
  float* acc = c.take<float>(arows * 128);
  float* ml = c.take<float>(arows * 2);
  const int64_t part_floats = block_part_floats(w, M);
  float* part = c.take<float>(part_floats);
  const int64_t NQKV = qkv_width(w), QD = (int64_t)Hq * 128;
  const int64_t layer_kv = B * Hkv * cap * 128;

  if (st->c_base && st->c_src && st->c_cnt)
    launch_kv_compact(st->k_cache, st->v_cache, w->n_layers, B, Hkv, cap, st->c_base, st->c_src,
                      st->c_cnt, T, s);
  // Projections whose tile grid splits K (the tree-verification rows) leave fp32 partials and
  // their consumer sums them in split order: q/k norm + RoPE for qkv, the residual add + RMSNorm
  // for o and down -- the same bits as a split reduce kernel, one launch fewer each.
  // `pend` = splits of down partials not yet folded into the residual x.
  int pend = 0;
  launch_embed(st->tokens, w->embed, st->x, M, V, H, H, s);
  for (int64_t l = 0; l < w->n_layers; ++l) {
    bf16_t* kc = st->k_cache + l * layer_kv;
    bf16_t* vc = st->v_cache + l * layer_kv;
    if (pend)
      launch_part_add_rmsnorm(part, pend, M, st->x, w->ln1 + l * H, st->xn, H, w->eps, s);
    else
      launch_add_rmsnorm(nullptr, st->x, w->ln1 + l * H, nullptr, st->xn, M, H, H, H, w->eps, s);
    const int sq = gemm_tile_partials(st->xn, H, M, w->w_qkv + l * NQKV * H, NQKV, H, part,
                                      part_floats, s);
    if (sq) {
      launch_qk_norm_rope_part(part, sq, w->q_norm + l * 128, w->k_norm + l * 128, st->cos, st->sin,
                               cap, st->base, st->depth, st->causal ? POS_CHUNK : POS_TREE, st->q,
                               kc, vc, B, T, Hq, Hkv, cap, w->eps, s);
    } else {
      launch_gemm(st->xn, H, M, w->w_qkv + l * NQKV * H, NQKV, H, st->qkv, NQKV, nullptr, 0,
                  EPI_NONE, nullptr, nullptr, nullptr, s, part, part_floats);
      launch_qk_norm_rope(st->qkv, NQKV, w->q_norm + l * 128, w->k_norm + l * 128, st->cos,
                          st->sin, cap, st->base, st->depth, st->causal ? POS_CHUNK : POS_TREE,
                          st->q, kc, vc, B, T, Hq, Hkv, cap, w->eps, s);
    }
    launch_block_attn(st->q, kc, vc, st->base, st->causal ? nullptr : st->anc, B, T, Hq, Hkv, cap,
                      acc, ml, st->attn, s);
    const int so = gemm_tile_partials(st->attn, QD, M, w->w_o + l * H * QD, H, QD, part,
                                      part_floats, s);
    if (so) {
      launch_part_add_rmsnorm(part, so, M, st->x, w->ln2 + l * H, st->xn, H, w->eps, s);
    } else {
      launch_gemm(st->attn, QD, M, w->w_o + l * H * QD, H, QD, st->x, H, st->x, H, EPI_RES,
                  nullptr, nullptr, nullptr, s, part, part_floats);
      launch_add_rmsnorm(nullptr, st->x, w->ln2 + l * H, nullptr, st->xn, M, H, H, H, w->eps, s);
    }
    launch_gemm(st->xn, H, M, w->w_gu + l * 2 * I * H, I, H, st->act, I, nullptr, 0, EPI_SWIGLU,
                nullptr, nullptr, nullptr, s);
    pend = gemm_tile_partials(st->act, I, M, w->w_down + l * H * I, H, I, part, part_floats, s);
    if (!pend)
      launch_gemm(st->act, I, M, w->w_down + l * H * I, H, I, st->x, H, st->x, H, EPI_RES, nullptr,
                  nullptr, nullptr, s, part, part_floats);
  }
  if (st->lm_mode == QD_LM_NONE) return launched();   // K/V only (x is not read afterwards)
  if (pend) {
    // the last down partials: residual + final norm for every row, then the normalised rows
    launch_part_add_rmsnorm(part, pend, M, st->x, w->final_norm, st->xn, H, w->eps, s);
    if (st->lm_mode == QD_LM_LAST)
      return lm_head_normed_strided(st->xn + (T - 1) * H, T * H, lm_weight(w), V, H, B,
                                    st->out_tok, lw, s);
    return lm_head_normed_strided(st->xn, H, lm_weight(w), V, H, M, st->out_tok, lw, s);
  }
  if (st->lm_mode == QD_LM_LAST)
    return lm_head(st->x + (T - 1) * H, T * H, lm_weight(w), V, H, B, w->final_norm, w->eps,
                   st->out_tok, nullptr, nullptr, lw, s);
  return lm_head(st->x, H, lm_weight(w), V, H, M, w->final_norm, w->eps, st->out_tok, nullptr, nullptr,
                 lw, s);
}

// ------------------------------------------------------------------ plan queries (host only)
int qd_gemm_rows_plan(int64_t M, int64_t N, int64_t K, int32_t epi, int64_t part_floats,
                      int32_t partials_only, int64_t* out) {
  if (!out || M <= 0 || N <= 0 || K <= 0 || epi < EPI_NONE || epi > EPI_SWIGLU) return QD_EARG;
  if (epi == EPI_SWIGLU && partials_only) return QD_EARG;
  return gemm_rows_query(M, N, K, epi, partials_only != 0, part_floats, out);
}

// ------------------------------------------------------------------ graphs
int qd_graph_begin(void* stream) {
  if (!stream) return QD_EARG;  // the legacy null stream cannot be captured
  return qd_err(hipStreamBeginCapture(S(stream), hipStreamCaptureModeRelaxed));
}

int qd_graph_end(void* stream, void** exec_out) {
  if (!stream || !exec_out) return QD_EARG;
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture(S(stream), &g);
  if (e != hipSuccess) return qd_err(e);
  hipGraphExec_t ex = nullptr;
  e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (e != hipSuccess) return qd_err(e);
  *exec_out = ex;
  return QD_OK;
}

int qd_graph_launch(void* exec, void* stream) {
  if (!exec) return QD_EARG;
  return qd_err(hipGraphLaunch(reinterpret_cast<hipGraphExec_t>(exec), S(stream)));
}

int qd_graph_destroy(void* exec) {
  if (!exec) return QD_OK;
  return qd_err(hipGraphExecDestroy(reinterpret_cast<hipGraphExec_t>(exec)));
}

}  // extern "C"
