"""Tensor-level wrappers of the libqdecode kernels.

torch is used for device memory and the current stream only: every wrapper checks dtype,
device and shape on the host, hands raw pointers to the C ABI and raises QDError on a non-zero
status.  Outputs and workspaces may be passed in (stable addresses for graph capture); when
omitted they are allocated here (workspaces zero-filled, as the ABI requires).

Reference counterparts (Yokanater/htn-2026):
  embed_gather       F.embedding / embed_ss      engine/engine.py:338, kernels/fast.py:53-76
  add_rmsnorm        rms_norm_rows (+ residual)  kernels/rmsnorm.py:15-53, gemv.py:50-51
  qk_norm_rope       qk_norm_rope_cache, tree_qk kernels/fused.py:84-98, tree.py:198-204
  swiglu             silu_mul                    kernels/fused.py:101-120
  linear             Gemv / FastGemm             kernels/gemv.py:161-234, fast.py:161-213
  lm_head_argmax     LmHeadArgmax / FastLmHead   kernels/gemv.py:237-287, fast.py:439-465
  decode_attention   FastAttention               kernels/fast.py:353-376
  block_attention    TreeAttention               kernels/tree.py:166-195
  kv_compact         compact                     kernels/tree.py:207-211
"""

import torch

from . import _lib
from ._lib import EPI_NONE, EPI_RES, EPI_SWIGLU, POS_ROW, POS_SHARED, POS_T, POS_TREE  # noqa: F401

BF16 = torch.bfloat16


def stream_ptr():
    return torch.cuda.current_stream().cuda_stream


def _ptr(t):
    return None if t is None else t.data_ptr()


def _check(t, dtype, name, device=None):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be on a HIP device, got {t.device}")
    if device is not None and t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")


def _rows(t, name):
    if t.dim() < 1 or t.stride(-1) != 1:
        raise ValueError(f"{name} must have a unit last stride")
    return t.reshape(-1, t.shape[-1]) if t.dim() != 2 else t


def workspace(nbytes, device):
    return torch.zeros(max(int(nbytes), 256), dtype=torch.uint8, device=device)


def embed_gather(ids, table, out=None):
    _check(ids, torch.int64, "ids")
    _check(table, BF16, "table", ids.device)
    ids = ids.reshape(-1).contiguous()
    V, H = table.shape
    if out is None:
        out = torch.empty((ids.numel(), H), dtype=BF16, device=ids.device)
    _check(out, BF16, "out", ids.device)
    _lib.call("qd_embed_gather", ids.data_ptr(), table.data_ptr(), out.data_ptr(), ids.numel(), V,
              H, out.stride(0), stream_ptr())
    return out


def add_rmsnorm(residual, w, eps, x=None, res_out=None, y=None):
    """(res_out, y) with res_out = bf16(x + residual) (or None when x is None) and
    y = RMSNorm(res_out or residual; w)."""
    _check(residual, BF16, "residual")
    _check(w, BF16, "w", residual.device)
    r2 = _rows(residual, "residual")
    rows, H = r2.shape
    if x is not None:
        _check(x, BF16, "x", residual.device)
        x2 = _rows(x, "x")
        if x2.shape != r2.shape or x2.stride(0) != r2.stride(0):
            raise ValueError("x and residual must have the same shape and row stride")
        if res_out is None:
            res_out = torch.empty_like(r2)
    if y is None:
        y = torch.empty((rows, H), dtype=BF16, device=residual.device)
    _check(y, BF16, "y", residual.device)
    if res_out is not None and res_out.stride(0) != r2.stride(0):
        raise ValueError("res_out must share residual's row stride")
    _lib.call("qd_add_rmsnorm", _ptr(x), r2.data_ptr(), w.data_ptr(), _ptr(res_out),
              y.data_ptr(), rows, H, r2.stride(0), y.stride(0), float(eps), stream_ptr())
    return res_out, y


def rmsnorm(x, w, eps, y=None):
    return add_rmsnorm(x, w, eps, y=y)[1]


def qk_norm_rope(qkv, q_norm_w, k_norm_w, cos, sin, pos, mode, q_out, k_cache, v_cache, batch, T,
                 n_q_heads, n_kv_heads, eps, depth=None):
    """qkv [B*T, (Hq + 2 Hkv) * 128]; q_out [B, T, Hq, 128]; k/v cache [B, Hkv, cap, 128]."""
    _check(qkv, BF16, "qkv")
    for n, t in (("q_norm_w", q_norm_w), ("k_norm_w", k_norm_w), ("cos", cos), ("sin", sin),
                 ("q_out", q_out), ("k_cache", k_cache), ("v_cache", v_cache)):
        _check(t, BF16, n, qkv.device)
    if pos is not None:
        _check(pos, torch.int64, "pos", qkv.device)
    if depth is not None:
        _check(depth, torch.int64, "depth", qkv.device)
    if q_out.numel() < batch * T * n_q_heads * 128:
        raise ValueError("q_out too small")
    cap = k_cache.shape[-2]
    _lib.call("qd_qk_norm_rope", qkv.data_ptr(), qkv.stride(0), q_norm_w.data_ptr(),
              k_norm_w.data_ptr(), cos.data_ptr(), sin.data_ptr(), cos.shape[0], _ptr(pos),
              _ptr(depth), int(mode), q_out.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
              batch, T, n_q_heads, n_kv_heads, cap, float(eps), stream_ptr())
    return q_out


def swiglu(gu, out=None):
    _check(gu, BF16, "gu")
    g2 = _rows(gu, "gu")
    rows, two_i = g2.shape
    inter = two_i // 2
    if out is None:
        out = torch.empty((rows, inter), dtype=BF16, device=gu.device)
    _check(out, BF16, "out", gu.device)
    _lib.call("qd_swiglu", g2.data_ptr(), g2.stride(0), out.data_ptr(), out.stride(0), rows, inter,
              stream_ptr())
    return out


def linear(x, w, epilogue=EPI_NONE, norm_w=None, eps=1e-6, res=None, out=None, ws=None):
    """out[m, n] = epi(sum_k xin[m, k] w[n, k]); SwiGLU: w is [2N, K] (gate | up)."""
    _check(x, BF16, "x")
    _check(w, BF16, "w", x.device)
    x2 = _rows(x, "x")
    rows, K = x2.shape
    n_out = w.shape[0] // 2 if epilogue == EPI_SWIGLU else w.shape[0]
    if w.shape[1] != K or not w.is_contiguous():
        raise ValueError(f"w must be contiguous [N, {K}]")
    if out is None:
        out = torch.empty((rows, n_out), dtype=BF16, device=x.device)
    _check(out, BF16, "out", x.device)
    if res is not None:
        _check(res, BF16, "res", x.device)
    need = _lib.LIB.qd_linear_workspace_bytes(rows, n_out, K, 1 if norm_w is not None else 0)
    if need and ws is None:
        ws = workspace(need, x.device)
    _lib.call("qd_linear", x2.data_ptr(), x2.stride(0), w.data_ptr(), n_out, K, out.data_ptr(),
              out.stride(0), rows, _ptr(norm_w), float(eps), int(epilogue), _ptr(res),
              res.stride(0) if res is not None else 0, _ptr(ws),
              ws.numel() if ws is not None else 0, stream_ptr())
    return out


def lm_head_argmax(x, w, norm_w, eps, tok=None, pos=None, logits=None, ws=None):
    _check(x, BF16, "x")
    x2 = _rows(x, "x")
    rows, K = x2.shape
    V = w.shape[0]
    if tok is None:
        tok = torch.empty((rows,), dtype=torch.int64, device=x.device)
    if logits is not None:
        _check(logits, torch.float32, "logits", x.device)
    need = _lib.LIB.qd_lm_head_workspace_bytes(rows, V, K)
    if ws is None:
        ws = workspace(need, x.device)
    _lib.call("qd_lm_head_argmax", x2.data_ptr(), x2.stride(0), w.data_ptr(), V, K, rows,
              norm_w.data_ptr(), float(eps), tok.data_ptr(), _ptr(pos), _ptr(logits),
              ws.data_ptr(), ws.numel(), stream_ptr())
    return tok


def decode_attention(qkv, q_norm_w, k_norm_w, cos, sin, pos, k_cache, v_cache, n_q_heads,
                     n_kv_heads, eps, out=None, ws=None):
    """qkv [B, (Hq + 2 Hkv) * 128]; k/v cache [B, Hkv, cap, 128]; out [B, Hq, 128]."""
    _check(qkv, BF16, "qkv")
    _check(pos, torch.int64, "pos", qkv.device)
    B = qkv.shape[0]
    cap = k_cache.shape[-2]
    if out is None:
        out = torch.empty((B, n_q_heads, 128), dtype=BF16, device=qkv.device)
    need = _lib.LIB.qd_decode_attn_workspace_bytes(B, n_q_heads, n_kv_heads, cap)
    if ws is None:
        ws = workspace(need, qkv.device)
    _lib.call("qd_decode_attn", qkv.data_ptr(), qkv.stride(0), q_norm_w.data_ptr(),
              k_norm_w.data_ptr(), cos.data_ptr(), sin.data_ptr(), pos.data_ptr(),
              k_cache.data_ptr(), v_cache.data_ptr(), B, n_q_heads, n_kv_heads, cap, float(eps),
              out.data_ptr(), ws.data_ptr(), ws.numel(), stream_ptr())
    return out


def block_attention(q, k_cache, v_cache, base, anc=None, out=None, ws=None):
    """q [B, T, Hq, 128]; k/v cache [B, Hkv, cap, 128]; base int64 [B]; anc uint64-as-int64
    [B, T] or None (causal)."""
    _check(q, BF16, "q")
    B, T, Hq, _ = q.shape
    Hkv, cap = k_cache.shape[1], k_cache.shape[2]
    if out is None:
        out = torch.empty_like(q)
    if anc is not None:
        _check(anc, torch.int64, "anc", q.device)
    need = _lib.LIB.qd_block_attn_workspace_bytes(B, T, Hq, cap)
    if ws is None:
        ws = workspace(need, q.device)
    _lib.call("qd_block_attn", q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
              base.data_ptr(), _ptr(anc), B, T, Hq, Hkv, cap, out.data_ptr(), ws.data_ptr(),
              ws.numel(), stream_ptr())
    return out


def kv_compact(k_all, v_all, base, src, cnt):
    L, B, Hkv, cap, _ = k_all.shape
    T = src.shape[-1]
    _lib.call("qd_kv_compact", k_all.data_ptr(), v_all.data_ptr(), L, B, Hkv, cap,
              base.data_ptr(), src.data_ptr(), cnt.data_ptr(), T, stream_ptr())


SIGMA_S = (8.0 * (65536.0 ** 2 - 1.0) / 12.0) ** 0.5


def synth_scale(std):
    """fp32 multiplier of the counter-based generator (std / exact sigma of the 8-term sum)."""
    import numpy as np
    return float(np.float32(std / SIGMA_S))


def synth_bf16(out, seed, stream, start=0, std=0.02):
    _check(out, BF16, "out")
    if not out.is_contiguous():
        raise ValueError("out must be contiguous")
    _lib.call("qd_synth_bf16", out.data_ptr(), out.numel(), seed, stream, start, synth_scale(std),
              stream_ptr())
    return out


def fill_bf16(out, value_bits):
    _check(out, BF16, "out")
    _lib.call("qd_fill_bf16", out.data_ptr(), out.numel(), int(value_bits), stream_ptr())
    return out
