"""ctypes binding of libqdecode.so (include/qdecode.h).

The library is the only compute path: importing this module on a machine where the library
was not built raises ImportError, and every non-zero return code raises QDError.  There is no
CPU or torch fallback.
"""

import ctypes as C
import os

HERE = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.environ.get("QDECODE_LIB", os.path.join(HERE, "libqdecode.so"))

QD_EARG, QD_EWS, QD_ESTATE, QD_ESCRATCH = -1, -2, -3, -4
QD_NOALLOC_SCRATCH_BYTES = 16 * 1024 * 1024
EPI_NONE, EPI_RES, EPI_SWIGLU = 0, 1, 2
POS_T, POS_SHARED, POS_ROW, POS_TREE = 0, 1, 2, 3
LM_ALL, LM_LAST, LM_NONE = 0, 1, 2

p, i32, i64, u64, f32 = C.c_void_p, C.c_int32, C.c_int64, C.c_uint64, C.c_float


class QDError(RuntimeError):
    """A libqdecode entry point returned a non-zero status."""

    def __init__(self, fn, rc):
        names = {QD_EARG: "invalid argument", QD_EWS: "workspace too small",
                 QD_ESTATE: "invalid state",
                 QD_ESCRATCH: "step needs more than the library's static scratch"}
        super().__init__(f"{fn} failed: {names.get(rc, f'hipError {rc}')} (rc={rc})")
        self.rc = rc


class Weights(C.Structure):
    """qd_weights (include/qdecode.h)."""
    _fields_ = [("n_layers", i32), ("hidden", i32), ("inter", i32), ("vocab", i32),
                ("n_q_heads", i32), ("n_kv_heads", i32), ("head_dim", i32), ("eps", f32),
                ("embed", p), ("final_norm", p), ("w_qkv", p), ("w_o", p), ("w_gu", p),
                ("w_down", p), ("ln1", p), ("ln2", p), ("q_norm", p), ("k_norm", p),
                ("lm_head", p)]


class DecodeState(C.Structure):
    """qd_decode_state (include/qdecode.h)."""
    _fields_ = [("batch", i32), ("cap", i64), ("k_cache", p), ("v_cache", p), ("cos", p),
                ("sin", p), ("tok", p), ("pos", p), ("x", p), ("qkv", p), ("attn", p),
                ("act", p), ("workspace", p), ("workspace_bytes", i64)]


class BlockState(C.Structure):
    """qd_block_state (include/qdecode.h)."""
    _fields_ = [("batch", i32), ("T", i32), ("causal", i32), ("lm_mode", i32), ("cap", i64),
                ("k_cache", p), ("v_cache", p), ("cos", p), ("sin", p), ("tokens", p),
                ("base", p), ("depth", p), ("anc", p), ("c_base", p), ("c_src", p),
                ("c_cnt", p), ("out_tok", p), ("x", p), ("xn", p), ("qkv", p), ("q", p),
                ("attn", p), ("act", p), ("workspace", p), ("workspace_bytes", i64)]


SIGNATURES = {
    "qd_version": ([], C.c_char_p),
    "qd_embed_gather": ([p, p, p, i64, i64, i64, i64, p], i32),
    "qd_add_rmsnorm": ([p, p, p, p, p, i64, i64, i64, i64, f32, p], i32),
    "qd_qk_norm_rope": ([p, i64, p, p, p, p, i64, p, p, i32, p, p, p, i64, i64, i64, i64, i64,
                         f32, p], i32),
    "qd_swiglu": ([p, i64, p, i64, i64, i64, p], i32),
    "qd_linear_workspace_bytes": ([i64, i64, i64, i32], i64),
    "qd_linear": ([p, i64, p, i64, i64, p, i64, i64, p, f32, i32, p, i64, p, i64, p], i32),
    "qd_lm_head_workspace_bytes": ([i64, i64, i64], i64),
    "qd_lm_head_argmax": ([p, i64, p, i64, i64, i64, p, f32, p, p, p, p, i64, p], i32),
    "qd_decode_attn_workspace_bytes": ([i64, i64, i64, i64], i64),
    "qd_decode_attn": ([p, i64, p, p, p, p, p, p, p, i64, i64, i64, i64, f32, p, p, i64, p], i32),
    "qd_block_attn_workspace_bytes": ([i64, i64, i64, i64], i64),
    "qd_block_attn": ([p, p, p, p, p, i64, i64, i64, i64, i64, p, p, i64, p], i32),
    "qd_kv_compact": ([p, p, i64, i64, i64, i64, p, p, p, i64, p], i32),
    "qd_synth_bf16": ([p, i64, u64, u64, u64, f32, p], i32),
    "qd_fill_bf16": ([p, i64, C.c_uint16, p], i32),
    "qd_read_probe": ([p, i64, i32, p, p], i32),
    "qd_decode_workspace_bytes": ([C.POINTER(Weights), i64, i64], i64),
    "qd_decode_step": ([C.POINTER(Weights), C.POINTER(DecodeState), p], i32),
    "qd_decode_step_noalloc": ([C.POINTER(Weights), C.POINTER(DecodeState), p], i32),
    "qd_mega_supported": ([C.POINTER(Weights), i64], i32),
    "qd_mega_workspace_bytes": ([C.POINTER(Weights), i64, i64], i64),
    "qd_mega_ctl_offset": ([C.POINTER(Weights), i64, i64], i64),
    "qd_mega_step": ([C.POINTER(Weights), C.POINTER(DecodeState), p], i32),
    "qd_block_workspace_bytes": ([C.POINTER(Weights), i64, i64, i64], i64),
    "qd_block_workspace_bytes_lm": ([C.POINTER(Weights), i64, i64, i64, i32], i64),
    "qd_block_step": ([C.POINTER(Weights), C.POINTER(BlockState), p], i32),
    "qd_gemm_rows_plan": ([i64, i64, i64, i32, i64, i32, C.POINTER(i64)], i32),
    "qd_graph_begin": ([p], i32),
    "qd_graph_end": ([p, C.POINTER(C.c_void_p)], i32),
    "qd_graph_launch": ([p, p], i32),
    "qd_graph_destroy": ([p], i32),
}


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built: run `python htn-2026_amd/build.py` "
                          "(or __graft_entry__.build()); there is no fallback path")
    lib = C.CDLL(LIB_PATH)
    for name, (args, res) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    return lib


LIB = _load()


def call(name, *args):
    """Call an int-returning entry point and raise QDError on a non-zero status."""
    rc = getattr(LIB, name)(*args)
    if rc != 0:
        raise QDError(name, rc)
    return rc
