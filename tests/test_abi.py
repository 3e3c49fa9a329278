"""CPU: the C-ABI library loads, exports every entry point include/qdecode.h declares, and
rejects invalid arguments before touching the device."""

import ctypes as C
import os
import re

import pytest

from helpers import ROOT

HEADER = os.path.join(ROOT, "include", "qdecode.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qd_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from qdecode import _lib
    return _lib


def test_every_declared_symbol_is_exported(lib):
    syms = declared_symbols()
    assert len(syms) >= 20
    for s in syms:
        assert hasattr(lib.LIB, s), s
    # and every exported binding is declared
    assert set(lib.SIGNATURES) <= set(syms)


def test_version(lib):
    assert b"gfx950" in lib.LIB.qd_version()


def test_argument_errors_without_device(lib):
    L = lib.LIB
    EARG, EWS = lib.QD_EARG, lib.QD_EWS
    assert L.qd_embed_gather(None, None, None, 4, 151936, 2560, 2560, None) == EARG
    assert L.qd_embed_gather(None, None, None, 0, 151936, 2560, 2560, None) == 0   # empty: no-op
    assert L.qd_embed_gather(None, None, None, 4, 151936, 2561, 2561, None) == EARG  # hidden % 8
    assert L.qd_add_rmsnorm(None, None, None, None, None, 2, 2560, 2560, 2560, 1e-6, None) == EARG
    assert L.qd_add_rmsnorm(None, None, None, None, None, 2, 2560, 2048, 2560, 1e-6, None) == EARG
    assert L.qd_swiglu(None, 100, None, 50, 1, 50, None) == EARG                    # inter % 8
    assert L.qd_linear(None, 2560, None, 10, 2560, None, 10, 1, None, 1e-6, 5, None, 0, None, 0,
                       None) == EARG                                                # bad epilogue
    assert L.qd_linear(None, 100, None, 10, 100, None, 10, 1, None, 1e-6, 0, None, 0, None, 0,
                       None) == EARG                                                # k % 128
    assert L.qd_qk_norm_rope(None, 6144, None, None, None, None, 10, None, None, 9, None, None, None,
                             1, 1, 32, 8, 10, 1e-6, None) == EARG                  # bad mode
    assert L.qd_decode_attn(None, 6144, None, None, None, None, None, None, None, 1, 30, 8, 10,
                            1e-6, None, None, 0, None) == EARG                     # Hq != 4 Hkv
    assert L.qd_block_attn(None, None, None, None, C.c_void_p(8), 1, 65, 32, 8, 100, None, None, 0,
                           None) == EARG                                           # T > 64 w/ anc
    ws = L.qd_lm_head_workspace_bytes(1, 151936, 2560)
    assert ws > 0
    x = C.c_void_p(256)
    assert L.qd_lm_head_argmax(x, 2560, x, 151936, 2560, 1, x, 1e-6, x, None, None, x, ws - 1,
                               None) == EWS
    assert L.qd_graph_begin(None) == EARG
    assert L.qd_graph_destroy(None) == 0
    sink = C.c_void_p(256)
    assert L.qd_read_probe(x, 1000, 64, sink, None) == EARG                         # bytes % 16
    assert L.qd_read_probe(C.c_void_p(264), 1024, 64, sink, None) == EARG           # misaligned
    assert L.qd_read_probe(x, 1024, 0, sink, None) == EARG                          # grid < 1
    assert L.qd_read_probe(x, 1024, 64, None, None) == EARG                         # no sink
    assert L.qd_read_probe(None, 0, 64, sink, None) == 0                            # nothing to read


def test_workspace_sizes(lib):
    L = lib.LIB
    w = lib.Weights(36, 2560, 9728, 151936, 32, 8, 128, 1e-6, *([256] * 10))
    b1 = L.qd_decode_workspace_bytes(C.byref(w), 1, 768)
    b32 = L.qd_decode_workspace_bytes(C.byref(w), 32, 2176)
    assert 0 < b1 < b32 < 1 << 30
    assert L.qd_block_workspace_bytes(C.byref(w), 4, 64, 8512) > 0
    assert L.qd_decode_attn_workspace_bytes(1, 32, 8, 768) >= 32 * 128 * 4
    bad = lib.Weights(36, 2560, 9728, 151936, 32, 8, 64, 1e-6, *([256] * 10))     # head_dim 64
    st = lib.DecodeState()
    assert L.qd_decode_step(C.byref(bad), C.byref(st), None) == lib.QD_EARG


def test_noalloc_scratch_limits(lib):
    """The documented limits of qd_decode_step_noalloc's static array at Qwen3-4B's shape:
    batch 32 up to cap 106496 and batch 64 up to 40960 fit, one more key does not."""
    L = lib.LIB
    w = lib.Weights(36, 2560, 9728, 151936, 32, 8, 128, 1e-6, *([256] * 10))
    lim = lib.QD_NOALLOC_SCRATCH_BYTES
    assert lim == 16 << 20
    for B, cap in ((32, 106496), (64, 40960)):
        assert L.qd_decode_workspace_bytes(C.byref(w), B, cap) <= lim
        assert L.qd_decode_workspace_bytes(C.byref(w), B, cap + 1) > lim
    assert L.qd_decode_workspace_bytes(C.byref(w), 1, 1 << 20) <= lim       # B = 1: 8.6 MB


def test_block_workspace_sizes(lib):
    """The block step's workspace at the benchmark shapes (no device here: 256 CUs assumed).
    Attention split partials exist only where the launch splits the keys and never grow with
    the context; a prefill runner (QD_LM_LAST) reserves LM-head room for one row per sequence."""
    L = lib.LIB
    w = lib.Weights(36, 2560, 9728, 151936, 32, 8, 128, 1e-6, *([256] * 10))
    al = lambda n: (n + 255) // 256 * 256                                       # noqa: E731
    # config-5 verify: 4 sequences x 8 KV heads x 1 query block = 32 workgroups per key split,
    # so 256 / 32 = 8 splits; 4 * 64 rows * 32 heads * 8 splits partial rows of 128 + 2 floats
    rows = 4 * 64 * 32 * 8
    assert L.qd_block_attn_workspace_bytes(4, 64, 32, 8512) == al(rows * 512) + al(rows * 8)
    # prefill chunks of 32768 rows: >= 256 workgroups with one split, no partials at any context
    for cap in (2176, 8512, 131328):
        assert L.qd_block_attn_workspace_bytes(32, 1024, 32, cap) == 0
    verify = L.qd_block_workspace_bytes_lm(C.byref(w), 4, 64, 8512, lib.LM_ALL)
    assert verify == L.qd_block_workspace_bytes(C.byref(w), 4, 64, 8512) < 100 << 20
    for B, T in ((4, 8192), (32, 1024), (1, 32768), (8, 4096)):
        sizes = [L.qd_block_workspace_bytes_lm(C.byref(w), B, T, cap, lib.LM_LAST)
                 for cap in (T + 256, 32768 + 256, 131072 + 256)]
        assert sizes[0] == sizes[1] == sizes[2] < 64 << 20, (B, T, sizes)
        none = L.qd_block_workspace_bytes_lm(C.byref(w), B, T, T + 256, lib.LM_NONE)
        every = L.qd_block_workspace_bytes_lm(C.byref(w), B, T, T + 256, lib.LM_ALL)
        assert none <= sizes[0] < every
    assert L.qd_block_workspace_bytes_lm(C.byref(w), 4, 64, 8512, 3) == 0              # bad mode


def test_missing_library_raises(tmp_path):
    """The product path has no fallback: a missing library is an ImportError."""
    import subprocess
    import sys
    code = ("import os, sys; os.environ['QDECODE_LIB'] = sys.argv[1]; "
            "sys.path.insert(0, sys.argv[2]); import qdecode._lib")
    r = subprocess.run([sys.executable, "-c", code, str(tmp_path / "none.so"),
                        os.path.join(ROOT, "htn-2026_amd")], capture_output=True, text=True)
    assert r.returncode != 0 and "ImportError" in r.stderr
