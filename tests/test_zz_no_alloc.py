"""GPU: qd_decode_step_noalloc (the decode step for callers that cannot allocate, its split
partials in the library's static device scratch) against qd_decode_step with a caller
workspace, through the C ABI: bit-identical tokens, positions, residual stream and K/V caches
after every step.

* The first test makes the process's first call of the entry point inside a hipGraph capture
  (no other test file calls it), so the array's address is resolved during the capture; the
  graph is then replayed with eager qd_decode_step work and synchronisation between replays.
* Then calls in a row on shrinking shapes, each running on scratch contents the one before
  left behind: B = 64 (tiled GEMMs, partials in the array), 8 and 3 (skinny GEMMs), 1 (GEMV).
* The size limit is refused before any launch."""

import ctypes as C

import pytest
import torch

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"\n[case] {msg}", flush=True)


@pytest.fixture(scope="module")
def mods():
    import engine  # noqa: F401  (puts qdecode on the path and loads the library)
    from qdecode import _lib
    from qdecode import model as M
    return _lib, M


@pytest.fixture(scope="module")
def model2(mods):
    _, M = mods
    return M.Qwen3Model.synthetic(n_layers=2, seed=0)


def _prefilled_pair(M, _lib, model, B, S, cap, seed):
    stream = torch.cuda.Stream()
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, model.V, (B, S), generator=g)
    kv_a = M.KVState(model, B, cap)
    with torch.cuda.stream(stream):
        pr = M.BlockRunner(kv_a, stream, S, causal=True, lm_mode=_lib.LM_LAST)
        pr.tokens.view(-1)[:B * S].copy_(ids.view(-1).to(model.device))
        pr.base.fill_(0)
        pr.enqueue(S)
        kv_a.tok.copy_(pr.out_tok)
        kv_a.pos.fill_(S)
    stream.synchronize()
    kv_b = M.KVState(model, B, cap)
    for name in ("k", "v", "tok", "pos"):
        getattr(kv_b, name).copy_(getattr(kv_a, name))
    torch.cuda.synchronize()
    return stream, kv_a, kv_b


def _noalloc_state(_lib, kv, m):
    """A qd_decode_state with no workspace (the entry point brings its own)."""
    B, dev = kv.B, m.device
    bufs = {"x": torch.empty((B, m.H), dtype=torch.bfloat16, device=dev),
            "qkv": torch.empty((B, (m.Hq + 2 * m.Hkv) * 128), dtype=torch.bfloat16, device=dev),
            "attn": torch.empty((B, m.Hq * 128), dtype=torch.bfloat16, device=dev),
            "act": torch.empty((B, m.I), dtype=torch.bfloat16, device=dev)}
    st = _lib.DecodeState(B, kv.cap, kv.k.data_ptr(), kv.v.data_ptr(), kv.cos.data_ptr(),
                          kv.sin.data_ptr(), kv.tok.data_ptr(), kv.pos.data_ptr(),
                          bufs["x"].data_ptr(), bufs["qkv"].data_ptr(), bufs["attn"].data_ptr(),
                          bufs["act"].data_ptr(), None, 0)
    return st, bufs


def _same(ra, kv_a, kv_b, bufs_b, step):
    assert torch.equal(kv_a.tok, kv_b.tok), f"step {step}: tok {kv_a.tok} vs {kv_b.tok}"
    assert torch.equal(kv_a.pos, kv_b.pos), f"step {step}: pos"
    assert torch.equal(ra.x.view(torch.int16), bufs_b["x"].view(torch.int16)), f"step {step}: x"
    assert torch.equal(kv_a.k.view(torch.int16), kv_b.k.view(torch.int16)), f"step {step}: K"
    assert torch.equal(kv_a.v.view(torch.int16), kv_b.v.view(torch.int16)), f"step {step}: V"


def test_noalloc_first_call_captured_in_graph(mods, model2):
    _lib, M = mods
    B, S, steps = 4, 96, 4
    cap = S + steps + 1
    say(f"qd_decode_step_noalloc captured into a hipGraph on its first call: B={B}, S={S}, "
        f"{steps} replays against eager qd_decode_step")
    stream, kv_a, kv_b = _prefilled_pair(M, _lib, model2, B, S, cap, seed=77)
    ra = M.DecodeRunner(kv_a, stream, mega=False)
    st_b, bufs_b = _noalloc_state(_lib, kv_b, model2)
    torch.cuda.synchronize()
    s = stream.cuda_stream
    _lib.call("qd_graph_begin", s)
    try:
        rc = _lib.LIB.qd_decode_step_noalloc(C.byref(model2.qd), C.byref(st_b), s)
    finally:
        ex = C.c_void_p()
        rc_end = _lib.LIB.qd_graph_end(s, C.byref(ex))
    assert rc == 0 and rc_end == 0, (rc, rc_end)
    try:
        for step in range(steps):
            with torch.cuda.stream(stream):
                ra.enqueue()
                _lib.call("qd_graph_launch", ex, s)
            stream.synchronize()
            _same(ra, kv_a, kv_b, bufs_b, step)
    finally:
        _lib.LIB.qd_graph_destroy(ex)


@pytest.mark.parametrize("B,S,steps", [(64, 80, 3), (8, 300, 4), (3, 40, 3), (1, 50, 3)],
                         ids=["first-B64", "then-B8", "then-B3", "then-B1"])
def test_noalloc_step_matches_decode_step(mods, model2, B, S, steps):
    _lib, M = mods
    cap = S + steps + 1
    say(f"qd_decode_step_noalloc vs qd_decode_step: 2 layers, B={B}, S={S}, {steps} steps")
    need = _lib.LIB.qd_decode_workspace_bytes(C.byref(model2.qd), B, cap)
    assert 0 < need <= _lib.QD_NOALLOC_SCRATCH_BYTES
    stream, kv_a, kv_b = _prefilled_pair(M, _lib, model2, B, S, cap, seed=B * 1000 + S)
    ra = M.DecodeRunner(kv_a, stream, mega=False)
    st_b, bufs_b = _noalloc_state(_lib, kv_b, model2)
    torch.cuda.synchronize()
    for step in range(steps):
        with torch.cuda.stream(stream):
            ra.enqueue()
            _lib.call("qd_decode_step_noalloc", C.byref(model2.qd), C.byref(st_b),
                      stream.cuda_stream)
        stream.synchronize()
        _same(ra, kv_a, kv_b, bufs_b, step)


def test_noalloc_rejects_steps_beyond_its_scratch(mods, model2):
    """A shape whose split partials exceed the static array is refused before any launch."""
    _lib, M = mods
    B, cap = 64, 100000
    say(f"qd_decode_step_noalloc B={B} cap={cap}: QD_ESCRATCH")
    assert _lib.LIB.qd_decode_workspace_bytes(C.byref(model2.qd), B, cap) > \
        _lib.QD_NOALLOC_SCRATCH_BYTES
    dummy = torch.zeros(16, dtype=torch.int64, device=model2.device)
    p = dummy.data_ptr()
    st = _lib.DecodeState(B, cap, p, p, p, p, p, p, p, p, p, p, None, 0)
    rc = _lib.LIB.qd_decode_step_noalloc(C.byref(model2.qd), C.byref(st),
                                         torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == _lib.QD_ESCRATCH
    assert torch.count_nonzero(dummy) == 0
