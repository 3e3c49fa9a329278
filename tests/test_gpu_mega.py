"""GPU parity of the persistent decode step (qd_mega_step) with the per-launch step
(qd_decode_step): bit-identical tokens, final residual, positions and K/V caches, step after
step.  At B = 1 over attention split plans of 1 split, several splits (merge), and more units
than workgroups; at 17 and 32 sequences (the batched persistent kernel) at short and ~2100-key
contexts; plus hipGraph replays over 36 layers, the bad-position error path and the bounded
waits (forced from the host through the error word)."""

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
def model4(mods):
    _lib, M = mods
    m = M.Qwen3Model.synthetic(n_layers=4, seed=0)
    if not _lib.LIB.qd_mega_supported(C.byref(m.qd), 1):
        pytest.skip("persistent step unsupported on this device")
    return m


def _prefilled_pair(M, _lib, model, S, cap, seed, B=1):
    """Two KV states holding the same causal prefill of B random prompts (tok/pos set)."""
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


def _assert_same(ra, rb, kv_a, kv_b, step):
    assert torch.equal(kv_a.tok, kv_b.tok), f"step {step}: tok {kv_a.tok} vs {kv_b.tok}"
    assert torch.equal(kv_a.pos, kv_b.pos), f"step {step}: pos"
    assert torch.equal(ra.x.view(torch.int16), rb.x.view(torch.int16)), f"step {step}: residual"
    assert torch.equal(kv_a.k.view(torch.int16), kv_b.k.view(torch.int16)), f"step {step}: K cache"
    assert torch.equal(kv_a.v.view(torch.int16), kv_b.v.view(torch.int16)), f"step {step}: V cache"


@pytest.mark.parametrize("S,N", [(40, 24), (600, 168), (8300, 12)],
                         ids=["one-split", "six-splits", "two-units-per-wg"])
def test_mega_matches_decode_step(mods, model4, S, N):
    _lib, M = mods
    cap = M.kv_capacity(S, N)
    say(f"mega vs per-launch step: 4 layers, S={S}, N={N}, cap={cap}")
    stream, kv_a, kv_b = _prefilled_pair(M, _lib, model4, S, cap, seed=S)
    ra = M.DecodeRunner(kv_a, stream, mega=False)
    rb = M.DecodeRunner(kv_b, stream, mega=True)
    torch.cuda.synchronize()
    for step in range(N - 1):
        with torch.cuda.stream(stream):
            ra.enqueue()
            rb.enqueue()
        stream.synchronize()
        _assert_same(ra, rb, kv_a, kv_b, step)
    epoch, err = rb.mega_status()
    assert err == 0 and epoch == N - 1


def test_mega_graph_replay_36_layers(mods):
    _lib, M = mods
    say("mega graph replays vs per-launch step: 36 layers, S=512, 24 steps")
    model = M.Qwen3Model.synthetic(n_layers=36, seed=1)
    if not _lib.LIB.qd_mega_supported(C.byref(model.qd), 1):
        pytest.skip("persistent step unsupported on this device")
    S, N = 512, 25
    stream, kv_a, kv_b = _prefilled_pair(M, _lib, model, S, M.kv_capacity(S, N), seed=7)
    ra = M.DecodeRunner(kv_a, stream, mega=False)
    rb = M.DecodeRunner(kv_b, stream, mega=True)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        ra.capture()
        rb.capture()
    for step in range(N - 1):
        with torch.cuda.stream(stream):
            ra.replay()
            rb.replay()
        stream.synchronize()
        _assert_same(ra, rb, kv_a, kv_b, step)
        # eager work between replays: the graph must not depend on it
        torch.zeros(1 << 20, device=model.device).add_(1.0)
        torch.cuda.synchronize()
    epoch, err = rb.mega_status()
    assert err == 0 and epoch == N - 1
    ra.close()
    rb.close()


def test_mega_bad_position_sets_error(mods, model4):
    _lib, M = mods
    say("mega with pos == cap: error word 2, nothing written")
    S, N = 40, 8
    stream, _, kv = _prefilled_pair(M, _lib, model4, S, M.kv_capacity(S, N), seed=3)
    r = M.DecodeRunner(kv, stream, mega=True)
    kv.pos.fill_(kv.cap)
    tok0, k0 = kv.tok.clone(), kv.k.clone()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        r.enqueue()
    epoch, err = r.mega_status()
    assert err == 2 and epoch == 0
    assert torch.equal(kv.tok, tok0) and torch.equal(kv.k, k0)
    assert int(kv.pos.item()) == kv.cap
    with pytest.raises(RuntimeError):
        r.check()


def test_mega_waits_are_bounded(mods, model4):
    """A preset error word makes every wait give up after a bounded number of polls: the step
    still completes, in bounded time, and reports the error."""
    _lib, M = mods
    say("mega with the error word preset: completes, error stays set")
    S, N = 40, 8
    stream, _, kv = _prefilled_pair(M, _lib, model4, S, M.kv_capacity(S, N), seed=4)
    r = M.DecodeRunner(kv, stream, mega=True)
    r.err_word.fill_(1)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        r.enqueue()
    epoch, err = r.mega_status()
    assert err == 1 and epoch == 1
    assert 0 <= int(kv.tok.item()) < model4.V


def test_engine_persistent_error_is_not_yielded_and_recovers(mods):
    """Engine.generate reads the persistent step's error word with every step's ids
    (engine.py:1038-1045 checks the megakernel flag before trusting T6).  The word is set from
    the host while step 4 runs, so step 5 runs with every wait giving up: generate yields steps
    0-4 (all equal to a clean run) and raises before step 5's ids.  The workspace is zeroed, the
    engine drops the persistent tier, and the next call emits the clean run's ids again through
    the bit-identical per-launch step."""
    _lib, M = mods
    from engine import Engine
    say("Engine.generate with the error word set mid-stream: no post-error ids, recovery")
    eng = Engine.synthetic(n_layers=4, seed=0)
    eng.tree_mode = "0"
    prompt = [list(range(200, 240))]
    clean = list(eng.generate(prompt, 12))
    if not eng.shape.decode.mega:
        pytest.skip("persistent step unsupported on this device")
    got = []
    with pytest.raises(RuntimeError, match="persistent decode step 5 failed"):
        for i, step in enumerate(eng.generate(prompt, 12)):
            got.append(step)
            if i == 3:           # step 4 is already enqueued: the word is set behind it
                with torch.cuda.stream(eng.stream):
                    eng.shape.decode.err_word.fill_(1)
    assert got == clean[:5]
    assert eng.mega is False and eng.mega_errors[-1][3:] == (5, 1)
    epoch, err = eng.shape.decode.mega_status()
    assert (epoch, err) == (0, 0)                  # the failed runner's workspace was zeroed
    again = list(eng.generate(prompt, 12))
    assert not eng.shape.decode.mega and again == clean


def test_engine_mega_matches_per_launch(mods, monkeypatch):
    _lib, M = mods
    from engine import Engine
    say("Engine.generate with and without the persistent step: identical tokens")
    prompt = [list(range(100, 164))]
    monkeypatch.setenv("QD_MEGA", "1")
    e1 = Engine.synthetic(n_layers=4, seed=0)
    t1 = list(e1.generate(prompt, 20))
    assert e1.shape.decode.mega or not _lib.LIB.qd_mega_supported(C.byref(e1.model.qd), 1)
    monkeypatch.setenv("QD_MEGA", "0")
    e2 = Engine.synthetic(n_layers=4, seed=0)
    t2 = list(e2.generate(prompt, 20))
    assert not e2.shape.decode.mega
    assert t1 == t2


# ------------------------------------------------------------------ batched persistent step
@pytest.fixture(scope="module")
def model4b(mods):
    _lib, M = mods
    m = M.Qwen3Model.synthetic(n_layers=4, seed=0)
    if not _lib.LIB.qd_mega_supported(C.byref(m.qd), 32):
        pytest.skip("batched persistent step unsupported on this device")
    return m


@pytest.mark.parametrize("B,S,N", [(32, 40, 12), (17, 40, 8), (32, 2100, 6)],
                         ids=["b32-short", "b17-short", "b32-2100-keys"])
def test_mega_batch_matches_decode_step(mods, model4b, B, S, N):
    _lib, M = mods
    cap = M.kv_capacity(S, N)
    say(f"batched mega vs per-launch step: 4 layers, B={B}, S={S}, N={N}, cap={cap}")
    stream, kv_a, kv_b = _prefilled_pair(M, _lib, model4b, S, cap, seed=S + B, B=B)
    ra = M.DecodeRunner(kv_a, stream, mega=False)
    rb = M.DecodeRunner(kv_b, stream, mega=True)
    assert rb.mega
    torch.cuda.synchronize()
    for step in range(N - 1):
        with torch.cuda.stream(stream):
            ra.enqueue()
            rb.enqueue()
        stream.synchronize()
        _assert_same(ra, rb, kv_a, kv_b, step)
    epoch, err = rb.mega_status()
    assert err == 0 and epoch == N - 1


def test_mega_batch_default_and_cap_limit(mods, model4b, monkeypatch):
    """The batched persistent step runs only when asked for (QD_MEGA_BATCH=1), and then only where
    one attention key split covers the cap."""
    _lib, M = mods
    say("batched mega default: off; with QD_MEGA_BATCH=1 on at cap 2200, off at cap 5000")
    monkeypatch.delenv("QD_MEGA_BATCH", raising=False)
    assert not M.mega_default(model4b, 32, 2200)
    monkeypatch.setenv("QD_MEGA_BATCH", "1")
    assert M.mega_default(model4b, 32, 2200)
    assert not M.mega_default(model4b, 32, 5000)
    assert not M.mega_default(model4b, 16, 2200)


def test_mega_batch_graph_replay_36_layers(mods):
    _lib, M = mods
    say("batched mega graph replays vs per-launch step: 36 layers, B=32, S=256, 8 steps")
    model = M.Qwen3Model.synthetic(n_layers=36, seed=1)
    if not _lib.LIB.qd_mega_supported(C.byref(model.qd), 32):
        pytest.skip("batched persistent step unsupported on this device")
    B, S, N = 32, 256, 9
    stream, kv_a, kv_b = _prefilled_pair(M, _lib, model, S, M.kv_capacity(S, N), seed=9, B=B)
    ra = M.DecodeRunner(kv_a, stream, mega=False)
    rb = M.DecodeRunner(kv_b, stream, mega=True)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        ra.capture()
        rb.capture()
    for step in range(N - 1):
        with torch.cuda.stream(stream):
            ra.replay()
            rb.replay()
        stream.synchronize()
        _assert_same(ra, rb, kv_a, kv_b, step)
        torch.zeros(1 << 20, device=model.device).add_(1.0)
        torch.cuda.synchronize()
    epoch, err = rb.mega_status()
    assert err == 0 and epoch == N - 1
    ra.close()
    rb.close()


def test_mega_batch_bad_position_sets_error(mods, model4b):
    """pos == cap: the persistent kernel writes nothing and reports error 2 (the LM head after it
    still runs, as in the per-launch step, and its token is not to be used)."""
    _lib, M = mods
    say("batched mega with pos == cap: error word 2, K/V untouched")
    B, S, N = 32, 40, 8
    stream, _, kv = _prefilled_pair(M, _lib, model4b, S, M.kv_capacity(S, N), seed=5, B=B)
    r = M.DecodeRunner(kv, stream, mega=True)
    kv.pos.fill_(kv.cap)
    k0, v0 = kv.k.clone(), kv.v.clone()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        r.enqueue()
    epoch, err = r.mega_status()
    assert err == 2 and epoch == 0
    assert torch.equal(kv.k, k0) and torch.equal(kv.v, v0)
    with pytest.raises(RuntimeError):
        r.check()


def test_mega_batch_waits_are_bounded(mods, model4b):
    """A preset error word makes every wait of the batched kernel give up after a bounded number
    of polls: the step completes and reports the error."""
    _lib, M = mods
    say("batched mega with the error word preset: completes, error stays set")
    B, S, N = 32, 40, 8
    stream, _, kv = _prefilled_pair(M, _lib, model4b, S, M.kv_capacity(S, N), seed=6, B=B)
    r = M.DecodeRunner(kv, stream, mega=True)
    r.err_word.fill_(1)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        r.enqueue()
    epoch, err = r.mega_status()
    assert err == 1 and epoch == 1
    assert ((kv.tok >= 0) & (kv.tok < model4b.V)).all()

