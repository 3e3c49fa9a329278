"""GPU parity of the persistent decode step (qd_mega_step) with the per-launch step
(qd_decode_step): bit-identical tokens, final residual, positions and K/V caches, step after
step.  At B = 1 over attention split plans of 1 split, several splits (merge), and more units
than workgroups; plus hipGraph replays over 36 layers, the bad-position error path and the
bounded waits (forced from the host through the error word); other batch sizes are refused."""

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
    rb.direct = False                # replay the captured one-node graph, not a direct launch
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


def test_persistent_step_is_batch_one_only(mods, model4):
    """The persistent entry points serve B = 1 only: other batch sizes are refused (the
    per-launch step serves them), and the host never picks them."""
    _lib, M = mods
    say("qd_mega_supported / workspace / ctl offset refuse B != 1")
    for B in (2, 17, 32):
        assert _lib.LIB.qd_mega_supported(C.byref(model4.qd), B) == 0
        assert _lib.LIB.qd_mega_workspace_bytes(C.byref(model4.qd), B, 2200) == 0
        assert _lib.LIB.qd_mega_ctl_offset(C.byref(model4.qd), B, 2200) == -1
        assert not M.mega_default(model4, B, 2200)
    assert _lib.LIB.qd_mega_supported(C.byref(model4.qd), 1) == 1
    assert M.mega_default(model4, 1, 2200)
