"""CPU: the tree-verification loop (qdecode.tree.stream_tree) end to end against a stand-in for
the device forward.

The stand-in sees only what the device would see -- the staged input block (tokens, depths,
ancestor masks, base slots, compaction lists) -- and keeps one simulated cache per sequence
holding a token id per slot.  Each forward first applies the staged compaction, then writes the
tree's tokens at base + i, and answers for node i with the model's greedy next token after the
context it can attend to: cache slots [0, base) followed by its ancestors' block slots in depth
order.  A wrong compaction list, base slot, mask or depth changes that context, and with it the
emitted ids, so the test pins the host loop's encoding as well as its emission order.
"""

import random

import numpy as np
import pytest

from qdecode import tree as tr
from qdecode.draft import LookaheadDrafter
from qdecode.inputs import BlockInputs

JUNK = 999_983                      # the model's answer off the reference text


class _Forward:
    def __init__(self, sh):
        self.sh = sh
        self.host = BlockInputs(sh.B, sh.tree_T)
        self.arrays = self.host.arrays()

    def run(self):
        sh, a, T = self.sh, self.arrays, self.sh.tree_T
        out = np.zeros((sh.B, T), dtype=np.int64)
        for b in range(sh.B):
            cache = sh.cache[b]
            cb, cnt = int(a["c_base"][b]), int(a["c_cnt"][b])
            src = a["c_src"][b, :cnt].tolist()
            assert 1 <= cnt <= T and src[0] == 0
            for k in range(cnt):                          # in order, as qd_kv_compact does
                assert 0 <= cb + src[k] < sh.cap and cb + k < sh.cap
                cache[cb + k] = cache[cb + src[k]]
            base = int(a["base"][b])
            assert 0 <= base and base + T <= sh.cap       # every slot inside the cache
            for i in range(T):
                cache[base + i] = int(a["tokens"][b, i])
            for i in range(T):
                m = int(a["anc"][b, i]) & ((1 << 64) - 1)
                anc = sorted((j for j in range(T) if m >> j & 1), key=lambda j: a["depth"][b, j])
                assert [int(a["depth"][b, j]) for j in anc] == list(range(len(anc)))
                assert anc[0] == 0 and anc[-1] == i       # root ... self
                ctx = cache[:base] + [cache[base + j] for j in anc]
                out[b, i] = sh.model(b, ctx)
        return out


class _Shape:
    """The parts of the engine's per-shape state that stream_tree uses."""

    def __init__(self, texts, S, N, T):
        self.texts = texts
        self.B, self.S, self.N, self.tree_T = len(texts), S, N, T
        self.cap = S + N + T                              # model.kv_capacity(S, N, extra=T)
        self.cache = None
        self.fwd = None

    def model(self, b, ctx):
        text = self.texts[b]
        n = len(ctx)
        return text[n] if n < len(text) and ctx == text[:n] else JUNK

    def start(self, ids):
        self.cache = [list(map(int, r)) + [-1] * (self.cap - self.S) for r in ids.tolist()]

    def first_token(self):
        return [self.model(b, self.cache[b][:self.S]) for b in range(self.B)]

    def tree_pass(self):
        if self.fwd is None:
            self.fwd = _Forward(self)
        return self.fwd


class _Engine:
    tree_stats = None


def _run(texts, S, N, T, drafter):
    import torch
    sh = _Shape(texts, S, N, T)
    ids = torch.tensor([t[:S] for t in texts], dtype=torch.int64)
    eng = _Engine()
    out = list(tr.stream_tree(eng, sh, ids, N, drafter))
    return out, eng.tree_stats


def _texts(seed, n):
    rng = random.Random(seed)
    rep7 = [rng.randrange(40) for _ in range(7)] * 40
    noise = [rng.randrange(40) for _ in range(280)]
    rep5 = [rng.randrange(40) for _ in range(5)] * 56
    return [rep7[:n], noise[:n], rep5[:n]]


@pytest.mark.parametrize("T", [16, 64])
def test_stream_tree_emits_greedy_columns(T):
    S, N = 24, 60
    texts = _texts(1, 240)
    out, stats = _run(texts, S, N, T, LookaheadDrafter())
    assert len(out) == N and all(len(c) == 3 for c in out)
    for t, col in enumerate(out):
        assert col == [texts[b][S + t] for b in range(3)], t
    # the noisy row takes ~1 id per pass and sets the pass count; the repetitive rows finish
    # early and are not staged again
    assert len(stats["host_ms"]) == stats["passes"]
    assert len(stats["accepted"]) < 3 * stats["passes"]
    assert sum(stats["accepted"]) >= 3 * (N - 1)
    # without the noisy row, whole runs of drafted ids are accepted per pass
    out, stats = _run([texts[0], texts[2]], S, N, T, LookaheadDrafter())
    for t, col in enumerate(out):
        assert col == [texts[0][S + t], texts[2][S + t]]
    assert stats["passes"] < (N - 1) // 3


def test_stream_tree_random_drafts_and_plain_callables():
    S, N, T = 10, 20, 64
    texts = _texts(2, 120)
    out, stats = _run(texts, S, N, T, tr.random_tree_drafter(3, vocab=40))
    for t, col in enumerate(out):
        assert col == [texts[b][S + t] for b in range(3)]
    assert stats["passes"] >= 1


def _decoy_then_truth(texts, depth=4):
    """A drafter whose trees hold a wrong branch first and the true continuation second, so
    the accepted nodes sit at indices > their depth and every compaction really moves K/V."""
    def drafter(seq, T):
        t = tr.Tree(seq[-1])
        t.add_path([JUNK - 1, JUNK - 2, JUNK - 3], T)
        for x in texts:
            if x[:len(seq)] == list(seq):
                t.add_path(x[len(seq):len(seq) + depth], T)
                break
        t.pad(T)
        return t
    return drafter


@pytest.mark.parametrize("T", [8, 64])
def test_stream_tree_compaction_moves_accepted_nodes(T):
    S, N = 16, 40
    texts = _texts(4, 200)
    out, stats = _run(texts, S, N, T, _decoy_then_truth(texts))
    for t, col in enumerate(out):
        assert col == [texts[b][S + t] for b in range(3)], t
    assert max(stats["accepted"]) == 5 and stats["passes"] <= (N - 1 + 4) // 5 + 1


def test_stream_tree_single_token_and_tiny_trees():
    S, T = 12, 2
    texts = _texts(3, 80)
    out, stats = _run(texts, S, 1, T, LookaheadDrafter())
    assert out == [[texts[b][S] for b in range(3)]] and stats is None
    out, stats = _run(texts, S, 9, T, LookaheadDrafter())
    for t, col in enumerate(out):
        assert col == [texts[b][S + t] for b in range(3)]


def test_row_state_compaction_plan():
    """After a pass the compaction moves the accepted nodes to the slots right after the old
    root, and the next tree's root sits right after them."""
    t = tr.Tree(5)
    a = t.add(0, 6)
    t.add(0, 7)
    c = t.add(a, 8)
    t.pad(8)
    row = tr.RowState([1, 2, 3, 5], 3, tr._FnSource(lambda seq, T: t, None))
    arr = BlockInputs(1, 8).arrays()
    row.stage(arr, 0, 8, 7)
    assert arr["base"][0] == 3 and arr["c_cnt"][0] == 1 and arr["c_base"][0] == 3
    g = [6, 9, 9, 9, 9, 9, 9, 9]
    g[a], g[c] = 8, 4
    assert row.settle(g) == 3                             # 6 (root), 8 (after a), 4 (after c)
    assert row.text == [1, 2, 3, 5, 6, 8, 4] and row.slot == 6
    row.stage(arr, 0, 8, 7)
    assert arr["c_base"][0] == 3 and arr["c_cnt"][0] == 3
    assert arr["c_src"][0].tolist() == [0, a, c, 0, 0, 0, 0, 0]
    assert arr["base"][0] == 6
