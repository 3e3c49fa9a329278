"""CPU: draft-tree construction, ancestor masks and the greedy accept walk
(engine/spec.py:18-55, 124-150) against brute force."""

import numpy as np
import pytest

from qdecode import tree as tr


def brute_anc(tree, i):
    m, n = 0, i
    while n >= 0:
        m |= 1 << n
        n = tree.parent[n]
    return m


def test_branching_4422_truncated_to_64():
    rng = np.random.default_rng(0)
    t = tr.branching_tree(7, 64, (4, 4, 2, 2), lambda n: rng.integers(0, 151936, size=n))
    assert len(t.tokens) == 64 and t.n_real == 64
    depths = np.bincount(t.depth)
    assert depths.tolist() == [1, 4, 16, 32, 11]            # 1 + 4 + 16 + 32 = 53, then 11 leaves
    for i in range(64):
        assert t.anc[i] == brute_anc(t, i)
        assert t.parent[i] < i                              # parents precede children
        assert t.depth[i] <= i
    assert max(t.anc) >= 1 << 63                            # needs the full 64-bit mask
    assert all(-(1 << 63) <= a < 1 << 63 for a in t.anc_i64())


def test_full_4422_tree_has_117_nodes():
    rng = np.random.default_rng(1)
    t = tr.Tree(0)
    frontier = [0]
    for fan in (4, 4, 2, 2):
        nxt = []
        for p in frontier:
            for tok in rng.integers(0, 1 << 30, size=fan):
                if len(t.tokens) < 64:
                    nxt.append(t.add(p, tok))
        frontier = nxt
    assert len(t.tokens) == 64
    assert 1 + 4 + 16 + 32 + 64 == 117


def test_pad_is_unreachable():
    t = tr.Tree(5)
    t.add(0, 9)
    t.pad(6)
    assert len(t.tokens) == 6
    g = [5, 0, 0, 0, 0, 0]                                  # argmax after root is 5 = pad token
    emitted, path = tr.accept(t, g)
    assert emitted == [5] and path == []                    # pads are not children
    assert t.anc[3] == 1 | 1 << 3


def test_accept_walk_brute_force():
    rng = np.random.default_rng(3)
    for trial in range(200):
        vocab = 5
        t = tr.branching_tree(int(rng.integers(vocab)), 30, (3, 2, 2, 2),
                              lambda n: rng.integers(0, vocab, size=n))
        g = rng.integers(0, vocab, size=len(t.tokens)).tolist()
        emitted, path = tr.accept(t, g)
        # brute force: follow the model's choice while a child carries it
        node, want = 0, [g[0]]
        while True:
            kids = [c for c in range(1, t.n_real) if t.parent[c] == node and t.tokens[c] == want[-1]]
            if not kids:
                break
            node = kids[0]
            want.append(g[node])
        assert emitted == want
        assert len(path) == len(emitted) - 1
        for k, n in enumerate(path):
            assert t.depth[n] == k + 1 and n >= k + 1       # compaction sources are >= targets


def test_tree_caps_at_64():
    t = tr.Tree(0)
    for i in range(63):
        t.add(0, i + 1)
    with pytest.raises(ValueError):
        t.add(0, 1000)


def test_random_drafter_is_seeded():
    a = tr.random_tree_drafter(5)([1, 2, 3], 64)
    b = tr.random_tree_drafter(5)([1, 2, 3], 64)
    assert a.tokens == b.tokens and a.tokens[0] == 3
