"""Host-side draft sources for tree speculation (qdecode/draft.py; the reference's
engine/spec.py:58-150) and the greedy accept walk, on the CPU with a mock greedy model: the
emitted text must be exactly the model's greedy text whatever the drafts, and the sources must
find the continuations they are meant to find (repeated n-grams, pooled predictions, the Jacobi
window), so acceptance rises above one token per pass on text that allows it."""

import os
import sys

import pytest

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                                "htn-2026_amd"))

from qdecode.draft import LookaheadDrafter, RowDraft  # noqa: E402
from qdecode.tree import Tree, accept  # noqa: E402


def test_ngram_candidates_follow_earlier_occurrences():
    seq = [5, 1, 2, 3, 9, 7, 1, 2, 3]
    d = RowDraft(seq)
    cands = d.candidates(3)
    # 3-gram (1, 2, 3) occurred at positions 1..3, followed by 9, 7, 1; 2-gram (2, 3) likewise
    assert cands[0] == [9, 7, 1] and cands[1] == [9, 7, 1]
    # most recent occurrence first, at most MAX_OCC kept
    seq2 = [4, 8] * 6
    d2 = RowDraft(seq2)
    assert len(d2.follow[2][(4, 8)]) == 3
    assert d2.candidates(2)[0] == seq2[d2.follow[3][(8, 4, 8)][-1]:][:2]


def test_index_is_incremental():
    seq = [1, 2, 3]
    d = RowDraft(seq)
    assert (1, 2) in d.follow[2] and (2, 3) not in d.follow[2]    # 3 has no successor yet
    seq += [1, 2]
    d.index()
    assert d.follow[2][(2, 3)] == [3] and d.follow[3][(1, 2, 3)] == [3]
    # the last 3 tokens (3, 1, 2) never occurred before; (1, 2) did, followed by 3, 1, 2
    assert d.candidates(3) == [[3, 1, 2]]


def test_pool_chain_and_jacobi_window():
    seq = [10, 11]
    d = RowDraft(seq)
    tree = d.draft(8, 4)                       # no candidates: a chain repeating the last token
    assert tree.tokens[:5] == [11, 11, 11, 11, 11] and tree.depth[:5] == [0, 1, 2, 3, 4]
    assert d.chain == [1, 2, 3, 4]
    g = [12, 20, 21, 22, 23] + [0] * 3         # the model's argmax after each node
    emitted, path = accept(tree, g)
    assert emitted == [12] and path == []
    d.observe(tree, g, path)
    # pool: (10, 11) -> 12 from the root; chain nodes (11, 11) -> ..
    assert d.pool[(10, 11)] == 12
    # window: predictions at the chain nodes beyond the accepted prefix (none accepted)
    assert d.window == [20, 21, 22, 23]
    seq.extend(emitted)
    d.index()
    cands = d.candidates(4)
    assert cands[0] == [20, 21, 22, 23]


def test_trie_respects_size_and_depth():
    seq = list(range(100)) + list(range(50))
    d = RowDraft(seq)
    tree = d.draft(16, 5)
    assert len(tree.tokens) == 16
    assert max(tree.depth[:tree.n_real]) <= 5
    # parents precede children and masks are ancestor-or-self
    for i in range(1, tree.n_real):
        p = tree.parent[i]
        assert p < i and tree.depth[i] == tree.depth[p] + 1
        assert tree.anc[i] == tree.anc[p] | (1 << i)


def _simulate(text, prompt_len, T, N, drafter):
    """CPU stand-in for stream_tree with a model whose greedy next token after any context
    that is a prefix of `text` is the next token of `text` (and a fixed junk token otherwise).
    Returns (emitted ids, tokens per pass)."""
    def model_next(ctx):
        n = len(ctx)
        return text[n] if n < len(text) and ctx == text[:n] else 999_999
    seq = text[:prompt_len] + [model_next(text[:prompt_len])]
    rows = drafter.rows([seq])
    per_pass = []
    while len(seq) - prompt_len < N:
        tree = rows[0].draft(T, min(T - 1, drafter.max_depth))
        g = []
        for i in range(T):                   # the argmax after node i given its ancestors
            path, n = [], i
            while n > 0:
                path.append(tree.tokens[n])
                n = tree.parent[n]
            g.append(model_next(seq + path[::-1]))
        emitted, path = accept(tree, g)
        rows[0].observe(tree, g, path)
        seq.extend(emitted)
        rows[0].index()
        per_pass.append(len(emitted))
    return seq[prompt_len:prompt_len + N], per_pass


@pytest.mark.parametrize("T", [8, 64])
def test_emitted_text_is_exactly_greedy(T):
    import random
    rng = random.Random(5)
    text = [rng.randrange(50) for _ in range(400)]       # little structure: few drafts hit
    out, per_pass = _simulate(text, 40, T, 200, LookaheadDrafter())
    assert out == text[40:240]
    assert all(k >= 1 for k in per_pass)


def test_repetitive_text_is_accepted_in_long_runs():
    base = [3, 14, 15, 92, 65, 35, 89, 79, 32, 38]
    text = base * 40
    out, per_pass = _simulate(text, 25, 64, 300, LookaheadDrafter())
    assert out == text[25:325]
    assert sum(per_pass) / len(per_pass) > 6          # n-gram matches verify whole runs


def test_jacobi_and_pool_converge_on_a_markov_text():
    # next token is a function of the last token only: after one visit the pool predicts it
    nxt = {i: (7 * i + 3) % 101 for i in range(101)}
    text = [0]
    for _ in range(600):
        text.append(nxt[text[-1]])
    out, per_pass = _simulate(text, 5, 32, 400, LookaheadDrafter())
    assert out == text[5:405]
    late = per_pass[len(per_pass) // 2:]
    assert sum(late) / len(late) > 4


def test_drafter_interface():
    d = LookaheadDrafter(max_depth=7)
    rows = d.rows([[1, 2, 3], [4, 5]])
    assert len(rows) == 2 and all(isinstance(r, RowDraft) for r in rows)
    assert isinstance(rows[1].draft(8, 7), Tree)
