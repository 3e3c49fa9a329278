"""Host side of exact token-tree speculative decoding.

``Tree`` and the greedy accept walk restate the reference's tree encoding and walk
(engine/spec.py:18-55, 124-150): they define which ids are emitted.  The mask is 64 bits wide
(the reference's int32 caps trees at 32 nodes, engine.py:166-169), so a 64-node tree verifies
in one block forward.  The verification loop (``stream_tree``, the counterpart of the
reference's engine.py:830-908) is built around per-sequence ``RowState`` objects and one
pinned input block per forward (``TreePass``).  Draft sources are pluggable:
``random_tree_drafter`` builds the benchmark's uniformly random 4-4-2-2 trees;
``draft.LookaheadDrafter`` restates the reference's window / n-gram / prediction-pool sources
(a stateful drafter: ``rows(seqs)`` gives per-sequence sources that draft a tree, observe the
verified argmaxes and index the emitted text).

Node 0 is the last emitted token (its K/V is not cached yet); parents precede children, so
node index >= depth.  Node i is rotated at base + depth_i, written to cache slot base + i,
and sees cached slots < base plus the block slots of its ancestors.  After verification the
accepted path (root, n_1, .., n_a) is compacted to slots base .. base + a by the next block
forward (qd_kv_compact), and the emitted tokens are exactly the model's greedy choices.
"""

import time

import numpy as np
import torch

from .inputs import BlockInputs


class Tree:
    __slots__ = ("tokens", "depth", "parent", "anc", "children", "n_real")

    def __init__(self, root):
        self.tokens, self.depth, self.parent = [int(root)], [0], [-1]
        self.anc = [1]
        self.children = [{}]
        self.n_real = 1

    def add(self, parent, tok):
        """Child of `parent` with token `tok` (merged with an existing equal child)."""
        tok = int(tok)
        hit = self.children[parent].get(tok)
        if hit is not None:
            return hit
        i = len(self.tokens)
        if i >= 64:
            raise ValueError("a tree holds at most 64 nodes (64-bit ancestor mask)")
        self.tokens.append(tok)
        self.depth.append(self.depth[parent] + 1)
        self.parent.append(parent)
        self.anc.append(self.anc[parent] | (1 << i))
        self.children.append({})
        self.children[parent][tok] = i
        self.n_real = len(self.tokens)
        return i

    def add_path(self, toks, T):
        node, nodes = 0, []
        for t in toks:
            if len(self.tokens) >= T and int(t) not in self.children[node]:
                break
            node = self.add(node, t)
            nodes.append(node)
        return nodes

    def pad(self, T):
        """Fill to T nodes with inert leaves under the root that `accept` can never reach
        (spec.py:41-49)."""
        root = self.tokens[0]
        while len(self.tokens) < T:
            i = len(self.tokens)
            self.tokens.append(root)
            self.depth.append(1)
            self.parent.append(0)
            self.anc.append(1 | (1 << i))
            self.children.append({})

    def anc_i64(self):
        """Masks as int64 two's complement (the device reads them as uint64)."""
        return [a - (1 << 64) if a >= 1 << 63 else a for a in self.anc]


def accept(tree, g):
    """Greedy accept walk (spec.py:124-135): g[i] = model argmax after node i.  Returns the
    emitted tokens (g of the root, then of every accepted node) and the accepted node path."""
    emitted, path, node = [int(g[0])], [], 0
    while True:
        nxt = tree.children[node].get(emitted[-1])
        if nxt is None:
            return emitted, path
        path.append(nxt)
        node = nxt
        emitted.append(int(g[nxt]))


def branching_tree(root, T, branching, draw):
    """BFS-ordered tree with the given branching per level, truncated to T nodes; ``draw(n)``
    returns n draft token ids."""
    tree = Tree(root)
    frontier = [0]
    for fan in branching:
        nxt = []
        for p in frontier:
            for tok in draw(fan):
                if len(tree.tokens) >= T:
                    break
                before = len(tree.tokens)
                i = tree.add(p, tok)
                if len(tree.tokens) > before:
                    nxt.append(i)
        frontier = nxt
        if len(tree.tokens) >= T:
            break
    tree.pad(T)
    return tree


def random_tree_drafter(seed, vocab=151936, branching=(4, 4, 2, 2)):
    """The benchmark's draft source: uniformly random ids in a 4-4-2-2 tree (root + the first
    T-1 BFS nodes of the 117-node tree).  The ids of one tree are drawn in a single call."""
    rng = np.random.default_rng(seed)
    full = 1
    width = 1
    for fan in branching:
        width *= fan
        full += width

    def drafter(seq, T):
        ids = iter(rng.integers(0, vocab, size=full).tolist())
        return branching_tree(seq[-1], T, branching, lambda n: [next(ids) for _ in range(n)])
    return drafter


# ----------------------------------------------------------------------------------------------
# The verification loop.  Its state is per sequence (``RowState``: text, draft source, the tree
# in flight, the cache slot of its root and the compaction that the next forward applies); the
# device side is one BlockRunner and a pinned twin of its input block (``TreePass``), so every
# pass moves all inputs host -> device in one copy and all argmaxes back in one copy.
# ----------------------------------------------------------------------------------------------

class _FnSource:
    """A plain ``drafter(text, T) -> Tree`` seen as a per-sequence source with no state."""

    def __init__(self, fn, text):
        self.fn, self.text = fn, text

    def draft(self, T, depth):
        return self.fn(self.text, T)

    def observe(self, tree, g, path):
        pass

    def index(self):
        pass


class RowState:
    """One sequence under tree verification.

    ``text`` is prompt + emitted ids (shared with the draft source); ``slot`` is the cache slot
    of the next tree's node 0, which is always the last emitted id, so slot = len(text) - 1;
    ``moves`` = (slot of the verified tree, its accepted node indices) is the compaction that
    the next forward performs first (node k of the accepted path goes to slot + k)."""

    __slots__ = ("text", "n_prompt", "source", "tree", "slot", "moves")

    def __init__(self, text, n_prompt, source):
        self.text, self.n_prompt, self.source = text, n_prompt, source
        self.tree = None
        self.slot = len(text) - 1
        self.moves = (self.slot, [0])            # identity until a tree has been verified

    @property
    def emitted(self):
        return len(self.text) - self.n_prompt

    def stage(self, arr, b, T, depth):
        """Draft this pass's tree and write it, its slot and the pending compaction into row b
        of the host input arrays (``BlockInputs.arrays()`` of the pinned twin)."""
        tree = self.source.draft(T, depth)
        if len(tree.tokens) != T:
            raise ValueError(f"draft tree has {len(tree.tokens)} nodes, the forward takes {T}")
        self.tree = tree
        arr["tokens"][b] = tree.tokens
        arr["depth"][b] = tree.depth
        arr["anc"][b] = np.array(tree.anc, dtype=np.uint64).view(np.int64)
        arr["base"][b] = self.slot
        at, nodes = self.moves
        arr["c_base"][b] = at
        arr["c_src"][b, :len(nodes)] = nodes
        arr["c_src"][b, len(nodes):] = 0
        arr["c_cnt"][b] = len(nodes)

    def settle(self, g):
        """Take the model's argmax after every node of the tree in flight (``g``, T ids):
        append the accepted ids to the text and plan their compaction.  Returns how many ids
        this pass emitted for the sequence."""
        out, path = accept(self.tree, g)
        self.source.observe(self.tree, g, path)
        self.moves = (self.slot, [0] + path)
        self.text.extend(out)
        self.source.index()
        self.slot = len(self.text) - 1
        return len(out)


class TreePass:
    """One tree-verification forward per call: the pinned input twin of ``runner`` is copied to
    the device in one transfer, the forward (compaction first) is replayed, and the per-node
    argmaxes come back in one transfer; ``run()`` returns them as a [B, T] numpy array."""

    def __init__(self, runner, stream):
        self.runner, self.stream = runner, stream
        B, T = runner.kv.B, runner.t_max
        self.B, self.T = B, T
        self.host = BlockInputs(B, T, pinned=True)
        self.arrays = self.host.arrays()
        self.out = torch.empty((B * T,), dtype=torch.int64, pin_memory=True)
        self.out_np = self.out.numpy().reshape(B, T)
        self.done = torch.cuda.Event()

    def run(self):
        with torch.cuda.stream(self.stream):
            self.runner.inputs.block.copy_(self.host.block, non_blocking=True)
            self.runner.launch(self.T, compact=True)
            self.out.copy_(self.runner.out_tok, non_blocking=True)
            self.done.record(self.stream)
        self.done.synchronize()
        return self.out_np


def stream_tree(engine, sh, ids, N, drafter):
    """Prefill, then one verification forward of a T-node draft tree per sequence per pass
    until every sequence has N ids; yields exactly N lists of B ids, each column as soon as
    every sequence has it (the reference's loop: engine/engine.py:830-908).

    A sequence that already has N ids is not staged again: its row of the input block keeps
    the last tree it verified, at the same slots (all inside its cache), and its outputs are
    ignored -- its cache is no longer read.  ``engine.tree_stats`` records the passes, the ids
    each sequence took per pass and the host time per pass (staging + accept walks)."""
    B, S, T = sh.B, sh.S, sh.tree_T
    sh.start(ids)
    first = sh.first_token()
    yield first
    if N == 1:
        return
    texts = [list(map(int, r)) + [t] for r, t in zip(ids.tolist(), first)]
    if hasattr(drafter, "rows"):
        sources = drafter.rows(texts)
    else:
        sources = [_FnSource(drafter, tx) for tx in texts]
    rows = [RowState(tx, S, src) for tx, src in zip(texts, sources)]
    depth = min(T - 1, getattr(drafter, "max_depth", T - 1))
    tp = sh.tree_pass()
    stats = {"passes": 0, "accepted": [], "host_ms": []}
    sent = 1
    while sent < N:
        t0 = time.perf_counter()
        live = [b for b in range(B) if rows[b].emitted < N]
        for b in live:
            rows[b].stage(tp.arrays, b, T, depth)
        t1 = time.perf_counter()
        g = tp.run()
        t2 = time.perf_counter()
        for b in live:
            stats["accepted"].append(rows[b].settle(g[b].tolist()))
        stats["passes"] += 1
        stats["host_ms"].append((t1 - t0 + time.perf_counter() - t2) * 1e3)
        ready = min(N, min(r.emitted for r in rows))
        for t in range(sent, ready):
            yield [r.text[S + t] for r in rows]
        sent = max(sent, ready)
    engine.tree_stats = stats
