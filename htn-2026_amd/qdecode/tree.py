"""Host side of exact token-tree speculative decoding.

Restates the reference's ``Tree`` and greedy accept walk (engine/spec.py:18-55, 124-150) and
its verify loop (engine/engine.py:830-908) with two MI355X-side changes:
  * the ancestor-or-self mask is 64 bits wide (the reference's int32 caps trees at 32 nodes,
    engine.py:166-169), so a 64-node tree verifies in one block forward;
  * draft sources are pluggable: ``random_tree_drafter`` builds the benchmark's uniformly
    random 4-4-2-2 trees; ``draft.LookaheadDrafter`` restates the reference's window / n-gram
    / prediction-pool sources (a stateful drafter: ``rows(seqs)`` gives per-sequence sources
    that draft a tree, observe the verified argmaxes and index the emitted text).

Node 0 is the last emitted token (its K/V is not cached yet); parents precede children, so
node index >= depth.  Node i is rotated at base + depth_i, written to cache slot base + i,
and sees cached slots < base plus the block slots of its ancestors.  After verification the
accepted path (root, n_1, .., n_a) is compacted to slots base .. base + a by the next block
forward (qd_kv_compact), and the emitted tokens are exactly the model's greedy choices.
"""

import numpy as np
import torch


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
    T-1 BFS nodes of the 117-node tree)."""
    rng = np.random.default_rng(seed)

    def drafter(seq, T):
        return branching_tree(seq[-1], T, branching, lambda n: rng.integers(0, vocab, size=n))
    return drafter


def stream_tree(engine, sh, ids, N, drafter):
    """Prefill, then verify one draft tree per sequence per block forward until every row has
    N tokens; yields exactly N lists of B ids (engine.py:830-908)."""
    B, S, T = sh.B, sh.S, sh.tree_T
    tr = sh.tree
    stream = engine.stream
    with torch.cuda.stream(stream):
        sh.ids_host.copy_(ids)
        sh.ids.copy_(sh.ids_host, non_blocking=True)
        sh.run_prefill()
        sh.host[0].copy_(sh.kv.tok, non_blocking=True)
        sh.events[0].record(stream)
    sh.events[0].synchronize()
    first = sh.host[0].tolist()
    yield first
    if N == 1:
        return
    seqs = [list(map(int, r)) + [t] for r, t in zip(ids.tolist(), first)]
    rows = drafter.rows(seqs) if hasattr(drafter, "rows") else None
    depth = min(T - 1, getattr(drafter, "max_depth", T - 1))
    c_base, c_src, c_cnt = [S] * B, [[0] * T for _ in range(B)], [1] * B
    pin = lambda shape, dt: torch.empty(shape, dtype=dt, pin_memory=True)  # noqa: E731
    h_tok, h_depth, h_anc = pin((B, T), torch.int64), pin((B, T), torch.int64), pin((B, T), torch.int64)
    h_base, h_cb, h_cs, h_cc = pin((B,), torch.int64), pin((B,), torch.int64), pin((B, T), torch.int32), pin((B,), torch.int32)
    h_out = pin((B * T,), torch.int64)
    ev = torch.cuda.Event()
    yielded = 1
    stats = {"passes": 0, "accepted": []}
    while yielded < N:
        stats["passes"] += 1
        trees, bases = [], []
        for b in range(B):
            sq = seqs[b]
            if len(sq) - S >= N:                 # done: verify an inert tree at a safe slot
                tree = Tree(sq[-1])
                tree.pad(T)
                trees.append(None)
                bases.append(S)
            else:
                tree = rows[b].draft(T, depth) if rows else drafter(sq, T)
                trees.append(tree)
                bases.append(len(sq) - 1)
            h_tok[b] = torch.tensor(tree.tokens, dtype=torch.int64)
            h_depth[b] = torch.tensor(tree.depth, dtype=torch.int64)
            h_anc[b] = torch.tensor(tree.anc_i64(), dtype=torch.int64)
        h_base.copy_(torch.tensor(bases, dtype=torch.int64))
        h_cb.copy_(torch.tensor(c_base, dtype=torch.int64))
        h_cs.copy_(torch.tensor(c_src, dtype=torch.int32))
        h_cc.copy_(torch.tensor(c_cnt, dtype=torch.int32))
        with torch.cuda.stream(stream):
            for d, h in ((tr.tokens, h_tok), (tr.depth, h_depth), (tr.anc, h_anc), (tr.base, h_base),
                         (tr.c_base, h_cb), (tr.c_src, h_cs), (tr.c_cnt, h_cc)):
                d.copy_(h, non_blocking=True)
            tr.launch(T, compact=True)
            h_out.copy_(tr.out_tok, non_blocking=True)
            ev.record(stream)
        ev.synchronize()
        g = h_out.tolist()
        for b in range(B):
            tree = trees[b]
            if tree is None:
                c_cnt[b] = 1
                continue
            gb = g[b * T:(b + 1) * T]
            emitted, path = accept(tree, gb)
            c_base[b] = bases[b]
            c_src[b] = [0] + path + [0] * (T - 1 - len(path))
            c_cnt[b] = len(path) + 1
            if rows:
                rows[b].observe(tree, gb, path)
            seqs[b].extend(emitted)
            if rows:
                rows[b].index()
            stats["accepted"].append(len(emitted))
        while yielded < N and all(len(sq) - S > yielded for sq in seqs):
            yield [sq[S + yielded] for sq in seqs]
            yielded += 1
    engine.tree_stats = stats
