"""Draft sources for exact token-tree speculation (engine/spec.py:1-150 of the reference).

Per sequence and verification pass, candidate continuations of the current text come from
  1. the lookahead (Jacobi) window: the model's own predictions at the nodes of the previous
     tree's first candidate path that lie beyond what was accepted -- iterated pass after pass
     this converges on the text the model will produce (spec.py:3-4, 140-149);
  2. earlier occurrences of the text's last 3 tokens, then of its last 2, in prompt + emitted
     text: what followed them (the most recent MAX_OCC occurrences each, spec.py:5, 70-92);
  3. a pool of the model's predictions at every verified node, keyed by (parent token, token):
     the n-grams that verification yields for free, chained from the text's last two tokens
     (spec.py:6-7, 108-115, 136-143).
They are merged into one trie of at most T nodes (node 0 = the last emitted token), at most
MAX_DEPTH deep, the first candidate first (its nodes are the next window's source).  With no
candidate at all the trie is a chain repeating the last token (spec.py:117-118), which seeds the
Jacobi iteration.  Which tokens are emitted never depends on the drafts: verification accepts
exactly the model's greedy choices (tree.accept), so drafts only change how many tokens one
forward yields.
"""

from .tree import Tree

MAX_OCC = 3        # occurrences kept per n-gram (spec.py:16)
MAX_DEPTH = 12     # longest candidate path (engine.py:833)


class RowDraft:
    """Candidate sources for one sequence.  ``seq`` (prompt + emitted ids) is shared with the
    caller, which appends the emitted ids after ``observe`` and then calls ``index``."""

    def __init__(self, seq, max_occ=MAX_OCC):
        self.seq = seq
        self.max_occ = max_occ
        self.follow = {3: {}, 2: {}}   # n -> {last n tokens: positions of the token after them}
        self.pool = {}                 # (parent token, token) -> the model's next token
        self.window = []               # Jacobi window (predicted continuation)
        self.chain = []                # the first candidate's nodes in the last drafted tree
        self.indexed = 1               # n-grams ending before this position are indexed
        self.index()

    def index(self):
        """Index every n-gram (n = 2, 3) whose following token is already known."""
        seq = self.seq
        for end in range(self.indexed, len(seq) - 1):    # n-gram seq[end-n+1 .. end]
            for n, table in self.follow.items():
                if end + 1 < n:
                    continue
                occ = table.setdefault(tuple(seq[end + 1 - n:end + 1]), [])
                occ.append(end + 1)
                if len(occ) > self.max_occ:
                    occ.pop(0)
        self.indexed = max(self.indexed, len(seq) - 1)

    def candidates(self, depth):
        """Candidate continuations in priority order (window, 3-gram, 2-gram, pool chain)."""
        seq, out = self.seq, []
        if self.window:
            out.append(self.window[:depth])
        for n in (3, 2):
            if len(seq) >= n:
                for p in reversed(self.follow[n].get(tuple(seq[-n:]), ())):
                    out.append(seq[p:p + depth])
        if len(seq) >= 2:
            chain, a, b = [], seq[-2], seq[-1]
            while len(chain) < depth and (a, b) in self.pool:
                c = self.pool[(a, b)]
                chain.append(c)
                a, b = b, c
            if chain:
                out.append(chain)
        return out

    def draft(self, T, depth):
        """The trie of this pass (padded to T nodes)."""
        tree = Tree(self.seq[-1])
        cands = self.candidates(depth) or [[self.seq[-1]] * depth]
        self.chain = []
        for i, c in enumerate(cands):
            nodes = tree.add_path(c, T)
            if i == 0:
                self.chain = nodes
            if len(tree.tokens) >= T:
                break
        tree.pad(T)
        return tree

    def observe(self, tree, g, path):
        """After verification (``g`` = the model's argmax after every node, ``path`` = the
        accepted nodes, before the emitted ids are appended to ``seq``): pool every real node's
        prediction and advance the window along the first candidate."""
        tok, parent = tree.tokens, tree.parent
        for i in range(tree.n_real):
            if i == 0 and len(self.seq) < 2:
                continue
            pt = self.seq[-2] if i == 0 else tok[parent[i]]
            self.pool[(pt, tok[i])] = int(g[i])
        a, chain = len(path), self.chain
        self.window = [int(g[c]) for c in chain[a:]] if len(chain) > a and chain[:a] == path else []


class LookaheadDrafter:
    """The reference's draft sources as a stateful drafter for ``Engine.generate_tree``:
    ``rows(seqs)`` gives one ``RowDraft`` per sequence for one generate call."""

    def __init__(self, max_depth=MAX_DEPTH, max_occ=MAX_OCC):
        self.max_depth = max_depth
        self.max_occ = max_occ

    def rows(self, seqs):
        return [RowDraft(s, self.max_occ) for s in seqs]
