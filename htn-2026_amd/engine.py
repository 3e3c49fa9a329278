"""Qwen3 greedy decode engine for one MI355X -- drop-in for the reference's decode path.

Interface (Yokanater/htn-2026 engine/engine.py:232-293, 1105-1132; QWEN_ENGINE_CONTRACT.md:22-36):

    from engine import Engine               # this directory on sys.path, as the reference's
    eng = Engine(model_path)                # local HF checkpoint dir (config.json + safetensors)
    for step in eng.generate(input_ids, max_new_tokens):
        ...                                 # list of B greedy ids, exactly max_new_tokens times

Semantics kept from the reference: equal-length prompts, no EOS stop, exactly N yields (none
for N <= 0), prompt state reset on every call, the GPU kept one step ahead of the host with a
pinned ring and one event per step (engine.py:719-757).  The decode step is the fused T5
layout (engine.py:463-477) recorded once as a hipGraph; the prompt runs as causal chunks through
the block forward.  All arithmetic is in libqdecode.so (hand-written gfx950 HIP): there is no
transformers model, no torch compute and no fallback tier -- a missing library raises at import.
"""

import gc
import os
import sys
import time

import torch

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

from qdecode import _lib  # noqa: E402
from qdecode import draft as _draft  # noqa: E402
from qdecode import model as _model  # noqa: E402
from qdecode import tree as _tree  # noqa: E402

DEVICE = os.environ.get("ENGINE_DEVICE", "cuda:0")
# Tree speculation in generate() (engine.py:87, 910-936): "auto" decides per shape on its first
# call (the reference's warmup gate), "1" always, "0" never.
TREE_MODE = os.environ.get("ENGINE_TREE", "auto")
TREE_CHECK_TOKENS = 128   # tokens the gate generates each way (engine.py:88)
TREE_MIN_GAIN = 0.92      # keep trees only below this fraction of the plain wall time (engine.py:89)
TREE_MAX_ROWS = 64        # verification rows B * T: the weight-streaming GEMM regime


class _Shape:
    """Buffers, runners and graphs for one (B, S, N, mode)."""

    def __init__(self, model, stream, B, S, N, tree_T=0, prefill_rows=None, mega=None):
        self.B, self.S, self.N, self.tree_T = B, S, N, tree_T
        cap = _model.kv_capacity(S, N, extra=tree_T)
        self.kv = _model.KVState(model, B, cap)
        self.stream = stream
        self.chunk = _model.prefill_chunk(B, S, prefill_rows or _model.PREFILL_ROWS)
        self.prefill = _model.BlockRunner(self.kv, stream, self.chunk, causal=True,
                                           lm_mode=_lib.LM_LAST)
        self.decode = _model.DecodeRunner(self.kv, stream, mega=mega)
        self.tree = (_model.BlockRunner(self.kv, stream, tree_T, causal=False, lm_mode=_lib.LM_ALL)
                     if tree_T else None)
        self.ids = torch.zeros((B, S), dtype=torch.int64, device=model.device)
        self.ids_host = torch.empty((B, S), dtype=torch.int64, pin_memory=True)
        self.host = torch.empty((max(N, 1), B), dtype=torch.int64, pin_memory=True)
        # the persistent step's error word after every step (checked before that step's ids)
        self.err_host = torch.zeros((max(N, 1),), dtype=torch.int32, pin_memory=True)
        self.events = [torch.cuda.Event() for _ in range(max(N, 1))]
        self.graph_ready = False
        self._tree_pass = None

    def start(self, ids, decode_next=False):
        """Enqueue the prompt (one host-to-device copy), its causal prefill and the first
        token's readback into host row 0 (``events[0]`` marks it); with ``decode_next`` also set
        pos = S and record the decode-step graph (once per shape).  Does not wait."""
        with torch.cuda.stream(self.stream):
            self.ids_host.copy_(ids)
            self.ids.copy_(self.ids_host, non_blocking=True)
            self.run_prefill()
            self.host[0].copy_(self.kv.tok, non_blocking=True)
            self.events[0].record(self.stream)
            if decode_next:
                self.kv.pos.fill_(self.S)
                if not self.graph_ready:
                    # the step reads tok/pos from the device; capture once per shape
                    self.decode.capture()
                    self.graph_ready = True

    def first_token(self):
        """Wait for the prefill's token (enqueued by ``start``) and return it (B ids)."""
        self.events[0].synchronize()
        return self.host[0].tolist()

    def tree_pass(self):
        """The tree runner's host twin (created on first use)."""
        if self._tree_pass is None:
            self._tree_pass = _tree.TreePass(self.tree, self.stream)
        return self._tree_pass

    def run_prefill(self):
        """Causal chunks of the prompt: KV [0, S) and the first greedy token into kv.tok."""
        B, S, c = self.B, self.S, self.chunk
        pr = self.prefill
        for c0 in range(0, S, c):
            T = min(c, S - c0)
            # the block step reads tokens as [B, T] contiguous
            pr.tokens.view(-1)[:B * T].view(B, T).copy_(self.ids[:, c0:c0 + T])
            pr.base.fill_(c0)
            # only the chunk holding the last prompt token needs the LM head
            pr.launch(T, lm_mode=_lib.LM_LAST if c0 + T == S else _lib.LM_NONE)
        self.kv.tok.copy_(pr.out_tok)


class Engine:
    def __init__(self, model_path: str, device: str = DEVICE) -> None:
        self.device = torch.device(device)
        torch.cuda.set_device(self.device)
        self.model = (_model.Qwen3Model.from_checkpoint(model_path, self.device)
                      if model_path is not None else None)
        self._init_common()

    @classmethod
    def synthetic(cls, n_layers=36, seed=1, device=DEVICE):
        """Engine over seeded random-init weights generated on the device (benchmark configs)."""
        eng = cls.__new__(cls)
        eng.device = torch.device(device)
        torch.cuda.set_device(eng.device)
        eng.model = _model.Qwen3Model.synthetic(n_layers=n_layers, seed=seed, device=eng.device)
        eng._init_common()
        return eng

    def _init_common(self):
        self.stream = torch.cuda.Stream(device=self.device)   # default priority
        self.shape = None
        self.tree_T = int(os.environ.get("ENGINE_TREE_T", "0"))
        self.prefill_budget_rows = None    # rows per causal prefill chunk (None: PREFILL_ROWS)
        self.tree_stats = None
        self.tree_mode = TREE_MODE
        self.tree_on = {}                  # (B, S, N) -> the gate's decision
        self.tree_log = {}                 # (B, S, N) -> what the gate measured
        # Persistent-step tier (engine.py:1038-1045 drops T6 when its error flag fires): None
        # lets the runner choose (qd_mega_step at B = 1); False after a persistent step
        # reported an error, so every later shape runs the bit-identical per-launch step.
        self.mega = None
        self.mega_errors = []              # (B, S, N, step, error word) of each failure

    # -------------------------------------------------------------- state
    def _state(self, B, S, N, tree_T=None):
        """Buffers for (B, S, N) with a tree runner of tree_T nodes (default self.tree_T)."""
        tree_T = self.tree_T if tree_T is None else tree_T
        sh = self.shape
        if sh is not None and (sh.B, sh.S, sh.N, sh.tree_T) == (B, S, N, tree_T) and \
                not (self.mega is False and sh.decode.mega):
            return sh
        if sh is not None:
            sh.decode.close()
        self.shape = None
        gc.collect()
        torch.cuda.empty_cache()
        with torch.cuda.stream(self.stream):
            sh = _Shape(self.model, self.stream, B, S, N, tree_T, self.prefill_budget_rows,
                        mega=self.mega)
        self.stream.synchronize()
        self.shape = sh
        return sh

    @staticmethod
    def _check_ids(input_ids, vocab):
        if not input_ids or not isinstance(input_ids, (list, tuple)):
            raise ValueError("input_ids must be a non-empty list of token-id lists")
        S = len(input_ids[0])
        if S == 0 or any(len(r) != S for r in input_ids):
            raise ValueError("every sequence in input_ids must have the same, non-zero length")
        t = torch.tensor(input_ids, dtype=torch.int64)
        if int(t.min()) < 0 or int(t.max()) >= vocab:
            raise IndexError(f"token ids must lie in [0, {vocab})")
        return t

    # -------------------------------------------------------------- API
    def generate(self, input_ids, max_new_tokens):
        N = int(max_new_tokens)
        if N <= 0:
            return
        ids = self._check_ids(input_ids, self.model.V)
        B, S = ids.shape
        T = self._tree_width(B, N)
        gc_was = gc.isenabled()
        gc.disable()
        try:
            sh = self._state(B, S, N, T)
            key = (B, S, N)
            if T and key not in self.tree_on:
                if self.tree_mode == "1":
                    self.tree_on[key] = True
                else:
                    # the reference disables tree speculation when its gate fails for any
                    # reason (engine.py:934-936); plain decode then serves this shape
                    try:
                        self.tree_on[key] = self._decide_tree(sh, ids, min(N, TREE_CHECK_TOKENS))
                    except Exception as exc:          # noqa: BLE001  (logged, tier dropped)
                        self.tree_on[key] = False
                        self.tree_log[key] = {"on": False, "error": repr(exc)[:200]}
                        sh = self._state(B, S, N, T)
            if T and self.tree_on[key]:
                yield from _tree.stream_tree(self, sh, ids, N, _draft.LookaheadDrafter())
            else:
                yield from self._stream_plain(sh, ids, N)
        finally:
            if gc_was:
                gc.enable()

    def _tree_width(self, B, N):
        """Verification tree size for tree speculation in generate() (0: off): as many nodes as
        keep B * T within TREE_MAX_ROWS, between 8 and 64 (the ancestor mask is 64 bits)."""
        if self.tree_mode == "0" or N <= 1 or B * 8 > TREE_MAX_ROWS:
            return 0
        return min(64, TREE_MAX_ROWS // B)

    def _decide_tree(self, sh, ids, n):
        """The warmup gate (engine.py:910-936): n tokens with tree speculation and n plain on
        the same buffers; keep trees only if they emit exactly the plain greedy ids and take
        less than TREE_MIN_GAIN of the plain wall time (best of two runs each, timed only when
        the ids agree: otherwise trees are off whatever their speed)."""
        def run(tree):
            t0 = time.perf_counter()
            it = (_tree.stream_tree(self, sh, ids, n, _draft.LookaheadDrafter()) if tree
                  else self._stream_plain(sh, ids, n))
            out = list(it)
            return out, time.perf_counter() - t0
        plain, _ = run(False)
        tree, _ = run(True)
        exact = tree == plain
        acc = (self.tree_stats or {}).get("accepted") or [1]
        ms_tree = ms_plain = None
        if exact:                  # the timing only chooses between two paths with the same ids
            ms_tree = round(min(run(True)[1] for _ in range(2)) * 1e3, 3)
            ms_plain = round(min(run(False)[1] for _ in range(2)) * 1e3, 3)
        on = exact and ms_tree < TREE_MIN_GAIN * ms_plain
        self.tree_log[(sh.B, sh.S, sh.N)] = {
            "tokens": n, "exact": exact, "tree_ms": ms_tree, "plain_ms": ms_plain,
            "accept_mean": round(sum(acc) / len(acc), 3), "T": sh.tree_T, "on": on}
        return on

    def _stream_plain(self, sh, ids, N):
        """Prefill, then N-1 graph replays of the decode step; the host yields step t-1 while
        the device runs step t (engine.py:719-757)."""
        sh.start(ids, decode_next=N > 1)
        err = sh.decode.err_word
        for t in range(1, N):
            with torch.cuda.stream(self.stream):
                sh.decode.replay()
                sh.host[t].copy_(sh.kv.tok, non_blocking=True)
                if err is not None:       # the persistent step's error word, read with its ids
                    sh.err_host[t:t + 1].copy_(err, non_blocking=True)
                sh.events[t].record(self.stream)
            sh.events[t - 1].synchronize()
            self._check_step(sh, t - 1)
            yield sh.host[t - 1].tolist()
        sh.events[N - 1].synchronize()
        self._check_step(sh, N - 1)
        yield sh.host[N - 1].tolist()

    def _check_step(self, sh, t):
        """Raise before step t's ids are handed out if the persistent step reported an error
        (a hand-off wait expired or pos fell outside the cache).  The error word stays set from
        the failing step on, so no id of that step or a later one is yielded.  The runner's
        workspace is zeroed (epoch, error word and hand-off words start clean) and the engine
        drops the persistent tier: every later call runs the per-launch step, which is
        bit-identical to it."""
        if sh.decode.err_word is None or t == 0:      # step 0 comes from the prefill
            return
        code = int(sh.err_host[t])
        if code == 0:
            return
        self.stream.synchronize()
        sh.decode.reset()
        self.mega = False
        self.mega_errors.append((sh.B, sh.S, sh.N, t, code))
        raise RuntimeError(f"persistent decode step {t} failed (error word {code}); no ids of it "
                           "were yielded and later calls run the per-launch decode step")

    # -------------------------------------------------------------- tree speculation
    def generate_tree(self, input_ids, max_new_tokens, drafter=None, T=64):
        """Exact token-tree speculative decoding (engine.py:830-908): every step verifies a
        T-node draft tree per sequence in one block forward and emits the longest
        greedy-matching path.  ``drafter``: ``draft.LookaheadDrafter`` (the default: window,
        n-gram and prediction-pool sources) or any ``drafter(seq, T) -> tree.Tree``."""
        N = int(max_new_tokens)
        if N <= 0:
            return
        ids = self._check_ids(input_ids, self.model.V)
        B, S = ids.shape
        if not 2 <= T <= 64:
            raise ValueError("T must lie in [2, 64] (64-bit ancestor masks)")
        sh = self._state(B, S, N, T)
        yield from _tree.stream_tree(self, sh, ids, N, drafter or _draft.LookaheadDrafter())
