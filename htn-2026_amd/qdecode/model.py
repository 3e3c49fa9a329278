"""Device-resident Qwen3 decoder: packed weights, KV cache, step runners and hipGraphs.

Weights are stacked per kind exactly as the reference packs them (engine/engine.py:250-282):
  w_qkv [L, (Hq + 2 Hkv) * 128, H] = q | k | v,  w_o [L, H, Hq * 128],
  w_gu  [L, 2 I, H] = gate | up,                 w_down [L, H, I],
  ln1 / ln2 [L, H], q_norm / k_norm [L, 128], embed [V, H] (tied lm_head), final_norm [H].
The KV cache is [L, B, Hkv, cap, 128] bf16 per K and V (engine.py:178-181).

``DecodeRunner`` owns the per-step buffers of one batch size and replays the whole decode
step as one hipGraph: at B = 1 on a device that supports it the persistent step (qd_mega_step,
one launch; ``QD_MEGA=0`` selects the per-launch step), otherwise qd_decode_step
(embed, 5-7 launches per layer, LM head + argmax + pos += 1);
``BlockRunner`` runs T tokens per sequence through every layer (tree verification, or a causal
chunk of the prompt).  Every launch goes to the runner's own HIP stream (default priority).
"""

import ctypes as C
import os

import torch

from . import _lib, ops
from .checkpoint import SafeTensors, read_config
from .inputs import BlockInputs

BF16 = torch.bfloat16

QWEN3_4B = {"hidden_size": 2560, "intermediate_size": 9728, "num_hidden_layers": 36,
            "num_attention_heads": 32, "num_key_value_heads": 8, "head_dim": 128,
            "vocab_size": 151936, "rms_norm_eps": 1e-6, "rope_theta": 5000000.0,
            "tie_word_embeddings": True}

# tensor ids of the synthetic generator (one stream per HF parameter)
_SYNTH_KIND = {"q_proj": 0, "k_proj": 1, "v_proj": 2, "o_proj": 3, "gate_proj": 4, "up_proj": 5,
               "down_proj": 6}


def synth_stream(name):
    if name == "model.embed_tokens.weight":
        return 1
    parts = name.split(".")
    return 16 + 16 * int(parts[2]) + _SYNTH_KIND[parts[4]]


def rope_tables(n_pos, theta, dim=128):
    """cos, sin [n_pos, dim] bf16 (host).  Same arithmetic as the reference's rotary module
    (engine/engine.py:182-185 -> TF:modeling_qwen3.py:104-137): fp32 inverse frequencies
    theta^(-2i/dim), one fp32 product per angle, cos/sin in fp32, rounded to bf16.  Computed
    once per state on the host; the decode kernels read the table."""
    inv = 1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.int64).to(torch.float32) / dim))
    pos = torch.arange(n_pos, dtype=torch.int64).to(torch.float32)
    freqs = pos[:, None] * inv[None, :]
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(BF16), emb.sin().to(BF16)


class Qwen3Model:
    """Packed, stacked bf16 weights on one device and their qd_weights view."""

    def __init__(self, cfg, device):
        self.cfg = dict(cfg)
        self.device = torch.device(device)
        c = self.cfg
        L, H, I, V = (c["num_hidden_layers"], c["hidden_size"], c["intermediate_size"],
                      c["vocab_size"])
        Hq, Hkv, D = c["num_attention_heads"], c["num_key_value_heads"], c["head_dim"]
        if D != 128 or Hq != 4 * Hkv:
            raise ValueError("the kernels implement head_dim 128 with 4 query heads per KV head")
        self.L, self.H, self.I, self.V, self.Hq, self.Hkv = L, H, I, V, Hq, Hkv
        self.eps = c["rms_norm_eps"]
        self.theta = c["rope_theta"]
        new = lambda *s: torch.empty(s, dtype=BF16, device=self.device)  # noqa: E731
        self.embed = new(V, H)
        self.final_norm = new(H)
        self.w_qkv = new(L, (Hq + 2 * Hkv) * D, H)
        self.w_o = new(L, H, Hq * D)
        self.w_gu = new(L, 2 * I, H)
        self.w_down = new(L, H, I)
        self.ln1, self.ln2 = new(L, H), new(L, H)
        self.q_norm, self.k_norm = new(L, D), new(L, D)
        # the output projection: the embedding itself when tied (engine.py:246-247), else its
        # own [V, H] tensor (lm_head.weight)
        self.tied = bool(c.get("tie_word_embeddings", True))
        self.lm_head = self.embed if self.tied else new(V, H)
        self.qd = _lib.Weights(
            L, H, I, V, Hq, Hkv, D, self.eps, self.embed.data_ptr(), self.final_norm.data_ptr(),
            self.w_qkv.data_ptr(), self.w_o.data_ptr(), self.w_gu.data_ptr(),
            self.w_down.data_ptr(), self.ln1.data_ptr(), self.ln2.data_ptr(),
            self.q_norm.data_ptr(), self.k_norm.data_ptr(),
            None if self.tied else self.lm_head.data_ptr())

    # -------------------------------------------------------------- where each HF tensor lives
    def slots(self):
        """(HF parameter name, destination view) for every parameter of the checkpoint."""
        D = 128
        nq, nkv = self.Hq * D, self.Hkv * D
        out = [("model.embed_tokens.weight", self.embed), ("model.norm.weight", self.final_norm)]
        if not self.tied:
            out.append(("lm_head.weight", self.lm_head))
        for i in range(self.L):
            p = f"model.layers.{i}."
            out += [
                (p + "self_attn.q_proj.weight", self.w_qkv[i, :nq]),
                (p + "self_attn.k_proj.weight", self.w_qkv[i, nq:nq + nkv]),
                (p + "self_attn.v_proj.weight", self.w_qkv[i, nq + nkv:]),
                (p + "self_attn.o_proj.weight", self.w_o[i]),
                (p + "mlp.gate_proj.weight", self.w_gu[i, :self.I]),
                (p + "mlp.up_proj.weight", self.w_gu[i, self.I:]),
                (p + "mlp.down_proj.weight", self.w_down[i]),
                (p + "input_layernorm.weight", self.ln1[i]),
                (p + "post_attention_layernorm.weight", self.ln2[i]),
                (p + "self_attn.q_norm.weight", self.q_norm[i]),
                (p + "self_attn.k_norm.weight", self.k_norm[i]),
            ]
        return out

    @classmethod
    def from_checkpoint(cls, path, device="cuda:0"):
        """Load a local HF checkpoint (engine.py:237-247 without transformers): every tensor of
        ``slots()`` must be present with its HF shape; an untied checkpoint must hold
        ``lm_head.weight``."""
        cfg = read_config(path)
        st = SafeTensors(path)
        if not cfg["tie_word_embeddings"] and "lm_head.weight" not in st:
            raise ValueError("tie_word_embeddings is false but the checkpoint has no lm_head.weight")
        m = cls(cfg, device)
        for name, dst in m.slots():
            if name not in st:
                raise KeyError(f"checkpoint {path} lacks {name}")
            t = st.get(name)
            if tuple(t.shape) != tuple(dst.shape):
                raise ValueError(f"{name}: checkpoint shape {tuple(t.shape)} != {tuple(dst.shape)}")
            dst.copy_(t.to(BF16), non_blocking=False)
        torch.cuda.synchronize(m.device)
        return m

    @classmethod
    def synthetic(cls, n_layers=36, seed=1, std=0.02, device="cuda:0", cfg=None):
        """Seeded random-init weights generated on the device by qd_synth_bf16 (norm weights
        1.0); bit-identical to the CPU generator in oracle/synth.py."""
        c = dict(cfg or QWEN3_4B)
        c["num_hidden_layers"] = n_layers
        m = cls(c, device)
        with torch.cuda.device(m.device):
            for name, dst in m.slots():
                if name.endswith("norm.weight"):
                    ops.fill_bf16(dst, 0x3F80)
                else:
                    ops.synth_bf16(dst, seed, synth_stream(name), 0, std)
            torch.cuda.synchronize(m.device)
        return m

    @property
    def weight_bytes(self):
        """Algorithmic weight bytes read by one decode step (all projections + the LM head)."""
        return 2 * (self.w_qkv.numel() + self.w_o.numel() + self.w_gu.numel() + self.w_down.numel()
                    + self.lm_head.numel())

    @property
    def kv_bytes_per_token(self):
        return self.L * 2 * self.Hkv * 128 * 2


class KVState:
    """KV cache + RoPE tables + device token/position state for B sequences of capacity cap."""

    def __init__(self, model, batch, cap):
        self.model, self.B, self.cap = model, batch, cap
        dev = model.device
        shape = (model.L, batch, model.Hkv, cap, 128)
        self.k = torch.zeros(shape, dtype=BF16, device=dev)
        self.v = torch.zeros(shape, dtype=BF16, device=dev)
        cos, sin = rope_tables(cap, model.theta)
        self.cos, self.sin = cos.to(dev), sin.to(dev)
        self.tok = torch.zeros((batch,), dtype=torch.int64, device=dev)
        self.pos = torch.zeros((1,), dtype=torch.int64, device=dev)


def mega_default(model, batch, cap=None):
    """Whether a decode step of `batch` sequences runs as the persistent kernel by default: at
    B = 1 when the device and shape support it, unless QD_MEGA=0 is set.  (A batched form for
    17..32 sequences was bit-identical to the per-launch step and not faster on MI355X, 3.99
    against 3.87 ms per B = 32 step: every hand-off waited for the slowest of up to 256
    producers plus a memory round trip queued behind the weight stream, which cost what the
    launch boundaries did; it was removed.)"""
    if os.environ.get("QD_MEGA", "1") == "0" or batch != 1:
        return False
    if not _lib.LIB.qd_mega_supported(C.byref(model.qd), batch):
        return False
    return cap is None or _lib.LIB.qd_mega_workspace_bytes(C.byref(model.qd), batch, cap) > 0


class DecodeRunner:
    """One greedy decode step for all B sequences, eager or as a hipGraph: the persistent
    qd_mega_step (mega=True, B = 1) or qd_decode_step.  mega=None picks mega_default()."""

    def __init__(self, kv, stream, mega=None):
        m = kv.model
        self.kv, self.model, self.stream = kv, m, stream
        B, dev = kv.B, m.device
        self.mega = mega_default(m, B, kv.cap) if mega is None else bool(mega)
        self.x = torch.empty((B, m.H), dtype=BF16, device=dev)
        self.qkv = torch.empty((B, (m.Hq + 2 * m.Hkv) * 128), dtype=BF16, device=dev)
        self.attn = torch.empty((B, m.Hq * 128), dtype=BF16, device=dev)
        self.act = torch.empty((B, m.I), dtype=BF16, device=dev)
        nbytes = _lib.LIB.qd_decode_workspace_bytes(C.byref(m.qd), B, kv.cap)
        self.ctl = None
        if self.mega:
            nbytes = _lib.LIB.qd_mega_workspace_bytes(C.byref(m.qd), B, kv.cap)
            if nbytes <= 0:
                raise _lib.QDError("qd_mega_workspace_bytes", _lib.QD_EARG)
            self.ctl_off = _lib.LIB.qd_mega_ctl_offset(C.byref(m.qd), B, kv.cap)
        # zero-filled once: the persistent step's epoch and hand-off words start at 0
        self.ws = torch.zeros((nbytes,), dtype=torch.uint8, device=dev)
        # device view of the persistent step's error word (None for qd_decode_step)
        self.err_word = (self.ws[self.ctl_off + 4:self.ctl_off + 8].view(torch.int32)
                         if self.mega else None)
        self.st = _lib.DecodeState(
            B, kv.cap, kv.k.data_ptr(), kv.v.data_ptr(), kv.cos.data_ptr(), kv.sin.data_ptr(),
            kv.tok.data_ptr(), kv.pos.data_ptr(), self.x.data_ptr(), self.qkv.data_ptr(),
            self.attn.data_ptr(), self.act.data_ptr(), self.ws.data_ptr(), nbytes)
        self.graph = None
        self.direct = True       # the persistent step replays as a direct launch (see replay)

    def enqueue(self):
        fn = "qd_mega_step" if self.mega else "qd_decode_step"
        _lib.call(fn, C.byref(self.model.qd), C.byref(self.st), self.stream.cuda_stream)

    def mega_status(self):
        """(epoch, error) words of the persistent step (synchronises the runner's stream)."""
        if not self.mega:
            return 0, 0
        self.stream.synchronize()
        w = self.ws[self.ctl_off:self.ctl_off + 8].view(torch.int32).cpu().tolist()
        return w[0], w[1]

    def check(self):
        """Raise if a persistent step reported an error (expired hand-off wait or bad pos)."""
        _, err = self.mega_status()
        if err:
            raise RuntimeError(f"persistent decode step failed (error word {err})")

    def reset(self):
        """Zero the workspace on the runner's stream: the persistent step's epoch, error word
        and both hand-off copies start clean, as before the first step."""
        with torch.cuda.stream(self.stream):
            self.ws.zero_()
        self.stream.synchronize()

    def capture(self):
        """Record one step into a hipGraph (the step has no host inputs: tok/pos are on device)."""
        s = self.stream.cuda_stream
        _lib.call("qd_graph_begin", s)
        try:
            self.enqueue()
        finally:
            ex = C.c_void_p()
            rc = _lib.LIB.qd_graph_end(s, C.byref(ex))
        if rc != 0:
            raise _lib.QDError("qd_graph_end", rc)
        self.graph = ex

    def replay(self):
        """One decode step on the runner's stream: the captured graph, or a direct launch when
        nothing was captured or the step is the persistent kernel with ``direct`` set (one
        kernel either way; back to back, a direct launch of it leaves ~5 us less between steps
        than a one-node graph: 1.4163 against 1.4211 ms per config-3 step on MI355X)."""
        if self.graph is None or (self.mega and self.direct):
            self.enqueue()
        else:
            _lib.call("qd_graph_launch", self.graph, self.stream.cuda_stream)

    def close(self):
        if self.graph is not None:
            _lib.LIB.qd_graph_destroy(self.graph)
            self.graph = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class BlockRunner:
    """T_max tokens per sequence through every layer (qd_block_step): causal prompt chunks
    (prefill) or tree verification with ancestor masks."""

    use_graphs = True        # launch() replays recorded hipGraphs (False: kernel by kernel)

    def __init__(self, kv, stream, t_max, causal, lm_mode):
        m = kv.model
        self.kv, self.model, self.stream = kv, m, stream
        self.t_max, self.causal, self.lm_mode = t_max, causal, lm_mode
        B, dev = kv.B, m.device
        M = B * t_max
        e = lambda *s: torch.empty(s, dtype=BF16, device=dev)  # noqa: E731
        self.x, self.xn = e(M, m.H), e(M, m.H)
        self.qkv = e(M, (m.Hq + 2 * m.Hkv) * 128)
        self.q, self.attn = e(M, m.Hq * 128), e(M, m.Hq * 128)
        self.act = e(M, m.I)
        self.inputs = BlockInputs(B, t_max, device=dev)
        inp = self.inputs
        self.tokens, self.base, self.depth, self.anc = inp.tokens, inp.base, inp.depth, inp.anc
        self.c_base, self.c_src, self.c_cnt = inp.c_base, inp.c_src, inp.c_cnt
        self.out_tok = torch.zeros((M if lm_mode == _lib.LM_ALL else B,), dtype=torch.int64,
                                   device=dev)
        # sized for the runner's own LM mode (a prefill runner ranks one row per sequence, or
        # none) and every T <= t_max; a launch asking for more fails with QD_EWS
        nbytes = _lib.LIB.qd_block_workspace_bytes_lm(C.byref(m.qd), B, t_max, kv.cap, lm_mode)
        self.ws = torch.zeros((nbytes,), dtype=torch.uint8, device=dev)
        # hipGraphs of the forward, one per (T, compact, lm_mode): the forward reads every input
        # (tokens, base, depth, anc, compaction lists) from these device buffers, so a replay
        # after the buffers are rewritten runs the new inputs (engine.py:685-713 captures its
        # prefill / verify / tree forwards the same way)
        self.graphs = {}

    def state(self, T, compact=False, lm_mode=None):
        kv = self.kv
        return _lib.BlockState(
            kv.B, T, 1 if self.causal else 0, self.lm_mode if lm_mode is None else lm_mode, kv.cap,
            kv.k.data_ptr(), kv.v.data_ptr(), kv.cos.data_ptr(), kv.sin.data_ptr(),
            self.tokens.data_ptr(), self.base.data_ptr(),
            None if self.causal else self.depth.data_ptr(),
            None if self.causal else self.anc.data_ptr(),
            self.c_base.data_ptr() if compact else None, self.c_src.data_ptr() if compact else None,
            self.c_cnt.data_ptr() if compact else None, self.out_tok.data_ptr(),
            self.x.data_ptr(), self.xn.data_ptr(), self.qkv.data_ptr(), self.q.data_ptr(),
            self.attn.data_ptr(), self.act.data_ptr(), self.ws.data_ptr(), self.ws.numel())

    def enqueue(self, T=None, compact=False, lm_mode=None):
        """One forward, launched kernel by kernel on the runner's stream."""
        T = self.t_max if T is None else T
        if not 0 < T <= self.t_max:
            raise ValueError(f"T={T} outside (0, {self.t_max}]")
        st = self.state(T, compact, lm_mode)
        _lib.call("qd_block_step", C.byref(self.model.qd), C.byref(st), self.stream.cuda_stream)

    def launch(self, T=None, compact=False, lm_mode=None):
        """One forward as a graph replay (recorded on the first call with these arguments), or
        kernel by kernel when use_graphs is off.  Same kernels, same bits either way."""
        T = self.t_max if T is None else T
        if not self.use_graphs:
            return self.enqueue(T, compact, lm_mode)
        key = (T, bool(compact), self.lm_mode if lm_mode is None else lm_mode)
        g = self.graphs.get(key)
        if g is None:
            s = self.stream.cuda_stream
            _lib.call("qd_graph_begin", s)
            try:
                self.enqueue(T, compact, lm_mode)
            finally:
                ex = C.c_void_p()
                rc = _lib.LIB.qd_graph_end(s, C.byref(ex))
            if rc != 0:
                raise _lib.QDError("qd_graph_end", rc)
            g = self.graphs[key] = ex
        _lib.call("qd_graph_launch", g, self.stream.cuda_stream)

    def close(self):
        for g in self.graphs.values():
            _lib.LIB.qd_graph_destroy(g)
        self.graphs = {}

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# Rows per causal prefill forward.  32768 = 128 blocks of the prefill GEMM's 256-row tiles: every
# projection's tile grid is a whole number of rounds over 256 CUs (qkv 3072 tiles, o / down 1280,
# gate/up 9728), and four prompts of 8192 tokens go through in one chunk.
# Measured on MI355X (prefill + first token, second of three runs): 4 x 8192 0.330 s (6144 rows:
# 0.342, 8192: 0.356, 12288: 0.335, 16384: 0.330, 24576: 0.336); 32 x 2048 0.515 s (6144: 0.541,
# 8192: 0.578, 12288: 0.521, 16384: 0.527, 24576: 0.524).  The block step's buffers grow with it
# (1.91 GB of activations at 32768 rows; its workspace stays at ~34 MB whatever the context).
PREFILL_ROWS = 32768


def prefill_chunk(B, S, budget_rows=PREFILL_ROWS):
    """Prompt tokens per sequence per causal chunk: at most budget_rows rows per forward."""
    return max(1, min(S, budget_rows // max(B, 1)))


def kv_capacity(S, N, extra=0):
    return S + max(N, 1) + extra
