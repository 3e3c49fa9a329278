"""Op-by-op torch-CPU restatement of the Qwen3 forward used by the reference's decode path --
TEST INFRASTRUCTURE ONLY (never imported by the product path).

The reference engine (Yokanater/htn-2026 engine/engine.py) takes its arithmetic from the
third-party ``transformers`` Qwen3ForCausalLM (pinned 4.51.3, requirements.txt:10; the
container has 5.15.0 whose Qwen3 ops are unchanged).  Each function below restates one
transformers op with the rounding points the reference's kernels document:

  rmsnorm          TF:modeling_qwen3.py:59-64; reference engine/kernels/rmsnorm.py:26-31
                   (fp32 reduce, normalise in fp32, ROUND TO BF16, then multiply the bf16 weight)
  rope_tables      TF:modeling_qwen3.py:104-137 (fp32 inv_freq / angles, cos/sin -> bf16);
                   reference engine/engine.py:182-185
  apply_rope       TF:modeling_qwen3.py:140-170; reference engine/kernels/fused.py:72-74
                   (every product and the sum are bf16 tensors)
  qk_norm_rope     TF:modeling_qwen3.py:252-257 + the two above; fused.py:24-98
  swiglu           TF:modeling_qwen3.py:81-83; fused.py:101-110 (silu in fp32 -> bf16, * up -> bf16)
  linear           nn.Linear (bf16 in/out, fp32 accumulate); gemv.py:1-9
  attention        SDPA / eager GQA, TF:modeling_qwen3.py:185-207; decode_attn.py:7-11
                   (fp32 scores, fp32 softmax, P rounded to bf16 before P@V, /l in fp32)
  Qwen3Ref.forward TF:modeling_qwen3.py:241-323, 423, 494-495 (decoder layer order, final norm,
                   tied lm_head); chunk form with explicit cache slots, RoPE positions and a
                   visibility mask so that prefill, decode and tree verification
                   (engine/kernels/tree.py:1-11) share one statement
  greedy           engine/engine.py:963-972 (_native greedy KV-cache loop)
  teacher_force    engine/engine.py:974-996 (margin of emitted tokens under a full forward)

How each is pinned (tests/test_oracle.py):
  rmsnorm, rope_tables, apply_rope, qk_norm_rope, swiglu, linear, attention, one decoder
  layer, and the 4-layer greedy loop (config 1: tokens, top-8 logits, margins) are compared
  with golden vectors that tests/golden/make_golden.py wrote by running transformers'
  own modules on the same inputs;
  closed forms: rmsnorm of a constant row, rope at position 0 (identity), norm preservation
  of the rotation, silu(0) = 0, a single visible key returns its V, identical keys return
  mean(V), attention against torch.nn.functional.scaled_dot_product_attention;
  the tree forward is checked against the chain (causal) forward on a chain-shaped tree and
  against sequential decode on every root-to-leaf path.
"""

import math

import numpy as np
import torch
import torch.nn.functional as F

BF16 = torch.bfloat16
F32 = torch.float32


def bf(x):
    """Round fp32 values through bf16 (RNE) and back."""
    return x.to(BF16).to(F32)


def bits_to_bf16(bits):
    """numpy uint16 bf16 bit patterns -> torch bf16 tensor (same shape)."""
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(BF16)


def bf16_to_bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


# ------------------------------------------------------------------ ops
def rmsnorm(x, w, eps=1e-6):
    xf = x.to(F32)
    var = xf.pow(2).mean(-1, keepdim=True)
    xf = xf * torch.rsqrt(var + eps)
    return w * xf.to(BF16)


def add_rmsnorm(x, residual, w, eps=1e-6):
    """Residual add then RMSNorm: r' = bf16(x + r) (the decoder layer's `residual + h`),
    y = rmsnorm(r').  Returns (r', y)."""
    r = x + residual
    return r, rmsnorm(r, w, eps)


def rope_inv_freq(theta=5000000.0, dim=128):
    return 1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.int64).to(F32) / dim))


def rope_tables(n_pos, theta=5000000.0, dim=128):
    """cos, sin [n_pos, dim] bf16 for absolute positions 0..n_pos-1."""
    inv = rope_inv_freq(theta, dim)
    pos = torch.arange(n_pos, dtype=torch.int64).to(F32)
    freqs = pos[:, None] * inv[None, :]                 # one fp32 product per element
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(BF16), emb.sin().to(BF16)


def rotate_half(x):
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def apply_rope(x, cos, sin):
    """x [..., D] bf16; cos/sin broadcastable bf16."""
    return (x * cos) + (rotate_half(x) * sin)


def qk_norm_rope(q, k, qn, kn, cos, sin, eps=1e-6):
    """q [B, T, Hq, D], k [B, T, Hkv, D] bf16; cos/sin [B, T, D] bf16 (per-token positions).
    Returns (q', k') of the same shapes."""
    c, s = cos[:, :, None, :], sin[:, :, None, :]
    return apply_rope(rmsnorm(q, qn, eps), c, s), apply_rope(rmsnorm(k, kn, eps), c, s)


def swiglu(g, u):
    return F.silu(g) * u


def linear(x, w):
    return F.linear(x, w)


def repeat_kv(x, n_rep):
    b, h, s, d = x.shape
    return x[:, :, None].expand(b, h, n_rep, s, d).reshape(b, h * n_rep, s, d)


def attention(q, k, v, visible, scale=None):
    """q [B, Hq, T, D]; k, v [B, Hkv, S, D] bf16; visible bool broadcastable to [B, 1, T, S].
    fp32 scores and softmax, P rounded to bf16 before P @ V, fp32 accumulate, / l, -> bf16."""
    hq, hkv, d = q.shape[1], k.shape[1], q.shape[-1]
    scale = d ** -0.5 if scale is None else scale
    kf = repeat_kv(k, hq // hkv).to(F32)
    vf = repeat_kv(v, hq // hkv).to(F32)
    s = (q.to(F32) @ kf.transpose(-1, -2)) * scale
    s = s.masked_fill(~visible, float("-inf"))
    m = s.amax(-1, keepdim=True)
    p = torch.exp(s - m)
    l = p.sum(-1, keepdim=True)
    o = (bf(p) @ vf) / l
    return o.to(BF16)


def argmax_lowest(logits):
    """Greedy id per row; lowest index among exact ties (torch.argmax semantics)."""
    return torch.argmax(logits.to(F32), dim=-1)


# ------------------------------------------------------------------ model
class Qwen3Ref:
    """Qwen3 decoder on CPU with a static KV cache [L, B, Hkv, cap, D] (bf16)."""

    def __init__(self, params, cfg):
        self.cfg = cfg
        self.L = cfg["num_hidden_layers"]
        self.H = cfg["hidden_size"]
        self.Hq = cfg["num_attention_heads"]
        self.Hkv = cfg["num_key_value_heads"]
        self.D = cfg["head_dim"]
        self.eps = cfg["rms_norm_eps"]
        self.theta = cfg["rope_theta"]
        self.p = params
        self.embed = params["model.embed_tokens.weight"]
        # untied checkpoints carry their own output projection (TF:modeling_qwen3.py:494-495)
        self.lm_head = params.get("lm_head.weight", self.embed)

    @classmethod
    def from_synth(cls, seed, n_layers, tied=True):
        from . import synth
        cfg = dict(synth.QWEN3_4B)
        cfg["num_hidden_layers"] = n_layers
        cfg["tie_word_embeddings"] = tied
        params = {n: bits_to_bf16(synth.param_bits(seed, n, s))
                  for n, s in synth.param_shapes(cfg).items()}
        return cls(params, cfg)

    def new_cache(self, B, cap):
        shape = (self.L, B, self.Hkv, cap, self.D)
        return torch.zeros(shape, dtype=BF16), torch.zeros(shape, dtype=BF16)

    def layer_params(self, i):
        p = f"model.layers.{i}."
        g = lambda n: self.p[p + n]  # noqa: E731
        return (g("input_layernorm.weight"), g("self_attn.q_proj.weight"), g("self_attn.k_proj.weight"),
                g("self_attn.v_proj.weight"), g("self_attn.q_norm.weight"), g("self_attn.k_norm.weight"),
                g("self_attn.o_proj.weight"), g("post_attention_layernorm.weight"),
                g("mlp.gate_proj.weight"), g("mlp.up_proj.weight"), g("mlp.down_proj.weight"))

    def forward(self, ids, rope_pos, slots, visible, cache, last_only=False, return_hidden=False):
        """ids, rope_pos, slots int64 [B, T]; visible bool [B, T, cap] over cache slots (after
        this chunk's K/V are written).  Writes K/V at ``slots``.  Returns bf16 logits
        [B, T, V] (or [B, 1, V] with last_only)."""
        kc, vc = cache
        B, T = ids.shape
        cap = kc.shape[3]
        cos_t, sin_t = rope_tables(int(rope_pos.max()) + 1, self.theta, self.D)
        cos, sin = cos_t[rope_pos], sin_t[rope_pos]                 # [B, T, D]
        x = self.embed[ids]                                          # [B, T, H]
        bidx = torch.arange(B)[:, None].expand(B, T)
        for i in range(self.L):
            ln1, wq, wk, wv, qn, kn, wo, ln2, wg, wu, wd = self.layer_params(i)
            h = rmsnorm(x, ln1, self.eps)
            q = linear(h, wq).view(B, T, self.Hq, self.D)
            k = linear(h, wk).view(B, T, self.Hkv, self.D)
            v = linear(h, wv).view(B, T, self.Hkv, self.D)
            q, k = qk_norm_rope(q, k, qn, kn, cos, sin, self.eps)
            kc[i][bidx, :, slots] = k                                 # [B, T, Hkv, D] at slot
            vc[i][bidx, :, slots] = v
            a = attention(q.transpose(1, 2), kc[i], vc[i], visible[:, None, :, :])
            x = x + linear(a.transpose(1, 2).reshape(B, T, self.Hq * self.D), wo)
            h = rmsnorm(x, ln2, self.eps)
            x = x + linear(swiglu(linear(h, wg), linear(h, wu)), wd)
        if last_only:
            x = x[:, -1:]
        h = rmsnorm(x, self.p["model.norm.weight"], self.eps)
        logits = linear(h, self.lm_head)
        return (logits, x) if return_hidden else logits

    def decoder_layer(self, i, x):
        """Layer i on hidden states x [B, T, H] at positions 0..T-1, causal, no cache
        (TF:modeling_qwen3.py:294-323)."""
        B, T, _ = x.shape
        cos_t, sin_t = rope_tables(T, self.theta, self.D)
        pos = torch.arange(T)[None, :].expand(B, T)
        cos, sin = cos_t[pos], sin_t[pos]
        ln1, wq, wk, wv, qn, kn, wo, ln2, wg, wu, wd = self.layer_params(i)
        h = rmsnorm(x, ln1, self.eps)
        q = linear(h, wq).view(B, T, self.Hq, self.D)
        k = linear(h, wk).view(B, T, self.Hkv, self.D)
        v = linear(h, wv).view(B, T, self.Hkv, self.D)
        q, k = qk_norm_rope(q, k, qn, kn, cos, sin, self.eps)
        visible = torch.tril(torch.ones((T, T), dtype=torch.bool))[None, None]
        a = attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), visible)
        x = x + linear(a.transpose(1, 2).reshape(B, T, self.Hq * self.D), wo)
        h = rmsnorm(x, ln2, self.eps)
        return x + linear(swiglu(linear(h, wg), linear(h, wu)), wd)

    # -------------------------------------------------------------- drivers
    def prefill(self, ids, cache, base=0, last_only=True):
        B, T = ids.shape
        cap = cache[0].shape[3]
        pos = base + torch.arange(T)[None, :].expand(B, T)
        j = torch.arange(cap)
        visible = (j[None, None, :] <= pos[:, :, None]).expand(B, T, cap)
        return self.forward(ids, pos, pos, visible, cache, last_only=last_only)

    def decode(self, tok, pos, cache):
        """tok int64 [B]; pos int (same for every row)."""
        B = tok.shape[0]
        cap = cache[0].shape[3]
        p = torch.full((B, 1), pos, dtype=torch.int64)
        visible = (torch.arange(cap)[None, None, :] <= pos).expand(B, 1, cap)
        return self.forward(tok[:, None], p, p, visible, cache)[:, 0]

    def greedy(self, prompt, n_new, cap=None):
        """engine.py:963-972 semantics: prefill then n_new-1 cached decode steps; returns
        (tokens [B, n_new] int64, logits list of [B, V] bf16 per step)."""
        prompt = torch.as_tensor(prompt, dtype=torch.int64)
        B, S = prompt.shape
        cache = self.new_cache(B, cap or S + n_new)
        logits = self.prefill(prompt, cache)[:, -1]
        toks, outs = [argmax_lowest(logits)], [logits]
        for t in range(1, n_new):
            logits = self.decode(toks[-1], S + t - 1, cache)
            toks.append(argmax_lowest(logits))
            outs.append(logits)
        return torch.stack(toks, 1), outs

    def teacher_logits(self, prompt, toks):
        """bf16 logits [B, n, V] at every emitted position of one causal forward over
        prompt + toks[:-1] (the judge's teacher-forced replay, engine.py:974-996)."""
        prompt = torch.as_tensor(prompt, dtype=torch.int64)
        toks = torch.as_tensor(toks, dtype=torch.int64)
        B, S = prompt.shape
        n = toks.shape[1]
        ids = torch.cat([prompt, toks[:, :-1]], 1)
        cache = self.new_cache(B, S + n)
        return self.prefill(ids, cache, last_only=False)[:, S - 1:]

    def teacher_force(self, prompt, toks):
        """(max logit - logit of the emitted token) as fp32 [B, n] under teacher forcing."""
        toks = torch.as_tensor(toks, dtype=torch.int64)
        logits = self.teacher_logits(prompt, toks).to(F32)
        return logits.max(-1).values - logits.gather(-1, toks[..., None])[..., 0]

    def verify_tree(self, tokens, depth, anc, base, cache):
        """Tree verification (engine/kernels/tree.py:1-11): node t of row b is rotated at
        base[b] + depth[b, t], written to slot base[b] + t, and sees cached slots < base[b]
        plus block slot base[b] + j iff bit j of anc[b, t].  Returns bf16 logits [B, T, V]."""
        tokens = torch.as_tensor(tokens, dtype=torch.int64)
        B, T = tokens.shape
        cap = cache[0].shape[3]
        base = torch.as_tensor(base, dtype=torch.int64)
        depth = torch.as_tensor(depth, dtype=torch.int64)
        rope_pos = base[:, None] + depth
        slots = base[:, None] + torch.arange(T)[None, :]
        j = torch.arange(cap)[None, None, :] - base[:, None, None]    # block index of each slot
        bits = torch.zeros((B, T, cap), dtype=torch.bool)
        anc_np = np.asarray(anc, dtype=np.uint64)
        for b in range(B):
            for t in range(T):
                a = int(anc_np[b, t])
                for jj in range(T):
                    if (a >> jj) & 1:
                        bits[b, t, int(base[b]) + jj] = True
        visible = (j < 0) | bits
        return self.forward(tokens, rope_pos, slots, visible, cache)
