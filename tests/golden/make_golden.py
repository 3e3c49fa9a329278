"""Write the golden vectors that pin the CPU oracle (oracle/qwen3_ref.py).

The reference (Yokanater/htn-2026) takes its arithmetic from the third-party
``transformers`` Qwen3ForCausalLM (pinned 4.51.3 in requirements.txt:10; this container has
5.15.0, whose Qwen3 ops are unchanged).  Its own tests hold no golden vectors for the engine,
so this script runs transformers' modules -- in this container, on the CPU, on seeded inputs
and on the seeded synthetic checkpoint -- and stores their inputs and outputs:

  ops.npz       per-op vectors: Qwen3RMSNorm (hidden and per-head), Qwen3RotaryEmbedding
                tables, apply_rotary_pos_emb, silu(gate) * up (Qwen3MLP's act), torch SDPA over
                repeat_kv (the "sdpa" attention path, decode and causal), and one full
                Qwen3DecoderLayer of the config-1 checkpoint
  config1.json  config 1 (4 layers, seed 0, B=1, 128 prompt ids, 32 greedy tokens): the greedy
                ids of transformers' KV-cache loop (engine/engine.py:963-972), the top-8 logits
                and ids and the top-1 minus top-2 margin of every step, plus sha256 of
                selected weights

bf16 arrays are stored as uint16 bit patterns.  Run from the repo root:
    make -C oracle && python tests/golden/make_golden.py
"""

import hashlib
import json
import os
import sys
import tempfile

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import synth  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))
BF16 = torch.bfloat16


def bits(t):
    return t.detach().contiguous().to(BF16).view(torch.int16).numpy().view(np.uint16)


def randn(g, *shape, scale=1.0, shift=0.0):
    return (torch.randn(shape, generator=g) * scale + shift).to(BF16)


def main():
    from transformers import Qwen3Config, Qwen3ForCausalLM
    from transformers.activations import ACT2FN
    from transformers.models.qwen3 import modeling_qwen3 as mq

    torch.set_num_threads(os.cpu_count() or 8)
    g = torch.Generator().manual_seed(20260)
    ops = {}

    # --- Qwen3RMSNorm on hidden rows and on 128-wide heads
    norm = mq.Qwen3RMSNorm(2560, eps=1e-6).to(BF16)
    with torch.no_grad():
        norm.weight.copy_(randn(g, 2560, scale=0.1, shift=1.0))
    x = randn(g, 4, 2560)
    x[3] = 0.75                                         # constant row (closed form check too)
    with torch.no_grad():
        y = norm(x)
    ops.update(rms_x=bits(x), rms_w=bits(norm.weight), rms_y=bits(y))
    hn = mq.Qwen3RMSNorm(128, eps=1e-6).to(BF16)
    with torch.no_grad():
        hn.weight.copy_(randn(g, 128, scale=0.2, shift=1.0))
    qh = randn(g, 2, 3, 32, 128, scale=2.0)
    with torch.no_grad():
        ops.update(hrms_x=bits(qh), hrms_w=bits(hn.weight), hrms_y=bits(hn(qh)))

    # --- rotary tables at selected absolute positions (theta 5e6, head_dim 128)
    cfg = Qwen3Config(hidden_size=2560, intermediate_size=9728, num_hidden_layers=1,
                      num_attention_heads=32, num_key_value_heads=8, head_dim=128,
                      vocab_size=151936, rms_norm_eps=1e-6, rope_theta=5000000.0,
                      tie_word_embeddings=True, max_position_embeddings=40960)
    rot = mq.Qwen3RotaryEmbedding(cfg)
    pos = torch.tensor([[0, 1, 2, 127, 128, 511, 767, 2047, 2175, 8191, 8447, 8511, 40000]])
    cos, sin = rot(torch.empty(1, dtype=BF16), pos)
    ops.update(rope_pos=pos[0].numpy(), rope_cos=bits(cos[0]), rope_sin=bits(sin[0]),
               rope_inv_freq=rot.inv_freq.float().numpy())

    # --- apply_rotary_pos_emb on normed q/k at per-token positions
    ppos = torch.tensor([[0, 5, 129, 4097, 8191]])
    c5, s5 = rot(torch.empty(1, dtype=BF16), ppos)
    q = randn(g, 1, 32, 5, 128, scale=1.5)
    k = randn(g, 1, 8, 5, 128, scale=1.5)
    qe, ke = mq.apply_rotary_pos_emb(q, k, c5, s5)
    ops.update(ar_pos=ppos[0].numpy(), ar_q=bits(q), ar_k=bits(k), ar_qo=bits(qe), ar_ko=bits(ke))

    # --- Qwen3MLP activation product: act_fn(gate) * up
    gt = randn(g, 2, 9728, scale=3.0)
    gt[0, :8] = torch.tensor([0.0, -0.0, 1e-3, -1e-3, 20.0, -20.0, 88.0, -88.0], dtype=BF16)
    up = randn(g, 2, 9728, scale=3.0)
    act = ACT2FN["silu"](gt) * up
    ops.update(mlp_g=bits(gt), mlp_u=bits(up), mlp_act=bits(act))

    # --- SDPA over repeat_kv (transformers' "sdpa" path): decode (1 query) and causal (6)
    qd = randn(g, 2, 32, 1, 128)
    kd = randn(g, 2, 8, 37, 128)
    vd = randn(g, 2, 8, 37, 128)
    od = torch.nn.functional.scaled_dot_product_attention(
        qd, mq.repeat_kv(kd, 4), mq.repeat_kv(vd, 4), scale=128 ** -0.5)
    ops.update(sd_q=bits(qd), sd_k=bits(kd), sd_v=bits(vd), sd_o=bits(od))
    qc = randn(g, 1, 32, 6, 128)
    kc = randn(g, 1, 8, 6, 128)
    vc = randn(g, 1, 8, 6, 128)
    oc = torch.nn.functional.scaled_dot_product_attention(
        qc, mq.repeat_kv(kc, 4), mq.repeat_kv(vc, 4), is_causal=True, scale=128 ** -0.5)
    ops.update(sc_q=bits(qc), sc_k=bits(kc), sc_v=bits(vc), sc_o=bits(oc))

    with tempfile.TemporaryDirectory() as ckpt:
        synth.write_checkpoint(ckpt, seed=0, n_layers=4)
        model = Qwen3ForCausalLM.from_pretrained(ckpt, dtype=BF16, attn_implementation="sdpa",
                                                 local_files_only=True).eval()
        assert model.lm_head.weight.data_ptr() == model.model.embed_tokens.weight.data_ptr()

        # --- one decoder layer (layer 0) over 6 tokens at positions 0..5, no cache
        lay = model.model.layers[0]
        xl = randn(g, 1, 6, 2560)
        p6 = torch.arange(6)[None]
        pe = model.model.rotary_emb(xl, p6)
        with torch.no_grad():
            yl = lay(xl, attention_mask=None, position_ids=p6, position_embeddings=pe)
        yl = yl[0] if isinstance(yl, tuple) else yl
        ops.update(layer_x=bits(xl), layer_y=bits(yl))

        # --- config 1: greedy KV-cache loop exactly as engine.py:963-972
        prompt = synth.prompt_ids(0, 1, 128)
        cur = torch.tensor(prompt)
        cache = None
        toks, top_v, top_i, margins = [], [], [], []
        with torch.inference_mode():
            for _ in range(32):
                out = model(input_ids=cur, past_key_values=cache, use_cache=True,
                            logits_to_keep=1, return_dict=True)
                lg = out.logits[:, -1, :]
                cur = lg.argmax(dim=-1, keepdim=True)
                cache = out.past_key_values
                tv, ti = lg.float().topk(8, dim=-1)
                toks.append(int(cur[0, 0]))
                top_v.append(tv[0].tolist())
                top_i.append(ti[0].tolist())
                margins.append(float(tv[0, 0] - tv[0, 1]))
        sd = model.state_dict()
        sha = {n: hashlib.sha256(bits(sd[n]).tobytes()).hexdigest()
               for n in ["model.embed_tokens.weight", "model.layers.0.self_attn.q_proj.weight",
                         "model.layers.3.mlp.down_proj.weight", "model.norm.weight"]}
        import transformers
        meta = {"config": "config 1: 4 layers, seed 0, B=1, S=128, N=32", "seed": 0,
                "n_layers": 4, "prompt": prompt.tolist(), "tokens": [toks], "top_values": top_v,
                "top_ids": top_i, "margins": margins, "weight_sha256": sha,
                "generator": "oracle/synth.py", "transformers": transformers.__version__,
                "torch": torch.__version__}
    with open(os.path.join(OUT, "config1.json"), "w") as f:
        json.dump(meta, f)
    np.savez_compressed(os.path.join(OUT, "ops.npz"), **ops)
    print("tokens", toks)
    print("min margin", min(margins))


if __name__ == "__main__":
    main()
