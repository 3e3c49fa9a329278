"""Write depth_noise.json: how far two equally valid restatements of the same bf16 model
disagree at the benchmark's depth -- the floor under any token rule applied to a 36-layer run.

Variant A is the oracle as pinned (oracle/qwen3_ref.py: softmax against each row's global
maximum).  Variant B changes one rounding order and nothing else: the online softmax of the
flash decomposition over 64-key blocks (running maximum, P rounded to bf16 against it, O and l
rescaled as the maximum moves) -- the form every split-K / tiled attention kernel computes.
Both run one causal forward over the config-3 prompt and the stored oracle run's tokens
(depth.json: 36 layers, seed 1, prompt seed 301, 512 ids + 31 greedy tokens) and are compared
at every position: how much the top-2 gap moves between them, where their argmax differs, and
B's argmax deficit under A -- how far below A's argmax the token that a valid implementation
picks can sit -- and the largest logit difference over the whole vocabulary at each position.
Variant C adds the other reordering a kernel implementation makes: every projection (and the
LM head) summed as fp32 partials over 512-wide K ranges.  ``logit_floor`` is the larger of the
B and C full-vocabulary differences: the logit bar for a 36-layer run.

Run from the repo root (about a minute on 8 cores):
    make -C oracle && python tests/golden/make_depth_noise.py
"""

import json
import os
import sys

import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import qwen3_ref as R  # noqa: E402
from oracle import synth  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
F32 = torch.float32
BLOCK = 64


def attention_online(q, k, v, visible, scale=None):
    """R.attention's arithmetic with the softmax taken online over BLOCK-key blocks."""
    hq, hkv, d = q.shape[1], k.shape[1], q.shape[-1]
    scale = d ** -0.5 if scale is None else scale
    kf = R.repeat_kv(k, hq // hkv).to(F32)
    vf = R.repeat_kv(v, hq // hkv).to(F32)
    s = (q.to(F32) @ kf.transpose(-1, -2)) * scale
    s = s.masked_fill(~visible, float("-inf"))
    m = torch.full(s.shape[:-1] + (1,), -1e30)
    l = torch.zeros_like(m)
    o = torch.zeros(s.shape[:-1] + (d,))
    for j in range(0, s.shape[-1], BLOCK):
        sj = s[..., j:j + BLOCK]
        mn = torch.maximum(m, sj.amax(-1, keepdim=True))
        a = torch.exp(m - mn)
        p = torch.exp(sj - mn)
        l = l * a + p.sum(-1, keepdim=True)
        o = o * a + R.bf(p) @ vf[..., j:j + BLOCK, :]
        m = mn
    return (o / l).to(torch.bfloat16)


def linear_splitk(x, w, chunk=512):
    """R.linear's arithmetic (bf16 operands, fp32 products and sums, one bf16 rounding) with K
    summed as fp32 partial dot products over `chunk`-wide K ranges, added in order -- the
    split-K accumulation of the MFMA kernels, a valid reordering of the same sum."""
    xf, wf = x.to(F32), w.to(F32)
    acc = None
    for k0 in range(0, x.shape[-1], chunk):
        part = xf[..., k0:k0 + chunk] @ wf[:, k0:k0 + chunk].T
        acc = part if acc is None else acc + part
    return acc.to(torch.bfloat16)


def main():
    torch.set_num_threads(os.cpu_count() or 8)
    depth = json.load(open(os.path.join(HERE, "depth.json")))
    c = depth["config3"]
    prompt = torch.as_tensor(synth.prompt_ids(c["seed"], c["B"], c["S"])[:1])
    toks = torch.tensor([c["rows"][0]["tokens"]])
    ids = torch.cat([prompt, toks[:, :-1]], 1)                    # every position is a sample
    ref = R.Qwen3Ref.from_synth(1, 36)
    logits = {}
    for name, att, lin in (("A", R.attention, R.linear), ("B", attention_online, R.linear),
                           ("C", attention_online, linear_splitk)):
        saved = R.attention, R.linear
        R.attention, R.linear = att, lin
        try:
            logits[name] = ref.prefill(ids, ref.new_cache(1, ids.shape[1]), last_only=False)[0].float()
        finally:
            R.attention, R.linear = saved
    la, lb, lc = logits["A"], logits["B"], logits["C"]
    absdiff_c = (la - lc).abs().amax(-1)
    arg_c = lc.argmax(-1)
    deficit_c = la.max(-1).values - la.gather(-1, arg_c[:, None])[:, 0]
    va, vb = la.topk(2, -1).values, lb.topk(2, -1).values
    gap_a, gap_b = va[:, 0] - va[:, 1], vb[:, 0] - vb[:, 1]
    arg_a, arg_b = la.argmax(-1), lb.argmax(-1)
    deficit = la.max(-1).values - la.gather(-1, arg_b[:, None])[:, 0]   # B's pick under A
    change = (gap_a - gap_b).abs()
    absdiff = (la - lb).abs().amax(-1)                                # per position, full vocab
    diff = (arg_a != arg_b).nonzero()[:, 0].tolist()
    out = {"run": "config3: the 512 prompt ids + the stored oracle run's first 31 tokens "
                  "(depth.json), logits at every position",
           "variant_A": "oracle/qwen3_ref.py attention (global row maximum)",
           "variant_B": f"online softmax over {BLOCK}-key blocks, otherwise identical",
           "positions": int(ids.shape[1]),
           "max_gap_change": float(change.max()),
           "gap_change_quantiles": {q: float(change.quantile(q)) for q in (0.5, 0.9, 0.99)},
           "argmax_differs": len(diff),
           "max_deficit_B_under_A": float(deficit.max()),
           "max_abs_logit_diff": float(absdiff.max()),
           "abs_logit_diff_quantiles": {q: float(absdiff.quantile(q)) for q in (0.5, 0.9, 0.99)},
           "variant_C": "variant B with every projection summed as fp32 partials over 512-wide "
                        "K ranges (split-K order), otherwise identical",
           "argmax_differs_C": int((la.argmax(-1) != arg_c).sum()),
           "max_deficit_C_under_A": float(deficit_c.max()),
           "max_abs_logit_diff_C": float(absdiff_c.max()),
           "abs_logit_diff_quantiles_C": {q: float(absdiff_c.quantile(q)) for q in (0.5, 0.9, 0.99)},
           "logit_floor": float(max(absdiff.max(), absdiff_c.max())),
           "differing": [{"pos": i, "gap_A": float(gap_a[i]), "gap_B": float(gap_b[i]),
                          "deficit_B_under_A": float(deficit[i])} for i in diff]}
    with open(os.path.join(HERE, "depth_noise.json"), "w") as f:
        json.dump(out, f, indent=1)
    print(json.dumps(out, indent=1))


if __name__ == "__main__":
    main()
