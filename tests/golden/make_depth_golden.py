"""Write depth.json: the CPU oracle's greedy decode at the benchmark configs' real depth and
context, for the GPU tests to compare against without re-running 36 layers over 8192 tokens on
the GPU box's host.

The oracle (oracle/qwen3_ref.py) is pinned op by op and at 4 layers against transformers'
Qwen3 (tests/test_oracle.py, golden vectors from make_golden.py); depth and context only
repeat those ops.  This script runs it on the seeded 36-layer checkpoint (seed 1, the one
configs 3-5 name) for:

  config3  B=1, 512 prompt ids, 32 greedy tokens
  config4  rows 0 and 31 of B=32 x 2048 prompt ids, 4 greedy tokens (rows are independent)
  config5  rows 0 and 1 of B=4 x 8192 prompt ids, 8 greedy tokens

and stores, per row, the prompt's generator seed, the greedy ids, and per step the top-2
logits (bf16 values as floats) and their ids.  Prompts are ``synth.prompt_ids(seed, B, S)``.
The prompt is prefilled in causal chunks of 1024 tokens (the same function; it bounds the
fp32 score matrices), then decoded one token at a time with the KV cache (engine.py:963-972).

Run from the repo root (about 10 minutes on 8 cores):
    make -C oracle && python tests/golden/make_depth_golden.py
"""

import json
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import qwen3_ref as R  # noqa: E402
from oracle import synth  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "depth.json")
CHUNK = 1024

# name -> (prompt seed, B, S, N, rows kept)
CONFIGS = {
    "config3": (301, 1, 512, 32, [0]),
    "config4": (401, 32, 2048, 4, [0, 31]),
    "config5": (501, 4, 8192, 8, [0, 1]),
}


def greedy_row(ref, prompt, n_new):
    """Greedy decode of one prompt row: (ids, per-step top-2 values and ids)."""
    S = prompt.shape[0]
    cache = ref.new_cache(1, S + n_new)
    cap = S + n_new
    j = torch.arange(cap)
    for c0 in range(0, S, CHUNK):
        ids = prompt[None, c0:c0 + CHUNK]
        T = ids.shape[1]
        pos = c0 + torch.arange(T)[None, :]
        vis = j[None, None, :] <= pos[:, :, None]
        logits = ref.forward(ids, pos, pos, vis, cache, last_only=True)[:, -1]
    toks, top_v, top_i = [], [], []
    for t in range(n_new):
        if t:
            logits = ref.decode(torch.tensor([toks[-1]]), S + t - 1, cache)
        v, i = logits.float().topk(2, dim=-1)
        top_v.append(v[0].tolist())
        top_i.append(i[0].tolist())
        toks.append(int(R.argmax_lowest(logits)[0]))
    return toks, top_v, top_i


def main():
    torch.set_num_threads(os.cpu_count() or 8)
    t0 = time.time()
    ref = R.Qwen3Ref.from_synth(1, 36)
    print(f"weights ready in {time.time() - t0:.1f} s", flush=True)
    out = {"weights": "synth seed 1, 36 layers, std 0.02, norm weights 1, tied",
           "prompt": "synth.prompt_ids(seed, B, S)[row]", "chunk": CHUNK}
    for name, (seed, B, S, N, rows) in CONFIGS.items():
        prompts = torch.as_tensor(synth.prompt_ids(seed, B, S))
        recs = []
        for r in rows:
            t1 = time.time()
            toks, tv, ti = greedy_row(ref, prompts[r], N)
            recs.append({"row": r, "tokens": toks, "top2_values": tv, "top2_ids": ti,
                         "margins": [a - b for a, b in tv]})
            print(f"{name} row {r}: {toks} ({time.time() - t1:.1f} s)", flush=True)
        out[name] = {"seed": seed, "B": B, "S": S, "N": N, "rows": recs}
        with open(OUT, "w") as f:
            json.dump(out, f, indent=1)
    print(f"wrote {OUT} in {time.time() - t0:.1f} s", flush=True)


if __name__ == "__main__":
    main()
