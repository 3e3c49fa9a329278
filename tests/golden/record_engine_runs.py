"""Record the engine's greedy ids at the 36-layer benchmark shapes whose teacher-forced oracle
check is too long for a GPU test (prompts of 2048 and 8192 tokens through 36 layers on the
host): make_depth_golden.py then teacher-forces exactly these ids on the CPU oracle and stores
the per-step top-2 gap and the emitted id's deficit, and tests/test_gpu_depth.py checks that
the engine still emits these ids.

  config4  B=32, S=2048 (prompt seed 401), 8 plain greedy tokens, all 32 rows
  config5  B=4, S=8192 (prompt seed 501), 32 tokens, all 4 rows: tree verification with
           random 4-4-2-2 drafts (random_tree_drafter(5), 64-node trees) and plain decode

Runs on the GPU (needs the built library):
    python tests/golden/record_engine_runs.py [out.json]      (default tests/golden/engine_runs.json)
"""

import hashlib
import json
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "htn-2026_amd"))

RUNS = {"config4": (401, 32, 2048, 8), "config5": (501, 4, 8192, 32)}


def main():
    import numpy as np

    from engine import Engine
    from oracle import synth
    from qdecode import tree as tr
    out_path = sys.argv[1] if len(sys.argv) > 1 else os.path.join(ROOT, "tests", "golden",
                                                                   "engine_runs.json")
    eng = Engine.synthetic(n_layers=36, seed=1)
    eng.tree_mode = "0"
    out = {}
    for name, (seed, B, S, N) in RUNS.items():
        prompt = synth.prompt_ids(seed, B, S).tolist()
        print(f"[record] {name}: B={B} S={S} N={N} plain", flush=True)
        rec = {"seed": seed, "B": B, "S": S, "N": N,
               "plain": np.array(list(eng.generate(prompt, N))).T.tolist()}
        if name == "config5":
            print(f"[record] {name}: tree verification, random 4-4-2-2 drafts", flush=True)
            rec["tree"] = np.array(list(eng.generate_tree(prompt, N, tr.random_tree_drafter(5),
                                                          T=64))).T.tolist()
            rec["tree_passes"] = eng.tree_stats["passes"]
        out[name] = rec
        eng.shape = None
    lib = os.path.join(ROOT, "htn-2026_amd", "libqdecode.so")
    out["library_sha256"] = hashlib.sha256(open(lib, "rb").read()).hexdigest()
    with open(out_path, "w") as f:
        json.dump(out, f)
    print(f"[record] wrote {out_path}", flush=True)


if __name__ == "__main__":
    main()
