"""Shared comparison helpers for the parity tests (bf16 ulp distances, margin rule)."""

import json
import os
import subprocess

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")


def ensure_oracle_built():
    lib = os.path.join(ROOT, "oracle", "_build", "libcsynth.so")
    if not os.path.exists(lib):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)


def bf16_ulp(x):
    """ulp of bf16 at |x| (fp32 tensor); normal range only, floor at 2^-133."""
    ax = x.abs().clamp(min=2.0 ** -126)
    return torch.pow(2.0, torch.floor(torch.log2(ax)) - 7)


def ulp_diff(a, b):
    """Elementwise |a - b| in bf16 ulps of max(|a|, |b|)."""
    a, b = a.float(), b.float()
    return (a - b).abs() / bf16_ulp(torch.maximum(a.abs(), b.abs()))


def assert_ulp(a, b, max_ulp, what="", abs_floor=0.0):
    """|a - b| <= max_ulp bf16 ulps (or <= abs_floor) everywhere."""
    a, b = a.float(), b.float()
    d = (a - b).abs()
    bad = (d > max_ulp * bf16_ulp(torch.maximum(a.abs(), b.abs()))) & (d > abs_floor)
    if bad.any():
        i = int(bad.flatten().nonzero()[0])
        raise AssertionError(f"{what}: {int(bad.sum())} elements beyond {max_ulp} ulp; first at "
                             f"{i}: {a.flatten()[i].item()} vs {b.flatten()[i].item()} "
                             f"(max ulp {ulp_diff(a, b).max().item():.2f})")


# Cross-implementation noise floor for the oracle-side token rule: the oracle (torch CPU,
# oneDNN accumulation order) and transformers' own run already disagree by up to 2 bf16 ulp of
# the top logit (tests/test_oracle.py: the golden ids sit up to 0.0625 below the oracle's
# argmax), so against the oracle a "near tie" is a top-2 gap within 2 ulp at |logit| < 8.
ORACLE_TIE = 0.0625 + 1e-6

# At the benchmarks' depth (36 layers) the floor is measured, not assumed: two equally valid
# restatements of the oracle -- softmax against the global row maximum, and the online softmax
# over 64-key blocks that tiled kernels compute -- teacher-forced over the config-3 run disagree
# on the argmax at 39 of 543 positions, with the second one's choice up to 0.15625 (5 bf16 ulp
# at |logit| < 8) below the first one's argmax (tests/golden/depth_noise.json, written by
# tests/golden/make_depth_noise.py).  A 36-layer run is held to that floor: an implementation
# as valid as the oracle itself would fail anything tighter.
DEPTH_NOISE = json.load(open(os.path.join(GOLDEN, "depth_noise.json")))
DEPTH_TIE = DEPTH_NOISE["max_deficit_B_under_A"] + 1e-6


def margin_report(tokens, ref_logits, margin=1e-2):
    """The north-star token rule on teacher-forced reference logits: at every step where the
    reference's top-2 margin exceeds `margin`, the emitted token must be the reference argmax;
    elsewhere it must be one of the near-tied tokens.  Returns a dict: ``bad`` the violating
    steps as (index, top-2 gap, emitted token's deficit); ``steps`` the steps judged;
    ``near`` the steps whose reference gap is within `margin` (where the allowance applies);
    ``used`` the steps that emitted a near-tied token other than the reference argmax."""
    bad, near, used = [], 0, 0
    lg = ref_logits.float()
    top2 = lg.topk(2, dim=-1).values
    gap = top2[..., 0] - top2[..., 1]
    best = lg.max(-1).values
    for idx in np.ndindex(*tokens.shape):
        t = int(tokens[idx])
        val = float(lg[idx][t])
        deficit = float(best[idx]) - val
        if float(gap[idx]) > margin:
            if deficit != 0:
                bad.append((idx, float(gap[idx]), deficit))
        else:
            near += 1
            if deficit > margin:
                bad.append((idx, float(gap[idx]), deficit))
            elif deficit > 0:
                used += 1
    return {"bad": bad, "steps": int(np.prod(tokens.shape)), "near": near, "used": used}


def allowance_bound(steps):
    """How many of `steps` judged steps may emit a near-tied id other than the reference
    argmax at 36 layers: the larger rate at which a valid restatement of the oracle disagrees
    with it on the argmax (depth_noise.json: 39 and 47 of 543 positions for variants B and C),
    plus three Poisson standard deviations and one.  A regression that moves many near-tie
    choices fails it even though each single choice stays within DEPTH_TIE."""
    worst = max(DEPTH_NOISE["argmax_differs"], DEPTH_NOISE["argmax_differs_C"])
    mean = steps * worst / DEPTH_NOISE["positions"]
    return int(mean + 3.0 * mean ** 0.5 + 1.0)


def margin_rule(tokens, ref_logits, margin=1e-2, what=""):
    """margin_report's violations; prints how many steps the near-tie allowance covered.  With
    margin >= DEPTH_TIE (a 36-layer run) the number of steps that used the allowance is held
    to allowance_bound() as well (reported as one more violation)."""
    rep = margin_report(tokens, ref_logits, margin)
    print(f"[margin] {what} steps {rep['steps']} near-ties {rep['near']} "
          f"allowance used {rep['used']} violations {len(rep['bad'])}", flush=True)
    bad = list(rep["bad"])
    if margin >= DEPTH_TIE - 1e-6 and rep["used"] > allowance_bound(rep["steps"]):
        bad.append(("allowance used", rep["used"], allowance_bound(rep["steps"])))
    return bad


def fixture_rule(tokens, rec, tie=None):
    """Compare one row of emitted ids with a stored oracle greedy run (tests/golden/depth.json
    record: tokens, top2_values, top2_ids, margins).  The ids must be identical step by step;
    the first difference is allowed only at a step whose oracle top-2 margin is within `tie`
    (default ORACLE_TIE) and only if the emitted id is the other of the oracle's top two (at an
    exact tie the oracle picks the lower index and the top-2 listing may name either first) --
    after that the prefixes differ and the stored run no longer applies.  Returns the number of
    steps checked (all of them when the ids agree throughout)."""
    tie = ORACLE_TIE if tie is None else tie
    ref = rec["tokens"]
    for i, (t, r) in enumerate(zip(tokens, ref)):
        if int(t) == r:
            continue
        m = rec["margins"][i]
        assert m <= tie and int(t) in rec["top2_ids"][i], (
            f"step {i}: emitted {int(t)}, oracle {r} with top-2 margin {m:.4f} "
            f"(top two {rec['top2_ids'][i]})")
        print(f"[fixture] near tie at step {i} (margin {m:.4f}): checked {i + 1} steps",
              flush=True)
        return i + 1
    print(f"[fixture] all {len(ref)} steps identical", flush=True)
    return len(ref)


def engine_step_logits(eng, prompt, N):
    """Run the engine's own prefill and N - 1 decode steps (the graph replays generate()
    performs) for a [B, S] prompt, and after every step recompute that step's logits from the
    final residual it left: qd_lm_head_argmax over the step's x rows with the final RMSNorm,
    fp32 logits before bf16 rounding.  Step 0's residual is the prefill's last prompt row per
    sequence.  Returns (emitted ids [B, N], recomputed argmax ids [B, N], fp32 logits
    [B, N, V]) on the host."""
    from qdecode import _lib, ops
    ids = torch.as_tensor(np.asarray(prompt), dtype=torch.int64)
    B, S = ids.shape
    sh = eng._state(B, S, N, 0)
    m, st = eng.model, eng.stream
    H, V = m.H, m.V
    logits = torch.empty((N, B, V), dtype=torch.float32, device=m.device)
    arg = torch.empty((N, B), dtype=torch.int64, device=m.device)
    emitted = torch.empty((N, B), dtype=torch.int64, device=m.device)
    ws = ops.workspace(_lib.LIB.qd_lm_head_workspace_bytes(B, V, H), m.device)
    sh.start(ids, decode_next=N > 1)
    T_last = S - (S - 1) // sh.chunk * sh.chunk              # rows of the last prefill chunk
    with torch.cuda.stream(st):
        last = sh.prefill.x[:B * T_last].view(B, T_last, H)[:, T_last - 1]
        emitted[0].copy_(sh.kv.tok)
        ops.lm_head_argmax(last, m.lm_head, m.final_norm, m.eps, tok=arg[0], logits=logits[0],
                           ws=ws)
        for t in range(1, N):
            sh.decode.replay()
            emitted[t].copy_(sh.kv.tok)
            ops.lm_head_argmax(sh.decode.x, m.lm_head, m.final_norm, m.eps, tok=arg[t],
                               logits=logits[t], ws=ws)
    st.synchronize()
    sh.decode.check()
    return (emitted.T.cpu().numpy(), arg.T.cpu().numpy(),
            logits.transpose(0, 1).contiguous().cpu())
