"""GPU end-to-end parity of the Engine (drop-in for engine/engine.py's Engine) against the golden
transformers run (tests/golden/config1.json) and the CPU oracle.

Token rule (north star): ids identical at every step where the reference top-2 margin exceeds
1e-2.  The reference logits for a step are taken teacher-forced on the engine's own prefix
(the judge's replay, QWEN_ENGINE_CONTRACT.md:105-123), so a legitimate near-tie flip is judged
on what was actually generated.  Against the stored golden run, whose margins are bf16 logit
differences, a margin of at most one bf16 ulp of the top logit counts as a tie (it bounds the
fp32 margin by nothing: any summation order may flip it)."""

import hashlib
import json
import os

import numpy as np
import pytest
import torch

from helpers import GOLDEN, ORACLE_TIE, bf16_ulp, ensure_oracle_built, margin_rule
from oracle import qwen3_ref as R
from oracle import synth

pytestmark = pytest.mark.gpu
CFG1 = json.load(open(os.path.join(GOLDEN, "config1.json")))


def say(msg):
    print(f"\n[case] {msg}", flush=True)


@pytest.fixture(scope="module")
def Engine():
    from engine import Engine as E
    return E


@pytest.fixture(scope="module")
def eng4(Engine):
    say("Engine.synthetic(4 layers, seed 0)")
    return Engine.synthetic(n_layers=4, seed=0)


@pytest.fixture(scope="module")
def ref4():
    ensure_oracle_built()
    return R.Qwen3Ref.from_synth(0, 4)


def test_device_weights_match_golden_run(eng4):
    say("device-generated weights == golden run's weights (sha256)")
    slots = dict(eng4.model.slots())
    for name, digest in CFG1["weight_sha256"].items():
        t = slots[name].contiguous().cpu().view(torch.int16).numpy().view(np.uint16)
        assert hashlib.sha256(t.tobytes()).hexdigest() == digest, name


def test_config1_greedy(eng4, ref4):
    say("config 1: 4 layers, B=1, S=128, N=32")
    prompt = CFG1["prompt"]
    steps = list(eng4.generate(prompt, 32))
    assert len(steps) == 32 and all(len(s) == 1 for s in steps)
    toks = np.array(steps).T                                     # [B, N]
    gold = np.array(CFG1["tokens"])
    # The golden margins are differences of bf16 logits.  At |logit| ~ 4 the bf16 spacing is
    # 0.03125, above the rule's 1e-2, and a one-ulp bf16 gap can come from an fp32 gap of any
    # size down to ~1e-6 -- so a margin of at most one ulp of the top logit is a rounding tie
    # that any fp32 summation order may flip.  Wider margins must match.
    def tied(i):
        top = torch.tensor(CFG1["top_values"][i][0], dtype=torch.float32)
        return CFG1["margins"][i] <= max(1e-2, float(bf16_ulp(top)))
    first_tie = next((i for i in range(32) if tied(i)), 32)
    assert np.array_equal(toks[0, :first_tie], gold[0, :first_tie]), (toks, gold)
    # the north-star rule against transformers itself: the prefix is identical to the golden
    # run up to the first divergence, so the golden margins apply there verbatim
    div = next((i for i in range(32) if toks[0, i] != gold[0, i]), 32)
    if div < 32:
        assert tied(div), f"diverged at step {div}, golden margin {CFG1['margins'][div]}"
    # What the engine achieves on MI355X: all 32 ids equal transformers' own greedy ids,
    # including the exact bf16 tie at step 6 (resolved to the lowest index, as torch.argmax
    # does).  The decode path is deterministic, so this is asserted outright.
    assert np.array_equal(toks[0], gold[0]), f"ids {toks[0].tolist()} != golden {gold[0].tolist()}"
    tl = ref4.teacher_logits(np.array(prompt), toks)
    bad = margin_rule(toks, tl, margin=ORACLE_TIE, what="config 1 vs oracle")
    worst = float((tl.float().max(-1).values - tl.float().gather(-1, torch.as_tensor(toks)[..., None])[..., 0]).max())
    print(f"config1 tokens {toks[0].tolist()} worst teacher-forced margin {worst:.4f} "
          f"violations {bad}", flush=True)
    assert bad == []


def test_config1_logits_against_transformers(eng4, ref4):
    """Logits end to end at config 1: after every step the fp32 logits recomputed from the
    step's final residual (qd_lm_head_argmax, final RMSNorm included) are compared with
      * transformers' own logits (the golden run's top-8 values at the golden top-8 ids, bf16):
        the engine's bf16-rounded logits within 2 bf16 ulp -- the bar the CPU oracle itself
        meets against transformers (tests/test_oracle.py); the fp32 max-abs is reported;
      * the CPU oracle's fp32 logits (same ids teacher-forced, final RMSNorm, fp32 product with
        the tied embedding) over the whole vocabulary: max-abs reported per step;
    and their argmax (bf16-rounded, lowest index) is the id the step emitted."""
    say("config 1: per-step logits vs transformers' top-8 and the oracle's full vocabulary")
    from helpers import engine_step_logits
    emitted, arg, lg = engine_step_logits(eng4, CFG1["prompt"], 32)        # prompt: [1, 128]
    assert np.array_equal(emitted, arg), (emitted, arg)
    gold = np.array(CFG1["tokens"])
    assert np.array_equal(emitted, gold), "the config-1 ids differ from the golden run"
    ids = torch.tensor(CFG1["top_ids"])                                   # [32, 8]
    want = torch.tensor(CFG1["top_values"], dtype=torch.float32)
    got = lg[0].gather(-1, ids)
    err = (got - want).abs()
    ulps = (got.to(torch.bfloat16).float() - want).abs() / bf16_ulp(want)
    print(f"vs transformers top-8: fp32 max-abs per step "
          f"{[round(float(e), 4) for e in err.max(-1).values]}; overall {float(err.max()):.4f}; "
          f"bf16-rounded max {float(ulps.max()):.1f} ulp", flush=True)
    # the oracle's fp32 logits along the same ids
    prompt = torch.tensor(CFG1["prompt"])
    seq = torch.cat([prompt, torch.as_tensor(gold)[:, :-1]], 1)
    S, cap = prompt.shape[1], seq.shape[1]
    pos = torch.arange(cap)[None]
    vis = torch.arange(cap)[None, None, :] <= pos[:, :, None]
    with torch.inference_mode():
        _, x = ref4.forward(seq, pos, pos, vis, ref4.new_cache(1, cap), return_hidden=True)
        h = R.rmsnorm(x, ref4.p["model.norm.weight"], ref4.eps)[0, S - 1:]
        ref32 = h.float() @ ref4.lm_head.float().T                        # [32, V]
    d = (lg[0] - ref32).abs().amax(-1)
    print(f"vs oracle fp32, whole vocabulary: max-abs per step "
          f"{[round(float(e), 4) for e in d]}; overall {float(d.max()):.4f}", flush=True)
    oracle_tf = (ref32.gather(-1, ids) - want).abs().max()
    print(f"oracle fp32 vs transformers top-8 (the implementation floor): {float(oracle_tf):.4f}",
          flush=True)
    assert float(ulps.max()) <= 2.0


def test_generate_resets_state_and_is_deterministic(eng4):
    say("generate x3 with an intervening prompt: identical ids")
    p1 = synth.prompt_ids(11, 1, 40).tolist()
    p2 = synth.prompt_ids(12, 1, 40).tolist()
    a = list(eng4.generate(p1, 12))
    b = list(eng4.generate(p2, 12))
    c = list(eng4.generate(p1, 12))
    assert a == c and a != b
    assert list(eng4.generate(p1, 0)) == []
    assert list(eng4.generate(p1, 1)) == a[:1]


def test_prefill_chunking_is_invariant(eng4, ref4):
    """Chunks of 7 / 64 / 96 tokens per sequence run the projections through different GEMM
    kernels (LDS-staged for <= 64 rows, register-blocked above), whose fp32 summation orders
    differ in the last bits: every chunking must emit a greedy decode under the margin rule, and
    the chunkings must agree on every step before a row's first oracle tie."""
    say("prefill chunk sizes 7 / 64 / whole prompt: same ids up to oracle ties")
    p = synth.prompt_ids(13, 2, 96)
    outs = []
    for rows in (14, 128, 4096):
        eng4.prefill_budget_rows = rows
        eng4.shape = None
        outs.append(np.array(list(eng4.generate(p.tolist(), 6))).T)   # [B, N]
    eng4.prefill_budget_rows = None
    eng4.shape = None
    for rows, toks in zip((14, 128, 4096), outs):
        tl = ref4.teacher_logits(p, toks)
        bad = margin_rule(toks, tl, margin=ORACLE_TIE, what=f"prefill budget {rows} rows")
        assert bad == [], f"budget {rows} rows: {bad}"
        if rows == 4096:
            top2 = tl.float().topk(2, dim=-1).values
            gap = (top2[..., 0] - top2[..., 1]).numpy()
    for b in range(p.shape[0]):
        first_tie = next((i for i in range(6) if gap[b, i] <= ORACLE_TIE), 6)
        for toks in outs[:2]:
            assert np.array_equal(toks[b, :first_tie], outs[2][b, :first_tie]), (b, outs)


@pytest.fixture(scope="module")
def eng2(Engine):
    say("Engine.synthetic(2 layers, seed 1)")
    return Engine.synthetic(n_layers=2, seed=1)


@pytest.fixture(scope="module")
def ref2():
    ensure_oracle_built()
    return R.Qwen3Ref.from_synth(1, 2)


@pytest.mark.parametrize("B,S,N", [(2, 33, 8), (5, 40, 6), (32, 64, 6), (64, 24, 4), (80, 16, 4)])
def test_batched_decode_paths(eng2, ref2, B, S, N):
    """Vector path B <= 2; LDS-staged MFMA GEMMs + streaming LM head 3..64 rows (16-, 32- and
    two 32-row activation tiles); the tiled GEMMs past 64 rows."""
    say(f"batched decode B={B} S={S} N={N}")
    prompt = synth.prompt_ids(20 + B, B, S)
    toks = np.array(list(eng2.generate(prompt.tolist(), N))).T
    tl = ref2.teacher_logits(prompt, toks)
    bad = margin_rule(toks, tl, margin=ORACLE_TIE, what=f"batched B={B}")
    assert bad == [], bad


def test_tree_verification_is_exact(eng2, ref2):
    say("tree verification B=2 S=48 N=20 T=64 random 4-4-2-2 drafts")
    from qdecode import tree as tr
    prompt = synth.prompt_ids(30, 2, 48)
    plain = np.array(list(eng2.generate(prompt.tolist(), 20))).T
    # drafts: the true greedy continuation as one branch of each tree, random ids elsewhere
    rng = np.random.default_rng(0)
    cont = {b: prompt[b].tolist() + plain[b].tolist() for b in range(2)}

    def drafter(seq, T):
        t = tr.branching_tree(seq[-1], T, (4, 4, 2, 2), lambda n: rng.integers(0, 151936, size=n))
        b = next(i for i in range(2) if cont[i][:48] == list(seq[:48]))   # the row, by its prompt
        # the plain run's continuation while the tree run still follows it (a near-tie flip
        # between the two kernels' summation orders ends that; random drafts from then on)
        truth = cont[b][len(seq):len(seq) + 4] if cont[b][:len(seq)] == list(seq) else []
        t2 = tr.Tree(seq[-1])
        if truth:
            t2.add_path(truth, T)
        for i in range(1, len(t.tokens)):
            if len(t2.tokens) >= T:
                break
            if t.parent[i] == 0:
                t2.add(0, t.tokens[i])
        t2.pad(T)
        return t2

    got = np.array(list(eng2.generate_tree(prompt.tolist(), 20, drafter, T=64))).T
    stats = eng2.tree_stats
    print(f"tree passes {stats['passes']} accepted {stats['accepted']}", flush=True)
    assert stats["passes"] < 19                      # the true branch was accepted at least once
    tl = ref2.teacher_logits(prompt, got)
    assert margin_rule(got, tl, margin=ORACLE_TIE, what="tree, true branch drafted") == []
    if not np.array_equal(got, plain):              # only a genuine near-tie may differ
        div = np.argwhere(got != plain)[0]
        print(f"tree vs plain first differ at {div.tolist()}", flush=True)


def test_tree_random_drafts_config5_shape(eng2, ref2):
    say("tree verification with purely random drafts B=4 S=40 N=6")
    from qdecode import tree as tr
    prompt = synth.prompt_ids(31, 4, 40)
    got = np.array(list(eng2.generate_tree(prompt.tolist(), 6, tr.random_tree_drafter(1), T=64))).T
    tl = ref2.teacher_logits(prompt, got)
    assert margin_rule(got, tl, margin=ORACLE_TIE, what="tree, random drafts") == []


def test_generate_tree_modes(eng2, ref2):
    """generate() with tree speculation forced on (the lookahead / n-gram / pool drafter) emits
    greedy ids under the margin rule; the warmup gate decides once per shape, records what it
    measured, and either way returns the plain greedy ids of its own check."""
    say("generate: ENGINE_TREE=1 (lookahead drafts), then the auto gate, B=2 S=48 N=24")
    prompt = synth.prompt_ids(41, 2, 48)
    mode = eng2.tree_mode
    try:
        eng2.tree_mode = "0"
        plain = np.array(list(eng2.generate(prompt.tolist(), 24))).T
        eng2.tree_mode, eng2.tree_on = "1", {}
        tree = np.array(list(eng2.generate(prompt.tolist(), 24))).T
        assert eng2.tree_stats["passes"] >= 1 and sum(eng2.tree_stats["accepted"]) >= 23
        tl = ref2.teacher_logits(prompt, tree)
        assert margin_rule(tree, tl, margin=ORACLE_TIE, what="generate, trees forced on") == []
        eng2.tree_mode, eng2.tree_on = "auto", {}
        auto = np.array(list(eng2.generate(prompt.tolist(), 24))).T
        log = eng2.tree_log[(2, 48, 24)]
        print(f"gate: {log}", flush=True)
        assert log["T"] == 32 and log["tokens"] == 24 and log["on"] == eng2.tree_on[(2, 48, 24)]
        assert log["on"] <= log["exact"]
        assert np.array_equal(auto, plain) or (log["on"] and np.array_equal(auto, tree))
    finally:
        eng2.tree_mode, eng2.tree_on = mode, {}


def test_block_forward_graphs_match_eager(eng2):
    """The prefill and tree-verify forwards replayed from hipGraphs (one per (T, compaction, LM
    mode), recorded on first use) emit exactly the ids of the same forwards launched kernel by
    kernel.  Every tree pass rewrites the runner's input buffers (tokens, base, depths, masks,
    compaction lists) with host copies and synchronises on its output before the next replay,
    and each later pass depends on every earlier pass's accepted tokens and compacted K/V, so
    comparing the streams checks every replay against eager execution; the second graph run on
    a shape replays the graphs the first one recorded."""
    say("graphs vs eager: generate_tree B=4 S=40 N=12 (random drafts), generate B=2 S=200 in "
        "two prefill chunks")
    from qdecode import model as M
    from qdecode import tree as tr
    prompt = synth.prompt_ids(51, 4, 40).tolist()
    prompt2 = synth.prompt_ids(52, 2, 200).tolist()
    mode = eng2.tree_mode
    runs = {}
    try:
        eng2.tree_mode = "0"
        for use in (False, True):
            M.BlockRunner.use_graphs = use
            eng2.shape = None
            t = [list(eng2.generate_tree(prompt, 12, tr.random_tree_drafter(3), T=64))
                 for _ in range(2)]
            ntree = len(eng2.shape.tree.graphs) + len(eng2.shape.prefill.graphs)
            eng2.prefill_budget_rows = 256                  # two causal chunks of 128 tokens
            eng2.shape = None
            p = [list(eng2.generate(prompt2, 8)) for _ in range(2)]
            npre = len(eng2.shape.prefill.graphs)
            eng2.prefill_budget_rows = None
            runs[use] = (t, p, ntree, npre)
    finally:
        M.BlockRunner.use_graphs = True
        eng2.tree_mode = mode
        eng2.prefill_budget_rows = None
        eng2.shape = None
    te, pe, nte, npe = runs[False]
    tg, pg, ntg, npg = runs[True]
    assert nte == npe == 0 and ntg == 2 and npg == 2     # tree: prefill + verify; 2 chunks
    assert te[0] == te[1] == tg[0] == tg[1]
    assert pe[0] == pe[1] == pg[0] == pg[1]


def _device_bits(t):
    return t.contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("shards,rope_form,tied", [(3, "parameters", True), (1, "theta", False)],
                         ids=["sharded-rope_parameters-tied", "single-file-untied"])
def test_checkpoint_load_is_bit_exact(Engine, tmp_path, shards, rope_form, tied):
    """Engine(model_path) over an HF directory written by the generator: every device tensor
    equals the generator's bits (synth.param_bits), the RoPE base comes from either config form,
    and the decoded ids follow the oracle built from the same bits (the untied case decodes
    through its own lm_head.weight, in the persistent step and the prefill's LM head)."""
    say(f"Engine(model_path): {shards} shard(s), rope form {rope_form}, tied={tied}, 1 layer")
    ensure_oracle_built()
    cfg = synth.write_checkpoint(str(tmp_path), seed=5, n_layers=1, shards=shards,
                                 rope_form=rope_form, tied=tied)
    eng = Engine(str(tmp_path))
    m = eng.model
    assert m.cfg["rope_theta"] == 5000000.0 and m.L == 1 and m.tied is tied
    shapes = synth.param_shapes(cfg)
    names = [n for n, _ in m.slots()]
    assert sorted(names) == sorted(shapes)
    for name, dst in m.slots():
        assert np.array_equal(_device_bits(dst), synth.param_bits(5, name, shapes[name])), name
    p = synth.prompt_ids(40, 1, 24)
    toks = np.array(list(eng.generate(p.tolist(), 5))).T
    ref = R.Qwen3Ref.from_synth(5, 1, tied=tied)
    tl = ref.teacher_logits(p, toks)
    assert margin_rule(toks, tl, margin=ORACLE_TIE, what=f"checkpoint tied={tied}") == []


def test_invalid_inputs_raise(eng2):
    say("invalid input ids raise on the host")
    with pytest.raises(IndexError):
        list(eng2.generate([[0, 151936]], 2))
    with pytest.raises(ValueError):
        list(eng2.generate([[1, 2], [3]], 2))
