"""Decode benchmark on one MI355X: Qwen3-4B-shaped bf16 greedy decode through the HIP engine.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-b32] [--no-tree] [--no-cpu]
                    [--no-layer] [--no-api] [--no-gemm]

Workloads (the benchmark's configurations 2-5; configuration 1 is the CPU parity case):
  value  config 3 -- 36 layers, B=1, prompt 512, up to 256 new tokens: decode tok/s over K timed
         steps (one step = the whole decode step -- embed, 36 layers, LM head + argmax --
         as one launch of the persistent kernel, or one hipGraph replay of the per-launch
         step with QD_MEGA=0), after W warm-up steps; inputs resident in HBM.
  b32    config 4 -- 36 layers, B=32, prompts of 2048, up to 128 new tokens (same method).
  tree   config 5 -- tree verification, B=4, context 8192, 64-node random trees: the verify
         forward timed with HIP events (bytes/s and MFMA TFLOP/s), plus an end-to-end
         generate_tree of 256 tokens (tokens per pass, host ms per pass, wall-clock tok/s) and,
         beside it, plain B=4 decode of the same prompt and length through generate().
  api    configs 3 and 4 through Engine.generate, measured the reference's way: batch x output
         tokens / total generate wall time, prefill included (first call and warm call).
  layer_kernels  config 2 -- embedding gather, residual-add + RMSNorm, QK-norm + RoPE (+ K/V
         write), SwiGLU at B in {1, 8, 64}: us per launch (1000 launches in one hipGraph) and
         algorithmic GB/s.
  layer_kernels_large  the same four kernels at row counts that move >= 100 MB per launch
         (where bandwidth, not launch latency, binds): GB/s, fraction of 8 TB/s, and a device
         copy of the same bytes as the read+write yardstick.
  prefill_gemm  the four projections of a prefill chunk (32768 rows, the engine's chunk) through
         qd_linear (the 256 x 256-tile MFMA kernel) and, beside them, torch.matmul (hipBLASLt)
         on the same operands: us per launch and TFLOP/s against the 2.5 PFLOP/s bf16 dense peak.
  step_ms  per-step spread (median, p90, min, max) of the same K steps replayed again with an
         event after each step (the headline timing has no events between steps).
Weights are seeded random-init N(0, 0.02) generated on the device; prompt ids uniform.

cpu_baseline_configs: config 1 in full and config 4's decode step (capped) on the CPU oracle.

Roofline: at B=1 the step is ONE kernel (mega_step_kernel, the persistent decode step), so
the dominant kernel is the step itself: achieved = algorithmic bytes per step (weights + the
KV read, averaged over the timed steps) / mean launch duration, timed live with HIP events on
the engine's stream around the K graph replays (one kernel node each).  With QD_MEGA=0 (the
per-launch step) the dominant kernel is the gate/up GEMV + SwiGLU, timed as a hipGraph of its 36
per-layer launches (each on its own layer's weights, so nothing is cache resident) replayed R
times; that figure is always reported as ``gemv_gate_up``.  ``traffic`` is HBM bytes per launch
from rocprofv3 FETCH_SIZE / WRITE_SIZE scaled by a 512 MiB copy (profiles/).  cpu_baseline
times the CPU oracle (oracle/qwen3_ref.py, same architecture and generator) on this host's
cores on a bounded sample.
"""

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "htn-2026_amd"))

PEAK_HBM_GBS = 8000.0
PEAK_BF16_TFLOPS = 2500.0
# HBM bytes per gate/up launch at B=1, from two rocprofv3 --pmc passes over this script
# (`--calib-copy-mib 512`): FETCH_SIZE 48,703.0 KiB x 1.99986 + WRITE_SIZE 38.0 KiB x 1.0, the
# factors being what the same counters read for a 512 MiB device copy.  Summary and commands:
# profiles/gemv_gate_up_b1_traffic.md.
GU_TRAFFIC_B1 = 99_775_769
# HBM bytes per persistent-step launch at B=1 (config 3), same method (FETCH_SIZE 4,001,519.25
# KiB x 1.99983 + WRITE_SIZE 19,108.1 KiB), mean over the profiled steps at positions 512..520;
# summary and commands: profiles/mega_step_b1_traffic.md.
MEGA_TRAFFIC_B1 = 8_213_971_655
METRIC = "decode tok/s (Qwen3-4B bf16, B=1 & B=32) + achieved HBM GB/s vs peak"


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def decode_run(eng, B, S, N, warmup, steps, seed):
    """Prefill once, W untimed decode steps, then exactly K timed steps (graph replays)."""
    import numpy as np
    import torch
    K = min(steps, N - 1 - warmup)
    if K <= 0:
        raise ValueError(f"steps + warmup must be < {N}")
    rng = np.random.default_rng(seed)
    ids = torch.as_tensor(rng.integers(0, eng.model.V, size=(B, S)), dtype=torch.int64)
    sh = eng._state(B, S, N)
    st = eng.stream
    t0 = time.perf_counter()
    with torch.cuda.stream(st):
        sh.ids.copy_(ids)
        sh.run_prefill()
        sh.kv.pos.fill_(S)
        if not sh.graph_ready:
            sh.decode.capture()
            sh.graph_ready = True
    st.synchronize()
    prefill_s = time.perf_counter() - t0
    with torch.cuda.stream(st):
        for _ in range(warmup):
            sh.decode.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    w0 = time.perf_counter()
    with torch.cuda.stream(st):
        e0.record(st)
        for _ in range(K):
            sh.decode.replay()
        e1.record(st)
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    sh.decode.check()                                   # persistent step: no expired wait
    ms = e0.elapsed_time(e1) / K
    # per-step spread: the same K steps again (pos rewound to the same context range), an
    # event after every replay; kept out of the headline timing above
    with torch.cuda.stream(st):
        sh.kv.pos.fill_(S + warmup)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(K + 1)]
    with torch.cuda.stream(st):
        ev[0].record(st)
        for i in range(K):
            sh.decode.replay()
            ev[i + 1].record(st)
    torch.cuda.synchronize()
    sh.decode.check()
    per = np.sort(np.array([ev[i].elapsed_time(ev[i + 1]) for i in range(K)]))
    spread = {"median": round(float(np.median(per)), 5),
              "p90": round(float(per[min(K - 1, int(0.9 * K))]), 5),
              "min": round(float(per[0]), 5), "max": round(float(per[-1]), 5)}
    ctx_mean = S + warmup + (K - 1) / 2.0 + 1           # keys read per step, averaged
    kv_bytes = B * ctx_mean * eng.model.kv_bytes_per_token
    step_bytes = eng.model.weight_bytes + kv_bytes
    return sh, {"B": B, "S": S, "K": K, "ms_per_step": ms, "wall_ms_per_step": wall * 1e3 / K,
                "step_ms": spread,
                "step": "qd_mega_step (persistent)" if sh.decode.mega else "qd_decode_step",
                "mega": sh.decode.mega,
                "tok_s": B * 1e3 / ms, "prefill_s": prefill_s, "bytes_per_step": step_bytes,
                "achieved_gbs": step_bytes / (ms * 1e-3) / 1e9}


def api_run(eng, B, S, N, seed, what):
    """The reference's own measure (QWEN_ENGINE_CONTRACT.md:93,102): batch x output tokens /
    total Engine.generate time, prefill included, through the drop-in API as a user gets it
    (tree speculation gate on its default, ``ENGINE_TREE=auto``).  The first call on a shape
    also captures the decode graph and runs the tree gate where it applies; it is reported
    apart, and the second call (same shape, a different prompt) is the measured one."""
    import numpy as np
    rng = np.random.default_rng(seed)
    out = {"workload": what, "B": B, "prompt_len": S, "new_tokens": N}
    for key in ("first_call", "warm"):
        prompt = rng.integers(0, eng.model.V, size=(B, S)).tolist()
        t0 = time.perf_counter()
        n = 0
        first_tok = None
        for step in eng.generate(prompt, N):
            n += 1
            if first_tok is None:
                first_tok = time.perf_counter() - t0
        wall = time.perf_counter() - t0
        assert n == N
        out[key] = {"wall_s": round(wall, 4), "tok_s": round(B * N / wall, 1),
                    "first_token_s": round(first_tok, 4)}
    out["tree_gate"] = eng.tree_log.get((B, S, N))
    out["value"], out["unit"] = out["warm"]["tok_s"], "tok/s"
    return out


def tree_run(eng, B=4, S=8192, T=64, K=20, warmup=3, N_e2e=256, seed=5):
    """Config 5: tree verification.  Prefill B prompts of S tokens, draft one random T-node tree
    per sequence (qdecode.tree.random_tree_drafter, branching 4-4-2-2), then time K replays of
    the verify forward (qd_block_step over B*T rows: every weight once + every row's K/V) with
    HIP events on the engine's stream.  Then an end-to-end generate_tree of N_e2e tokens (wall
    clock, drafting / accept walk / per-pass sync included) for tokens per pass."""
    import numpy as np
    import torch
    from qdecode import tree as tr
    rng = np.random.default_rng(seed)
    ids = torch.as_tensor(rng.integers(0, eng.model.V, size=(B, S)), dtype=torch.int64)
    eng.tree_T = T
    try:
        eng.shape = None
        sh = eng._state(B, S, N_e2e)
    finally:
        eng.tree_T = 0
    st = eng.stream
    t0 = time.perf_counter()
    with torch.cuda.stream(st):
        sh.ids.copy_(ids)
        sh.run_prefill()
    st.synchronize()
    prefill_s = time.perf_counter() - t0
    first = sh.kv.tok.cpu().tolist()
    drafter = tr.random_tree_drafter(seed)
    trees = [drafter(list(map(int, ids[b])) + [first[b]], T) for b in range(B)]
    run = sh.tree
    with torch.cuda.stream(st):
        run.tokens.copy_(torch.tensor([t.tokens for t in trees], dtype=torch.int64))
        run.depth.copy_(torch.tensor([t.depth for t in trees], dtype=torch.int64))
        run.anc.copy_(torch.tensor([t.anc_i64() for t in trees], dtype=torch.int64))
        run.base.fill_(S)
        for _ in range(warmup):
            run.launch(T)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(st):
        e0.record(st)
        for _ in range(K):
            run.launch(T)
        e1.record(st)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / K
    m = eng.model
    ctx = S + T
    kv_bytes = B * S * m.kv_bytes_per_token
    nbytes = m.weight_bytes + kv_bytes
    dense = 36 * (6144 * 2560 + 2560 * 4096 + 19456 * 2560 + 2560 * 9728) + m.V * m.H
    gemm_flop = 2.0 * B * T * dense
    attn_flop = 4.0 * B * T * 32 * 128 * ctx * m.L
    # end to end (same shape, host loop included): tree verification of N_e2e tokens, then
    # plain B=4 decode of the same prompt and N_e2e (the comparison that matters when random
    # drafts accept ~1 token per pass)
    prompt = ids.tolist()
    w0 = time.perf_counter()
    out = list(eng.generate_tree(prompt, N_e2e, tr.random_tree_drafter(seed + 1), T=T))
    wall = time.perf_counter() - w0
    stats = eng.tree_stats
    acc = stats["accepted"]
    host_ms = stats["host_ms"]
    mode = eng.tree_mode
    try:
        eng.tree_mode = "0"
        eng.shape = None
        list(eng.generate(prompt, N_e2e))                 # shape + graph capture, untimed
        p0 = time.perf_counter()
        plain = list(eng.generate(prompt, N_e2e))
        plain_wall = time.perf_counter() - p0
    finally:
        eng.tree_mode = mode
    return {"workload": f"config 5: tree verification, B={B}, context {S}, {T}-node random "
                        f"4-4-2-2 trees", "verify_ms": round(ms, 4), "verify_steps": K,
            "bytes_per_verify": int(nbytes), "achieved_gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "gemm_tflop_per_verify": round(gemm_flop / 1e12, 3),
            "attn_tflop_per_verify": round(attn_flop / 1e12, 3),
            "achieved_tflops": round((gemm_flop + attn_flop) / (ms * 1e-3) / 1e12, 1),
            "mfma_frac": round((gemm_flop + attn_flop) / (ms * 1e-3) / 2.5e15, 4),
            "prefill_s": round(prefill_s, 3),
            "e2e": {"new_tokens": N_e2e, "passes": stats["passes"],
                    "tokens_per_pass": round(sum(acc) / max(len(acc), 1), 3),
                    "host_ms_per_pass": round(sum(host_ms) / max(len(host_ms), 1), 4),
                    "wall_s": round(wall, 3), "tok_s": round(B * len(out) / wall, 1)},
            "plain_e2e": {"new_tokens": N_e2e, "wall_s": round(plain_wall, 3),
                          "tok_s": round(B * len(plain) / plain_wall, 1),
                          "note": "generate() with trees off, same prompt, prefill included"}}


def time_gu_kernel(eng, sh, reps=20):
    """Mean duration of the gate/up GEMV + SwiGLU launch (B rows) over all layers' weights."""
    import ctypes as C

    import torch
    from qdecode import _lib, ops
    m, st, dec = eng.model, eng.stream, sh.decode
    with torch.cuda.stream(st):
        _lib.call("qd_graph_begin", st.cuda_stream)
        try:
            for l in range(m.L):
                ops.linear(dec.x, m.w_gu[l], ops.EPI_SWIGLU, norm_w=m.ln2[l], eps=m.eps, out=dec.act)
        finally:
            ex = C.c_void_p()
            rc = _lib.LIB.qd_graph_end(st.cuda_stream, C.byref(ex))
        if rc != 0:
            raise _lib.QDError("qd_graph_end", rc)
        for _ in range(2):
            _lib.call("qd_graph_launch", ex, st.cuda_stream)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(st):
        e0.record(st)
        for _ in range(reps):
            _lib.call("qd_graph_launch", ex, st.cuda_stream)
        e1.record(st)
    torch.cuda.synchronize()
    _lib.LIB.qd_graph_destroy(ex)
    us = e0.elapsed_time(e1) * 1e3 / (reps * m.L)
    B = sh.B
    nbytes = 2 * (2 * m.I * m.H + B * m.H + m.H + B * m.I)   # W_gate|W_up + x + norm w + act
    return us, nbytes


def time_read_ceiling(eng, reps=20, grids=(768, 2048, 4864), bufs=None):
    """The read rate one launch can reach over the gate/up GEMV's weight bytes (or over each of
    `bufs`, equal-sized contiguous tensors): qd_read_probe (non-temporal 16-byte loads, nothing
    computed or written) over the same 36 layers' W_gate|W_up, captured as one hipGraph of 36
    launches like time_gu_kernel and replayed; the best of the grids.  Returns (us per launch,
    grid, bytes per launch)."""
    import ctypes as C

    import torch
    from qdecode import _lib
    m, st = eng.model, eng.stream
    sink = torch.zeros(1, dtype=torch.int32, device=m.device)
    bufs = [m.w_gu[l] for l in range(m.L)] if bufs is None else bufs
    nbytes = bufs[0].numel() * bufs[0].element_size()
    best = None
    for g in grids:
        with torch.cuda.stream(st):
            _lib.call("qd_graph_begin", st.cuda_stream)
            try:
                for w in bufs:
                    assert w.is_contiguous() and w.numel() * w.element_size() == nbytes
                    _lib.call("qd_read_probe", w.data_ptr(), nbytes, g, sink.data_ptr(),
                              st.cuda_stream)
            finally:
                ex = C.c_void_p()
                rc = _lib.LIB.qd_graph_end(st.cuda_stream, C.byref(ex))
            if rc != 0:
                raise _lib.QDError("qd_graph_end", rc)
            for _ in range(2):
                _lib.call("qd_graph_launch", ex, st.cuda_stream)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(st):
            e0.record(st)
            for _ in range(reps):
                _lib.call("qd_graph_launch", ex, st.cuda_stream)
            e1.record(st)
        torch.cuda.synchronize()
        _lib.LIB.qd_graph_destroy(ex)
        us = e0.elapsed_time(e1) * 1e3 / (reps * len(bufs))
        if best is None or us < best[0]:
            best = (us, g)
    return best[0], best[1], nbytes


def read_floors(eng, kv_bytes):
    """The streaming floor of one launch of each B=32 decode-step size: qd_read_probe over each
    projection's 36 per-layer weight tensors, and over four buffers of one layer's K/V bytes,
    best of grids 256-4096 (what a launch of that many bytes can read at all, ramp-up and drain
    included)."""
    import torch
    m = eng.model
    grids = (256, 512, 1024, 2048, 4096)
    out = {}
    for name, t in (("qkv", m.w_qkv), ("o", m.w_o), ("gate_up", m.w_gu), ("down", m.w_down)):
        us, g, nb = time_read_ceiling(eng, reps=10, grids=grids, bufs=[t[l] for l in range(m.L)])
        out[name] = {"bytes": nb, "us": round(us, 3), "grid": g,
                     "tb_s": round(nb / (us * 1e-6) / 1e12, 3)}
    kv = torch.empty((4, int(kv_bytes) // 2), dtype=torch.bfloat16, device=m.device)
    us, g, nb = time_read_ceiling(eng, reps=10, grids=grids, bufs=[kv[i] for i in range(4)])
    out["kv_layer"] = {"bytes": nb, "us": round(us, 3), "grid": g,
                       "tb_s": round(nb / (us * 1e-6) / 1e12, 3)}
    del kv
    return out


def layer_kernels(reps=1000):
    """Config 2: the fused layer kernels on their own, B in {1, 8, 64}, synthetic bf16 N(0, 1)
    activations, positions uniform on [0, 8192).  Each kernel is captured `reps` times into one
    hipGraph (fixed inputs and outputs) and the graph replayed; us_per_launch = replay time /
    reps, so it includes the per-node launch cost of a graph (~1.6 us), which at these sizes
    (10 KB - 3.7 MB) is most of it.  Bytes are the algorithmic ones: gather 2 B 5120;
    add+RMSNorm 4 B 5120 + 5120; QK-norm+RoPE (q, k, v read and written) 2 B 48 256 + 2 B 256
    (cos/sin rows); SwiGLU 3 B 19456."""
    import ctypes as C

    import torch
    from qdecode import _lib, ops
    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(7)
    bf = torch.bfloat16
    H, I, V, Hq, Hkv, cap = 2560, 9728, 151936, 32, 8, 8192
    table = torch.randn((V, H), generator=g, device=dev).to(bf)
    w = torch.ones(H, dtype=bf, device=dev)
    cos = torch.randn((cap, 128), generator=g, device=dev).to(bf)
    sin = torch.randn((cap, 128), generator=g, device=dev).to(bf)
    qn = torch.ones(128, dtype=bf, device=dev)
    st = torch.cuda.Stream()
    out = []
    for B in (1, 8, 64):
        ids = torch.randint(0, V, (B,), generator=g, device=dev)
        emb = torch.empty((B, H), dtype=bf, device=dev)
        x = torch.randn((B, H), generator=g, device=dev).to(bf)
        r = torch.randn((B, H), generator=g, device=dev).to(bf)
        ro, y = torch.empty_like(r), torch.empty_like(r)
        qkv = torch.randn((B, (Hq + 2 * Hkv) * 128), generator=g, device=dev).to(bf)
        pos = torch.randint(0, cap, (B,), generator=g, device=dev)
        q_out = torch.empty((B, 1, Hq, 128), dtype=bf, device=dev)
        kc = torch.zeros((B, Hkv, cap, 128), dtype=bf, device=dev)
        vc = torch.zeros_like(kc)
        gu = torch.randn((B, 2 * I), generator=g, device=dev).to(bf)
        act = torch.empty((B, I), dtype=bf, device=dev)
        cases = [
            ("embed_gather", 2 * B * H * 2, lambda: ops.embed_gather(ids, table, out=emb)),
            ("add_rmsnorm", 4 * B * H * 2 + H * 2,
             lambda: ops.add_rmsnorm(r, w, 1e-6, x=x, res_out=ro, y=y)),
            ("qk_norm_rope", 2 * B * 48 * 256 + 2 * B * 256,
             lambda: ops.qk_norm_rope(qkv, qn, qn, cos, sin, pos, ops.POS_ROW, q_out, kc, vc,
                                      B, 1, Hq, Hkv, 1e-6)),
            ("swiglu", 3 * B * I * 2, lambda: ops.swiglu(gu, out=act)),
        ]
        for name, nbytes, fn in cases:
            torch.cuda.synchronize()
            with torch.cuda.stream(st):
                fn()                                     # argument checks outside the capture
                _lib.call("qd_graph_begin", st.cuda_stream)
                try:
                    for _ in range(reps):
                        fn()
                finally:
                    ex = C.c_void_p()
                    rc = _lib.LIB.qd_graph_end(st.cuda_stream, C.byref(ex))
                if rc != 0:
                    raise _lib.QDError("qd_graph_end", rc)
                _lib.call("qd_graph_launch", ex, st.cuda_stream)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            with torch.cuda.stream(st):
                e0.record(st)
                for _ in range(3):
                    _lib.call("qd_graph_launch", ex, st.cuda_stream)
                e1.record(st)
            torch.cuda.synchronize()
            _lib.LIB.qd_graph_destroy(ex)
            us = e0.elapsed_time(e1) * 1e3 / (3 * reps)
            out.append({"kernel": name, "B": B, "us_per_launch": round(us, 3), "bytes": nbytes,
                        "achieved_gbs": round(nbytes / (us * 1e-6) / 1e9, 1)})
        del kc, vc
    return out


def _graph_time_us(fn, reps, rounds=5):
    """Mean µs of one fn() call: fn captured `reps` times into a hipGraph on a side stream,
    replayed `rounds` times between HIP events on that stream."""
    import ctypes as C

    import torch
    from qdecode import _lib
    st = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(st):
        fn()                                             # argument checks outside the capture
        _lib.call("qd_graph_begin", st.cuda_stream)
        try:
            for _ in range(reps):
                fn()
        finally:
            ex = C.c_void_p()
            rc = _lib.LIB.qd_graph_end(st.cuda_stream, C.byref(ex))
        if rc != 0:
            raise _lib.QDError("qd_graph_end", rc)
        _lib.call("qd_graph_launch", ex, st.cuda_stream)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(st):
        e0.record(st)
        for _ in range(rounds):
            _lib.call("qd_graph_launch", ex, st.cuda_stream)
        e1.record(st)
    torch.cuda.synchronize()
    _lib.LIB.qd_graph_destroy(ex)
    return e0.elapsed_time(e1) * 1e3 / (rounds * reps)


def layer_kernels_large(reps=20, scale=1):
    """The config-2 layer kernels at row counts where bandwidth binds (>= 100 MB per launch;
    the config's own B <= 64 moves 10 KB - 3.7 MB): embedding gather of 16384 ids, add +
    RMSNorm of 8192 rows, QK-norm + RoPE + K/V write of 8192 token rows (one sequence at
    positions 0..8191, i.e. the whole config-2 position range), SwiGLU of 4096 rows; with
    scale=4, four times those rows (the prefill chunk's 32768 rows for the norms).  Bytes
    are algorithmic (every input read once, every output written once).  `copy_gbs` is a
    device-to-device copy of the same number of bytes (half read, half written) by the
    runtime, the read+write stream these kernels compare to; `frac` is of 8 TB/s."""
    import torch
    from qdecode import ops
    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(11)
    bf = torch.bfloat16
    H, I, V, Hq, Hkv = 2560, 9728, 151936, 32, 8
    out = []

    def record(name, rows, nbytes, fn):
        us = _graph_time_us(fn, reps)
        src = torch.empty(nbytes // 4, dtype=torch.int16, device=dev)
        dst = torch.empty_like(src)
        cus = _graph_time_us(lambda: dst.copy_(src), reps)
        del src, dst
        gbs = nbytes / (us * 1e-6) / 1e9
        out.append({"kernel": name, "rows": rows, "bytes": nbytes, "us_per_launch": round(us, 2),
                    "achieved_gbs": round(gbs, 1), "frac": round(gbs / 8000.0, 4),
                    "copy_gbs": round(nbytes / (cus * 1e-6) / 1e9, 1)})

    table = torch.randn((V, H), generator=g, device=dev).to(bf)
    n = 16384 * scale
    ids = torch.randint(0, V, (n,), generator=g, device=dev)
    emb = torch.empty((n, H), dtype=bf, device=dev)
    record("embed_gather", n, 2 * n * H * 2, lambda: ops.embed_gather(ids, table, out=emb))
    del table, emb

    n = 8192 * scale
    x = torch.randn((n, H), generator=g, device=dev).to(bf)
    r = torch.randn((n, H), generator=g, device=dev).to(bf)
    w = torch.ones(H, dtype=bf, device=dev)
    ro, y = torch.empty_like(r), torch.empty_like(r)
    record("add_rmsnorm", n, 4 * n * H * 2 + H * 2,
           lambda: ops.add_rmsnorm(r, w, 1e-6, x=x, res_out=ro, y=y))
    del x, r, ro, y

    T = 8192 * scale
    qkv = torch.randn((T, (Hq + 2 * Hkv) * 128), generator=g, device=dev).to(bf)
    cos = torch.randn((T, 128), generator=g, device=dev).to(bf)
    sin = torch.randn((T, 128), generator=g, device=dev).to(bf)
    qn = torch.ones(128, dtype=bf, device=dev)
    q_out = torch.empty((1, T, Hq, 128), dtype=bf, device=dev)
    kc = torch.zeros((1, Hkv, T, 128), dtype=bf, device=dev)
    vc = torch.zeros_like(kc)
    zero = torch.zeros(1, dtype=torch.int64, device=dev)
    record("qk_norm_rope", T, 2 * T * (Hq + 2 * Hkv) * 128 * 2 + T * 2 * 128 * 2,
           lambda: ops.qk_norm_rope(qkv, qn, qn, cos, sin, zero, ops.POS_SHARED, q_out, kc, vc,
                                    1, T, Hq, Hkv, 1e-6))
    del qkv, q_out, kc, vc

    n = 4096 * scale
    gu = torch.randn((n, 2 * I), generator=g, device=dev).to(bf)
    act = torch.empty((n, I), dtype=bf, device=dev)
    record("swiglu", n, 3 * n * I * 2, lambda: ops.swiglu(gu, out=act))
    return out


def prefill_gemm(rows=32768, reps=20):
    """The four projections at a prefill chunk's row count through qd_linear (RMSNorm-free
    operands: the GEMM alone) and torch.matmul (hipBLASLt) on the same operands; synthetic bf16
    N(0, 1) activations, N(0, 0.02) weights.  HIP events on the current stream (the one both
    calls launch on) around `reps` back-to-back launches after 5 warm-up launches."""
    import torch
    from qdecode import ops
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(21)
    shapes = [("qkv", 6144, 2560, ops.EPI_NONE), ("o", 2560, 4096, ops.EPI_NONE),
              ("gate_up_swiglu", 2 * 9728, 2560, ops.EPI_SWIGLU), ("down", 2560, 9728, ops.EPI_NONE)]

    def timed(fn):
        for _ in range(5):
            fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / reps

    out = []
    for name, n_w, K, epi in shapes:
        x = torch.randn(rows, K, device=dev, dtype=torch.bfloat16, generator=g)
        w = torch.randn(n_w, K, device=dev, dtype=torch.bfloat16, generator=g) * 0.02
        y = torch.empty(rows, n_w // 2 if epi == ops.EPI_SWIGLU else n_w, device=dev,
                        dtype=torch.bfloat16)
        yb = torch.empty(rows, n_w, device=dev, dtype=torch.bfloat16)
        flop = 2.0 * rows * n_w * K
        need = ops._lib.LIB.qd_linear_workspace_bytes(rows, y.shape[1], K, 0)
        ws = ops.workspace(need, dev) if need else None
        us = timed(lambda: ops.linear(x, w, epi, out=y, ws=ws))
        ub = timed(lambda: torch.matmul(x, w.t(), out=yb))
        out.append({"gemm": name, "rows": rows, "n": n_w, "k": K, "us_per_launch": round(us, 1),
                    "tflops": round(flop / us / 1e6, 1),
                    "frac": round(flop / us / 1e6 / PEAK_BF16_TFLOPS, 4),
                    "hipblaslt_us": round(ub, 1), "hipblaslt_tflops": round(flop / ub / 1e6, 1)})
        del x, w, y, yb, ws
        torch.cuda.empty_cache()
    return out


def cpu_baseline(budget_s=15.0, prompt_len=512):
    """The CPU oracle (torch CPU, oneDNN bf16) on the same 36-layer architecture and
    generator: prefill config 3's 512-token prompt (untimed), then time greedy decode steps for
    ~budget_s, on the host's CPU share (OMP_NUM_THREADS threads: 16 per GPU on the GPU box)."""
    import numpy as np
    import torch
    sys.path.insert(0, ROOT)
    from oracle import qwen3_ref, synth
    lib = os.path.join(ROOT, "oracle", "_build", "libcsynth.so")
    if not os.path.exists(lib):
        import subprocess
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = os.cpu_count()
    t0 = time.perf_counter()
    ref = qwen3_ref.Qwen3Ref.from_synth(1, 36)
    gen_s = time.perf_counter() - t0
    prompt = torch.as_tensor(synth.prompt_ids(1, 1, prompt_len))
    max_steps = 400
    cap = prompt_len + max_steps + 1
    cache = ref.new_cache(1, cap)
    with torch.inference_mode():
        lg = ref.prefill(prompt, cache)
        tok = qwen3_ref.argmax_lowest(lg[:, -1])
        n, t1 = 0, time.perf_counter()
        while n < 3 or (time.perf_counter() - t1 < budget_s and n < max_steps):
            lg = ref.decode(tok, prompt_len + n, cache)
            tok = qwen3_ref.argmax_lowest(lg)
            n += 1
        dt = time.perf_counter() - t1
    cpu = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            cpu = next(l.split(":", 1)[1].strip() for l in f if l.startswith("model name"))
    except Exception:
        pass
    return {"value": n / dt, "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": (f"oracle/qwen3_ref.py greedy decode, 36-layer Qwen3-4B shape, B=1, "
                       f"{n} steps after a {prompt_len}-token prefill ({dt:.1f} s; weight "
                       f"generation {gen_s:.1f} s and the prefill untimed); "
                       f"torch {torch.__version__} CPU on "
                       f"{threads} threads (the host's CPU share; {affinity} in the affinity "
                       f"mask) of {cpu}")}


def cpu_config1():
    """Config 1 in full on the CPU oracle: 4 layers (seed 0), B=1, 128-token prompt, 32 greedy
    tokens, prefill included (the reference's CPU path, engine.py:963-972)."""
    import torch
    sys.path.insert(0, ROOT)
    from oracle import qwen3_ref, synth
    ref = qwen3_ref.Qwen3Ref.from_synth(0, 4)
    prompt = torch.as_tensor(synth.prompt_ids(0, 1, 128))
    with torch.inference_mode():
        t0 = time.perf_counter()
        toks, _ = ref.greedy(prompt, 32)
        dt = time.perf_counter() - t0
    return {"workload": "config 1: 4 layers, B=1, S=128, N=32, greedy with prefill (full run)",
            "value": round(32 / dt, 3), "unit": "tok/s", "wall_s": round(dt, 3),
            "cores": torch.get_num_threads(), "kind": "port"}


def cpu_config4(budget_s=12.0, B=32, ctx=2048):
    """Config 4's decode step on the CPU oracle, capped: B=32 sequences at context 2048, 36
    layers.  The 32 x 2048-token prefill (minutes on the host) is replaced by a KV cache
    filled with seeded bf16 values (the step's cost does not depend on them), then greedy
    decode steps are timed for ~budget_s."""
    import torch
    sys.path.insert(0, ROOT)
    from oracle import qwen3_ref
    ref = qwen3_ref.Qwen3Ref.from_synth(1, 36)
    g = torch.Generator().manual_seed(4)
    cap = ctx + 64
    kc, vc = ref.new_cache(B, cap)
    kc[:, :, :, :ctx].copy_(torch.randn(kc[:, :, :, :ctx].shape, generator=g).to(kc.dtype))
    vc[:, :, :, :ctx].copy_(torch.randn(vc[:, :, :, :ctx].shape, generator=g).to(vc.dtype))
    tok = torch.randint(0, ref.embed.shape[0], (B,), generator=g)
    n = 0
    with torch.inference_mode():
        t0 = time.perf_counter()
        while n < 2 or (time.perf_counter() - t0 < budget_s and n < 200):
            tok = qwen3_ref.argmax_lowest(ref.decode(tok, ctx + n, (kc, vc)))
            n += 1
        dt = time.perf_counter() - t0
    return {"workload": f"config 4 decode step, capped: 36 layers, B={B}, context {ctx} "
                        f"(KV cache filled with seeded values instead of the 32 x 2048 prefill), "
                        f"{n} steps ({dt:.1f} s)",
            "value": round(B * n / dt, 3), "unit": "tok/s", "ms_per_step": round(dt * 1e3 / n, 2),
            "cores": torch.get_num_threads(), "kind": "port"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--b32-steps", type=int, default=100)
    ap.add_argument("--no-b32", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-tree", action="store_true")
    ap.add_argument("--no-layer", action="store_true", help="skip the config-2 kernel microbench")
    ap.add_argument("--no-api", action="store_true", help="skip the Engine.generate runs")
    ap.add_argument("--no-gemm", action="store_true", help="skip the prefill GEMM comparison")
    ap.add_argument("--tree-steps", type=int, default=20, help="timed verify forwards")
    ap.add_argument("--tree-e2e", type=int, default=256, help="tokens of the end-to-end tree run")
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="first run one plain device copy of this many MiB: the reference "
                         "dispatch that scales rocprofv3 FETCH_SIZE / WRITE_SIZE to bytes")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build is single-GPU (the decode path would shard "
              "by sequence, one full weight copy per GPU, with no collective). Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)
    import torch
    from engine import Engine

    torch.cuda.set_device(0)
    if a.calib_copy_mib > 0:
        n = a.calib_copy_mib << 19                     # bf16 elements
        src = torch.ones(n, dtype=torch.bfloat16, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"calibration copy: {a.calib_copy_mib} MiB read + {a.calib_copy_mib} MiB written")
        del src, dst
    t0 = time.perf_counter()
    eng = Engine.synthetic(n_layers=36, seed=1)
    log(f"weights generated on device in {time.perf_counter() - t0:.1f}s "
        f"({eng.model.weight_bytes / 1e9:.3f} GB per step)")

    sh, r1 = decode_run(eng, B=1, S=512, N=256, warmup=a.warmup, steps=a.steps, seed=3)
    log(f"B=1: {r1['ms_per_step']:.4f} ms/step, {r1['tok_s']:.1f} tok/s, "
        f"{r1['achieved_gbs']:.0f} GB/s, prefill {r1['prefill_s']:.2f}s")
    us, gu_bytes = time_gu_kernel(eng, sh)
    log(f"gate/up GEMV: {us:.2f} us/launch, {gu_bytes / (us * 1e-6) / 1e9:.0f} GB/s")
    ceil_us, ceil_grid, ceil_bytes = time_read_ceiling(eng)
    log(f"read ceiling over the same weights: {ceil_us:.2f} us/launch, "
        f"{ceil_bytes / (ceil_us * 1e-6) / 1e9:.0f} GB/s (grid {ceil_grid})")

    layer = layer_large = None
    if not a.no_layer:
        eng.shape = None
        sh = None
        torch.cuda.empty_cache()
        layer = layer_kernels()
        for c in layer:
            log(f"config 2 {c['kernel']:>13} B={c['B']:>2}: {c['us_per_launch']:.2f} us/launch, "
                f"{c['achieved_gbs']:.0f} GB/s")
        torch.cuda.empty_cache()
        layer_large = layer_kernels_large()
        for c in layer_large:
            log(f"config 2 large {c['kernel']:>13} rows={c['rows']:>5}: {c['us_per_launch']:.2f} "
                f"us/launch, {c['achieved_gbs']:.0f} GB/s ({c['frac']:.3f} of peak; device copy "
                f"of the same bytes {c['copy_gbs']:.0f} GB/s)")
        torch.cuda.empty_cache()

    b32 = None
    if not a.no_b32:
        eng.shape = None
        sh = None
        torch.cuda.empty_cache()
        sh32, r32 = decode_run(eng, B=32, S=2048, N=128, warmup=10, steps=a.b32_steps, seed=4)
        log(f"B=32: {r32['ms_per_step']:.4f} ms/step, {r32['tok_s']:.1f} tok/s, "
            f"{r32['achieved_gbs']:.0f} GB/s, prefill {r32['prefill_s']:.2f}s")
        b32 = {"workload": "config 4: 36 layers, B=32, prompts 2048, N=128", "steps": r32["K"],
               "decode_step": r32["step"],
               "warmup": 10, "ms_per_step": round(r32["ms_per_step"], 5),
               "value": round(r32["tok_s"], 2), "unit": "tok/s", "step_ms": r32["step_ms"],
               "step_roofline": {"bound": "hbm", "achieved": round(r32["achieved_gbs"], 1),
                                 "peak": PEAK_HBM_GBS, "unit": "GB/s",
                                 "frac": round(r32["achieved_gbs"] / PEAK_HBM_GBS, 4),
                                 "bytes_per_step": int(r32["bytes_per_step"])},
               "prefill_s": round(r32["prefill_s"], 3)}
        # one layer's K/V read at the timed steps' mean context
        kv_layer = r32["B"] * (2048 + 10 + (r32["K"] - 1) / 2 + 1) * eng.model.kv_bytes_per_token / eng.model.L
        eng.shape = None
        del sh32
        torch.cuda.empty_cache()
        b32["read_floors"] = read_floors(eng, kv_layer // 16 * 16)
        log("B=32 read floors: " + ", ".join(f"{k} {v['us']} us" for k, v in b32["read_floors"].items()))
        torch.cuda.empty_cache()

    api = None
    if not a.no_api:
        eng.shape = None
        torch.cuda.empty_cache()
        api = {"config3": api_run(eng, 1, 512, 256, 13, "config 3 through Engine.generate: "
                                  "B=1, prompt 512, 256 new tokens")}
        log(f"API config 3: {api['config3']['warm']['tok_s']} tok/s (prefill included), first "
            f"call {api['config3']['first_call']['tok_s']}")
        if not a.no_b32:
            eng.shape = None
            torch.cuda.empty_cache()
            api["config4"] = api_run(eng, 32, 2048, 128, 14, "config 4 through Engine.generate: "
                                     "B=32, prompts 2048, 128 new tokens")
            log(f"API config 4: {api['config4']['warm']['tok_s']} tok/s (prefill included)")
        eng.shape = None
        torch.cuda.empty_cache()

    tree = None
    if not a.no_tree:
        eng.shape = None
        torch.cuda.empty_cache()
        tree = tree_run(eng, K=a.tree_steps, N_e2e=a.tree_e2e)
        log(f"tree verify (B=4, ctx 8192, T=64): {tree['verify_ms']:.3f} ms, "
            f"{tree['achieved_gbs']:.0f} GB/s, {tree['achieved_tflops']:.1f} TFLOP/s; "
            f"e2e {tree['e2e']['tok_s']} tok/s, prefill {tree['prefill_s']:.2f}s")
        eng.shape = None
        torch.cuda.empty_cache()

    pgemm = None
    if not a.no_gemm:
        eng.shape = None
        torch.cuda.empty_cache()
        pgemm = prefill_gemm()
        for c in pgemm:
            log(f"prefill GEMM {c['gemm']:>14}: {c['us_per_launch']:.1f} us, {c['tflops']:.0f} "
                f"TFLOP/s ({c['frac']:.3f} of 2.5 PF); hipBLASLt {c['hipblaslt_us']:.1f} us, "
                f"{c['hipblaslt_tflops']:.0f} TFLOP/s")
        torch.cuda.empty_cache()

    cpu = cpu_more = None
    if not a.no_cpu:
        eng = None
        torch.cuda.empty_cache()
        cpu = cpu_baseline(a.cpu_budget)
        log(f"cpu baseline: {cpu['value']:.3f} tok/s on {cpu['cores']} threads")
        cpu_more = {"config1": cpu_config1(), "config4": cpu_config4()}
        log(f"cpu config 1: {cpu_more['config1']['value']} tok/s; config 4 capped: "
            f"{cpu_more['config4']['value']} tok/s")

    gu_gbs = gu_bytes / (us * 1e-6) / 1e9
    gemv = {"bound": "hbm", "kernel": "gemv_kernel gate/up + SwiGLU (B=1, per-launch step)",
            "achieved": round(gu_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(gu_gbs / PEAK_HBM_GBS, 4), "traffic": GU_TRAFFIC_B1,
            "bytes_per_launch": gu_bytes, "us_per_launch": round(us, 3),
            # qd_read_probe over the same weight bytes: what one launch of this size can read
            "read_ceiling": {"us_per_launch": round(ceil_us, 3), "grid": ceil_grid,
                             "bytes_per_launch": ceil_bytes,
                             "achieved": round(ceil_bytes / (ceil_us * 1e-6) / 1e9, 1),
                             "frac": round(ceil_bytes / (ceil_us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4)},
            "of_read_ceiling": round(ceil_us / us, 4)}
    if r1["mega"]:
        roofline = {"bound": "hbm", "kernel": "mega_step_kernel (whole B=1 decode step)",
                    "achieved": round(r1["achieved_gbs"], 1), "peak": PEAK_HBM_GBS,
                    "unit": "GB/s", "frac": round(r1["achieved_gbs"] / PEAK_HBM_GBS, 4),
                    "traffic": MEGA_TRAFFIC_B1, "bytes_per_launch": int(r1["bytes_per_step"]),
                    "us_per_launch": round(r1["ms_per_step"] * 1e3, 2)}
    else:
        roofline = gemv
    line = {
        "metric": METRIC, "value": round(r1["tok_s"], 2), "unit": "tok/s", "n_gpus": 1,
        "steps": r1["K"], "warmup": a.warmup, "ms_per_step": round(r1["ms_per_step"], 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: seeded random-init bf16 weights N(0, 0.02) (norm weights 1), "
                "uniform prompt ids",
        "config": {"workload": "config 3: Qwen3-4B-shaped 36 layers, B=1, prompt 512, "
                               "N=256 greedy decode (steps timed after prefill)",
                   "batch": 1, "prompt_len": 512, "new_tokens": 256, "layers": 36,
                   "decode_step": r1["step"]},
        "roofline": roofline,
        "gemv_gate_up": gemv,
        "step_roofline": {"bound": "hbm", "achieved": round(r1["achieved_gbs"], 1),
                          "peak": PEAK_HBM_GBS, "unit": "GB/s",
                          "frac": round(r1["achieved_gbs"] / PEAK_HBM_GBS, 4),
                          "bytes_per_step": int(r1["bytes_per_step"])},
        "wall_ms_per_step": round(r1["wall_ms_per_step"], 5),
        "step_ms": r1["step_ms"],
        "prefill_s": round(r1["prefill_s"], 3),
        "b32": b32,
        "tree": tree,
        "prefill_gemm": pgemm,
        "layer_kernels": layer,
        "layer_kernels_large": layer_large,
        "api": api,
        "cpu_baseline": cpu,
        "cpu_baseline_configs": cpu_more,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
