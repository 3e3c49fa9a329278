"""GPU parity of each libqdecode kernel against the CPU oracle (oracle/qwen3_ref.py) on seeded
inputs.  Bars (north star): embedding gather, argmax index, K/V copies and the synthetic
generator bit-exact; fused layer kernels within 2 bf16 ulp (fp32 accumulate); fp32 logits
within 2e-2 max-abs."""

import os

import numpy as np
import pytest
import torch

from helpers import GOLDEN, assert_ulp, bf16_ulp
from oracle import qwen3_ref as R
from oracle import synth

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
BF = torch.bfloat16


@pytest.fixture(scope="module")
def ops():
    from qdecode import ops as o
    return o


def say(msg):
    print(f"\n[case] {msg}", flush=True)


def rnd(g, *shape, scale=1.0):
    return (torch.randn(shape, generator=g) * scale).to(BF)


def sync():
    torch.cuda.synchronize()


# ------------------------------------------------------------------ generator
def test_synth_bitexact(ops):
    for seed, sid, start, n in [(0, 1, 0, 1 << 20), (1, 16 + 16 * 35 + 6, 12345, 100003),
                                (0, 17, (1 << 31) - 50, 4096)]:
        say(f"synth seed={seed} stream={sid} start={start} n={n}")
        out = torch.empty(n, dtype=BF, device=DEV)
        ops.synth_bf16(out, seed, sid, start, 0.02)
        sync()
        got = out.cpu().view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(got, synth.normal_bf16_bits(seed, sid, start, n))


# ------------------------------------------------------------------ config 2 layer kernels
@pytest.mark.parametrize("B", [1, 8, 64])
def test_embed_gather_bitexact(ops, B):
    say(f"embed_gather B={B}")
    g = torch.Generator().manual_seed(B)
    table = rnd(g, 151936, 2560)
    ids = torch.randint(0, 151936, (B,), generator=g)
    ids[0] = 151935
    out = ops.embed_gather(ids.to(DEV), table.to(DEV))
    sync()
    assert torch.equal(out.cpu(), table[ids])


def test_embed_gather_out_of_range_row_is_zero(ops):
    say("embed_gather out-of-range id")
    table = torch.ones((64, 2560), dtype=BF, device=DEV)
    ids = torch.tensor([3, 64, -1], dtype=torch.int64, device=DEV)
    out = ops.embed_gather(ids, table)
    sync()
    assert torch.all(out[0] == 1) and torch.all(out[1:] == 0)


@pytest.mark.parametrize("B", [1, 8, 64])
def test_add_rmsnorm(ops, B):
    say(f"add_rmsnorm B={B}")
    g = torch.Generator().manual_seed(100 + B)
    x, r = rnd(g, B, 2560), rnd(g, B, 2560, scale=4.0)
    w = rnd(g, 2560, scale=0.1) + 1
    r_out, y = ops.add_rmsnorm(r.to(DEV), w.to(DEV), 1e-6, x=x.to(DEV))
    sync()
    r_ref, y_ref = R.add_rmsnorm(x, r, w)
    assert torch.equal(r_out.cpu(), r_ref)               # bf16(x + r): one rounding, exact
    assert_ulp(y.cpu(), y_ref, 2, "add_rmsnorm")
    y2 = ops.rmsnorm(r.to(DEV), w.to(DEV), 1e-6)         # no residual input
    sync()
    assert_ulp(y2.cpu(), R.rmsnorm(r, w), 2, "rmsnorm")


def test_add_rmsnorm_many_rows(ops):
    """Launches of more rows than 32 workgroups per CU take the multi-row kernel (each
    workgroup walks rows with the next row's loads in flight); its per-row arithmetic is the
    one-workgroup-per-row kernel's, so the bits are the same: 32 x CUs + 100 rows at once
    against the same rows in pieces of at most 2048 (the per-row kernel), with and without the
    residual input, also in place (res_out = residual), and within 2 ulp of the oracle."""
    n = 32 * torch.cuda.get_device_properties(0).multi_processor_count + 100
    say(f"add_rmsnorm {n} rows: multi-row kernel == per-row kernel, bitwise")
    g = torch.Generator().manual_seed(123)
    x, r = rnd(g, n, 2560).to(DEV), rnd(g, n, 2560, scale=4.0).to(DEV)
    w = (rnd(g, 2560, scale=0.1) + 1).to(DEV)
    r_all, y_all = ops.add_rmsnorm(r, w, 1e-6, x=x)
    y0_all = ops.rmsnorm(r, w, 1e-6)
    r_pc, y_pc, y0_pc = torch.empty_like(r), torch.empty_like(r), torch.empty_like(r)
    for a in range(0, n, 2048):
        b = min(n, a + 2048)
        ops.add_rmsnorm(r[a:b], w, 1e-6, x=x[a:b], res_out=r_pc[a:b], y=y_pc[a:b])
        ops.rmsnorm(r[a:b], w, 1e-6, y=y0_pc[a:b])
    rr = r.clone()                                       # in place: res_out = residual
    _, y_in = ops.add_rmsnorm(rr, w, 1e-6, x=x, res_out=rr)
    sync()
    assert torch.equal(r_all, r_pc) and torch.equal(rr, r_pc)
    assert torch.equal(y_all.view(torch.int16), y_pc.view(torch.int16))
    assert torch.equal(y_in.view(torch.int16), y_pc.view(torch.int16))
    assert torch.equal(y0_all.view(torch.int16), y0_pc.view(torch.int16))
    r_ref, y_ref = R.add_rmsnorm(x[:512].cpu(), r[:512].cpu(), w.cpu())
    assert torch.equal(r_all[:512].cpu(), r_ref)
    assert_ulp(y_all[:512].cpu(), y_ref, 2, "add_rmsnorm, many rows")


@pytest.mark.parametrize("B", [1, 8, 64])
def test_qk_norm_rope_kv_write(ops, B):
    say(f"qk_norm_rope B={B} positions U[0,8192)")
    g = torch.Generator().manual_seed(200 + B)
    Hq, Hkv, cap = 32, 8, 8192
    qkv = rnd(g, B, (Hq + 2 * Hkv) * 128, scale=2.0)
    qn, kn = rnd(g, 128, scale=0.2) + 1, rnd(g, 128, scale=0.2) + 1
    pos = torch.randint(0, cap, (B,), generator=g)
    cos, sin = R.rope_tables(cap)
    kc = torch.zeros((B, Hkv, cap, 128), dtype=BF, device=DEV)
    vc = torch.zeros_like(kc)
    q_out = torch.empty((B, 1, Hq, 128), dtype=BF, device=DEV)
    ops.qk_norm_rope(qkv.to(DEV), qn.to(DEV), kn.to(DEV), cos.to(DEV), sin.to(DEV), pos.to(DEV),
                     ops.POS_ROW, q_out, kc, vc, B, 1, Hq, Hkv, 1e-6)
    sync()
    q = qkv[:, :Hq * 128].view(B, 1, Hq, 128)
    k = qkv[:, Hq * 128:(Hq + Hkv) * 128].view(B, 1, Hkv, 128)
    v = qkv[:, (Hq + Hkv) * 128:].view(B, Hkv, 128)
    q_ref, k_ref = R.qk_norm_rope(q, k, qn, kn, cos[pos][:, None], sin[pos][:, None])
    assert_ulp(q_out.cpu(), q_ref, 2, "q")
    kcc, vcc = kc.cpu(), vc.cpu()
    bi = torch.arange(B)
    assert_ulp(kcc[bi, :, pos], k_ref[:, 0], 2, "k cache")
    assert torch.equal(vcc[bi, :, pos], v)               # V is copied as is
    mask = torch.ones((B, cap), dtype=torch.bool)
    mask[bi, pos] = False
    assert torch.all(kcc.permute(0, 2, 1, 3)[mask] == 0)  # nothing else written


@pytest.mark.parametrize("B", [1, 8, 64])
def test_swiglu(ops, B):
    say(f"swiglu B={B}")
    g = torch.Generator().manual_seed(300 + B)
    gu = rnd(g, B, 2 * 9728, scale=3.0)
    out = ops.swiglu(gu.to(DEV))
    sync()
    assert_ulp(out.cpu(), R.swiglu(gu[:, :9728], gu[:, 9728:]), 2, "swiglu")


def test_silu_every_bf16_input(ops):
    """bf16(silu(g)) over the whole domain -- all 65,536 bf16 bit patterns g -- equals the table
    recorded from the IEEE evaluation (tests/golden/record_silu_table.py; the CPU suite pins the
    table to the oracle's silu bit for bit), so the SwiGLU paths' cheaper evaluation with its
    near-midpoint fallback changes no result."""
    import sys
    sys.path.insert(0, GOLDEN)
    from record_silu_table import silu_table
    say("silu over all 65536 bf16 inputs against the recorded table")
    want = np.load(os.path.join(GOLDEN, "silu_bf16.npy"))
    got = silu_table(torch.device(DEV))
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{bad.size} inputs differ, first {[hex(int(x)) for x in bad[:8]]}"


# ------------------------------------------------------------------ projections
def exact_linear(x, w):
    """fp64 dot products of the bf16 inputs, rounded once to bf16 (and the fp64 values)."""
    acc = x.double() @ w.double().T
    return acc.to(torch.float32).to(BF), acc


SHAPES = {"qkv": (6144, 2560), "o": (2560, 4096), "gu": (9728, 2560), "down": (2560, 9728)}


# 1..2 rows: vector GEMV; 3..32: the skinny kernel (one workgroup per CU; 20 rows: a ragged
# second activation tile); 64: the LDS-staged MFMA kernel; 100, 256, 600 rows: the LDS-tiled
# kernel (128-row tiles with a ragged last tile; K split over workgroups with the fp32 partials
# summed by a second kernel where the tile grid is small: qkv / o / down at 100 and 256 rows,
# o / down at 600); 1040 rows: the 256 x 256-tile prefill kernel (four full row blocks and a
# ragged 16-row one)
@pytest.mark.parametrize("B", [1, 2, 3, 16, 20, 32, 64, 65, 100, 200, 256, 600, 1040])
@pytest.mark.parametrize("name", ["qkv", "o", "gu", "down"])
def test_linear_epilogues(ops, name, B):
    say(f"linear {name} B={B}")
    N, K = SHAPES[name]
    g = torch.Generator().manual_seed(1000 * B + sum(map(ord, name)))
    w = rnd(g, 2 * N if name == "gu" else N, K, scale=0.02)
    x = rnd(g, B, K)
    wd, xd = w.to(DEV), x.to(DEV)
    if name == "qkv":                                    # RMSNorm prologue, plain epilogue
        nw = rnd(g, K, scale=0.1) + 1
        out = ops.linear(xd, wd, ops.EPI_NONE, norm_w=nw.to(DEV), eps=1e-6)
        sync()
        want, _ = exact_linear(R.rmsnorm(x, nw).float(), w.float())
        # the normalised input itself may differ by 1 ulp (reduction order), hence 2 ulp + floor
        assert_ulp(out.cpu(), want, 2, "qkv", abs_floor=2 ** -9)
    elif name == "gu":                                   # RMSNorm prologue + SwiGLU epilogue
        nw = rnd(g, K, scale=0.1) + 1
        out = ops.linear(xd, wd, ops.EPI_SWIGLU, norm_w=nw.to(DEV), eps=1e-6)
        sync()
        h = R.rmsnorm(x, nw)
        if B >= 3:
            # From 3 rows on, the prologue is the standalone RMSNorm kernel (qd_add_rmsnorm).
            # Its rstd reduction order may move single elements by 1 ulp. Through a dot product,
            # that shifts gate/up by up to ~1e-2 absolute: large relative to a small `up`.  So the
            # epilogue is judged on the kernel's own normalised input, which must itself meet
            # the RMSNorm bar against the oracle (2 ulp: a flip of bf16(x rstd) is scaled by w
            # and rounded again).
            hg = ops.rmsnorm(xd, nw.to(DEV), 1e-6).cpu()
            sync()
            assert_ulp(hg, h, 2, "gate/up prologue")
            h = hg
        gate, _ = exact_linear(h.float(), w[:N].float())
        up, _ = exact_linear(h.float(), w[N:].float())
        want = R.swiglu(gate, up)
        # first-order propagation of one ulp in bf16(gate), bf16(up) and bf16(silu) plus two
        # output ulps: each input rounding may land on either side of a midpoint
        g, u = gate.float(), up.float()
        sg = torch.sigmoid(g)
        s = (g * sg).to(BF).float()
        dsilu = (sg * (1 + g * (1 - sg))).abs()
        got = out.cpu().float()
        bound = (u.abs() * (dsilu * bf16_ulp(g) + bf16_ulp(s)) + s.abs() * bf16_ulp(u)
                 + 2 * bf16_ulp(torch.maximum(got.abs(), want.float().abs())) + 2 ** -12)
        d = (got - want.float()).abs()
        assert bool((d <= bound).all()), f"gate/up: max excess {float((d - bound).max())}"
    else:                                                # residual epilogue, in place
        res = rnd(g, B, N, scale=2.0)
        xo = res.to(DEV).clone()
        ops.linear(xd, wd, ops.EPI_RES, res=xo, out=xo)
        sync()
        acc, _ = exact_linear(x.float(), w.float())
        want = (res.float() + acc.float()).to(BF)
        # bf16(res + bf16(acc)): one ulp of bf16(acc) may survive cancellation into the sum,
        # so the bound is ulp(acc) + 2 ulp(out)
        d = (xo.cpu().float() - want.float()).abs()
        bound = bf16_ulp(acc.float()) + 2 * bf16_ulp(torch.maximum(xo.cpu().float().abs(),
                                                                   want.float().abs()))
        assert bool((d <= bound).all()), f"{name}: max excess {float((d - bound).max())}"


# Ragged shapes across every dispatch range (vector GEMV, skinny MFMA, LDS-staged, all-rows with
# and without K splits and activation halves, 128 x 128 and 256 x 256 tiles): seeded random
# (rows, outputs, K, epilogue), against fp64 with test_linear_epilogues' bounds
_RNG = np.random.default_rng(2024)
RAGGED = [(int(_RNG.integers(1, 65) if i % 2 else _RNG.integers(65, 1101)),
           int(_RNG.choice([256, 512, 768, 1280])), int(_RNG.choice([128, 256, 640, 1152])),
           int(_RNG.integers(0, 3))) for i in range(24)]


@pytest.mark.parametrize("M,N,K,epi", RAGGED)
def test_linear_ragged_shapes(ops, M, N, K, epi):
    say(f"linear ragged M={M} N={N} K={K} epi={epi}")
    g = torch.Generator().manual_seed(M * 7919 + N * 31 + K + epi)
    w = rnd(g, 2 * N if epi == ops.EPI_SWIGLU else N, K, scale=0.05)
    x = rnd(g, M, K)
    xd, wd = x.to(DEV), w.to(DEV)
    if epi == ops.EPI_NONE:
        out = ops.linear(xd, wd, epi)
        sync()
        want, _ = exact_linear(x.float(), w.float())
        assert_ulp(out.cpu(), want, 2, "plain", abs_floor=2 ** -9)
    elif epi == ops.EPI_RES:
        res = rnd(g, M, N, scale=2.0)
        xo = res.to(DEV).clone()
        ops.linear(xd, wd, epi, res=xo, out=xo)
        sync()
        _, acc = exact_linear(x.float(), w.float())
        want = (res.float() + acc.float()).to(BF)
        d = (xo.cpu().float() - want.float()).abs()
        bound = bf16_ulp(acc.float()) + 2 * bf16_ulp(torch.maximum(xo.cpu().float().abs(),
                                                                   want.float().abs()))
        assert bool((d <= bound).all()), f"residual: max excess {float((d - bound).max())}"
    else:
        out = ops.linear(xd, wd, epi)
        sync()
        _, gate = exact_linear(x.float(), w[:N].float())
        _, up = exact_linear(x.float(), w[N:].float())
        want = R.swiglu(gate.float().to(BF), up.float().to(BF))
        # bf16(gate), bf16(up) may each sit one ulp off the fp64 rounding (fp32 accumulation),
        # propagated through silu and the product, plus two output ulps
        gf, uf = gate.float(), up.float()
        sg = torch.sigmoid(gf)
        sv = (gf * sg).to(BF).float()
        dsilu = (sg * (1 + gf * (1 - sg))).abs()
        got = out.cpu().float()
        bound = (uf.abs() * (dsilu * bf16_ulp(gf) + bf16_ulp(sv)) + sv.abs() * bf16_ulp(uf)
                 + 2 * bf16_ulp(torch.maximum(got.abs(), want.float().abs())) + 2 ** -12)
        d = (got - want.float()).abs()
        assert bool((d <= bound).all()), f"gate/up: max excess {float((d - bound).max())}"


# The 256 x 256-tile kernel's shortest pipelines (K = 128: its two K stages both loaded up front;
# K = 384: six) with a ragged last row block: plain against fp64, residual in place, and SwiGLU
# bit for bit against the oracle's SwiGLU of the same kernel's own gate and up projections (the
# gate / up rows reach it through the 64-deep stages' row mapping)
@pytest.mark.parametrize("K", [128, 384])
def test_big_tile_short_k(ops, K):
    M, N = 1100, 512
    say(f"256 x 256 tiles: M={M} N={N} K={K}")
    g = torch.Generator().manual_seed(77 + K)
    x = rnd(g, M, K)
    w = rnd(g, 2 * N, K, scale=0.05)
    xd, wd = x.to(DEV), w.to(DEV)
    plain = ops.linear(xd, wd, ops.EPI_NONE)
    sync()
    want, acc = exact_linear(x.float(), w.float())
    assert_ulp(plain.cpu(), want, 2, "plain", abs_floor=2 ** -9)
    res = rnd(g, M, N, scale=2.0)
    xo = res.to(DEV).clone()
    ops.linear(xd, wd[:N].contiguous(), ops.EPI_RES, res=xo, out=xo)
    sync()
    want_r = (res.float() + acc[:, :N].float()).to(BF)
    d = (xo.cpu().float() - want_r.float()).abs()
    bound = bf16_ulp(acc[:, :N].float()) + 2 * bf16_ulp(torch.maximum(xo.cpu().float().abs(),
                                                                       want_r.float().abs()))
    assert bool((d <= bound).all()), f"residual: max excess {float((d - bound).max())}"
    act = ops.linear(xd, wd, ops.EPI_SWIGLU)
    sync()
    pc = plain.cpu()
    want_s = R.swiglu(pc[:, :N], pc[:, N:])
    assert torch.equal(act.cpu().view(torch.int16), want_s.view(torch.int16))


# ------------------------------------------------------------------ LM head + argmax
# 1-2 rows: the vector kernel; 3-64: the weight-streaming MFMA kernel (16 / 32 / 64-row
# activation tiles); 72: the 128 x 128 tiled kernel; 160, 256: the 256 x 256 tile with the argmax
# epilogue (one partly filled / one full row block, and the vocabulary's last block half full)
@pytest.mark.parametrize("B", [1, 2, 8, 24, 40, 72, 160, 256])
def test_lm_head_argmax(ops, B):
    say(f"lm_head_argmax B={B}")
    g = torch.Generator().manual_seed(400 + B)
    V, K = 151936, 2560
    w = rnd(g, V, K, scale=0.02)
    x = rnd(g, B, K)
    nw = rnd(g, K, scale=0.1) + 1
    logits = torch.empty((B, V), dtype=torch.float32, device=DEV)
    pos = torch.zeros((1,), dtype=torch.int64, device=DEV)
    tok = ops.lm_head_argmax(x.to(DEV), w.to(DEV), nw.to(DEV), 1e-6, pos=pos, logits=logits)
    sync()
    h = R.rmsnorm(x, nw)
    exact = h.double() @ w.double().T
    lg = logits.cpu()
    assert float((lg.double() - exact).abs().max()) <= 2e-2      # north-star logits bar
    assert float((lg.double() - exact).abs().max()) <= 1e-3      # what fp32 accumulation gives
    # the index is bit-exact given the kernel's own bf16 logits (lowest index on ties)
    own = torch.argmax(lg.to(BF).float(), dim=-1)
    assert torch.equal(tok.cpu(), own)
    # and it is the oracle's argmax wherever the oracle's top-2 margin exceeds 1e-2
    ref = R.linear(h, w).float()
    top2 = ref.topk(2, dim=-1).values
    for b in range(B):
        if float(top2[b, 0] - top2[b, 1]) > 1e-2:
            assert int(tok[b]) == int(torch.argmax(ref[b]))
    assert int(pos.item()) == 1                                  # position advanced once


# Ragged vocabularies (multiples of 4 from 256 up) at row counts across the LM head's kernels:
# every kernel's last, partly filled vocabulary block
_RNG_LM = np.random.default_rng(31337)
RAGGED_LM = [(int(_RNG_LM.choice([1, 2, 5, 17, 33, 64, 100, 129, 200, 256])),
              int(_RNG_LM.integers(64, 12001)) * 4) for _ in range(8)]


@pytest.mark.parametrize("B,V", RAGGED_LM)
def test_lm_head_argmax_ragged_vocab(ops, B, V):
    say(f"lm_head_argmax ragged B={B} V={V}")
    g = torch.Generator().manual_seed(B * 131 + V)
    K = 2560
    w = rnd(g, V, K, scale=0.02)
    x = rnd(g, B, K)
    nw = rnd(g, K, scale=0.1) + 1
    logits = torch.empty((B, V), dtype=torch.float32, device=DEV)
    tok = ops.lm_head_argmax(x.to(DEV), w.to(DEV), nw.to(DEV), 1e-6, logits=logits)
    sync()
    exact = R.rmsnorm(x, nw).double() @ w.double().T
    lg = logits.cpu()
    assert float((lg.double() - exact).abs().max()) <= 2e-2      # north-star logits bar
    if B >= 3:
        # from 3 rows on the normalised input is the standalone RMSNorm kernel's, whose rstd
        # reduction may move single bf16 elements by one ulp (~1e-3 in a logit); against that
        # input the logits carry only fp32 accumulation error
        hk = ops.rmsnorm(x.to(DEV), nw.to(DEV), 1e-6).cpu()
        own_exact = hk.double() @ w.double().T
        assert float((lg.double() - own_exact).abs().max()) <= 1e-4
    assert torch.equal(tok.cpu(), torch.argmax(lg.to(BF).float(), dim=-1))


@pytest.mark.parametrize("B", [1, 8, 40, 72, 256])
def test_lm_head_ties_pick_lowest_index(ops, B):
    say(f"lm_head ties B={B}")
    V, K = 151936, 2560
    g = torch.Generator().manual_seed(7)
    w = rnd(g, V, K, scale=0.001)
    x = torch.ones((B, K), dtype=BF)
    nw = torch.ones(K, dtype=BF)
    # identical maximal rows in different workgroups / tiles: the lowest index must win
    for n in (150000, 77777, 40001, 151935):
        w[n] = 0.05
    tok = ops.lm_head_argmax(x.to(DEV), w.to(DEV), nw.to(DEV), 1e-6)
    sync()
    assert tok.cpu().tolist() == [40001] * B


# ------------------------------------------------------------------ attention
def p_round_bound(v, qkv=None):
    """Attention outputs differ from the oracle by where P is rounded to bf16: online softmax
    rounds exp(s - m_running), the oracle exp(s - m_global); each term moves by at most one
    bf16 rounding (2^-9 relative) on either side, so |do| <= 2^-8 max|V| (+ a 2^-12 floor)."""
    m = float(v.float().abs().max())
    if qkv is not None:
        m = max(m, float(qkv[:, 5120:].float().abs().max()))
    return 2 ** -8 * m + 2 ** -12


def decode_ref(qkv, qn, kn, cos, sin, kcache, vcache, pos):
    """Oracle: q/k norm + rope at pos, write K/V at pos, attend keys [0, pos]."""
    B = qkv.shape[0]
    q = qkv[:, :4096].view(B, 1, 32, 128)
    k = qkv[:, 4096:5120].view(B, 1, 8, 128)
    v = qkv[:, 5120:].view(B, 8, 128)
    qr, kr = R.qk_norm_rope(q, k, qn, kn, cos[pos][None, None].expand(B, 1, 128),
                            sin[pos][None, None].expand(B, 1, 128))
    kc, vc = kcache.clone(), vcache.clone()
    kc[:, :, pos] = kr[:, 0]
    vc[:, :, pos] = v
    vis = torch.zeros((1, 1, 1, kc.shape[2]), dtype=torch.bool)
    vis[..., :pos + 1] = True
    o = R.attention(qr.transpose(1, 2), kc, vc, vis)
    return o[:, :, 0], kc, vc


# Ragged blocks of tokens per sequence (the prefill / tree path: 8-token row blocks with a
# partial last one), per-row base positions: every token's q, K and V against the oracle, and no
# cache slot outside the block written
_RNG_QK = np.random.default_rng(99)
RAGGED_QK = [(int(_RNG_QK.integers(1, 5)), int(_RNG_QK.integers(1, 71))) for _ in range(6)]


@pytest.mark.parametrize("B,T", RAGGED_QK)
def test_qk_norm_rope_ragged_blocks(ops, B, T):
    Hq, Hkv, cap = 32, 8, 700
    say(f"qk_norm_rope ragged B={B} T={T} (per-row bases)")
    g = torch.Generator().manual_seed(900 + 7 * B + T)
    qkv = rnd(g, B * T, (Hq + 2 * Hkv) * 128, scale=2.0)
    qn, kn = rnd(g, 128, scale=0.2) + 1, rnd(g, 128, scale=0.2) + 1
    base = torch.randint(0, cap - T + 1, (B,), generator=g)
    cos, sin = R.rope_tables(cap)
    kc = torch.zeros((B, Hkv, cap, 128), dtype=BF, device=DEV)
    vc = torch.zeros_like(kc)
    q_out = torch.empty((B, T, Hq, 128), dtype=BF, device=DEV)
    ops.qk_norm_rope(qkv.to(DEV), qn.to(DEV), kn.to(DEV), cos.to(DEV), sin.to(DEV), base.to(DEV),
                     ops.POS_ROW, q_out, kc, vc, B, T, Hq, Hkv, 1e-6)
    sync()
    x = qkv.view(B, T, Hq + 2 * Hkv, 128)
    slots = base[:, None] + torch.arange(T)[None]                       # [B, T]
    c, sn = cos[slots][:, :, None, :], sin[slots][:, :, None, :]
    q_ref, k_ref = R.qk_norm_rope(x[:, :, :Hq], x[:, :, Hq:Hq + Hkv], qn, kn, cos[slots], sin[slots])

    def check(got, ref, h, nw, what):
        # the head's rstd may differ from the oracle's by its reduction order, moving a normalised
        # value by one ulp; where the rotation's two products cancel, that ulp of each product
        # survives into a small output: bound = 2 ulp(out) + ulp(y c) + ulp(rot(y) s)
        y = R.rmsnorm(h, nw).float()
        bound = (2 * bf16_ulp(torch.maximum(got.float().abs(), ref.float().abs()))
                 + bf16_ulp((y * c.float()).abs()) + bf16_ulp((R.rotate_half(y) * sn.float()).abs()))
        d = (got.float() - ref.float()).abs()
        assert bool((d <= bound).all()), f"{what}: max excess {float((d - bound).max())}"

    check(q_out.cpu(), q_ref, x[:, :, :Hq], qn, "q")
    kcc, vcc = kc.cpu(), vc.cpu()
    check(kcc.permute(0, 2, 1, 3).gather(1, slots[:, :, None, None].expand(B, T, Hkv, 128)), k_ref,
          x[:, :, Hq:Hq + Hkv], kn, "k cache")
    for b in range(B):
        sl = slice(int(base[b]), int(base[b]) + T)
        assert torch.equal(vcc[b, :, sl].transpose(0, 1), x[b, :, Hq + Hkv:])
        kcc[b, :, sl] = 0
        vcc[b, :, sl] = 0
    assert not bool(kcc.any()) and not bool(vcc.any())                 # nothing else written


@pytest.mark.parametrize("B", [1, 4])
def test_qk_norm_rope_matches_decode_unit_bitwise(ops, B):
    """The standalone q/k norm + RoPE kernel (prefill chunks, tree verification: 16 lanes per
    head) and the decode attention unit's prologue (one lane per dim pair; B = 1 the VALU unit
    shared with the persistent step, B = 4 the MFMA kernel) add the head's sum of squares in
    the same order: the K / V rows they write to the cache are bit-identical."""
    say(f"qk_norm_rope vs decode attention prologue, B={B}: identical K/V writes")
    g = torch.Generator().manual_seed(4242 + B)
    cap, pos = 600, 517
    qkv = rnd(g, B, 6144, scale=3.0).to(DEV)
    qn, kn = (rnd(g, 128, scale=0.2) + 1).to(DEV), (rnd(g, 128, scale=0.2) + 1).to(DEV)
    cos, sin = (t.to(DEV) for t in R.rope_tables(cap))
    p = torch.tensor([pos], dtype=torch.int64, device=DEV)
    k1 = torch.zeros((B, 8, cap, 128), dtype=BF, device=DEV)
    v1 = torch.zeros_like(k1)
    ops.decode_attention(qkv, qn, kn, cos, sin, p, k1, v1, 32, 8, 1e-6)
    k2, v2 = torch.zeros_like(k1), torch.zeros_like(k1)
    q_out = torch.empty((B, 1, 32, 128), dtype=BF, device=DEV)
    ops.qk_norm_rope(qkv, qn, kn, cos, sin, p, ops.POS_SHARED, q_out, k2, v2, B, 1, 32, 8, 1e-6)
    sync()
    assert torch.equal(k1.view(torch.int16), k2.view(torch.int16))
    assert torch.equal(v1.view(torch.int16), v2.view(torch.int16))


# B = 1 runs the VALU unit (shared with the persistent step); B >= 2 the MFMA kernel, whose
# 32-key tiles make pos = 0 / 31 / 32, the new key in the last split, and splits past pos (no
# keys at all: (2, 4100, 1000) has 13 splits, pos in the fourth) the edge cases
@pytest.mark.parametrize("B,cap,pos", [(1, 768, 0), (1, 768, 1), (1, 768, 63), (1, 768, 64),
                                       (1, 768, 640), (1, 768, 767), (4, 300, 129),
                                       (32, 2176, 2100), (2, 64, 0), (2, 100, 31), (2, 100, 32),
                                       (3, 4100, 4099), (8, 600, 257), (2, 4100, 1000),
                                       # config-5 context (B = 4, 8192 + a verify's slots)
                                       (4, 8512, 8447), (1, 8512, 8300)])
def test_decode_attention(ops, B, cap, pos):
    say(f"decode_attention B={B} cap={cap} pos={pos}")
    g = torch.Generator().manual_seed(500 + B + pos)
    qkv = rnd(g, B, 6144, scale=2.0)
    qn, kn = rnd(g, 128, scale=0.2) + 1, rnd(g, 128, scale=0.2) + 1
    cos, sin = R.rope_tables(cap)
    kcache = rnd(g, B, 8, cap, 128)
    vcache = rnd(g, B, 8, cap, 128)
    kcache[:, :, pos:] = 0
    vcache[:, :, pos:] = 0
    kd, vd = kcache.to(DEV), vcache.to(DEV)
    p = torch.tensor([pos], dtype=torch.int64, device=DEV)
    out = ops.decode_attention(qkv.to(DEV), qn.to(DEV), kn.to(DEV), cos.to(DEV), sin.to(DEV), p,
                               kd, vd, 32, 8, 1e-6)
    sync()
    o_ref, kc_ref, vc_ref = decode_ref(qkv, qn, kn, cos, sin, kcache, vcache, pos)
    assert torch.equal(vd.cpu(), vc_ref)
    assert_ulp(kd.cpu(), kc_ref, 2, "k cache")
    assert_ulp(out.cpu(), o_ref, 2, "attention out", abs_floor=p_round_bound(vcache, qkv))


# Ragged decode attention: seeded random batch (the VALU unit at B = 1, the MFMA kernel above),
# cache size and position, so the split plan, the last partial key tile and the split that holds
# the new key vary from case to case
_RNG_DA = np.random.default_rng(777)
RAGGED_DA = []
for _i in range(10):
    _B = 1 if _i % 3 == 0 else int(_RNG_DA.integers(2, 41))
    _cap = int(_RNG_DA.integers(33, 5001))
    RAGGED_DA.append((_B, _cap, int(_RNG_DA.integers(0, _cap))))


@pytest.mark.parametrize("B,cap,pos", RAGGED_DA)
def test_decode_attention_ragged(ops, B, cap, pos):
    test_decode_attention(ops, B, cap, pos)


@pytest.mark.parametrize("B", [1, 2])
@pytest.mark.parametrize("pos", [300, -1])
def test_decode_attention_position_outside_cache_writes_nothing(ops, B, pos):
    """A device position outside [0, cap) (B = 1: the VALU unit; B = 2: the MFMA kernel) ends
    every unit before any cache write: both caches come back unchanged."""
    say(f"decode_attention B={B} pos={pos} (cap 300): no K/V write")
    g = torch.Generator().manual_seed(77 + B)
    cap = 300
    qkv = rnd(g, B, 6144).to(DEV)
    qn = torch.ones(128, dtype=BF, device=DEV)
    cos, sin = (t.to(DEV) for t in R.rope_tables(cap))
    kd = rnd(g, B, 8, cap, 128).to(DEV)
    vd = rnd(g, B, 8, cap, 128).to(DEV)
    k0, v0 = kd.clone(), vd.clone()
    p = torch.tensor([pos], dtype=torch.int64, device=DEV)
    ops.decode_attention(qkv, qn, qn, cos, sin, p, kd, vd, 32, 8, 1e-6)
    sync()
    assert torch.equal(kd, k0) and torch.equal(vd, v0)


def test_decode_attention_repeat_is_deterministic(ops):
    say("decode_attention repeat x3 bit-identical (tickets reset)")
    g = torch.Generator().manual_seed(9)
    B, cap, pos = 2, 1024, 900
    qkv = rnd(g, B, 6144).to(DEV)
    qn = torch.ones(128, dtype=BF, device=DEV)
    cos, sin = (t.to(DEV) for t in R.rope_tables(cap))
    kd = rnd(g, B, 8, cap, 128).to(DEV)
    vd = rnd(g, B, 8, cap, 128).to(DEV)
    p = torch.tensor([pos], dtype=torch.int64, device=DEV)
    ws = ops.workspace(ops._lib.LIB.qd_decode_attn_workspace_bytes(B, 32, 8, cap), DEV)
    outs = [ops.decode_attention(qkv, qn, qn, cos, sin, p, kd, vd, 32, 8, 1e-6, ws=ws).cpu()
            for _ in range(3)]
    sync()
    # a ticket that was not reset would leave the merge undone and the fresh output garbage
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])


@pytest.mark.parametrize("mode", ["tree", "causal"])
def test_block_attention(ops, mode):
    say(f"block_attention {mode}")
    g = torch.Generator().manual_seed(600)
    B, T, cap = 2, 64 if mode == "tree" else 40, 1200
    base = torch.tensor([700, 1100], dtype=torch.int64) if mode == "tree" else torch.tensor([0, 333])
    base = base.clamp(max=cap - T)
    q = rnd(g, B, T, 32, 128)
    kc, vc = rnd(g, B, 8, cap, 128), rnd(g, B, 8, cap, 128)
    if mode == "tree":
        rng = np.random.default_rng(1)
        parent = [-1] + [int(rng.integers(0, i)) for i in range(1, T)]
        anc = []
        for i in range(T):
            m, n = 0, i
            while n >= 0:
                m |= 1 << n
                n = parent[n]
            anc.append(m)
        anc_t = torch.tensor([[a - (1 << 64) if a >= 1 << 63 else a for a in anc]] * B)
    out = ops.block_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), base.to(DEV),
                              anc_t.to(DEV) if mode == "tree" else None)
    sync()
    for b in range(B):
        vis = torch.zeros((T, cap), dtype=torch.bool)
        for t in range(T):
            vis[t, :base[b]] = True
            for jj in range(T):
                ok = ((anc[t] >> jj) & 1) if mode == "tree" else jj <= t
                if ok:
                    vis[t, base[b] + jj] = True
        o = R.attention(q[b:b + 1].transpose(1, 2), kc[b:b + 1], vc[b:b + 1], vis[None, None])
        assert_ulp(out[b].cpu(), o[0].transpose(0, 1), 2, f"block row {b}",
                   abs_floor=p_round_bound(vc))


def _tree_masks(T, seed):
    """Ancestor-or-self masks of a 4-4-2-2 draft tree truncated to T nodes in BFS order (the
    config-5 tree shape; tests/test_tree_host.py checks the builder)."""
    from qdecode import tree as tr
    rng = np.random.default_rng(seed)
    t = tr.branching_tree(0, T, (4, 4, 2, 2), lambda n: rng.integers(1, 1 << 30, size=n))
    return t.anc


def _block_ref_rows(q, kc, vc, base, anc, T):
    """Oracle output [B, T, Hq, 128] row by row (visibility from base and masks / causal)."""
    outs = []
    cap = kc.shape[2]
    for b in range(q.shape[0]):
        vis = torch.zeros((T, cap), dtype=torch.bool)
        vis[:, :int(base[b])] = True
        if anc is None:
            vis[:, int(base[b]):int(base[b]) + T] = torch.tril(torch.ones((T, T), dtype=torch.bool))
        else:
            for t in range(T):
                for jj in range(T):
                    if (anc[b][t] >> jj) & 1:
                        vis[t, int(base[b]) + jj] = True
        o = R.attention(q[b:b + 1].transpose(1, 2), kc[b:b + 1], vc[b:b + 1], vis[None, None])
        outs.append(o[0].transpose(0, 1))
    return outs


def test_block_attention_config5_verify(ops):
    """The config-5 verify launch at its real context: B = 4 trees of 64 nodes over 8192 cached
    keys and more (cap 8512 = 8192 prompt + 256 output + 64 tree slots), different random
    4-4-2-2 trees per row, bases up to the last legal slot.  B*Hkv = 32 query blocks give the
    launch's own plan of 8 key splits of 1088 keys each."""
    B, T, cap = 4, 64, 8512
    base = torch.tensor([8192, 8193, 8300, cap - T], dtype=torch.int64)
    say(f"block_attention config 5: B={B} T={T} cap={cap} bases {base.tolist()}")
    g = torch.Generator().manual_seed(8192)
    q = rnd(g, B, T, 32, 128, scale=2.0)
    kc, vc = rnd(g, B, 8, cap, 128), rnd(g, B, 8, cap, 128)
    anc = [_tree_masks(T, 100 + b) for b in range(B)]
    anc_t = torch.tensor([[a - (1 << 64) if a >= 1 << 63 else a for a in row] for row in anc])
    out = ops.block_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), base.to(DEV), anc_t.to(DEV))
    sync()
    for b, o in enumerate(_block_ref_rows(q, kc, vc, base, anc, T)):
        assert_ulp(out[b].cpu(), o, 2, f"verify row {b}", abs_floor=p_round_bound(vc))


def test_block_attention_causal_chunk_deep(ops):
    """A causal prefill chunk deep in a config-5 prompt: 1024 tokens per row at base 7168 over a
    cache of 8512 slots (one key split: 2 x 8 x 16 query blocks fill the chip)."""
    B, T, cap = 2, 1024, 8512
    base = torch.tensor([7168, 7168], dtype=torch.int64)
    say(f"block_attention causal chunk: B={B} T={T} base 7168 cap={cap}")
    g = torch.Generator().manual_seed(7168)
    q = rnd(g, B, T, 32, 128, scale=2.0)
    kc, vc = rnd(g, B, 8, cap, 128), rnd(g, B, 8, cap, 128)
    out = ops.block_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), base.to(DEV), None)
    sync()
    for b, o in enumerate(_block_ref_rows(q, kc, vc, base, None, T)):
        assert_ulp(out[b].cpu(), o, 2, f"chunk row {b}", abs_floor=p_round_bound(vc))


# Ragged block attention: seeded random batch, block length, cache size and per-row bases, tree
# (random 4-4-2-2 trees, up to 64 nodes) and causal (up to 300 tokens) -- partial key tiles, partial
# query blocks, and the launch's own split plan for each shape
_RNG_BA = np.random.default_rng(4242)
RAGGED_BA = []
for _i in range(10):
    _tree = _i % 2 == 0
    _B = int(_RNG_BA.integers(1, 4))
    _T = int(_RNG_BA.integers(1, 65) if _tree else _RNG_BA.integers(1, 301))
    _cap = int(_RNG_BA.integers(_T + 1, 3001))
    _bases = [int(_RNG_BA.integers(0, _cap - _T + 1)) for _ in range(_B)]
    RAGGED_BA.append(("tree" if _tree else "causal", _B, _T, _cap, tuple(_bases)))


@pytest.mark.parametrize("mode,B,T,cap,bases", RAGGED_BA)
def test_block_attention_ragged(ops, mode, B, T, cap, bases):
    say(f"block_attention ragged {mode}: B={B} T={T} cap={cap} bases {list(bases)}")
    g = torch.Generator().manual_seed(T * 1009 + cap)
    q = rnd(g, B, T, 32, 128, scale=2.0)
    kc, vc = rnd(g, B, 8, cap, 128), rnd(g, B, 8, cap, 128)
    base = torch.tensor(bases, dtype=torch.int64)
    anc = [_tree_masks(T, 300 + b) for b in range(B)] if mode == "tree" else None
    anc_t = (torch.tensor([[a - (1 << 64) if a >= 1 << 63 else a for a in row] for row in anc])
             if anc is not None else None)
    out = ops.block_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), base.to(DEV),
                              anc_t.to(DEV) if anc_t is not None else None)
    sync()
    for b, o in enumerate(_block_ref_rows(q, kc, vc, base, anc, T)):
        assert_ulp(out[b].cpu(), o, 2, f"ragged row {b}", abs_floor=p_round_bound(vc))


def test_kv_compact(ops):
    say("kv_compact")
    g = torch.Generator().manual_seed(700)
    L, B, cap, T = 3, 2, 200, 8
    k = rnd(g, L, B, 8, cap, 128).to(DEV)
    v = rnd(g, L, B, 8, cap, 128).to(DEV)
    k0, v0 = k.cpu(), v.cpu()
    base = torch.tensor([50, 120])
    src = torch.tensor([[0, 2, 3, 7, 0, 0, 0, 0], [0, 1, 5, 0, 0, 0, 0, 0]], dtype=torch.int32)
    cnt = torch.tensor([4, 3], dtype=torch.int32)
    ops.kv_compact(k, v, base.to(DEV), src.to(DEV), cnt.to(DEV))
    sync()
    ke, ve = k0.clone(), v0.clone()
    for b in range(B):
        for kk in range(1, int(cnt[b])):
            s = int(src[b, kk])
            ke[:, b, :, base[b] + kk] = ke[:, b, :, base[b] + s]
            ve[:, b, :, base[b] + kk] = ve[:, b, :, base[b] + s]
    assert torch.equal(k.cpu(), ke) and torch.equal(v.cpu(), ve)


# ------------------------------------------------------------------ read-stream probe
@pytest.mark.parametrize("nbytes,grid", [(16, 1), (1 << 20, 64), ((1 << 20) + 48, 4864)])
def test_read_probe_reads_and_writes_nothing(nbytes, grid):
    """qd_read_probe (the benchmark's read-ceiling kernel) runs over ragged sizes and grids
    larger than the data, leaves its input untouched and never writes the sink for real data."""
    from qdecode import _lib
    say(f"read probe {nbytes} B, grid {grid}")
    buf = torch.arange(nbytes // 2, dtype=torch.int16, device=DEV)
    before = buf.clone()
    sink = torch.full((1,), -7, dtype=torch.int32, device=DEV)
    _lib.call("qd_read_probe", buf.data_ptr(), nbytes, grid, sink.data_ptr(),
              torch.cuda.current_stream().cuda_stream)
    sync()
    assert int(sink.item()) == -7 and torch.equal(buf, before)
