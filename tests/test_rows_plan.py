"""CPU: every launch plan of the all-rows projection kernel (gemm_rows_kernel, gemm_tile.hip;
65..256 activation rows: the tree-verification GEMMs) covers its grid and keeps every load and
store inside its buffers.

The plans come from the built library itself (qd_gemm_rows_plan: the same decision function
the launchers call), so a change to the planner is checked as it ships.  What the kernel does
with a plan is modelled here from its index math (gemm_tile.hip gemm_rows_kernel: the
workgroup -> (weight block, K split, activation half) map, the staged-row offsets and the
epilogue's store pattern) and checked with numpy:
  * every (weight block, K split, activation half) is run by exactly one workgroup, and the
    padding workgroups of the two-halves grid exit;
  * every staged weight / activation row and K range lies inside its operand (32-bit offsets);
  * every output element (or fp32 partial of every split) is written exactly once, inside N x M
    (and inside the partial buffer's floats);
  * the stage buffers fit the LDS and the grid is one round of workgroups.
The plans run with no, half and full partial room, as the launchers can be called.
"""

import ctypes as C

import pytest

TK = 64            # K per stage (bf16)
LDS_BYTES = 160 * 1024
CUS = 256          # no device here: the library assumes 256 CUs
EPI_NONE, EPI_RES, EPI_SWIGLU = 0, 1, 2


def _plan(lib, M, N, K, epi, part_floats, partials_only):
    out = (C.c_int64 * 8)()
    rc = lib.LIB.qd_gemm_rows_plan(M, N, K, epi, part_floats, int(partials_only), out)
    keys = ("rows", "nt", "mt", "mh", "S", "ks_per", "grid", "lds")
    return rc, dict(zip(keys, list(out)))


def _check(P, M, N, K, epi, part_floats):
    """The kernel's index math for plan P (see the module docstring)."""
    sw = epi == EPI_SWIGLU
    split = P["S"] > 1
    rows, NT, MT, mh, S, ks_per, grid = (P[k] for k in ("rows", "nt", "mt", "mh", "S", "ks_per",
                                                         "grid"))
    WT = 2 * NT if (sw and not split) else NT
    WR, RM = 16 * WT, 128 * MT
    assert P["lds"] == 3 * (WR + RM) * 128 <= LDS_BYTES
    assert 16 * NT >= rows and rows % 4 == 0 and N % 4 == 0
    ksteps = K // TK
    nb = -(-N // rows)
    assert nb * S * mh <= CUS                               # one round of workgroups
    wbytes = (2 * N if sw else N) * K * 2
    assert wbytes < 1 << 32 and M * K * 2 < 1 << 32         # 32-bit load offsets
    seen = set()
    rects = {}                                              # (split, half) -> store rectangles
    for g in range(grid):
        blkid, mb = g, 0
        if mh > 1:
            slot = g >> 3
            mb = slot % mh
            blkid = (slot // mh) * 8 + (g & 7)
            if blkid >= nb * S:
                continue                                    # padding workgroup: exits
        rb, sp = divmod(blkid, S)
        assert (rb, sp, mb) not in seen
        seen.add((rb, sp, mb))
        m0, n0 = mb * RM, rb * rows
        nrows = min(rows, N - n0)
        assert 0 <= n0 < N and nrows >= 1
        kbeg = sp * ks_per
        kend = min(ksteps, kbeg + ks_per)
        assert 0 <= kbeg < kend                             # no empty split
        # staged rows: weight rows n0 + min(r, nrows - 1) (SwiGLU: gate rows r < 16 NT, up rows
        # + N), then activation rows min(m0 + r, M - 1); the last stage reads up to kend * TK
        wmax = n0 + min(16 * NT - 1 if (sw and not split) else WR - 1, nrows - 1)
        if sw and not split:
            wmax += N
        assert wmax * K * 2 + kend * TK * 2 <= wbytes
        assert m0 < M                                       # every half has rows
        # stores: activation rows m0 + 16 MT wave + 16 mt + c, columns n0 + 16 t + 4 q (.. + 3)
        m1 = min(m0 + 8 * 16 * MT, M)
        n1 = n0 + min(-(-nrows // 4) * 4, 16 * NT)
        assert n1 <= N
        rects.setdefault((sp, mb), []).append((m0, m1, n0, n1))
        if split and m0 < m1:
            last = ((sp * M + (m1 - 1)) * N + (n1 - 1))
            assert last < part_floats, ("partials past the buffer", last, part_floats)
    assert len(seen) == nb * S * mh
    # every split's stores tile M x N exactly once: the halves tile the rows, and within a
    # half the blocks tile the columns with the same row range
    for sp in range(S):
        edge = 0
        for mb in range(mh):
            rs = sorted(rects[(sp, mb)], key=lambda t: t[2])
            m0, m1 = rs[0][0], rs[0][1]
            assert m0 == edge and all((a, b) == (m0, m1) for a, b, _, _ in rs)
            edge = max(edge, m1)
            col = 0
            for _, _, n0, n1 in rs:
                assert n0 == col, ("column gap or overlap", sp, mb, n0, col)
                col = n1
            assert col == N
        assert edge == M


# the model's projections (N, K, epilogue) and the block step's partial-summing calls, plus
# small shapes that exercise the odd block heights
MODEL = [(6144, 2560, EPI_NONE), (2560, 4096, EPI_RES), (9728, 2560, EPI_SWIGLU),
         (2560, 9728, EPI_RES), (2560, 4096, EPI_NONE), (2560, 9728, EPI_NONE)]
SMALL = [(512, 256, EPI_NONE), (256, 512, EPI_RES), (1024, 1024, EPI_SWIGLU), (128, 128, EPI_NONE),
         (384, 640, EPI_RES), (640, 384, EPI_SWIGLU), (4096, 128, EPI_RES)]


def _launches(lib, shapes, Ms):
    n = 0
    for M in Ms:
        for N, K, epi in shapes:
            rc, full = _plan(lib, M, N, K, epi, 1 << 40, False)
            if rc != 1:
                continue
            need = full["S"] * M * N
            for part in (0, need // 2, need):
                for only in ((False, True) if epi != EPI_SWIGLU else (False,)):
                    rc, P = _plan(lib, M, N, K, epi, part, only)
                    assert rc in (0, 1)
                    if only:
                        # the block step's consumers take partials only when the plan splits
                        assert rc == (1 if full["S"] > 1 and part >= need else 0)
                    else:
                        assert rc == 1 and (P["S"] == 1 or part >= P["S"] * M * N)
                    if rc == 1:
                        _check(P, M, N, K, epi, part)
                        n += 1
    return n


def test_rows_plans_model_shapes_every_row_count(lib):
    assert _launches(lib, MODEL, range(65, 257)) > 1500


def test_rows_plans_small_shapes(lib):
    assert _launches(lib, SMALL, [65, 80, 96, 100, 127, 128, 129, 160, 200, 255, 256]) > 50


def test_rows_plan_query_limits(lib):
    assert _plan(lib, 64, 6144, 2560, EPI_NONE, 0, False)[0] == -1       # below the kernel
    assert _plan(lib, 257, 6144, 2560, EPI_NONE, 0, False)[0] == -1      # the tiled kernels
    assert _plan(lib, 256, 6144, 2560, EPI_NONE, 0, True)[0] == 0        # split but no room
    assert lib.LIB.qd_gemm_rows_plan(256, 6144, 2560, 7, 0, 0, (C.c_int64 * 8)()) == lib.QD_EARG
    assert lib.LIB.qd_gemm_rows_plan(256, 6144, 2560, EPI_SWIGLU, 0, 1,
                                     (C.c_int64 * 8)()) == lib.QD_EARG
    assert lib.LIB.qd_gemm_rows_plan(256, 6144, 2560, EPI_NONE, 0, 0, None) == lib.QD_EARG
    # the config-5 verify's plans (256 rows): two activation halves for every projection
    for N, K, epi in MODEL[:4]:
        rc, P = _plan(lib, 256, N, K, epi, 1 << 40, epi != EPI_SWIGLU)
        assert rc == 1 and P["mh"] == 2, (N, K, epi, P)


@pytest.fixture(scope="module")
def lib():
    from qdecode import _lib
    return _lib
