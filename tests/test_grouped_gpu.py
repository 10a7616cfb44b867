"""The grouped expert linear alone (lsk_grouped_gemm_w8a8 / lsk_grouped_gemm_mx): rows sorted by
expert, each expert's rows through its own weight with the v2.1 (int8) or MX (MXFP4) epilogue, bf16
out -- the per-expert int_mm + lin_epilogue(_b) / int_mm_mx + lin_epilogue_mx of moe_ref.py, bit for
bit against the oracle, expert by expert.  Row counts include empty experts, multi-tile experts and
counts below and above the ping-pong tile's switch (E x 128 rows)."""
import numpy as np
import pytest
import torch

from gpu_util import bits, dev, say, to_dev
from oracle import contract as C

pytestmark = pytest.mark.gpu

F32 = np.float32


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import lockstep_amd._lib as L
    L.load()


def _counts(g, E, R):
    """R rows over E experts, Zipf-skewed, two experts forced empty."""
    p = 1.0 / np.arange(1, E + 1) ** 1.1
    p = p[g.permutation(E)]
    p[:2] = 0.0
    c = g.multinomial(R, p / p.sum())
    return c.astype(np.int64)


@pytest.mark.parametrize("R,E,N,K,bias", [(300, 8, 192, 256, False), (40, 6, 96, 320, True),
                                          (2200, 12, 256, 512, False), (1600, 8, 320, 128, True),
                                          (256, 32, 400, 2880, True), (100, 16, 48, 208, False)])
def test_grouped_linear_int8(R, E, N, K, bias):
    from lockstep_amd import moe_ref as MR
    say("grouped int8", dict(R=R, E=E, N=N, K=K, bias=bias))
    g = np.random.default_rng(R + N)
    cnt = _counts(g, E, R)
    offs = np.concatenate([[0], np.cumsum(cnt)]).astype(np.int32)
    a8 = g.integers(-127, 128, (R, K), dtype=np.int8)
    asc = g.uniform(1e-3, 1e-1, R).astype(F32)
    experts = []
    for e in range(E):
        W = g.integers(-127, 128, (N, K), dtype=np.int8)
        ws = g.uniform(1e-3, 1e-2, N).astype(F32)
        b = g.standard_normal(N).astype(F32) if bias else None
        experts.append((W, ws, b))
    # only the w13 slot of the tables is used: w13col [K, N] views, a dummy w2
    dev_ex = [(to_dev(W).t(), to_dev(ws), to_dev(np.zeros((K, N // 2), np.int8)).t(), to_dev(np.ones(K, F32)),
               None if b is None else to_dev(b), None) for (W, ws, b) in experts]
    out = MR.grouped_linear(dev_ex, "w13", to_dev(a8), to_dev(asc), to_dev(offs))
    got = bits(out)
    for e, (W, ws, b) in enumerate(experts):
        r0, r1 = offs[e], offs[e + 1]
        if r1 == r0:
            continue
        acc = C.int_mm(a8[r0:r1], W.T)
        ref = C.lin_epilogue_b(acc, ws, asc[r0:r1], b) if bias else C.lin_epilogue(acc, ws, asc[r0:r1])
        assert np.array_equal(got[r0:r1], C.bf16_bits(ref)), "expert %d" % e


@pytest.mark.parametrize("R,E,N,K,bias,mxv", [(200, 6, 128, 256, False, 0), (1500, 8, 256, 320, True, 0),
                                              (256, 32, 384, 2880, True, 0), (100, 8, 400, 320, False, 0),
                                              (1500, 8, 256, 320, True, 3)])
def test_grouped_linear_mx(R, E, N, K, bias, mxv):
    """The grouped MX linear on the tiles and, for experts averaging at most 32 rows (256 rows over
    32 experts, 100 over 8) or under lsk_moe_mx_select(3) (full 128-row tiles, eight 16-row chunks
    each), on the skinny grouped MX GEMM reading the codes' skinny-layout copies."""
    from lockstep_amd import _lib as L
    from lockstep_amd import moe_ref as MR
    say("grouped mx", dict(R=R, E=E, N=N, K=K, bias=bias, mxv=mxv))
    g = np.random.default_rng(7 * R + N)
    cnt = _counts(g, E, R)
    offs = np.concatenate([[0], np.cumsum(cnt)]).astype(np.int32)
    a8 = g.integers(-127, 128, (R, K), dtype=np.int8)
    asc = g.uniform(1e-3, 1e-1, R).astype(F32)
    experts, dev_ex = [], []
    for e in range(E):
        codes = g.integers(0, 256, (N, K // 2), dtype=np.uint8)
        kx = (127 + g.integers(-8, 3, (N, K // 32))).astype(np.uint8)
        b = g.standard_normal(N).astype(F32) if bias else None
        experts.append((codes, kx, b))
        dummy = (to_dev(np.zeros((K, N // 4), np.uint8)), to_dev(np.full((K, N // 64), 127, np.uint8)))
        dev_ex.append(((to_dev(codes), to_dev(kx)), dummy, None if b is None else to_dev(b), None))
    tables = MR.ExpertTablesMX(dev_ex, packed=True)
    L.call("lsk_moe_mx_select", mxv)
    try:
        skinny = L.load().lsk_grouped_mx_reads_skinny(R, E, K, tables.lds13) == 1
        out = MR.grouped_linear_mx(tables, "w13", to_dev(a8), to_dev(asc), to_dev(offs))
    finally:
        L.call("lsk_moe_mx_select", 0)
    assert skinny == (R <= 32 * E or mxv == 3)
    assert (tables._skinny[0] is not None) == skinny
    got = bits(out)
    for e, (codes, kx, b) in enumerate(experts):
        r0, r1 = offs[e], offs[e + 1]
        if r1 == r0:
            continue
        m2, kexp = C.mx_to_m2(codes, kx)
        ref = C.lin_epilogue_mx(C.int_mm_mx(a8[r0:r1], m2, kexp), asc[r0:r1], b)
        assert np.array_equal(got[r0:r1], C.bf16_bits(ref)), "expert %d" % e


@pytest.mark.parametrize("variant", [0, 1, 5, 6, 7])
def test_grouped_linear_int8_tile_choice(variant):
    """The grouped linear on the register-staged tile (0), the 128x256 (1) and the 256x256 ping-pong
    tiles (5 persistent, 6 one tile per block) and the skinny grouped GEMM (7: experts of about 300
    rows in ten 32-row chunks), each chosen, with experts of several 256-row tiles and a bias: the
    oracle's bits."""
    from lockstep_amd import _lib as L
    from lockstep_amd import moe_ref as MR
    R, E, N, K = 1500, 5, 384, 448
    g = np.random.default_rng(91 + variant)
    cnt = _counts(g, E, R)
    offs = np.concatenate([[0], np.cumsum(cnt)]).astype(np.int32)
    a8 = g.integers(-127, 128, (R, K), dtype=np.int8)
    asc = g.uniform(1e-3, 1e-1, R).astype(F32)
    experts = [(g.integers(-127, 128, (N, K), dtype=np.int8), g.uniform(1e-3, 1e-2, N).astype(F32),
                g.standard_normal(N).astype(F32)) for _ in range(E)]
    dev_ex = [(to_dev(W).t(), to_dev(ws), to_dev(np.zeros((K, N // 2), np.int8)).t(), to_dev(np.ones(K, F32)),
               to_dev(b), None) for (W, ws, b) in experts]
    L.call("lsk_moe_select", variant)
    try:
        out = MR.grouped_linear(dev_ex, "w13", to_dev(a8), to_dev(asc), to_dev(offs))
    finally:
        L.call("lsk_moe_select", -1)
    got = bits(out)
    for e, (W, ws, b) in enumerate(experts):
        r0, r1 = offs[e], offs[e + 1]
        if r1 > r0:
            ref = C.lin_epilogue_b(C.int_mm(a8[r0:r1], W.T), ws, asc[r0:r1], b)
            assert np.array_equal(got[r0:r1], C.bf16_bits(ref)), "expert %d" % e


def test_grouped_linear_clamps_bad_offsets():
    """Offsets that decrease or run past R are made monotone and clamped to R on the device (a
    running maximum): experts come out empty or shortened, the rows they keep match the oracle, and
    nothing outside [0, R) is touched (the output has guard rows after R that stay as written)."""
    from lockstep_amd import moe_ref as MR
    R, E, N, K = 500, 6, 128, 256
    g = np.random.default_rng(77)
    offs = np.array([0, 100, 80, 300, 700, 650, 900], np.int32)       # -> 0 100 100 300 500 500 500
    co = np.minimum(np.maximum.accumulate(np.maximum(offs, 0)), R)
    a8 = g.integers(-127, 128, (R, K), dtype=np.int8)
    asc = g.uniform(1e-3, 1e-1, R).astype(F32)
    experts = [(g.integers(-127, 128, (N, K), dtype=np.int8), g.uniform(1e-3, 1e-2, N).astype(F32))
               for _ in range(E)]
    dev_ex = [(to_dev(W).t(), to_dev(ws), to_dev(np.zeros((K, N // 2), np.int8)).t(), to_dev(np.ones(K, F32)),
               None, None) for (W, ws) in experts]
    for variant in (-1, 0, 1, 5, 6):
        from lockstep_amd import _lib as L
        L.call("lsk_moe_select", variant)
        try:
            out = MR.grouped_linear(dev_ex, "w13", to_dev(a8), to_dev(asc), to_dev(offs))
        finally:
            L.call("lsk_moe_select", -1)
        got = bits(out)
        for e, (W, ws) in enumerate(experts):
            r0, r1 = co[e], co[e + 1]
            if r1 > r0:
                ref = C.lin_epilogue(C.int_mm(a8[r0:r1], W.T), ws, asc[r0:r1])
                assert np.array_equal(got[r0:r1], C.bf16_bits(ref)), (variant, e)
