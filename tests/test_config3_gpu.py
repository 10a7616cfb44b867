"""One Qwen2.5-7B-shaped decoder block's GEMMs through ref_block_v1, at 2048 and 8192 prefill rows.

Shapes (hidden 3584; 28 query heads and 4 KV heads of 128 -> qkv N = 4608; o_proj 3584; SwiGLU
intermediate 18944 -> gate+up N = 37888, down K = 18944), each GEMM fed a synthetic N(0,1)
binary32 activation [T, K] and an int8 weight uniform on [-127, 127]:

  pow2 form, the block's GEMM sites (reference/ref_block_v1.py:166-167, 191-193, 196-198,
      216-218): q8, ex = quant8_dyn(x); y = fl32(gemm_int(q8, W8)) * fl32(2^-(ex + ew)), binary32.
      The weight's exponent is ew = 7: quant8_dyn of the float weight W8 / 128 returns (W8, 7)
      whenever the weight holds a +-127, which these weights do.
  v2.1 form, the same shapes through lockstep_fullstack.w8a8_matmul with per-channel scales
      U(1e-3, 1e-2) and bf16 output (reference/lockstep_fullstack.py:503-530).

Checks per case: the exponent, and q, y on a seeded sample of rows (first, last and random) against
the oracle; for every row, the int32 accumulator's column sums and row sums against exact integer
identities (sum_m acc[m, n] = sum_k (sum_m q[m, k]) W[n, k], and the transpose), q against the
rounding rule evaluated in torch, and the fused POW2 / v2.1 outputs against the RAW accumulator
passed through a separate epilogue.
"""
import numpy as np
import pytest
import torch

from gpu_util import bits, dev, f32_bits, say
from oracle import contract as C

pytestmark = pytest.mark.gpu

F32 = np.float32
SHAPES = {"qkv": (4608, 3584), "o": (3584, 3584), "gate_up": (37888, 3584), "down": (3584, 18944)}
EW = 7


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import lockstep_amd._lib as L
    L.load()


def _inputs(T, name):
    N, K = SHAPES[name]
    g = np.random.Generator(np.random.PCG64(3000 + T + list(SHAPES).index(name)))
    x = g.standard_normal((T, K), dtype=np.float32)
    W8 = g.integers(-127, 128, (N, K), dtype=np.int8)
    W8[0, 0] = 127                                   # quant8_dyn(W8 / 128) = (W8, 7)
    ws = g.uniform(1e-3, 1e-2, N).astype(F32)
    rows = np.unique(np.concatenate([[0, 1, T - 1], g.choice(T, 21, replace=False)]))
    return x, W8, ws, rows


def _exact_rows(q_rows, W8):
    """Exact int32 products of a few quantised rows (float64 BLAS: every partial sum < 2^53)."""
    return C.int_mm(q_rows.astype(np.int8), W8.T, method="f64")


@pytest.mark.parametrize("T", [2048, 8192])
@pytest.mark.parametrize("name", list(SHAPES))
def test_qwen25_7b_block_gemm(T, name):
    from lockstep_amd import _lib as L
    from lockstep_amd import lockstep_fullstack as FS
    from lockstep_amd import ops
    from lockstep_amd import ref_block_v1 as RB

    N, K = SHAPES[name]
    say("config 3: %s T=%d (N=%d, K=%d)" % (name, T, N, K))
    x, W8, ws, rows = _inputs(T, name)
    xd = torch.from_numpy(x).to(dev())
    Wd = torch.from_numpy(W8).to(dev())
    wsd = torch.from_numpy(ws).to(dev())

    # ---- pow2 form through the fused site and through the drop-in's separate calls
    y, ex_dev = RB.linear_dyn(xd, Wd.t(), EW)
    q8, ex = RB.quant8_dyn(xd)
    assert int(ex_dev[0].item()) == ex
    m = F32(np.max(np.abs(x)))
    _, ex_ref = C.quant8_dyn(np.array([[m]], dtype=F32))   # the exponent depends on the maximum alone
    assert ex == ex_ref
    mrow = np.zeros((1, K), F32)
    mrow[0, 0] = m                                           # keeps the tensor maximum in the sample
    q_ref_rows, _ = C.quant8_dyn(np.concatenate([x[rows], mrow]))
    assert np.array_equal(bits(q8[rows]).astype(np.int64), q_ref_rows[:-1])
    # q for every row: the same rule in torch (one binary32 product by an exact power of two,
    # round half to even, clamp)
    q_t = torch.clamp(torch.round(xd * float(2.0 ** ex)), -127, 127).to(torch.int8)
    assert torch.equal(q8, q_t)
    del q_t
    y_ref_rows = C.dequant_pow2(_exact_rows(q_ref_rows[:-1], W8), ex + EW)
    assert np.array_equal(bits(y[rows]), f32_bits(y_ref_rows))
    y2 = RB.gemm_pow2(q8, ex, Wd.t(), EW)
    assert torch.equal(y.view(torch.int32), y2.view(torch.int32))
    del y2
    # every row: exact integer identities of the accumulator, and the fused epilogue against a
    # separate one over the RAW accumulator
    acc = ops.gemm(q8, Wd, L.EPI_RAW, L.LSK_I32)
    colsum = acc.sum(0, dtype=torch.int64).cpu().numpy()
    qsum = q8.sum(0, dtype=torch.int64).cpu().numpy()
    assert np.array_equal(colsum, W8.astype(np.int64) @ qsum)
    rowsum = acc.sum(1, dtype=torch.int64).cpu().numpy()
    wsum = W8.sum(0, dtype=np.int64)
    assert np.array_equal(rowsum, bits(q8).astype(np.int64) @ wsum)
    assert torch.equal(y.view(torch.int32), (acc.float() * float(2.0 ** -(ex + EW))).view(torch.int32))
    del y, q8

    # ---- v2.1 form, bf16 out
    yb = FS.w8a8_matmul(xd, Wd, wsd, out_dtype=torch.bfloat16)
    ref_b = C.w8a8_matmul(x[rows], W8, ws, None, "bf16")
    assert np.array_equal(bits(yb[rows]), ref_b)
    qr, asc = ops.rowquant(xd)
    acc = ops.gemm(qr, Wd, L.EPI_RAW, L.LSK_I32)
    yb2 = ops.epilogue(acc, L.EPI_V21, L.LSK_BF16, asc=asc, ws=wsd)
    assert torch.equal(yb.view(torch.int16), yb2.view(torch.int16))
    del acc, yb, yb2, qr
    torch.cuda.empty_cache()


def test_quant8_dyn_edge_cases():
    """Device quant8_dyn against the oracle: all-zero tensor (e = 0, q = 0), a maximum exactly at
    127 * 2^j (no decrement) and just above (decrement), the clip at e = -32 / 40, strided rows,
    and tails that are not a multiple of eight elements."""
    from lockstep_amd import ops
    from lockstep_amd import ref_block_v1 as RB

    g = np.random.default_rng(77)
    cases = [np.zeros((5, 7), F32),
             (g.standard_normal((3, 33)) * 0.01).astype(F32),
             np.full((2, 9), F32(127.0 * 2.0 ** -3)),
             np.full((2, 9), np.nextafter(F32(127.0 * 2.0 ** -3), F32(1))),
             (g.standard_normal((4, 16)) * 1e12).astype(F32),
             (g.standard_normal((4, 16)) * 1e-14).astype(F32),
             g.standard_normal((1, 1)).astype(F32),
             g.standard_normal((257, 1001)).astype(F32)]
    for x in cases:
        q_ref, e_ref = C.quant8_dyn(x)
        q, e = RB.quant8_dyn(torch.from_numpy(x).to(dev()))
        assert e == e_ref, (x.shape, e, e_ref)
        assert np.array_equal(bits(q).astype(np.int64), q_ref)
    # a strided view (row stride > K) takes the row-by-row kernels
    big = g.standard_normal((64, 300)).astype(F32)
    xs = torch.from_numpy(big).to(dev())[:, :250]
    q, e, er = ops.quant8_dyn(xs, erow=True)
    q_ref, e_ref = C.quant8_dyn(big[:, :250])
    assert int(e[0].item()) == e_ref and torch.all(er == e_ref)
    assert np.array_equal(bits(q).astype(np.int64), q_ref)
    # numpy in, numpy out (the reference's own types)
    q_np, e_np = RB.quant8_dyn(big)
    q_ref, e_ref = C.quant8_dyn(big)
    assert e_np == e_ref and np.array_equal(q_np, q_ref)


@pytest.mark.parametrize("T,N,K", [(301, 520, 3600), (256, 512, 64), (1000, 264, 208), (64, 320, 192),
                                   (24, 256, 128), (200, 130, 100), (513, 1000, 8)])
def test_linear_dyn_operand_layouts(T, N, K):
    """linear_dyn where the quantised operand takes the row-pair layout (ping-pong tiles: odd T, K
    not a multiple of 64, a single 64-byte chunk, partial tiles) and where it stays row-major (the
    128x128 tile, the decode GEMV, K % 16 != 0 on the generic kernel, K = 8), against the oracle;
    the quant-only and GEMM-only stages give the same y."""
    from lockstep_amd import ops
    from lockstep_amd import ref_block_v1 as RB

    say("linear_dyn layouts: T=%d N=%d K=%d" % (T, N, K))
    g = np.random.default_rng(T * 7 + K)
    x = g.standard_normal((T, K)).astype(F32)
    W8 = g.integers(-127, 128, (N, K), dtype=np.int8)
    xd, Wd = torch.from_numpy(x).to(dev()), torch.from_numpy(W8).to(dev())
    y, ex = RB.linear_dyn(xd, Wd.t(), 5)
    q_ref, e_ref = C.quant8_dyn(x)
    assert int(ex[0].item()) == e_ref
    ref = C.dequant_pow2(C.gemm_int(q_ref, W8.T.astype(np.int64)), e_ref + 5)
    assert np.array_equal(bits(y), f32_bits(ref))
    from lockstep_amd import _lib as L
    work = torch.empty((L.load().lsk_linear_dyn_workspace(T, K),), dtype=torch.uint8, device=dev())
    y2 = torch.full((T, N), float("nan"), device=dev())
    ex2 = torch.zeros((1,), dtype=torch.int32, device=dev())
    ops.linear_dyn(xd, Wd, 5, stages=1, work=work, y=y2, ex=ex2)
    assert int(ex2[0].item()) == e_ref and bool(torch.isnan(y2).all())
    ops.linear_dyn(xd, Wd, 5, stages=2, work=work, y=y2, ex=ex2)
    assert torch.equal(y2.view(torch.int32), y.view(torch.int32))


def test_pack_row_pairs_layout():
    """lsk_pack_row_pairs against the layout written out in numpy: element (n, k) at byte
    (n >> 1) * 2 kp + (k >> 6) * 128 + (n & 1) * 64 + (k & 63), kp = K rounded up to 64, padding 0;
    odd N, K not a multiple of 64, a strided weight."""
    from lockstep_amd import ops

    g = np.random.default_rng(9)
    for N, K, ld in [(257, 208, 208), (64, 64, 64), (3, 16, 48), (130, 1040, 1056)]:
        full = g.integers(-127, 128, (N, ld), dtype=np.int8)
        w = torch.from_numpy(full).to(dev())[:, :K]
        got = ops.pack_row_pairs(w).cpu().numpy()
        kp = (K + 63) // 64 * 64
        want = np.zeros(((N + 1) // 2) * 2 * kp, np.int8)
        n, k = np.meshgrid(np.arange(N), np.arange(K), indexing="ij")
        want[(n >> 1) * 2 * kp + (k >> 6) * 128 + (n & 1) * 64 + (k & 63)] = full[:, :K]
        assert np.array_equal(got, want), (N, K, ld)


def test_linear_dyn_weight_copy_follows_the_weight():
    """The row-pair weight copy linear_dyn keeps is remade when the weight changes in place (its
    version counter) and when another tensor takes the same storage address."""
    from lockstep_amd import ref_block_v1 as RB

    g = np.random.default_rng(10)
    T, N, K = 512, 258, 320
    x = g.standard_normal((T, K)).astype(F32)
    xd = torch.from_numpy(x).to(dev())
    W8 = g.integers(-127, 128, (N, K), dtype=np.int8)
    Wd = torch.from_numpy(W8).to(dev())
    q_ref, e_ref = C.quant8_dyn(x)

    def check(wnp, y):
        ref = C.dequant_pow2(C.gemm_int(q_ref, wnp.T.astype(np.int64)), e_ref + 7)
        assert np.array_equal(bits(y), f32_bits(ref))

    y, _ = RB.linear_dyn(xd, Wd.t(), 7)
    check(W8, y)
    Wd.neg_()                                   # in place: the cached copy is stale
    y, _ = RB.linear_dyn(xd, Wd.t(), 7)
    check(-W8, y)
    Wd[:, 5:9] = 3                              # in place through a view
    W2 = -W8
    W2[:, 5:9] = 3
    y, _ = RB.linear_dyn(xd, Wd.t(), 7)
    check(W2, y)
    ptr = Wd.data_ptr()
    del Wd
    torch.cuda.synchronize()
    W3 = g.integers(-127, 128, (N, K), dtype=np.int8)
    Wn = torch.empty((N, K), dtype=torch.int8, device=dev())
    Wn.copy_(torch.from_numpy(W3))              # often the freed block again
    say("same storage address reused: %s" % (Wn.data_ptr() == ptr))
    y, _ = RB.linear_dyn(xd, Wn.t(), 7)
    check(W3, y)


def test_linear_dyn_partial_tiles_and_graph_capture():
    """linear_dyn on shapes whose tiles are partial (general epilogue) and whole (fast POW2
    epilogue), and replayed from a captured HIP graph: every replay equals the eager result."""
    from lockstep_amd import ref_block_v1 as RB

    g = np.random.default_rng(5)
    for T, N, K in [(300, 200, 96), (512, 512, 256), (257, 640, 160)]:
        x = g.standard_normal((T, K)).astype(F32)
        W8 = g.integers(-127, 128, (N, K), dtype=np.int8)
        y, ex = RB.linear_dyn(torch.from_numpy(x).to(dev()), torch.from_numpy(W8).to(dev()).t(), 3)
        q_ref, e_ref = C.quant8_dyn(x)
        assert int(ex[0].item()) == e_ref
        ref = C.dequant_pow2(C.gemm_int(q_ref, W8.T.astype(np.int64)), e_ref + 3)
        assert np.array_equal(bits(y), f32_bits(ref)), (T, N, K)
    T, N, K = 512, 768, 512
    x = torch.from_numpy(g.standard_normal((T, K)).astype(F32)).to(dev())
    W = torch.from_numpy(g.integers(-127, 128, (N, K), dtype=np.int8)).to(dev())
    eager, _ = RB.linear_dyn(x, W.t(), 7)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        RB.linear_dyn(x, W.t(), 7)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out, _ = RB.linear_dyn(x, W.t(), 7)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), eager.view(torch.int32))
        x.mul_(1.0)            # eager work between replays


@pytest.mark.parametrize("T,N,K,scale", [(256, 512, 64, 1.0), (2048, 512, 3584, 1.0), (8192, 256, 3584, 1.0),
                                         (302, 520, 3584, 3e4), (1000, 264, 192, 1e-30), (64, 320, 3584, 0.0)])
def test_linear_dyn_single_pass_quant(T, N, K, scale):
    """linear_dyn with the one-pass quant8_dyn (lsk_quant8_dyn_single_pass(1): a cooperative launch
    holding x on chip; taken here for every shape, the largest at the on-chip capacity of a 256-CU
    part) against the oracle on a
    row sample and, bit for bit over every row, against the two-pass quantiser: tensors scaled so
    the exponent clips at -32 and at 40 (subnormal x), an all-zero tensor (e = 0), and an element
    whose scaled value is exactly 127."""
    from lockstep_amd import _lib as L
    from lockstep_amd import ref_block_v1 as RB
    say("linear_dyn one-pass quant: T=%d N=%d K=%d scale=%g" % (T, N, K, scale))
    g = np.random.default_rng(T + N + K)
    x = (g.standard_normal((T, K)) * scale).astype(F32)
    if scale == 1.0:
        x[3, 5] = F32(127.0 / 32.0)          # exactly 127 after scaling by 2^5 (max |x| < 4)
        x[np.abs(x) > 127.0 / 32.0] = F32(3.0)
    W8 = g.integers(-127, 128, (N, K), dtype=np.int8)
    xd, Wd = torch.from_numpy(x).to(dev()), torch.from_numpy(W8).to(dev())
    L.call("lsk_quant8_dyn_single_pass", 1)
    try:
        y1, e1 = RB.linear_dyn(xd, Wd.t(), 5)
    finally:
        L.call("lsk_quant8_dyn_single_pass", 0)
    y2, e2 = RB.linear_dyn(xd, Wd.t(), 5)
    assert int(e1[0].item()) == int(e2[0].item())
    assert torch.equal(y1.view(torch.int32), y2.view(torch.int32))
    rows = np.sort(np.random.default_rng(T).choice(T, min(T, 64), replace=False))
    q_ref, e_ref = C.quant8_dyn(x)
    assert int(e1[0].item()) == e_ref
    with np.errstate(over="ignore", invalid="ignore"):
        ref = C.dequant_pow2(C.gemm_int(q_ref[rows], W8.T.astype(np.int64)), e_ref + 5)
    assert np.array_equal(bits(y1)[rows], f32_bits(ref))


@pytest.mark.parametrize("T,N,K,scale", [(256, 512, 64, 1.0), (2048, 512, 3584, 1.0), (302, 520, 3584, 3e4),
                                         (6, 64, 64, 1e-30), (301, 520, 3600, 1.0), (1000, 264, 192, 0.0)])
def test_linear_dyn_quant_pass_variants(T, N, K, scale):
    """The quantise pass of linear_dyn's quant8_dyn in each form (lsk_quant8_dyn_variant 0: row
    pairs per block; 1: the walk in the order of q, taken for K % 64 == 0 and even T; 2: as 1 with
    ordinary loads) writes the same workspace bytes (partial maxima, exponents, q) and y: a tensor
    smaller than one block's threads, exponents clipped at 40 (subnormal x) and an all-zero tensor,
    and shapes that fall back to the row pairs (odd T, K % 64 != 0).  y against the oracle on a row
    sample."""
    from lockstep_amd import _lib as L
    from lockstep_amd import ops
    say("linear_dyn quant pass variants: T=%d N=%d K=%d scale=%g" % (T, N, K, scale))
    g = np.random.default_rng(T + 3 * K)
    x = (g.standard_normal((T, K)) * scale).astype(F32)
    W8 = g.integers(-127, 128, (N, K), dtype=np.int8)
    xd, Wd = torch.from_numpy(x).to(dev()), torch.from_numpy(W8).to(dev())
    nbytes = L.load().lsk_linear_dyn_workspace(T, K)
    got = []
    for v in (0, 1, 2):
        work = torch.full((nbytes,), 0x5A, dtype=torch.uint8, device=dev())
        y = torch.empty((T, N), dtype=torch.float32, device=dev())
        ex = torch.zeros((1,), dtype=torch.int32, device=dev())
        L.call("lsk_quant8_dyn_variant", v)
        try:
            ops.linear_dyn(xd, Wd, 5, stages=3, work=work, y=y, ex=ex)
        finally:
            L.call("lsk_quant8_dyn_variant", 1)
        got.append((work.cpu(), y.view(torch.int32).cpu(), int(ex[0].item())))
    for w, y, e in got[1:]:
        assert e == got[0][2] and torch.equal(w, got[0][0]) and torch.equal(y, got[0][1])
    q_ref, e_ref = C.quant8_dyn(x)
    assert got[0][2] == e_ref
    rows = np.sort(np.random.default_rng(T).choice(T, min(T, 48), replace=False))
    with np.errstate(over="ignore", invalid="ignore"):
        ref = C.dequant_pow2(C.gemm_int(q_ref[rows], W8.T.astype(np.int64)), e_ref + 5)
    assert np.array_equal(got[0][1].numpy()[rows].view(np.uint32), f32_bits(ref))
