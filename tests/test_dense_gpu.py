"""GPU parity of the dense contract path: bit equality with the oracle (and, through it, with
the reference's published conformance digests) on seeded inputs and edge shapes."""
import numpy as np
import pytest
import torch

from gpu_util import bf16_dev, bits, dev, f16_bits, f32_bits, say, to_dev
from oracle import contract as C
from vector_inputs import linear_inputs, load_vectors

pytestmark = pytest.mark.gpu

F32 = np.float32


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import lockstep_amd._lib as L
    L.load()


def _rng(seed):
    return np.random.default_rng(seed)


# ------------------------------------------------------------------ the published vectors
def test_conformance_vectors_on_gpu():
    from lockstep_amd import lockstep_fullstack as FS
    from lockstep_amd import moe_ref as MR
    V = load_vectors()
    _, x, W, bias = linear_inputs()
    xd = bf16_dev(x)
    q, asc = FS.quantize_rows_int8(xd.float())
    assert C.digest(bits(q), "int8") == V["act_quant.q"]["sha256"]
    assert C.digest(bits(asc).view(F32), "float32") == V["act_quant.asc"]["sha256"]
    W8, ws = FS.quantize_weight_int8(bf16_dev(W))
    assert C.digest(bits(W8), "int8") == V["weight_quant.w8"]["sha256"]
    assert C.digest(bits(ws).view(F32), "float32") == V["weight_quant.ws"]["sha256"]
    bd = to_dev(bias)
    y = FS.w8a8_matmul(xd, W8, ws, None, out_dtype=torch.bfloat16)
    assert C.digest(bits(y), "bfloat16") == V["linear.v2_1.no_bias"]["sha256"]
    yb = FS.w8a8_matmul(xd, W8, ws, bd, out_dtype=torch.bfloat16)
    assert C.digest(bits(yb), "bfloat16") == V["linear.v2_1.bias"]["sha256"]
    # moe_ref's separate int_mm + lin_epilogue(_b), and the fused form
    q2, asc2 = MR.rowquant(xd)
    acc = MR.int_mm(q2, W8.t())
    y2 = MR.lin_epilogue(acc, ws, asc2).to(torch.bfloat16)
    assert C.digest(bits(y2), "bfloat16") == V["linear.v2_1.no_bias"]["sha256"]
    y3 = MR.lin_epilogue_b(acc, ws, asc2, bd).to(torch.bfloat16)
    assert C.digest(bits(y3), "bfloat16") == V["linear.v2_1.bias"]["sha256"]
    y4 = MR.linear(q2, asc2, W8.t(), ws, bd).to(torch.bfloat16)
    assert C.digest(bits(y4), "bfloat16") == V["linear.v2_1.bias"]["sha256"]


# ------------------------------------------------------------------ row quant
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(1, 16), (3, 37), (7, 512), (33, 4096), (2, 18944), (0, 64), (64, 16), (65, 520),
                                   (200, 2048), (129, 4096), (70, 37)])
def test_rowquant_parity(dtype, shape):
    from lockstep_amd import moe_ref as MR
    say("rowquant", dtype, shape)
    r = _rng(hash((str(dtype), shape)) % 2**32)
    x = (r.standard_normal(shape) * 3).astype(F32)
    if shape[0] > 2:
        x[1] = 0.0
        x[2, :3] = [1e-30, -1e-40, 0.5]
    xt = torch.from_numpy(x).to(dtype)
    xr = xt.float().numpy()                      # the values the reference sees after .float()
    q, asc = MR.rowquant(xt.to(dev()))
    qo, asco = C.rowquant(xr)
    assert np.array_equal(bits(q), qo)
    assert np.array_equal(bits(asc), f32_bits(asco))


# ------------------------------------------------------------------ exact GEMM
GEMM_SHAPES = [
    (1, 1, 16), (1, 17, 64), (5, 16, 128), (16, 33, 144), (17, 64, 512), (31, 100, 2880),
    (32, 256, 4096), (33, 130, 256), (64, 64, 64), (127, 255, 1024), (128, 128, 128),
    (129, 257, 640), (300, 1000, 2048), (16, 3584, 3584),
]


@pytest.mark.parametrize("M,N,K", GEMM_SHAPES)
def test_int_mm_parity(M, N, K):
    from lockstep_amd import moe_ref as MR
    say("int_mm", M, N, K)
    r = _rng(M * 1000003 + N * 1009 + K)
    a = r.integers(-127, 128, (M, K), dtype=np.int8)
    w = r.integers(-127, 128, (N, K), dtype=np.int8)
    acc = MR.int_mm(to_dev(a), to_dev(w).t())
    assert np.array_equal(bits(acc), C.int_mm(a, w.T))


@pytest.mark.parametrize("M,N,K", [(3, 5, 7), (4, 9, 100), (17, 3, 33), (2, 2, 0)])
def test_int_mm_generic_path(M, N, K):
    """K not a multiple of 16 and K == 0 take the generic kernel; results stay exact."""
    from lockstep_amd import moe_ref as MR
    r = _rng(M + N + K)
    a = r.integers(-127, 128, (M, K), dtype=np.int8)
    w = r.integers(-127, 128, (N, K), dtype=np.int8)
    acc = MR.int_mm(to_dev(a), to_dev(w).t())
    assert np.array_equal(bits(acc), C.int_mm(a, w.T) if K else np.zeros((M, N), np.int32))


def test_int_mm_extremes_and_strided_operands():
    from lockstep_amd import moe_ref as MR
    K = 18944
    a = np.full((3, K), -127, np.int8)
    a[1] = 127
    w = np.full((20, K), 127, np.int8)
    acc = MR.int_mm(to_dev(a), to_dev(w).t())
    assert np.array_equal(bits(acc), C.int_mm(a, w.T))
    assert int(bits(acc)[0, 0]) == -K * 127 * 127
    # a [K, N] weight that is NOT the transpose of a row-major [N, K]: copied, same result
    r = _rng(99)
    a = r.integers(-127, 128, (40, 96), dtype=np.int8)
    b = r.integers(-127, 128, (96, 50), dtype=np.int8)
    acc = MR.int_mm(to_dev(a), to_dev(b))
    assert np.array_equal(bits(acc), C.int_mm(a, b))


# ------------------------------------------------------------------ epilogues
@pytest.mark.parametrize("M,N,K", [(1, 64, 256), (8, 100, 512), (32, 48, 1024), (200, 300, 768)])
@pytest.mark.parametrize("use_bias", [False, True])
@pytest.mark.parametrize("out", ["bf16", "f32", "f16"])
def test_w8a8_matmul_parity(M, N, K, use_bias, out):
    from lockstep_amd import lockstep_fullstack as FS
    say("w8a8_matmul", M, N, K, use_bias, out)
    r = _rng(M * 7 + N * 11 + K * 13 + use_bias)
    x = (r.standard_normal((M, K)) * 2).astype(F32)
    x[r.random((M, K)) < 0.001] = 20.0
    xb = C.bfr(x)
    W8 = r.integers(-127, 128, (N, K), dtype=np.int8)
    ws = r.uniform(1e-3, 1e-2, N).astype(F32)
    bias = (r.standard_normal(N) * 0.1).astype(F32) if use_bias else None
    tdt = {"bf16": torch.bfloat16, "f32": torch.float32, "f16": torch.float16}[out]
    y = FS.w8a8_matmul(bf16_dev(xb), to_dev(W8), to_dev(ws), to_dev(bias) if use_bias else None, out_dtype=tdt)
    ref = C.w8a8_matmul(xb, W8, ws, bias, out)
    if out == "f16":
        ref = f16_bits(ref)
    elif out == "f32":
        ref = f32_bits(ref)
    assert np.array_equal(bits(y), ref)


def test_w8a8_matmul_fp32_input_and_zero_rows():
    from lockstep_amd import lockstep_fullstack as FS
    r = _rng(5)
    x = r.standard_normal((2, 3, 256)).astype(F32)
    W8 = r.integers(-127, 128, (40, 256), dtype=np.int8)
    ws = r.uniform(1e-3, 1e-2, 40).astype(F32)
    y = FS.w8a8_matmul(to_dev(x), to_dev(W8), to_dev(ws))          # fp32 in, fp32 out, no rounding
    assert y.shape == (2, 3, 40) and y.dtype == torch.float32
    ref = C.w8a8_matmul(x.reshape(6, 256), W8, ws, None, "f32")
    assert np.array_equal(bits(y).reshape(6, 40), f32_bits(ref))
    z = FS.w8a8_matmul(to_dev(np.zeros((0, 256), F32)), to_dev(W8), to_dev(ws), out_dtype=torch.bfloat16)
    assert z.shape == (0, 40) and z.dtype == torch.bfloat16


def test_w8a8_linear_v2_order():
    from lockstep_amd import contract_common as CC
    r = _rng(6)
    lin = torch.nn.Linear(384, 72, bias=True).to(dev()).to(torch.bfloat16)
    Wf = lin.weight.data.float().cpu().numpy()
    bias = lin.bias.data.float().cpu().numpy()
    x = C.bfr((r.standard_normal((9, 384)) * 2).astype(F32))
    CC.w8a8_linear(lin)
    y = lin(bf16_dev(x))
    W8, ws = C.w8a8_linear_prepare(Wf)
    ref = C.w8a8_linear_fwd(x, W8, ws, bias, "bf16")
    assert y.dtype == torch.bfloat16
    assert np.array_equal(bits(y), ref)


# ------------------------------------------------------------------ pow2 (ref_block_v1)
def test_pow2_quant_and_gemm_parity():
    from lockstep_amd import ref_block_v1 as RB
    r = _rng(7)
    x = (r.standard_normal((64, 512)) * 3).astype(F32)
    Wt = (r.standard_normal((512, 192)) * 0.05).astype(F32)   # [K, N] as the block's weights
    qx, ex = RB.quant8_dyn(x)
    qo, eo = C.quant8_dyn(x)
    assert ex == eo and np.array_equal(qx, qo)
    qw, ew = RB.quant8_dyn(Wt)
    qwo, ewo = C.quant8_dyn(Wt)
    assert ew == ewo and np.array_equal(qw, qwo)
    acc = RB.gemm_int(qx, qw)
    assert np.array_equal(acc, C.gemm_int(qo, qwo))
    y = RB.gemm_pow2(qx, ex, qw, ew)
    assert np.array_equal(f32_bits(y), f32_bits(C.dequant_pow2(C.gemm_int(qo, qwo), eo + ewo)))
    qr, er = RB.quant8_rows(x)
    qro, ero = C.quant8_rows(x)
    assert np.array_equal(qr, qro) and np.array_equal(er, ero)
    qc, ec = RB.quant8_cols(Wt)
    qco, eco = C.quant8_cols(Wt)
    assert np.array_equal(qc, qco) and np.array_equal(ec, eco)
    y2 = RB.gemm_pow2(qr, er, qc, ec)
    ref2 = C.dequant_pow2(C.gemm_int(qro, qco), ero[:, None] + eco[None, :])
    assert np.array_equal(f32_bits(y2), f32_bits(ref2))
    assert RB.quant8_dyn(np.zeros((3, 4), F32))[1] == 0
    em = np.array([0.0, 127.0, 127.5, 1e-30, 3e38, 1e-40, 64.0], F32)
    assert np.array_equal(RB._e_from_max(em), C._e_from_max(em))


@pytest.mark.parametrize("M", [1, 2, 3, 4])
@pytest.mark.parametrize("N,K", [(1000, 4096), (77, 2880), (300, 1040), (520, 14336), (64, 16), (33, 32768)])
@pytest.mark.parametrize("xdt", ["f32", "bf16"])
def test_decode_w8a8_rows(M, N, K, xdt):
    """w8a8_matmul at M <= 4 (row quant, then the whole-row GEMV) against the oracle's rowquant +
    int_mm + epilogue: V21 with and without bias and V2, bf16 and binary32 out, K up to 32768.  x
    carries 20-sigma outliers, an exact amax of 127 in row 0 (asc = 1, so 2.5, -3.5, 0.5 and 126.5
    are rounding ties) and, for M >= 2, an all-zero last row (the 1e-8 floor)."""
    import lockstep_amd._lib as L
    from lockstep_amd import ops
    say("decode rows", M, N, K, xdt)
    r = _rng(1000 * M + N + K)
    x = (r.standard_normal((M, K)) * 2).astype(F32)
    out_idx = r.random((M, K)) < 1e-3
    x[out_idx] = np.sign(x[out_idx]) * 40.0
    if K >= 8:
        x[0, 1] = 127.0
        x[0, 2:6] = [2.5, -3.5, 0.5, 126.5]
    if M >= 2:
        x[M - 1] = 0.0
    if xdt == "bf16":
        x = C.bf16_to_f32(C.bf16_bits(x))
        xd = bf16_dev(x)
    else:
        xd = to_dev(x)
    W8 = r.integers(-127, 128, (N, K), dtype=np.int8)
    ws = r.uniform(1e-3, 1e-2, N).astype(F32)
    bias = (r.standard_normal(N) * 0.1).astype(F32)
    q, asc = C.rowquant(x)
    acc = C.int_mm(q, W8.T)
    Wd, wsd, bd = to_dev(W8), to_dev(ws), to_dev(bias)
    for order, b in ((L.EPI_V21, None), (L.EPI_V21, bias), (L.EPI_V2, bias)):
        for odt, name in ((L.LSK_BF16, "bf16"), (L.LSK_F32, "f32")):
            y = ops.w8a8_matmul(xd, Wd, wsd, None if b is None else bd, order, odt)
            f = C.epilogue_v21 if order == L.EPI_V21 else C.epilogue_v2
            ref = f(acc, ws, asc, b, name)
            want = ref if name == "bf16" else f32_bits(ref)
            assert np.array_equal(bits(y), want), (order, b is not None, name)


@pytest.mark.parametrize("M", [1, 4, 5, 8, 16, 17, 32])
@pytest.mark.parametrize("N,K", [(1000, 4096), (77, 2880), (3584, 3584), (33, 48), (1001, 1040), (520, 14336),
                                 (4100, 64), (16, 4096)])
def test_skinny_gemv_parity(M, N, K):
    """The skinny decode GEMV (activation rows staged in LDS, weight rows streamed into the MFMA B
    operand) forced for every M it fits (tile 19), reading the weight row-major and as its row-pair
    copy: V21 with bias and bf16 out, V2 with binary32 out, RAW int32 and POW2 with per-row
    exponents, against the oracle; K tails (K % 64 != 0), partial 16-row groups, an all-zero
    activation row."""
    from lockstep_amd import _lib as L
    from lockstep_amd import ops
    say("skinny", M, N, K)
    if M * ((K + 1023) // 1024 * 1024 + 16) > 160 * 1024:
        pytest.skip("A does not fit in LDS: the skinny GEMV is not taken at this shape")
    r = _rng(7 * M + 11 * N + K)
    a8 = r.integers(-127, 128, (M, K), dtype=np.int8)
    if M > 2:
        a8[M - 2] = 0
    W8 = r.integers(-127, 128, (N, K), dtype=np.int8)
    asc = r.uniform(1e-3, 1e-2, M).astype(F32)
    ws = r.uniform(1e-3, 1e-2, N).astype(F32)
    bias = (r.standard_normal(N) * 0.1).astype(F32)
    erow = r.integers(-20, 20, M).astype(np.int32)
    acc = C.int_mm(a8, W8.T)
    ad, Wd = to_dev(a8), to_dev(W8)
    Wp = ops.pack_row_pairs(Wd)
    # x whose row quant reproduces rows of a8 scaled: the row-pair copy is read through w8a8_matmul
    x = (r.standard_normal((M, K)) * 2).astype(F32)
    q, asc_q = C.rowquant(x)
    accq = C.int_mm(q, W8.T)
    L.call("lsk_gemm_select", 19)
    try:
        y = ops.gemm(ad, Wd, L.EPI_RAW, L.LSK_I32)
        assert np.array_equal(bits(y), acc), "raw"
        y = ops.gemm(ad, Wd, L.EPI_V21, L.LSK_BF16, asc=to_dev(asc), ws=to_dev(ws), bias=to_dev(bias))
        assert np.array_equal(bits(y), C.epilogue_v21(acc, ws, asc, bias, "bf16")), "v21"
        y = ops.gemm(ad, Wd, L.EPI_V2, L.LSK_F32, asc=to_dev(asc), ws=to_dev(ws))
        assert np.array_equal(bits(y), f32_bits(C.epilogue_v2(acc, ws, asc, None, "f32"))), "v2"
        y = ops.gemm(ad, Wd, L.EPI_POW2, L.LSK_F32, erow=to_dev(erow), shift=3)
        with np.errstate(over="ignore"):
            ref = C.dequant_pow2(acc, erow[:, None].astype(np.int64) + 3)
        assert np.array_equal(bits(y), f32_bits(ref)), "pow2"
        for wp in (None, Wp):
            y = ops.w8a8_matmul(to_dev(x), Wd, to_dev(ws), to_dev(bias), L.EPI_V21, L.LSK_BF16, w_pairs=wp)
            assert np.array_equal(bits(y), C.epilogue_v21(accq, ws, asc_q, bias, "bf16")), ("w8a8 v21", wp is None)
            y = ops.w8a8_matmul(to_dev(x), Wd, to_dev(ws), None, L.EPI_V2, L.LSK_F32, w_pairs=wp)
            assert np.array_equal(bits(y), f32_bits(C.epilogue_v2(accq, ws, asc_q, None, "f32"))), ("w8a8 v2",
                                                                                                  wp is None)
    finally:
        L.call("lsk_gemm_select", -1)


@pytest.mark.parametrize("tile", [1, 2, 3, 4, 12, 13, 17, 18])
def test_pow2_whole_tile_epilogue_exponent_range(tile):
    """The POW2 epilogue of whole ping-pong / four-wave tiles (binary32 out, per-row exponents,
    stored straight from the accumulators) over the whole exponent range: shift + erow from -140
    (factor 2^140 overflows: inf, NaN for a zero sum) through 0 to 126 .. 149 (subnormal factors,
    exact) and 150, 200 (factor 0)."""
    import lockstep_amd._lib as L
    from lockstep_amd import ops
    M, N, K, shift = 512, 512, 192, 7
    say("pow2 range", tile, M, N, K)
    r = _rng(900 + tile)
    a = r.integers(-127, 128, (M, K), dtype=np.int8)
    w = r.integers(-127, 128, (N, K), dtype=np.int8)
    a[5] = 0  # a zero row under every factor
    picks = np.array([-147, -135, -134, -100, -7, 0, 3, 30, 119, 120, 126, 130, 142, 143, 150, 193], np.int32)
    erow = r.choice(picks, M).astype(np.int32)
    erow[:len(picks)] = picks
    erow[5] = -147
    L.call("lsk_gemm_select", tile)
    try:
        y = ops.gemm(to_dev(a), to_dev(w), L.EPI_POW2, L.LSK_F32, erow=to_dev(erow), shift=shift)
        got = bits(y)
    finally:
        L.call("lsk_gemm_select", -1)
    with np.errstate(over="ignore", invalid="ignore"):
        ref = C.dequant_pow2(C.int_mm(a, w.T), erow[:, None].astype(np.int64) + shift)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got.view(F32)), nan)
    assert np.array_equal(got[~nan], f32_bits(ref)[~nan])
    assert nan[5].all() and np.isinf(ref[0]).any() and (ref[np.where(erow + shift > 149)[0]] == 0).all()


@pytest.mark.parametrize("M,N,K", [(512, 512, 384), (2048, 1536, 640), (1024, 2304, 3584)])
@pytest.mark.parametrize("blocks", [1, 3, 7])
def test_pow2_persistent_kernel(M, N, K, blocks):
    """The persistent POW2 kernel (whole 256 x 256 tiles, each block walking several tiles and
    issuing the next tile's first stages before storing the current one): bits equal to the
    one-tile-per-block launch and, on a row subset, to the oracle, with one block per CU (1) and
    with 3 or 7 blocks (many tiles per block, uneven counts)."""
    import lockstep_amd._lib as L
    from lockstep_amd import ops
    say("pow2 persistent", M, N, K, blocks)
    r = _rng(M + N + K + blocks)
    a = r.integers(-127, 128, (M, K), dtype=np.int8)
    w = r.integers(-127, 128, (N, K), dtype=np.int8)
    erow = r.integers(-20, 20, M).astype(np.int32)
    erow[:4] = [-150, 150, 130, -130]
    ad, wd, ed = to_dev(a), to_dev(w), to_dev(erow)
    L.call("lsk_gemm_persist", blocks)
    try:
        y = bits(ops.gemm(ad, wd, L.EPI_POW2, L.LSK_F32, erow=ed, shift=5))
        L.call("lsk_gemm_persist", 0)
        y0 = bits(ops.gemm(ad, wd, L.EPI_POW2, L.LSK_F32, erow=ed, shift=5))
    finally:
        L.call("lsk_gemm_persist", 1)
    assert np.array_equal(y, y0)
    rows = np.sort(np.concatenate([[0, 1, 2, 3, M - 1], r.choice(M, 12, replace=False)]))
    with np.errstate(over="ignore", invalid="ignore"):
        ref = C.dequant_pow2(C.int_mm(a[rows], w.T), erow[rows, None].astype(np.int64) + 5)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(y[rows].view(F32)), nan)
    assert np.array_equal(y[rows][~nan], f32_bits(ref)[~nan])


# ------------------------------------------------------------------ the dense configurations
def test_config1_o_proj_m16_bit_exact():
    """M=16 tokens, K=N=3584: x N(0,1) seed 0 quantised by the contract quantiser, W8 uniform
    [-127, 127], ws U(1e-3, 1e-2), bf16 output."""
    from lockstep_amd import lockstep_fullstack as FS
    from lockstep_amd import workloads as WL
    x, W8, ws = WL.dense_inputs(16, 3584, 3584, seed=0)
    y = FS.w8a8_matmul(to_dev(x), to_dev(W8), to_dev(ws), out_dtype=torch.bfloat16)
    assert np.array_equal(bits(y), C.w8a8_matmul(x, W8, ws, None, "bf16"))


@pytest.mark.parametrize("seed", [1, 2, 3, 4])
@pytest.mark.parametrize("M", [1, 8, 32])
@pytest.mark.parametrize("which", ["gate_up", "down"])
def test_config2_decode_bit_exact(M, which, seed):
    from lockstep_amd import lockstep_fullstack as FS
    from lockstep_amd import workloads as WL
    N, K = WL.LLAMA8B[which]
    say("config2 decode", which, M, N, K, "seed", seed)
    x, W8, ws = WL.dense_inputs(M, N, K, seed=seed, outliers=True)
    y = FS.w8a8_matmul(to_dev(x), to_dev(W8), to_dev(ws), out_dtype=torch.bfloat16)
    assert np.array_equal(bits(y), C.w8a8_matmul(x, W8, ws, None, "bf16"))


@pytest.mark.parametrize("seed", [1, 2, 3, 4])
@pytest.mark.parametrize("which", ["gate_up", "down"])
def test_config2_prefill_rows_and_chunk_invariance(which, seed):
    """M=2048: a seeded subset of 256 rows against the oracle; for every row the quantised rows
    against the oracle's quantiser, the int32 accumulator's column and row sums against exact
    integer identities, the fused v2.1 epilogue against the separate epilogue over that
    accumulator, and the whole result equal to the same rows computed in 64-row chunks (row
    independence: per-token scales, exact sums)."""
    from lockstep_amd import _lib as L
    from lockstep_amd import lockstep_fullstack as FS
    from lockstep_amd import ops
    from lockstep_amd import workloads as WL
    N, K = WL.LLAMA8B[which]
    M = 2048
    say("config2 prefill", which, M, N, K, "seed", seed)
    x, W8, ws = WL.dense_inputs(M, N, K, seed=seed, outliers=True)
    xd, Wd, wsd = to_dev(x), to_dev(W8), to_dev(ws)
    y = FS.w8a8_matmul(xd, Wd, wsd, out_dtype=torch.bfloat16)
    rows = np.sort(_rng(3 + seed).choice(M, 256, replace=False))
    ref = C.w8a8_matmul(x[rows], W8, ws, None, "bf16")
    assert np.array_equal(bits(y)[rows], ref)
    q, asc = ops.rowquant(xd)
    q_ref, asc_ref = C.rowquant(x)
    assert np.array_equal(bits(q), q_ref) and np.array_equal(bits(asc), f32_bits(asc_ref))
    acc = ops.gemm(q, Wd, L.EPI_RAW, L.LSK_I32)
    assert np.array_equal(acc.sum(0, dtype=torch.int64).cpu().numpy(), W8.astype(np.int64) @ q_ref.sum(0, dtype=np.int64))
    assert np.array_equal(acc.sum(1, dtype=torch.int64).cpu().numpy(), q_ref.astype(np.int64) @ W8.sum(0, dtype=np.int64))
    y2 = ops.epilogue(acc, L.EPI_V21, L.LSK_BF16, asc=asc, ws=wsd)
    assert torch.equal(y2.view(torch.int16), y.view(torch.int16))
    chunks = torch.cat([FS.w8a8_matmul(xd[i:i + 64], Wd, wsd, out_dtype=torch.bfloat16) for i in range(0, M, 64)])
    assert torch.equal(chunks.view(torch.int16), y.view(torch.int16))


@pytest.mark.parametrize("tile", [0, 1, 2, 3, 4, 5, 6, 7, 12, 13, 14, 15, 17, 18, 19])
@pytest.mark.parametrize("M,N,K", [(300, 1000, 2048), (129, 257, 640), (512, 520, 2880), (64, 64, 16),
                                   (1, 1000, 14336), (3, 77, 2880), (4, 300, 1040), (8, 1000, 4096),
                                   (17, 77, 2880), (32, 520, 14336), (5, 33, 48), (24, 32800, 320),
                                   (16, 700, 8192), (13, 129, 1040), (7, 1001, 14336)])
def test_every_tile_config_is_exact(tile, M, N, K):
    """The forced tile configurations produce the same bits (exact integer sums, any tiling)."""
    from lockstep_amd import _lib as L
    from lockstep_amd import lockstep_fullstack as FS
    say("tile", tile, M, N, K)
    r = _rng(M + 3 * N + 7 * K + tile)
    x = (r.standard_normal((M, K)) * 2).astype(F32)
    W8 = r.integers(-127, 128, (N, K), dtype=np.int8)
    ws = r.uniform(1e-3, 1e-2, N).astype(F32)
    bias = (r.standard_normal(N) * 0.1).astype(F32)
    L.call("lsk_gemm_select", tile)
    try:
        y = FS.w8a8_matmul(to_dev(x), to_dev(W8), to_dev(ws), to_dev(bias), out_dtype=torch.bfloat16)
        acc = FS._int_mm_exact(to_dev(C.rowquant(x)[0]), to_dev(W8).t())
    finally:
        L.call("lsk_gemm_select", -1)
    assert np.array_equal(bits(y), C.w8a8_matmul(x, W8, ws, bias, "bf16"))
    assert np.array_equal(bits(acc), C.int_mm(C.rowquant(x)[0], W8.T))


@pytest.mark.parametrize("tile", [1, 3, 4, 12, 13, 17, 18])
@pytest.mark.parametrize("out", ["bf16", "f32"])
def test_epilogue_special_scales(tile, out):
    """Scales that can make outputs infinite or NaN, placed so that some tiles hold none of them
    (those take the vectorised epilogue) and others do (the general one): every output equal to
    the oracle's (bf16 NaN as 0x7FC0; binary32 NaN compared as NaN, its payload is the
    platform's).  The clean tile also holds extreme but NaN-free scales: a subnormal ws and
    asc, zeros of both signs, ws = 2^95 against asc = 2^100 (infinite outputs)."""
    from lockstep_amd import _lib as L
    from lockstep_amd import ops
    say("epilogue special scales", tile, out)
    r = _rng(11 + tile)
    M = N = 512
    K = 256
    a8 = r.integers(-127, 128, (M, K), dtype=np.int8)
    W8 = r.integers(-127, 128, (N, K), dtype=np.int8)
    a8[7] = 0                                            # an all-zero accumulator row
    asc = r.uniform(1e-3, 1e-2, M).astype(F32)
    ws = r.uniform(1e-3, 1e-2, N).astype(F32)
    # NaN-free extremes in rows / columns 0..127
    ws[10] = F32(1e-40)
    ws[20] = F32(2.0 ** 95)
    ws[21] = F32(-3.0)
    asc[30] = F32(2.0 ** 100)
    asc[40] = F32(1e-41)
    asc[50] = F32(0.0)
    asc[51] = F32(-0.0)
    # scales that rule the fast path out, in rows / columns 384..511
    ws[400] = np.inf
    ws[401] = np.nan
    ws[402] = F32(2.0 ** 100)
    ws[403] = F32(2.0 ** 96)
    asc[450] = np.inf
    asc[451] = np.nan
    asc[452] = F32(0.0)
    a8[452] = a8[0]
    odt = {"bf16": L.LSK_BF16, "f32": L.LSK_F32}[out]
    L.call("lsk_gemm_select", tile)
    try:
        y = ops.gemm(to_dev(a8), to_dev(W8), L.EPI_V21, odt, asc=to_dev(asc), ws=to_dev(ws))
    finally:
        L.call("lsk_gemm_select", -1)
    acc = C.int_mm(a8, W8.T)
    with np.errstate(invalid="ignore", over="ignore"):
        ref = C.epilogue_v21(acc, ws, asc, None, out)
    got = bits(y)
    if out == "bf16":
        assert np.array_equal(got, ref)
    else:
        gf = got.view(F32)
        nan = np.isnan(ref)
        assert np.array_equal(np.isnan(gf), nan)
        assert np.array_equal(got[~nan], f32_bits(ref)[~nan])
    assert acc[30, 20] != 0 and np.isinf(C.out_to_f32(ref, out)[30, 20])  # the case is present


@pytest.mark.parametrize("N", [33024, 33064])
def test_column_split_into_whole_rounds_is_exact(N):
    """Shapes whose 256x256 tiles end in a partial round run as whole rounds of 256x256 tiles
    over the first columns plus 256x128 tiles over the rest; every epilogue sees shifted column
    operands (ws, bias, the outlier weights): the results equal the oracle's bit for bit."""
    from lockstep_amd import lockstep_fullstack as FS
    M, K = 300, 256
    say("column split", M, N, K)
    r = _rng(N)
    x = C.bfr((r.standard_normal((M, K)) * 2).astype(F32))
    W8 = r.integers(-127, 128, (N, K), dtype=np.int8)
    ws = r.uniform(1e-3, 1e-2, N).astype(F32)
    bias = (r.standard_normal(N) * 0.1).astype(F32)
    y = FS.w8a8_matmul(to_dev(x), to_dev(W8), to_dev(ws), to_dev(bias), out_dtype=torch.bfloat16)
    assert np.array_equal(bits(y), C.w8a8_matmul(x, W8, ws, bias, "bf16"))
    acc = FS._int_mm_exact(to_dev(C.rowquant(x)[0]), to_dev(W8).t())
    assert np.array_equal(bits(acc), C.int_mm(C.rowquant(x)[0], W8.T))
    oidx = np.array([3, 77, 200], dtype=np.int32)
    wo = C.bfr((r.standard_normal((N, 3)) * 0.05).astype(F32))
    yo = FS.w8a8_outlier_linear(bf16_dev(x), to_dev(oidx), bf16_dev(wo), to_dev(W8), to_dev(ws), to_dev(bias),
                                out_dtype=torch.bfloat16)
    assert np.array_equal(bits(yo), C.w8a8_outlier_linear(x, oidx, wo, W8, ws, bias, "bf16"))


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("K", [1024, 4104, 14336])
def test_rowquant_near_half_integer_quotients(dtype, K):
    """Values whose quotient x / asc lies on or next to a half-integer (x = fl32((n + 1/2) asc) and
    its neighbours, for every n in [-127, 126]) under several row maxima (asc exact, inexact,
    tiny, below the 1e-8 floor, huge): the quantisers round fl32(x / asc), which the fast
    reciprocal path must reproduce exactly, ties to even included."""
    from lockstep_amd import ops
    say("rowquant near ties", dtype, K)
    rows = []
    for amax in (127.0, 100.0, 3.3, 1e-3, 5e-9, 7e30, 0.7):
        a = np.float32(amax)
        s = np.float32(max(a, np.float32(1e-8)) / np.float32(127.0))
        vals = [a]
        for n in range(-127, 127):
            c = np.float32((n + 0.5) * np.float64(s))
            vals += [c, np.nextafter(c, np.float32(np.inf)), np.nextafter(c, np.float32(-np.inf))]
        v = np.array(vals, np.float32)
        v = v[np.abs(v) <= a]
        row = np.resize(v, K).astype(np.float32)
        row[0] = a
        rows.append(row)
    x = np.stack(rows)
    if dtype == "bf16":
        x = C.bf16_to_f32(C.bf16_bits(x))
        xd = bf16_dev(x)
    else:
        xd = to_dev(x)
    q, asc = ops.rowquant(xd)
    rq, rasc = C.rowquant(x)
    assert np.array_equal(bits(asc), f32_bits(rasc))
    assert np.array_equal(bits(q), rq)
    # the same rows one at a time through the one-row GEMV with the row quant fused in
    from lockstep_amd import lockstep_fullstack as FS
    r = _rng(K)
    N = 40
    W8 = r.integers(-127, 128, (N, K), dtype=np.int8)
    ws = r.uniform(1e-3, 1e-2, N).astype(F32)
    for i in range(x.shape[0]):
        y = FS.w8a8_matmul(xd[i:i + 1], to_dev(W8), to_dev(ws), out_dtype=torch.bfloat16)
        assert np.array_equal(bits(y), C.w8a8_matmul(x[i:i + 1], W8, ws, None, "bf16")), i


def test_bf16_conversion_instruction_equals_rne_on_every_binary32():
    """Every bf16 rounding of the library is gfx950's packed conversion instruction: it must give
    the round-to-nearest-even bits (torch's .to(bfloat16)) for every one of the 2^32 binary32
    patterns that is not a NaN, both halves of the pair, denormals included; and the library's
    conversion (that instruction, NaN -> 0x7FC0) must equal the bit method on all 2^32 patterns."""
    from lockstep_amd import _lib as L
    mism = torch.zeros(1, dtype=torch.int32, device=dev())
    first = torch.full((1,), -1, dtype=torch.int32, device=dev())    # 0xFFFFFFFF
    s = L.stream_of(mism)
    for c in range(4):
        L.call("lsk_bf16_cvt_check", c << 30, 1 << 30, L.ptr(mism), L.ptr(first), s)
    torch.cuda.synchronize()
    assert int(mism.item()) == 0, "%d patterns differ, first 0x%08x" % (int(mism.item()), int(first.item()) & 0xffffffff)


@pytest.mark.parametrize("xdt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("N,K", [(1, 16), (257, 1040), (3, 2048), (1000, 4096), (300, 5120), (4096, 14336),
                                 (77, 16384)])
def test_one_row_fused_rowquant_gemv(N, K, xdt):
    """w8a8_matmul with one activation row runs the row quant inside the whole-row GEMV (one
    launch: four-wave blocks up to K = 4096, sixteen-wave blocks up to 16384; two launches beyond):
    the oracle's bits for every order, bias and output
    type, near-tie activations, and the same bits as the two-launch path
    (lsk_gemm_fuse_rowquant(0))."""
    import lockstep_amd._lib as L
    from lockstep_amd import ops
    say("fused one-row GEMV", N, K, xdt)
    r = _rng(7 * N + K)
    x = (r.standard_normal((1, K)) * 3).astype(F32)
    x[0, : min(K, 6)] = [127.0, 2.5, -3.5, 0.5, 126.5, -40.0][: min(K, 6)]
    if xdt == "bf16":
        x = C.bf16_to_f32(C.bf16_bits(x))
        xd = bf16_dev(x)
    elif xdt == "f16":
        x = x.astype(np.float16).astype(F32)
        xd = to_dev(x.astype(np.float16))
    else:
        xd = to_dev(x)
    W8 = r.integers(-127, 128, (N, K), dtype=np.int8)
    ws = r.uniform(1e-3, 1e-2, N).astype(F32)
    bias = (r.standard_normal(N) * 0.1).astype(F32)
    q, asc = C.rowquant(x)
    acc = C.int_mm(q, W8.T)
    Wd, wsd, bd = to_dev(W8), to_dev(ws), to_dev(bias)
    for order, b in ((L.EPI_V21, None), (L.EPI_V21, bias), (L.EPI_V2, bias)):
        for odt, name in ((L.LSK_BF16, "bf16"), (L.LSK_F32, "f32")):
            y = ops.w8a8_matmul(xd, Wd, wsd, None if b is None else bd, order, odt)
            f = C.epilogue_v21 if order == L.EPI_V21 else C.epilogue_v2
            ref = f(acc, ws, asc, b, name)
            want = ref if name == "bf16" else f32_bits(ref)
            assert np.array_equal(bits(y), want), (order, b is not None, name)
            L.call("lsk_gemm_fuse_rowquant", 0)
            try:
                y2 = ops.w8a8_matmul(xd, Wd, wsd, None if b is None else bd, order, odt)
            finally:
                L.call("lsk_gemm_fuse_rowquant", 1)
            assert torch.equal(y.view(torch.int16) if name == "bf16" else y.view(torch.int32),
                               y2.view(torch.int16) if name == "bf16" else y2.view(torch.int32))
    # rows per wave 1, 2, 4, 8 (the whole-row GEMV's tuning control also sets the fused kernel's)
    for tile in (8, 9, 10, 11):
        L.call("lsk_gemm_select", tile)
        try:
            y = ops.w8a8_matmul(xd, Wd, wsd, bd, L.EPI_V21, L.LSK_BF16)
        finally:
            L.call("lsk_gemm_select", -1)
        assert np.array_equal(bits(y), C.epilogue_v21(acc, ws, asc, bias, "bf16")), tile


def test_mfma_bf16_acc_probe_exact_cases():
    """lsk_mfma_bf16_acc_probe (one v_mfma_f32_16x16x32_bf16 per case, D = A B^T + C) on cases whose
    every partial sum is an integer below 2^24, so any order of additions and roundings gives the
    exact value: the operand layout (a rows are M, b rows are N, K contiguous) and D's layout (row
    M, column N) against a float64 matmul, with C = 0 and with integer C."""
    from lockstep_amd import _lib as L
    g = np.random.default_rng(5)
    n = 64
    a = g.integers(-64, 65, (n, 16, 32)).astype(np.float32)
    b = g.integers(-64, 65, (n, 16, 32)).astype(np.float32)
    c = np.where(np.arange(n)[:, None, None] % 2 == 0, 0.0,
                 g.integers(-2 ** 20, 2 ** 20, (n, 16, 16))).astype(np.float32)
    to_bf = lambda x: torch.from_numpy((x.view(np.uint32) >> 16).astype(np.uint16).view(np.int16)).to(dev())  # noqa: E731
    ad, bd, cd = to_bf(a), to_bf(b), to_dev(c)
    d = torch.full((n, 16, 16), float("nan"), device=dev())
    L.call("lsk_mfma_bf16_acc_probe", L.ptr(ad), L.ptr(bd), L.ptr(cd), L.ptr(d), n, None)
    torch.cuda.synchronize()
    want = (np.einsum("nmk,njk->nmj", a.astype(np.float64), b.astype(np.float64)) + c).astype(np.float32)
    assert np.array_equal(f32_bits(d.cpu().numpy()), f32_bits(want))
