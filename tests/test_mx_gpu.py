"""GPU parity of the MXFP4 path: the MX-operand GEMM (ordered binary32 block updates), the exact
dequant, and the fused MoE layer with MXFP4 experts, against the oracle, bit for bit."""
import numpy as np
import pytest
import torch

from gpu_util import bf16_dev, bits, dev, f32_bits, say, to_dev
from moe_util import routing_device, routing_from_logits, u16
from oracle import contract as C

pytestmark = pytest.mark.gpu
F32 = np.float32
M2_SET = np.array([0, 1, 2, 3, 4, 6, 8, 12, -1, -2, -3, -4, -6, -8, -12], np.int8)


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _tab():
    from lockstep_amd import contract_common as CC
    return CC.table_on(dev())


def _pack(m2):
    """m2 int8 [..., K] -> packed codes (the oracle's inverse of mx_to_m2)."""
    a = np.abs(m2.astype(np.int64))
    mag = np.select([a == 0, a == 1, a == 2, a == 3, a == 4, a == 6, a == 8, a == 12], list(range(8)), -1)
    assert (mag >= 0).all()
    codes = (mag | np.where(m2 < 0, 8, 0)).astype(np.uint8)
    return (codes[..., 0::2] | (codes[..., 1::2] << 4)).astype(np.uint8)


@pytest.mark.parametrize("M,N,K", [(1, 16, 32), (3, 256, 64), (17, 100, 2880), (64, 520, 128), (130, 130, 320)])
@pytest.mark.parametrize("fmt", [0, 1])
def test_int_mm_mx_parity(M, N, K, fmt):
    from lockstep_amd import moe_ref as MR
    from lockstep_amd import ops
    say("int_mm_mx", M, N, K, fmt)
    r = np.random.default_rng(M * 7 + N + K + fmt)
    a = r.integers(-127, 128, (M, K), dtype=np.int8)
    m2 = r.choice(M2_SET, (N, K))
    kexp = r.integers(100, 150, (N, K // 32), dtype=np.uint8)
    ref = C.int_mm_mx(a, m2, kexp)
    if fmt == 0:
        acc = MR.int_mm_mx(to_dev(a), to_dev(m2), to_dev(kexp))
    else:
        acc = ops.gemm_mx(to_dev(a), to_dev(_pack(m2)), to_dev(kexp), 1)
    assert np.array_equal(bits(acc), f32_bits(ref))
    asc = r.uniform(1e-3, 1e-1, M).astype(F32)
    bias = (r.standard_normal(N) * 0.1).astype(F32)
    y = MR.lin_epilogue_mx(acc, to_dev(asc), to_dev(bias))
    assert np.array_equal(bits(y), f32_bits(C.lin_epilogue_mx(ref, asc, bias)))
    y2 = ops.gemm_mx(to_dev(a), to_dev(m2), to_dev(kexp), 0, asc=to_dev(asc), bias=to_dev(bias), epilogue=1)
    assert np.array_equal(bits(y2), f32_bits(C.lin_epilogue_mx(ref, asc, bias)))


def test_int_mm_mx_extreme_exponents():
    """Exponent bytes across the whole range: subnormal block scales (0, 1), ordinary ones, and
    bytes >= 240 whose products overflow to infinity exactly as the reference's."""
    from lockstep_amd import moe_ref as MR
    r = np.random.default_rng(5)
    M, N, K = 9, 40, 32 * 12
    a = r.integers(-127, 128, (M, K), dtype=np.int8)
    m2 = r.choice(M2_SET, (N, K))
    kexp = r.integers(0, 256, (N, K // 32), dtype=np.uint8)
    kexp[:, 0] = 0
    kexp[:, 1] = 1
    kexp[0, :] = 250
    with np.errstate(over="ignore", invalid="ignore"):
        ref = C.int_mm_mx(a, m2, kexp)
    acc = MR.int_mm_mx(to_dev(a), to_dev(m2), to_dev(kexp))
    got = bits(acc)
    refb = f32_bits(ref)
    nan_g = np.isnan(acc.cpu().numpy())
    assert np.array_equal(nan_g, np.isnan(ref))
    assert np.array_equal(got[~nan_g], refb[~nan_g])


def test_int_mm_mx_block_order_is_ascending():
    """The crafted negative control of the oracle: 2^24 + 1 - 2^24 in block order gives 0."""
    from lockstep_amd import moe_ref as MR
    a = np.zeros((1, 96), np.int8)
    a[0, [0, 32, 64]] = 1
    m2 = np.zeros((1, 96), np.int8)
    m2[0, 0], m2[0, 32], m2[0, 64] = 1, 1, -1
    kk = np.array([[152, 128, 152]], np.uint8)
    acc = MR.int_mm_mx(to_dev(a), to_dev(m2), to_dev(kk))
    assert float(acc.cpu()[0, 0]) == 0.0


def test_dequant_mxfp4_all_codes_and_exponents():
    from lockstep_amd import moe_mxfp4 as MX
    codes = np.tile(np.arange(16, dtype=np.uint8), 256 * 2)            # [8192]
    packed = (codes[0::2] | (codes[1::2] << 4)).astype(np.uint8).reshape(256, 16)
    scale = np.arange(256, dtype=np.uint8).reshape(256, 1)             # one block of 32 per row
    with np.errstate(over="ignore", invalid="ignore"):
        ref_bf = C.dequant_mxfp4(packed, scale)
        ref_f = C.dequant_mxfp4(packed, scale, out="f32")
    y = MX.dequant_mxfp4(to_dev(packed), to_dev(scale))
    assert np.array_equal(u16(y), ref_bf)
    yf = MX.dequant_mxfp4(to_dev(packed), to_dev(scale), out_dtype=torch.float32)
    got = yf.cpu().numpy()
    assert np.array_equal(np.isnan(got), np.isnan(ref_f))
    ok = ~np.isnan(got)
    assert np.array_equal(got.view(np.uint32)[ok], ref_f.view(np.uint32)[ok])
    vals = MX.fp4_values(to_dev(np.arange(16, dtype=np.uint8)))
    assert np.array_equal(bits(vals), f32_bits(C.fp4_values(np.arange(16))))
    assert MX.self_test(dev())


def _mx_case(T, E, k, H, I, seed, bias=False, act="silu", from_m2=True):
    from lockstep_amd import moe_ref as MR
    from lockstep_amd import workloads as WL
    say("mx moe case", dict(T=T, E=E, k=k, H=H, I=I, seed=seed, bias=bias, act=act, from_m2=from_m2))
    x, experts, logits = WL.moe_mx_inputs(T, E, k, H, I, seed=seed, bias=bias)
    idx, w = routing_from_logits(logits, k)
    oexp = []
    dexp = []
    for (p13, s13, p2, s2, b13, b2) in experts:
        m13, _ = C.mx_to_m2(p13, s13)
        m2_, _ = C.mx_to_m2(p2, s2)
        oexp.append(((m13, s13), (m2_, s2), b13, b2))
        d13 = to_dev(m13) if from_m2 else to_dev(p13)
        d2 = to_dev(m2_) if from_m2 else to_dev(p2)
        dexp.append(((d13, to_dev(s13)), (d2, to_dev(s2)), None if b13 is None else to_dev(b13),
                     None if b2 is None else to_dev(b2)))
    if not from_m2:
        dexp = MR.ExpertTablesMX(dexp, packed=True)
    oact = C.act_silu if act == "silu" else C.act_swigluoai
    dact = MR.act_silu if act == "silu" else MR.act_swigluoai
    ridx, rw = routing_device(idx, w)
    y, _, _ = MR.moe_forward_mx(bf16_dev(x), None, dexp, k, True, _tab(), 0, dact, routing=(ridx, rw))
    return x, oexp, idx, w, oact, u16(y)


def test_moe_mx_small():
    x, oexp, idx, w, oact, got = _mx_case(24, 8, 2, 256, 128, seed=1)
    assert np.array_equal(got, C.moe_forward_mx(x, oexp, idx, w, oact))


@pytest.mark.parametrize("T", [5, 300])
def test_moe_mx_step_by_step_activation(T):
    """Without the activation table (the skinny grouped GEMM at T = 5, tiles at T = 300) the same
    bits."""
    from lockstep_amd import moe_ref as MR
    MR.USE_ACT_TABLE = False
    try:
        x, oexp, idx, w, oact, got = _mx_case(T, 6, 2, 320, 192, seed=17, bias=True, act="swigluoai")
    finally:
        MR.USE_ACT_TABLE = True
    assert np.array_equal(got, C.moe_forward_mx(x, oexp, idx, w, oact))


def test_moe_mx_bias_swigluoai_packed_tables():
    x, oexp, idx, w, oact, got = _mx_case(40, 6, 3, 320, 192, seed=2, bias=True, act="swigluoai", from_m2=False)
    assert np.array_equal(got, C.moe_forward_mx(x, oexp, idx, w, oact))


def test_expert_block_mx_composed():
    from lockstep_amd import moe_ref as MR
    from lockstep_amd import workloads as WL
    x, experts, _ = WL.moe_mx_inputs(13, 1, 1, 256, 160, seed=3, bias=True)
    p13, s13, p2, s2, b13, b2 = experts[0]
    m13, _ = C.mx_to_m2(p13, s13)
    m2_, _ = C.mx_to_m2(p2, s2)
    y = MR.expert_block_mx(bf16_dev(x), (to_dev(m13), to_dev(s13)), (to_dev(m2_), to_dev(s2)), MR.act_swigluoai,
                           to_dev(b13), to_dev(b2))
    ref = C.expert_block_mx(x, (m13, s13), (m2_, s2), C.act_swigluoai, b13, b2)
    assert np.array_equal(bits(y), f32_bits(ref))


@pytest.mark.parametrize("T", [1, 32])
def test_config5_gpt_oss_full(T):
    from lockstep_amd import workloads as WL
    c = WL.GPT_OSS_20B
    x, oexp, idx, w, oact, got = _mx_case(T, c["E"], c["k"], c["H"], c["I"], seed=50 + T, act="swigluoai",
                                          from_m2=False)
    assert np.array_equal(got, C.moe_forward_mx(x, oexp, idx, w, oact))


def test_config5_t4096_token_subset():
    from lockstep_amd import workloads as WL
    c = WL.GPT_OSS_20B
    x, oexp, idx, w, oact, got = _mx_case(4096, c["E"], c["k"], c["H"], c["I"], seed=54, act="swigluoai",
                                          from_m2=False)
    rows = np.sort(np.random.default_rng(2).choice(4096, 128, replace=False))
    ref = C.moe_forward_mx(x[rows], oexp, idx[rows], w[rows], oact)
    assert np.array_equal(got[rows], ref)


def _skinny_layout(codes, K):
    """The skinny-layout copy of codes [rows, K/2] as lsk_mx_skinny_pack documents it, in numpy:
    per group of 16 rows, step of 4 blocks and row of the group, the 4 blocks' 16 code bytes in
    4-byte pieces ordered (k-quarter, block)."""
    rows = codes.shape[0]
    nb = K // 32
    G, nst = (rows + 15) // 16, (nb + 3) // 4
    c = np.zeros((G * 16, nst * 4, 16), np.uint8)
    c[:rows, :nb] = codes[:, :K // 2].reshape(rows, nb, 16)
    # [G, 16 rows, nst, 4 blocks, 4 quarters, 4 bytes] -> [G, nst, 16 rows, 4 quarters, 4 blocks, 4 bytes]
    c = c.reshape(G, 16, nst, 4, 4, 4).transpose(0, 2, 1, 4, 3, 5)
    return c.reshape(-1)


@pytest.mark.parametrize("rows,K,ldw", [(16, 128, 64), (37, 2880, 1440), (5, 96, 64), (64, 4096, 2048)])
def test_mx_skinny_pack(rows, K, ldw):
    """lsk_mx_skinny_pack against the layout restated in numpy: partial groups of 16 rows, partial
    steps of 4 blocks, a row stride above K/2; lsk_mx_skinny_bytes its size."""
    from lockstep_amd import _lib as L
    say("mx skinny pack", rows, K, ldw)
    rng = np.random.default_rng(rows * 7 + K)
    codes = rng.integers(0, 256, size=(rows, ldw), dtype=np.uint8)
    nbytes = L.load().lsk_mx_skinny_bytes(rows, K)
    exp = _skinny_layout(codes, K)
    assert nbytes == exp.size
    dc = torch.from_numpy(codes).cuda()
    out = torch.full((nbytes,), 0xA5, dtype=torch.uint8, device="cuda")
    L.call("lsk_mx_skinny_pack", dc.data_ptr(), ldw, rows, K, out.data_ptr(),
           torch.cuda.current_stream().cuda_stream)
    assert np.array_equal(out.cpu().numpy(), exp)


@pytest.mark.parametrize("T,E,k,H,I,big_exp,small_exp", [(32, 32, 4, 2880, 2880, False, False),
                                                         (100, 16, 2, 1088, 576, False, True),
                                                         (25, 8, 3, 2048, 3040, False, False),
                                                         (40, 8, 2, 1088, 576, True, True),
                                                         (1, 32, 4, 2880, 2880, False, False),
                                                         (2, 8, 2, 1088, 576, True, False),
                                                         (6, 16, 3, 2048, 3040, False, True),
                                                         (12, 4, 2, 1088, 576, False, False)])
def test_moe_mx_skinny(T, E, k, H, I, big_exp, small_exp):
    """The skinny grouped MX GEMM on the experts' skinny-layout code copies, taken by size from 2
    tokens (GPT-OSS-20B at 32 tokens; 16-row chunks, up to several per expert; whole and partial steps of 4 blocks; a bias; K up to 3040; exponent bytes
    >= 240, the multiply-then-add update), against the oracle and the tiled path
    (lsk_moe_select(0))."""
    from lockstep_amd import _lib as L
    from lockstep_amd import moe_ref as MR
    from lockstep_amd import workloads as WL
    say("mx skinny", dict(T=T, E=E, k=k, H=H, I=I, big_exp=big_exp, small_exp=small_exp))
    x, experts, logits = WL.moe_mx_inputs(T, E, k, H, I, seed=80 + T, bias=True)
    if big_exp:
        p13, s13, p2, s2, b13, b2 = experts[1]
        s2 = s2.copy()
        s2[::5, 2] = 241
        s2[::9, 7] = 250
        experts[1] = (p13, s13, p2, s2, b13, b2)
    if small_exp:
        # block scales 2^-128 and 2^-127 (binary32 subnormals) in every expert's gate/up and down
        for e in range(E):
            p13, s13, p2, s2, b13, b2 = experts[e]
            s13, s2 = s13.copy(), s2.copy()
            s13[::3, 1] = 0
            s13[1::4, 4] = 1
            s2[::5, 0] = 1
            s2[2::7, 3] = 0
            experts[e] = (p13, s13, p2, s2, b13, b2)
    idx, w = routing_from_logits(logits, k)
    oexp, dexp = [], []
    for (p13, s13, p2, s2, b13, b2) in experts:
        m13, _ = C.mx_to_m2(p13, s13)
        m2_, _ = C.mx_to_m2(p2, s2)
        oexp.append(((m13, s13), (m2_, s2), b13, b2))
        dexp.append(((to_dev(p13), to_dev(s13)), (to_dev(p2), to_dev(s2)), to_dev(b13), to_dev(b2)))
    dexp = MR.ExpertTablesMX(dexp, packed=True)
    mxv = 3 if T == 1 else 0            # one token takes the MX GEMV unless the skinny form is chosen
    assert L.load().lsk_moe_mx_reads_skinny(T, k, E, H, I, dexp.lds13, dexp.lds2, 0, mxv + 1) == 1
    assert L.load().lsk_moe_mx_reads_skinny(T, k, E, H, I, dexp.lds13, dexp.lds2, 2, 0) == 0
    assert dexp.mx_safe == (1 if big_exp else 0)
    ridx, rw = routing_device(idx, w)
    with MR.kernel_choice(mx=mxv):
        y, _, _ = MR.moe_forward_mx(bf16_dev(x), None, dexp, k, True, _tab(), 0, MR.act_swigluoai,
                                    routing=(ridx, rw))
    assert all(t is not None for t in dexp._skinny)  # the call made and read the copies
    L.call("lsk_moe_select", 0)
    try:
        yt, _, _ = MR.moe_forward_mx(bf16_dev(x), None, dexp, k, True, _tab(), 0, MR.act_swigluoai,
                                     routing=(ridx, rw))
    finally:
        L.call("lsk_moe_select", -1)
    with np.errstate(over="ignore", invalid="ignore"):
        ref = C.moe_forward_mx(x, oexp, idx, w, C.act_swigluoai)
    assert np.array_equal(u16(y), ref)
    assert np.array_equal(u16(yt), ref)


@pytest.mark.parametrize("E,k,H,I,big_exp,bad_slot", [(32, 4, 2880, 2880, False, False), (8, 3, 1088, 576, True, True),
                                                     (6, 2, 320, 192, False, True), (16, 4, 2048, 4160, True, False)])
def test_moe_mx_one_token_down_combine(E, k, H, I, big_exp, bad_slot):
    """One token of MXFP4 experts (k <= 4): the down GEMV of every slot and the ordered combine in
    one launch (a wave per slot, the slots added in ascending expert order), against the oracle and
    the slot-row path (lsk_moe_mx_select(3)): biases, the multiply-then-add update (exponent bytes
    >= 240), one-, two- and four-chunk K (I = 192, 576 / 2880, 4160), and a slot whose expert index
    is outside [0, E) (skipped, as the reference's loop over range(E) skips it)."""
    from lockstep_amd import moe_ref as MR
    from lockstep_amd import workloads as WL
    say("mx one token down + combine", dict(E=E, k=k, H=H, I=I, big_exp=big_exp, bad_slot=bad_slot))
    x, experts, logits = WL.moe_mx_inputs(1, E, k, H, I, seed=140 + E + k, bias=True)
    if big_exp:
        for e in range(E):
            p13, s13, p2, s2, b13, b2 = experts[e]
            s2 = s2.copy()
            s2[::5, 1] = 242
            experts[e] = (p13, s13, p2, s2, b13, b2)
    idx, w = routing_from_logits(logits, k)
    if bad_slot:
        idx = idx.copy()
        idx[0, 1] = E
    oexp, dexp = [], []
    for (p13, s13, p2, s2, b13, b2) in experts:
        m13, _ = C.mx_to_m2(p13, s13)
        m2_, _ = C.mx_to_m2(p2, s2)
        oexp.append(((m13, s13), (m2_, s2), b13, b2))
        dexp.append(((to_dev(p13), to_dev(s13)), (to_dev(p2), to_dev(s2)), to_dev(b13), to_dev(b2)))
    dexp = MR.ExpertTablesMX(dexp, packed=True)
    ridx, rw = routing_device(idx, w)
    y, _, _ = MR.moe_forward_mx(bf16_dev(x), None, dexp, k, True, _tab(), 0, MR.act_swigluoai, routing=(ridx, rw))
    with MR.kernel_choice(mx=3):
        y3, _, _ = MR.moe_forward_mx(bf16_dev(x), None, dexp, k, True, _tab(), 0, MR.act_swigluoai,
                                     routing=(ridx, rw))
    with np.errstate(over="ignore", invalid="ignore"):
        ref = C.moe_forward_mx(x, oexp, idx, w, C.act_swigluoai)
    assert np.array_equal(u16(y), ref)
    assert np.array_equal(u16(y3), ref)


@pytest.mark.parametrize("variant", [0, 2])
@pytest.mark.parametrize("big_exp", [False, True])
def test_moe_mx_tiles_and_gemv(variant, big_exp):
    """The MX layer on the tiled grouped GEMM (0) and on the decode GEMV (2), against the oracle:
    up to 12 rows per expert (the GEMV's row chunks), a bias, and optionally exponent bytes >= 240
    in some blocks of one expert's down projection (the separate multiply-then-add update; the
    overflowing products give infinities, and their sums in the combine NaNs, compared as bf16
    bits).  The gate/up stage stays finite: a NaN reaching the int8 requant has no defined
    int8 value in the reference's torch casts."""
    from lockstep_amd import _lib as L
    from lockstep_amd import moe_ref as MR
    from lockstep_amd import workloads as WL
    T, E, k, H, I = 12, 3, 2, 2112, 352
    say("mx tiles / gemv", variant, big_exp)
    x, experts, logits = WL.moe_mx_inputs(T, E, k, H, I, seed=61, bias=True)
    if big_exp:
        p13, s13, p2, s2, b13, b2 = experts[1]
        s2 = s2.copy()
        s2[::5, 2] = 241
        s2[::9, 7] = 250
        experts[1] = (p13, s13, p2, s2, b13, b2)
    idx, w = routing_from_logits(logits, k)
    oexp = []
    dexp = []
    for (p13, s13, p2, s2, b13, b2) in experts:
        m13, _ = C.mx_to_m2(p13, s13)
        m2_, _ = C.mx_to_m2(p2, s2)
        oexp.append(((m13, s13), (m2_, s2), b13, b2))
        dexp.append(((to_dev(p13), to_dev(s13)), (to_dev(p2), to_dev(s2)), to_dev(b13), to_dev(b2)))
    dexp = MR.ExpertTablesMX(dexp, packed=True)
    ridx, rw = routing_device(idx, w)
    L.call("lsk_moe_select", variant)
    try:
        y, _, _ = MR.moe_forward_mx(bf16_dev(x), None, dexp, k, True, _tab(), 0, MR.act_swigluoai,
                                    routing=(ridx, rw))
    finally:
        L.call("lsk_moe_select", -1)
    with np.errstate(over="ignore", invalid="ignore"):
        ref = C.moe_forward_mx(x, oexp, idx, w, C.act_swigluoai)
    assert np.array_equal(u16(y), ref)


@pytest.mark.parametrize("mxv", [0, 1, 2, 3])
@pytest.mark.parametrize("big_exp", [False, True])
def test_moe_mx_grouped_main_loops(mxv, big_exp):
    """Every main loop of the grouped MX GEMM (0 / 2: direct-to-LDS with a two / three-stage ring,
    1: register-staged; 3 past the skinny GEMM's 256 tokens: loop 0) on the tiled path against the
    oracle: several 128-row tiles per expert, a half 64-wide K stage in both
    projections (H = 352, I = 224), partial column tiles, biases, and optionally exponent bytes
    >= 240 (the multiply-then-add update)."""
    from lockstep_amd import _lib as L
    from lockstep_amd import moe_ref as MR
    from lockstep_amd import workloads as WL
    T, E, k, H, I = 600, 4, 2, 352, 224
    say("mx grouped main loop", mxv, big_exp)
    x, experts, logits = WL.moe_mx_inputs(T, E, k, H, I, seed=71, bias=True)
    if big_exp:
        p13, s13, p2, s2, b13, b2 = experts[2]
        s2 = s2.copy()
        s2[::7, 3] = 244
        experts[2] = (p13, s13, p2, s2, b13, b2)
    idx, w = routing_from_logits(logits, k)
    oexp, dexp = [], []
    for (p13, s13, p2, s2, b13, b2) in experts:
        m13, _ = C.mx_to_m2(p13, s13)
        m2_, _ = C.mx_to_m2(p2, s2)
        oexp.append(((m13, s13), (m2_, s2), b13, b2))
        dexp.append(((to_dev(p13), to_dev(s13)), (to_dev(p2), to_dev(s2)), to_dev(b13), to_dev(b2)))
    dexp = MR.ExpertTablesMX(dexp, packed=True)
    ridx, rw = routing_device(idx, w)
    L.call("lsk_moe_select", 0)
    L.call("lsk_moe_mx_select", mxv)
    try:
        y, _, _ = MR.moe_forward_mx(bf16_dev(x), None, dexp, k, True, _tab(), 0, MR.act_swigluoai,
                                    routing=(ridx, rw))
    finally:
        L.call("lsk_moe_select", -1)
        L.call("lsk_moe_mx_select", 0)
    with np.errstate(over="ignore", invalid="ignore"):
        ref = C.moe_forward_mx(x, oexp, idx, w, C.act_swigluoai)
    assert np.array_equal(u16(y), ref)
