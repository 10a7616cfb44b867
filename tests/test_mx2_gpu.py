"""GPU parity of the block-scaled activation path (moe_ref.blockquant / int_mm_mx2 /
expert_block_mx2 / moe_forward_mx2): block quant, the MX operand with per-row block exponents,
and the fused MoE layer, against the oracle, bit for bit.  The layer cases include rows whose
block exponents fall outside the window where the fused update on dequantised values is exact,
so that both grouped kernels (the fused one and the general per-row-exponent one) run, on tiles
that mix both kinds of row."""
import numpy as np
import pytest
import torch

from gpu_util import bf16_dev, bits, dev, f32_bits, say, to_dev
from moe_util import routing_device, routing_from_logits, u16
from oracle import contract as C
from test_oracle_mx2 import adversarial_maxima, blocks_with_maxima

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


def _bf16_vals(a):
    return C.bf16_to_f32(C.bf16_bits(a))


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_blockquant_adversarial_maxima(dtype):
    from lockstep_amd import moe_ref as MR
    say("blockquant adversarial", dtype)
    am = adversarial_maxima()
    x = blocks_with_maxima(am)
    n = x.shape[0] // 8 * 8
    x = x[:n].reshape(n // 8, 8 * 32)        # 8 blocks per row
    if dtype == "bf16":
        x = _bf16_vals(x)
        xd = bf16_dev(x)
    else:
        xd = to_dev(x)
    q, ka = MR.blockquant(xd)
    rq, rka = C.blockquant(x)
    assert np.array_equal(bits(ka), rka)
    assert np.array_equal(bits(q), rq)


@pytest.mark.parametrize("T,K", [(1, 32), (7, 2880), (33, 96), (300, 768)])
def test_blockquant_random(T, K):
    from lockstep_amd import moe_ref as MR
    say("blockquant", T, K)
    r = np.random.default_rng(T + K)
    x = (r.standard_normal((T, K)) * np.exp2(r.integers(-40, 40, (T, 1)))).astype(F32)
    x[0, :32] = 0.0                       # an all-zero block
    if T > 2:
        x[2, 32:64] = np.inf if K > 32 else x[2, 32:64]
    for vals, d in ((x, to_dev(x)), (_bf16_vals(x), bf16_dev(_bf16_vals(x)))):
        q, ka = MR.blockquant(d)
        rq, rka = C.blockquant(vals)
        assert np.array_equal(bits(ka), rka)
        assert np.array_equal(bits(q), rq)


def _pack(m2):
    a = np.abs(m2.astype(np.int64))
    mag = np.select([a == 0, a == 1, a == 2, a == 3, a == 4, a == 6, a == 8, a == 12], list(range(8)), -1)
    codes = (mag | np.where(m2 < 0, 8, 0)).astype(np.uint8)
    return (codes[..., 0::2] | (codes[..., 1::2] << 4)).astype(np.uint8)


@pytest.mark.parametrize("M,N,K", [(1, 16, 32), (3, 256, 64), (17, 100, 2880), (130, 130, 320)])
@pytest.mark.parametrize("fmt", [0, 1])
def test_int_mm_mx2_parity(M, N, K, fmt):
    from lockstep_amd import moe_ref as MR
    from lockstep_amd import ops
    say("int_mm_mx2", M, N, K, fmt)
    r = np.random.default_rng(M * 5 + N + K + fmt)
    x = (r.standard_normal((M, K)) * np.exp2(r.integers(-30, 30, (M, K // 32))).repeat(32, axis=1)).astype(F32)
    q, ka = C.blockquant(x)
    m2 = r.choice(M2_SET, (N, K))
    kexp = r.integers(100, 150, (N, K // 32), dtype=np.uint8)
    ref = C.int_mm_mx2(q, ka, m2, kexp)
    b = to_dev(m2) if fmt == 0 else to_dev(_pack(m2))
    acc = ops.gemm_mx2(to_dev(q), to_dev(ka), b, to_dev(kexp), fmt)
    assert np.array_equal(bits(acc), f32_bits(ref))
    if fmt == 0:
        assert np.array_equal(bits(MR.int_mm_mx2(to_dev(q), to_dev(ka), to_dev(m2), to_dev(kexp))), f32_bits(ref))
    bias = (r.standard_normal(N) * 0.1).astype(F32)
    y = ops.gemm_mx2(to_dev(q), to_dev(ka), b, to_dev(kexp), fmt, bias=to_dev(bias), epilogue=1)
    want = C.bfr((C.bfr(ref) + bias[None, :]).astype(F32))
    assert np.array_equal(bits(y), f32_bits(want))


def test_int_mm_mx2_extreme_exponents():
    """Row exponents over [-126, 127] against weight bytes over [0, 255]: products whose
    2^(ka + kexp - 128) underflows to 0, is subnormal, or overflows to infinity, and the NaNs of
    0 * inf, exactly as the reference's."""
    from lockstep_amd import ops
    r = np.random.default_rng(9)
    M, N, K = 12, 48, 32 * 10
    q = r.integers(-127, 128, (M, K), dtype=np.int8)
    q[3, :64] = 0
    ka = r.integers(-126, 128, (M, K // 32)).astype(np.int32)
    ka[0, :] = -126
    ka[1, :] = 127
    m2 = r.choice(M2_SET, (N, K))
    kexp = r.integers(0, 256, (N, K // 32), dtype=np.uint8)
    kexp[:, 0] = 0
    kexp[:, 1] = 255
    kexp[5, :] = 104
    with np.errstate(over="ignore", invalid="ignore"):
        ref = C.int_mm_mx2(q, ka, m2, kexp)
    acc = ops.gemm_mx2(to_dev(q), to_dev(ka), to_dev(m2), to_dev(kexp), 0)
    got = acc.cpu().numpy()
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(got[ok].view(np.uint32), ref[ok].view(np.uint32))


def test_expert_block_mx2_composed():
    from lockstep_amd import moe_ref as MR
    from lockstep_amd import workloads as WL
    x, experts, _ = WL.moe_mx_inputs(13, 1, 1, 256, 160, seed=3, bias=True)
    p13, s13, p2, s2, b13, b2 = experts[0]
    m13, _ = C.mx_to_m2(p13, s13)
    m2_, _ = C.mx_to_m2(p2, s2)
    y = MR.expert_block_mx2(bf16_dev(x), (to_dev(m13), to_dev(s13)), (to_dev(m2_), to_dev(s2)), MR.act_swigluoai,
                            to_dev(b13), to_dev(b2))
    ref = C.expert_block_mx2(x, (m13, s13), (m2_, s2), C.act_swigluoai, b13, b2)
    assert np.array_equal(bits(y), f32_bits(ref))


def _mx2_layer(T, E, k, H, I, seed, tiny_rows=0.0, low_exp=False, big_exp=False, bias=True, act="swigluoai",
               mxv=0, moe_force=-1):
    """The layer on device vs the oracle.  tiny_rows: fraction of tokens scaled by 2^-40 (block
    exponents far below the fused window when low_exp puts E8M0 bytes <= 10 into one expert's
    w13 and w2); big_exp: bytes >= 240 in one expert's w2 (the multiply-then-add update and a
    narrower window at the top).  moe_force: lsk_moe_select's variant (0 keeps decode-sized
    layers on the tiled kernels instead of the GEMV)."""
    from lockstep_amd import _lib as L
    from lockstep_amd import moe_ref as MR
    from lockstep_amd import workloads as WL
    say("mx2 layer", dict(T=T, E=E, k=k, H=H, I=I, seed=seed, tiny=tiny_rows, low=low_exp, big=big_exp, mxv=mxv))
    x, experts, logits = WL.moe_mx_inputs(T, E, k, H, I, seed=seed, bias=bias)
    r = np.random.default_rng(seed)
    if tiny_rows:
        rows = r.random(T) < tiny_rows
        x[rows] = (x[rows] * F32(2.0 ** -40)).astype(F32)
    if low_exp:
        p13, s13, p2, s2, b13, b2 = experts[0]
        s13, s2 = s13.copy(), s2.copy()
        s13[::3, 1] = 3
        s2[::4, 2] = 7
        experts[0] = (p13, s13, p2, s2, b13, b2)
    if big_exp:
        p13, s13, p2, s2, b13, b2 = experts[-1]
        s2 = s2.copy()
        s2[::7, 3] = 243
        experts[-1] = (p13, s13, p2, s2, b13, b2)
    idx, w = routing_from_logits(logits, k)
    oexp, dexp = [], []
    for (p13, s13, p2, s2, b13, b2) in experts:
        m13, _ = C.mx_to_m2(p13, s13)
        m2_, _ = C.mx_to_m2(p2, s2)
        oexp.append(((m13, s13), (m2_, s2), b13, b2))
        dexp.append(((to_dev(p13), to_dev(s13)), (to_dev(p2), to_dev(s2)),
                     None if b13 is None else to_dev(b13), None if b2 is None else to_dev(b2)))
    dexp = MR.ExpertTablesMX(dexp, packed=True)
    ridx, rw = routing_device(idx, w)
    oact = C.act_silu if act == "silu" else C.act_swigluoai
    dact = MR.act_silu if act == "silu" else MR.act_swigluoai
    L.call("lsk_moe_mx_select", mxv)
    L.call("lsk_moe_select", moe_force)
    try:
        y, _, _ = MR.moe_forward_mx2(bf16_dev(x), None, dexp, k, True, _tab(), 0, dact, routing=(ridx, rw))
    finally:
        L.call("lsk_moe_mx_select", 0)
        L.call("lsk_moe_select", -1)
    return x, oexp, idx, w, oact, u16(y), dexp


def _flagged_tokens(x, dexp):
    """tokens whose block exponents leave the fused window of the gate/up projection"""
    lo = -21 - dexp.kw_bounds[0]
    hi = min(111, (255 if dexp.mx_safe else 239) - dexp.kw_bounds[1])
    q, ka = C.blockquant(x)
    am = np.abs(x.reshape(x.shape[0], -1, 32)).max(axis=-1)
    return ((am > 0) & ((ka < lo) | (ka > hi))).any(axis=1)


def test_moe_mx2_small_fused_only():
    x, oexp, idx, w, oact, got, dexp = _mx2_layer(24, 8, 2, 256, 128, seed=1, act="silu", bias=False, moe_force=0)
    assert not _flagged_tokens(x, dexp).any()
    assert np.array_equal(got, C.moe_forward_mx2(x, oexp, idx, w, oact))


@pytest.mark.parametrize("mxv", [0, 1, 2])
@pytest.mark.parametrize("big_exp", [False, True])
def test_moe_mx2_mixed_tiles(mxv, big_exp):
    """Several 128-row tiles per expert, about 4% of tokens flagged: tiles with and without flagged
    rows, so the fused and the general kernels split each projection; a half K stage in both
    projections (H = 352, I = 224) and partial column tiles."""
    x, oexp, idx, w, oact, got, dexp = _mx2_layer(600, 4, 2, 352, 224, seed=71, tiny_rows=0.04, low_exp=True,
                                                  big_exp=big_exp, mxv=mxv)
    fl = _flagged_tokens(x, dexp)
    assert 0 < fl.sum() < 100
    with np.errstate(over="ignore", invalid="ignore"):
        ref = C.moe_forward_mx2(x, oexp, idx, w, oact)
    assert np.array_equal(got, ref)


def test_moe_mx2_every_row_general():
    """All tokens tiny with low weight exponents: every tile takes the general kernel."""
    x, oexp, idx, w, oact, got, dexp = _mx2_layer(150, 3, 2, 256, 160, seed=5, tiny_rows=1.0, low_exp=True)
    assert _flagged_tokens(x, dexp).all()
    assert np.array_equal(got, C.moe_forward_mx2(x, oexp, idx, w, oact))


@pytest.mark.parametrize("T", [1, 32])
@pytest.mark.parametrize("path", ["gemv", "tiled"])
def test_moe_mx2_gpt_oss_shapes(T, path):
    """Decode sizes through the grouped GEMV (forced at T = 32, past the default's 16-token switch)
    and through the tiled kernels.  K = 2880 (90 blocks): the GEMV's two-chunk form."""
    from lockstep_amd import workloads as WL
    c = WL.GPT_OSS_20B
    x, oexp, idx, w, oact, got, dexp = _mx2_layer(T, c["E"], c["k"], c["H"], c["I"], seed=80 + T, bias=True,
                                                  moe_force=2 if path == "gemv" else 0)
    assert np.array_equal(got, C.moe_forward_mx2(x, oexp, idx, w, oact))


@pytest.mark.parametrize("act", ["silu", "swigluoai"])
def test_moe_mx2_gemv_extreme_exponents(act):
    """The decode GEMV (forced at T = 48) on tiny rows (block exponents near -126), E8M0 bytes <= 10
    and >= 240 (products 2^(ka + k - 128) underflowing to subnormals and zero, and large ones), with
    K of 11 / 7 blocks (one-chunk form, four rows per pass)."""
    x, oexp, idx, w, oact, got, dexp = _mx2_layer(48, 4, 2, 352, 224, seed=91, tiny_rows=0.15, low_exp=True,
                                                  big_exp=True, act=act, moe_force=2)
    assert _flagged_tokens(x, dexp).any()
    with np.errstate(over="ignore", invalid="ignore"):
        ref = C.moe_forward_mx2(x, oexp, idx, w, oact)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("T", [2, 8, 16])
@pytest.mark.parametrize("H,I", [(352, 224), (4160, 128)])
def test_moe_mx2_gemv_token_counts(T, H, I):
    """The decode GEMV (forced; by default these token counts take the skinny grouped MX GEMM where
    its LDS allows, the GEMV otherwise) at T <= 16: T = 2 takes two rows
    per pass, T = 8 and 16 four (the per-row block exponents sa[m * kB + b] of every row of a pass).
    H = 352 (11 blocks) keeps the gate/up in the one-chunk form; H = 4160 (130 blocks, above 128)
    takes the four-chunk form with one row per pass, and I = 128 (4 blocks) the down projection's
    one-chunk form.  Tiny rows and extreme E8M0 bytes put the block products 2^(ka + k - 128) near
    both ends of the binary32 range.  (Every MX row count is a multiple of 32, so a GEMV column
    chunk of 8 or 16 columns is always whole.)"""
    x, oexp, idx, w, oact, got, dexp = _mx2_layer(T, 4, 2, H, I, seed=100 + T + H, tiny_rows=0.3, low_exp=True,
                                                  big_exp=True, moe_force=2)
    with np.errstate(over="ignore", invalid="ignore"):
        ref = C.moe_forward_mx2(x, oexp, idx, w, oact)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("T,E,k,H,I,tiny,low,big", [(32, 32, 4, 2880, 2880, 0.0, False, False),
                                                    (1, 32, 4, 2880, 2880, 0.0, False, False),
                                                    (40, 8, 2, 1088, 576, 0.0, False, True),
                                                    (8, 4, 2, 352, 224, 0.3, True, True),
                                                    (60, 6, 2, 352, 224, 0.05, True, False)])
def test_moe_mx2_skinny(T, E, k, H, I, tiny, low, big):
    """Block-scaled layers on the skinny grouped MX GEMM (the default from 2 tokens, and one token
    of GPT-OSS-20B): the dequantised rows through the fused update with no row scale, gate / up
    values through moe_act_h_kernel into h; with a flagged row (tiny rows against low E8M0 bytes)
    the general tile kernel takes every tile of that projection instead; exponent bytes >= 240
    (the multiply-then-add update)."""
    from lockstep_amd import _lib as L
    x, oexp, idx, w, oact, got, dexp = _mx2_layer(T, E, k, H, I, seed=120 + T, tiny_rows=tiny, low_exp=low,
                                                  big_exp=big, bias=True)
    assert L.load().lsk_moe_mx_reads_skinny(T, k, E, H, I, dexp.lds13, dexp.lds2, 0, 0) == 1
    assert all(t is not None for t in dexp._skinny)
    assert bool(_flagged_tokens(x, dexp).any()) == (tiny > 0)
    with np.errstate(over="ignore", invalid="ignore"):
        ref = C.moe_forward_mx2(x, oexp, idx, w, oact)
    assert np.array_equal(got, ref)


def test_moe_mx2_gpt_oss_t4096_token_subset():
    from lockstep_amd import workloads as WL
    c = WL.GPT_OSS_20B
    x, oexp, idx, w, oact, got, dexp = _mx2_layer(4096, c["E"], c["k"], c["H"], c["I"], seed=84, bias=True)
    rows = np.sort(np.random.default_rng(3).choice(4096, 24, replace=False))
    ref = C.moe_forward_mx2(x[rows], oexp, idx[rows], w[rows], oact)
    assert np.array_equal(got[rows], ref)


def test_zero_tokens_through_the_layers():
    """T = 0: the router, block quant, the block-scaled GEMM and the int8 / MXFP4 / MX2 layers return
    empty results of the right shape and dtype (the reference's functions do the same on an
    empty batch)."""
    from lockstep_amd import moe_ref as MR
    from lockstep_amd import workloads as WL
    from moe_util import device_experts
    say("zero tokens")
    E, k, H, I = 8, 2, 256, 128
    g0 = torch.empty((0, E), dtype=torch.bfloat16, device=dev())
    idx0, w0, _ = MR.router_from_logits(g0, k, True, _tab())
    assert idx0.shape == (0, k) and idx0.dtype == torch.int64 and w0.shape == (0, k) and w0.dtype == torch.bfloat16
    x0 = torch.empty((0, H), dtype=torch.bfloat16, device=dev())
    q0, ka0 = MR.blockquant(x0)
    assert q0.shape == (0, H) and ka0.shape == (0, H // 32)
    m2 = to_dev(np.ones((16, H), np.int8))
    kexp = to_dev(np.full((16, H // 32), 127, np.uint8))
    assert MR.int_mm_mx2(q0, ka0, m2, kexp).shape == (0, 16)

    x, experts, logits = WL.moe_inputs(4, E, k, H, I, seed=1)
    idx, w = routing_from_logits(logits, k)
    ridx, rw = routing_device(idx[:0], w[:0])
    y, _, _ = MR.moe_forward_b(x0, None, device_experts(experts), k, True, _tab(), 0, MR.act_silu, rot_blk=0,
                               routing=(ridx, rw))
    assert y.shape == (0, H) and y.dtype == torch.bfloat16

    x, experts, logits = WL.moe_mx_inputs(4, E, k, H, I, seed=1, bias=True)
    dexp = MR.ExpertTablesMX([((to_dev(p13), to_dev(s13)), (to_dev(p2), to_dev(s2)), to_dev(b13), to_dev(b2))
                              for (p13, s13, p2, s2, b13, b2) in experts], packed=True)
    for fwd in (MR.moe_forward_mx, MR.moe_forward_mx2):
        y, _, _ = fwd(x0, None, dexp, k, True, _tab(), 0, MR.act_swigluoai, routing=(ridx, rw))
        assert y.shape == (0, H) and y.dtype == torch.bfloat16
