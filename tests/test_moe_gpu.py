"""GPU parity of the contract v3 MoE path (router, activations, rotation, fused int8 layer)
against the oracle, bit for bit."""
import numpy as np
import pytest
import torch

from gpu_util import bf16_dev, bits, dev, f32_bits, say, to_dev
from moe_util import device_experts, oracle_experts, routing_device, routing_from_logits, u16
from oracle import contract as C
from vector_inputs import load_vectors, silu_r4_inputs

pytestmark = pytest.mark.gpu
F32 = np.float32


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _tab():
    from lockstep_amd import contract_common as CC
    return CC.table_on(dev())


# ------------------------------------------------------------------ elementwise operators
def test_silu_and_r4_digests_on_gpu():
    from lockstep_amd import lockstep_fullstack as FS
    from lockstep_amd import moe_ref as MR
    V = load_vectors()
    gate, up, v = silu_r4_inputs()
    s = FS.silu_contract(to_dev(gate))
    assert C.digest(bits(s).view(F32), "float32") == V["silu"]["sha256"]
    sm = (s * to_dev(up)).to(torch.bfloat16)
    assert C.digest(u16(sm), "bfloat16") == V["silu_mul"]["sha256"]
    am = MR.act_silu(to_dev(gate), to_dev(up)).to(torch.bfloat16)
    assert C.digest(u16(am), "bfloat16") == V["silu_mul"]["sha256"]
    r4 = FS.fwht_blocks(to_dev(v))
    assert C.digest(bits(r4).view(F32), "float32") == V["r4.block256"]["sha256"]


def test_activations_parity_wide_range():
    from lockstep_amd import moe_ref as MR
    r = np.random.default_rng(1)
    x = np.concatenate([r.standard_normal(20000) * 8, np.linspace(-40, 40, 4001),
                        [0.0, -0.0, 1e-39, -1e-39, 1e-30, 30.0, -30.0, 1e30, -1e30]]).astype(F32)
    u = C.bfr(r.standard_normal(x.size).astype(F32) * 5)
    xb = C.bfr(x)
    assert np.array_equal(bits(MR.sigmoid_contract(to_dev(x))), f32_bits(C.sigmoid_contract(x)))
    from lockstep_amd import lockstep_fullstack as FS
    assert np.array_equal(bits(FS.silu_contract(to_dev(x))), f32_bits(C.silu_contract(x)))
    assert np.array_equal(bits(MR.act_silu(to_dev(xb), to_dev(u))), f32_bits(C.act_silu(xb, u)))
    assert np.array_equal(bits(MR.act_swigluoai(to_dev(xb), to_dev(u))), f32_bits(C.act_swigluoai(xb, u)))


@pytest.mark.parametrize("blk", [64, 256])
def test_fwht_parity(blk):
    from lockstep_amd import lockstep_fullstack as FS
    r = np.random.default_rng(blk)
    x = (r.standard_normal((7, 768)) * 3).astype(F32)
    y = FS.fwht_blocks(to_dev(x), blk=blk, scale=1.0 / blk ** 0.5)
    assert np.array_equal(bits(y), f32_bits(C.fwht_blocks(x, blk, 1.0 / blk ** 0.5)))


# ------------------------------------------------------------------ router
@pytest.mark.parametrize("E,k", [(8, 2), (32, 4), (64, 6), (128, 8), (200, 8), (1000, 7)])
@pytest.mark.parametrize("renorm", [True, False])
def test_router_parity(E, k, renorm):
    from lockstep_amd import moe_ref as MR
    r = np.random.default_rng(E * 10 + k)
    T = 257
    g = C.bfr((r.standard_normal((T, E)) * 2).astype(F32))
    g[:40] = C.bfr((r.integers(-6, 6, (40, E)) / 4.0).astype(F32))     # tie-dense rows
    g[40] = 0.0                                                          # all tied
    idx, w, gb = MR.router_from_logits(to_dev(g), k, renorm, _tab())
    ridx, rw, rg = C.router_from_logits(g, k, renorm)
    assert np.array_equal(bits(idx), ridx)
    assert np.array_equal(u16(w), rw)
    assert np.array_equal(u16(gb), rg)
    dg = np.abs(r.standard_normal(5000) * 6).astype(F32)
    assert np.array_equal(bits(MR.table_scores(to_dev(dg), _tab())), C.table_scores(dg))


def test_router_from_hidden_states():
    from lockstep_amd import moe_ref as MR
    r = np.random.default_rng(3)
    T, H, E, k = 40, 256, 16, 4
    x = C.bfr(r.standard_normal((T, H)).astype(F32))
    gw = r.integers(-127, 128, (E, H), dtype=np.int8)
    gws = r.uniform(1e-3, 1e-2, E).astype(F32)
    gb = (r.standard_normal(E) * 0.1).astype(F32)
    idx, w, _ = MR.router(bf16_dev(x), to_dev(gw).t(), to_dev(gws), k, True, _tab())
    ridx, rw, _ = C.router(x, gw.T, gws, k, True)
    assert np.array_equal(bits(idx), ridx) and np.array_equal(u16(w), rw)
    idx, w, _ = MR.router_b(bf16_dev(x), to_dev(gw).t(), to_dev(gws), k, True, _tab(), 0, to_dev(gb))
    ridx, rw, _ = C.router(x, gw.T, gws, k, True, gate_bias=gb)
    assert np.array_equal(bits(idx), ridx) and np.array_equal(u16(w), rw)


# ------------------------------------------------------------------ the fused int8 layer
def _run_case(T, E, k, H, I, seed, bias=False, act="silu", rot_blk=0, zipf=True, shared=False,
              routing_override=None):
    from lockstep_amd import moe_ref as MR
    from lockstep_amd import workloads as WL
    say("moe case", dict(T=T, E=E, k=k, H=H, I=I, seed=seed, bias=bias, act=act, rot_blk=rot_blk))
    x, experts, logits = WL.moe_inputs(T, E, k, H, I, seed=seed, bias=bias, zipf=zipf)
    idx, w = routing_from_logits(logits, k) if routing_override is None else routing_override
    dx = bf16_dev(x)
    dexp = device_experts(experts)
    ridx, rw = routing_device(idx, w)
    oact = C.act_silu if act == "silu" else C.act_swigluoai
    dact = MR.act_silu if act == "silu" else MR.act_swigluoai
    sh_np = None
    if shared:
        sh_np = (np.random.default_rng(seed).standard_normal((T, H)) * 0.3).astype(F32)
    if bias or act != "silu" or rot_blk not in (0, 256):
        y, _, _ = MR.moe_forward_b(dx, None, dexp, k, True, _tab(), 0, dact, rot_blk=rot_blk, routing=(ridx, rw))
        ref = C.moe_forward_b(x, oracle_experts(experts, True), idx, w, oact, rot_blk=rot_blk)
    else:
        sfn = (lambda xx: to_dev(sh_np)) if shared else None
        y, _, _ = MR.moe_forward(dx, None, dexp, k, True, _tab(), 0, dact, shared=sfn, routing=(ridx, rw),
                                 rot=rot_blk == 256)
        ref = C.moe_forward(x, oracle_experts(experts), idx, w, act=oact, rot=rot_blk == 256, shared_out=sh_np)
    got = u16(y)
    assert got.shape == ref.shape
    bad = int((got != ref).sum())
    assert bad == 0, "%d of %d outputs differ" % (bad, got.size)


def test_moe_small():
    _run_case(24, 8, 2, 256, 128, seed=3)


def test_act_tables_over_every_bf16_gate():
    """lsk_act_table against the oracle for every non-NaN bf16 gate pattern (65282 values, both
    infinities included): SiLU's table is silu_contract(g) in binary32; SwiGLU-OAI's is the glu
    factor, which the oracle's act gives at u = 0 (bfr(1 * glu) = glu).  A NaN gate has no value in
    the reference (its table index is the int64 cast of NaN)."""
    from lockstep_amd import _lib as L
    from lockstep_amd import ops
    g = C.bf16_to_f32(np.arange(65536, dtype=np.uint32).astype(np.uint16))
    ok = ~np.isnan(g)
    with np.errstate(all="ignore"):
        want = {L.LSK_ACT_SILU: C.silu_contract(g[ok]),
                L.LSK_ACT_SWIGLUOAI: C.act_swigluoai(g[ok], np.zeros_like(g[ok]))}
    for act, ref in want.items():
        got = ops.act_table(dev(), act).cpu().numpy()[ok]
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), act


@pytest.mark.parametrize("variant", [0, 1, 2])
def test_moe_step_by_step_activation(variant):
    """The layer without the activation table (the epilogues evaluate every step) gives the same
    bits: the int8 kernels and the MXFP4 layer."""
    from lockstep_amd import _lib as L
    from lockstep_amd import moe_ref as MR
    MR.USE_ACT_TABLE = False
    L.call("lsk_moe_select", variant)
    try:
        _run_case(150, 6, 2, 320, 96, seed=14, bias=True, act="swigluoai")
        _run_case(40, 8, 3, 256, 192, seed=16)
    finally:
        MR.USE_ACT_TABLE = True
        L.call("lsk_moe_select", -1)


def test_moe_single_token_and_zero_load_experts():
    _run_case(1, 16, 4, 256, 128, seed=4)


def test_moe_skewed_multi_tile_expert():
    """Every token routed to experts {0, 1}: expert tiles of up to 300 rows (3 M-tiles)."""
    T, E, k = 300, 6, 2
    idx = np.tile(np.array([[1, 0]]), (T, 1)).astype(np.int64)
    w = C.bf16_bits(np.tile(np.array([[0.75, 0.25]], F32), (T, 1)))
    _run_case(T, E, k, 128, 64, seed=5, routing_override=(idx, w))


def test_moe_skipped_experts_out_of_range():
    """Routing entries outside [0, E) are skipped, as the reference's loop over range(E) does."""
    T, E, k = 20, 4, 3
    r = np.random.default_rng(6)
    idx = np.stack([r.permutation(6)[:k] for _ in range(T)]).astype(np.int64)   # some >= E
    w = C.bf16_bits(r.uniform(0, 1, (T, k)).astype(F32))
    _run_case(T, E, k, 128, 64, seed=6, routing_override=(idx, w))


@pytest.mark.parametrize("T,E,k", [(700, 16, 4), (513, 9, 3)])
def test_moe_multi_chunk_dispatch(T, E, k):
    """T > 256: per-chunk counts, the expert scan and per-chunk placement; every output against
    the oracle (Zipf-skewed routing, some experts never chosen)."""
    _run_case(T, E, k, 128, 64, seed=11 + T)


@pytest.mark.parametrize("variant", [0, 1, 2, 3, 4, 5, 6, 7])
def test_moe_grouped_gemm_variants(variant):
    """Every grouped-GEMM kernel (register-staged 128x128 tile, ping-pong 128x256 tile, the
    decode GEMV, the 128x256 tile on four waves, the ping-pong tile with 128-byte K stages, the
    256x256 tile persistent and one tile per block, the skinny grouped GEMM) gives the oracle's
    bits: skewed routing with multi-tile experts (the GEMV takes their rows eight at a time, the
    skinny kernel 32 at a time), empty experts, a bias and SwiGLU-OAI; an odd number of routed rows
    (the down tiles' row-pair operand ends in a half pair)."""
    from lockstep_amd import _lib as L
    L.call("lsk_moe_select", variant)
    try:
        _run_case(300, 12, 4, 256, 192, seed=13)
        _run_case(301, 8, 3, 256, 128, seed=17)
        _run_case(150, 6, 2, 320, 96, seed=14, bias=True, act="swigluoai")
        _run_case(5, 16, 4, 256, 128, seed=15)
        if variant in (1, 5, 6):
            # experts of several 256-row tiles and a partial last one, I not a multiple of 128
            _run_case(1100, 6, 3, 384, 320, seed=18)
            # both projections with K >= 384 (the persistent 256x256 kernel takes both)
            _run_case(1100, 6, 3, 448, 400, seed=19, bias=True, act="swigluoai")
    finally:
        L.call("lsk_moe_select", -1)


@pytest.mark.parametrize("pairs", [True, False])
@pytest.mark.parametrize("T", [2, 3, 9, 16, 17, 40, 64, 96, 200])
def test_moe_skinny_grouped(T, pairs):
    """The skinny grouped GEMM (the default for int8 layers from 2 tokens while the routed rows stay
    under 16 E; chosen here at every size), reading the experts' row-pair copies and their row-major
    weights: Zipf-skewed routing over 16 experts (some empty), H and I not multiples of 64 (partial
    last K steps of both projections), a bias with SwiGLU-OAI, and every token routed to the same
    two experts (up to 200 rows per expert: chunks of 32 rows, a partial last chunk), all against
    the oracle."""
    from lockstep_amd import moe_ref as MR
    prev = MR.ROW_PAIRS
    MR.ROW_PAIRS = pairs
    try:
        with MR.kernel_choice(moe=7):
            _run_case(T, 16, 4, 256, 128, seed=40 + T)
            _run_case(T, 8, 3, 272, 208, seed=50 + T, bias=True, act="swigluoai")
            idx = np.tile(np.array([[3, 1]]), (T, 1)).astype(np.int64)
            w = C.bf16_bits(np.tile(np.array([[0.625, 0.375]], F32), (T, 1)))
            _run_case(T, 4, 2, 320, 192, seed=60 + T, routing_override=(idx, w))
    finally:
        MR.ROW_PAIRS = prev


@pytest.mark.parametrize("variant", [5, 6])
def test_moe_256_tiles(variant):
    """The 256x256 expert tiles (chosen; persistent and one tile per block): Zipf-skewed experts of
    one to several 256-row tiles, with a bias and SwiGLU-OAI, and with the shared expert on."""
    from lockstep_amd import _lib as L
    L.call("lsk_moe_select", variant)
    try:
        _run_case(700, 8, 4, 256, 256, seed=31)
        _run_case(513, 4, 2, 512, 192, seed=32, bias=True, act="swigluoai")
        _run_case(900, 8, 2, 256, 128, seed=33, shared=True)
    finally:
        L.call("lsk_moe_select", -1)


def test_moe_per_call_kernel_choice():
    """lsk_moe_args.select / mx_select choose the kernels of one call (moe_ref.kernel_choice) over
    the thread's lsk_moe_select setting, with the oracle's bits, and leave that setting in place."""
    from lockstep_amd import _lib as L
    from lockstep_amd import moe_ref as MR
    L.call("lsk_moe_select", 2)            # the thread: the decode GEMV
    try:
        for v in (0, 1, 3, 4, 5, 6, 7, -1):
            with MR.kernel_choice(moe=v):
                _run_case(300, 12, 4, 256, 192, seed=13)
        _run_case(40, 8, 3, 256, 192, seed=16)   # the thread's setting again
    finally:
        L.call("lsk_moe_select", -1)


@pytest.mark.parametrize("T", [1, 3, 12])
def test_moe_gemv_wide_k(T):
    """The decode GEMV with K beyond one 1 KB lane sweep and not a multiple of it (H = 2064:
    three sweeps, the last partial; I = 1104: two), at one, up to four and up to eight rows per
    expert at a time."""
    _run_case(T, 8, 3, 2064, 1104, seed=21 + T)


def test_moe_multi_chunk_out_of_range_entries():
    """Routing entries outside [0, E) spread over several 256-token chunks are skipped."""
    T, E, k = 600, 5, 3
    r = np.random.default_rng(12)
    idx = np.stack([r.permutation(8)[:k] for _ in range(T)]).astype(np.int64)   # some >= E
    w = C.bf16_bits(r.uniform(0, 1, (T, k)).astype(F32))
    _run_case(T, E, k, 128, 64, seed=12, routing_override=(idx, w))


def test_moe_bias_swigluoai():
    _run_case(40, 8, 3, 256, 192, seed=7, bias=True, act="swigluoai")


def test_moe_shared_expert():
    _run_case(30, 8, 2, 256, 128, seed=8, shared=True)


@pytest.mark.parametrize("rot_blk", [256, 64])
def test_moe_rotation(rot_blk):
    _run_case(33, 8, 2, 512, 256, seed=9, rot_blk=rot_blk)


def test_expert_swiglu_and_block_composed():
    from lockstep_amd import moe_ref as MR
    from lockstep_amd import workloads as WL
    x, experts, _ = WL.moe_inputs(19, 1, 1, 256, 256, seed=10, bias=True)
    w13, ws13, w2, ws2, b13, b2 = experts[0]
    dx = bf16_dev(x)
    d = device_experts(experts)[0]
    for rot in (False, True):
        y = MR.expert_swiglu(dx, d[0], d[1], d[2], d[3], MR.act_silu, rot=rot)
        ref = C.expert_swiglu(x, w13.T, ws13, w2.T, ws2, act=C.act_silu, rot=rot)
        assert np.array_equal(bits(y), f32_bits(ref))
    y = MR.expert_block(dx, d[0], d[1], d[2], d[3], MR.act_swigluoai, d[4], d[5], rot_blk=64)
    ref = C.expert_block(x, w13.T, ws13, w2.T, ws2, C.act_swigluoai, b13, b2, rot_blk=64)
    assert np.array_equal(bits(y), f32_bits(ref))


# ------------------------------------------------------------------ the Qwen3-30B-A3B shapes (E=128, k=8, H=2048, I=768)
@pytest.mark.parametrize("T", [1, 32])
def test_config4_full_bit_exact(T):
    from lockstep_amd import workloads as WL
    c = WL.QWEN3_30B_A3B
    _run_case(T, c["E"], c["k"], c["H"], c["I"], seed=40 + T)


@pytest.mark.parametrize("variant", [-1, 5])
def test_config4_t4096_token_subset(variant):
    """T=4096 on the device; a seeded subset of tokens against the oracle run on just those
    tokens (a token's output depends only on its own row and routing).  Under the default choice
    and on the persistent 256x256 tiles (about a thousand tiles per projection: every block walks
    several)."""
    from lockstep_amd import moe_ref as MR
    from lockstep_amd import workloads as WL
    c = WL.QWEN3_30B_A3B
    T = 4096
    say("config4 T=4096", dict(variant=variant))
    x, experts, logits = WL.moe_inputs(T, c["E"], c["k"], c["H"], c["I"], seed=44)
    dx = bf16_dev(x)
    dexp = device_experts(experts)
    idx_d, w_d, _ = MR.router_from_logits(to_dev(logits), c["k"], True, _tab())
    idx, w = routing_from_logits(logits, c["k"])
    assert np.array_equal(bits(idx_d), idx) and np.array_equal(u16(w_d), w)
    loads = np.bincount(idx.reshape(-1), minlength=c["E"])
    say("expert loads: max %d, min %d, zero-load experts %d" % (loads.max(), loads.min(), (loads == 0).sum()))
    with MR.kernel_choice(moe=variant):
        y, _, _ = MR.moe_forward(dx, None, dexp, c["k"], True, _tab(), 0, MR.act_silu, routing=(idx_d, w_d))
    rows = np.sort(np.random.default_rng(1).choice(T, 512, replace=False))
    ref = C.moe_forward(x[rows], oracle_experts(experts), idx[rows], w[rows])
    assert np.array_equal(u16(y)[rows], ref)


def test_moe_decode_layers_replayed_from_a_graph():
    """The decode-sized layer (dispatch and row quant of x in one launch, then the GEMVs): layers
    of 1, 12 and 1 tokens in a row, then one layer captured in a HIP graph and replayed, with eager
    layers of another size between the replays; every output against the oracle."""
    from lockstep_amd import moe_ref as MR
    from lockstep_amd import workloads as WL

    def case(T, seed):
        x, experts, logits = WL.moe_inputs(T, 16, 4, 256, 128, seed=seed)
        idx, w = routing_from_logits(logits, 4)
        ref = C.moe_forward(x, oracle_experts(experts), idx, w, act=C.act_silu)
        ridx, rw = routing_device(idx, w)
        return bf16_dev(x), device_experts(experts), (ridx, rw), ref

    cases = [case(T, 60 + T) for T in (1, 12, 1)]
    for dx, dexp, rt, ref in cases:
        y, _, _ = MR.moe_forward(dx, None, dexp, 4, True, _tab(), 0, MR.act_silu, routing=rt)
        assert np.array_equal(u16(y), ref)
    dx, dexp, rt, ref = case(3, 70)
    other = case(7, 71)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        MR.moe_forward(dx, None, dexp, 4, True, _tab(), 0, MR.act_silu, routing=rt)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        yg, _, _ = MR.moe_forward(dx, None, dexp, 4, True, _tab(), 0, MR.act_silu, routing=rt)
    for _ in range(4):
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(u16(yg), ref)
        yo, _, _ = MR.moe_forward(other[0], None, other[1], 4, True, _tab(), 0, MR.act_silu, routing=other[2])
        assert np.array_equal(u16(yo), other[3])


@pytest.mark.parametrize("T", [1, 3, 4, 5, 40, 300])
def test_moe_forward_from_logits(T):
    """moe_forward(logits=...): the routing computed inside the layer (up to 4 tokens in the layer's
    first launch, a wave per token; beyond that by the router kernel first; past 256 tokens with
    the multi-chunk dispatch) against the oracle's router_from_logits and moe_forward: y, idx and
    w bit for bit, logits given as binary32 and as bf16."""
    from lockstep_amd import moe_ref as MR
    from lockstep_amd import workloads as WL
    say("moe from logits", T)
    x, experts, logits = WL.moe_inputs(T, 16, 4, 256, 128, seed=90 + T)
    idx, w = routing_from_logits(logits, 4)
    ref = C.moe_forward(x, oracle_experts(experts), idx, w, act=C.act_silu)
    dx, dexp = bf16_dev(x), device_experts(experts)
    for g in (to_dev(logits), bf16_dev(logits)):
        y, di, dw = MR.moe_forward(dx, None, dexp, 4, True, _tab(), 0, MR.act_silu, logits=g)
        assert np.array_equal(u16(y), ref)
        assert np.array_equal(di.cpu().numpy(), idx)
        assert np.array_equal(u16(dw), w)


@pytest.mark.parametrize("T,E,k,H,I", [(300, 128, 8, 2048, 128), (260, 200, 6, 4096, 64), (400, 64, 2, 1040, 64)])
def test_moe_route_and_row_quant_in_one_launch(T, E, k, H, I):
    """Past 256 tokens the router and the row quant of x run in one launch (a wave per token;
    E up to 256, H up to 4096, H % 8 == 0): y, idx and w equal the oracle's and the two-launch
    path's (lsk_moe_fuse_route(0)), for one to eight chunks of 512 values per lane and 64 to 256
    experts."""
    from lockstep_amd import _lib as L
    from lockstep_amd import moe_ref as MR
    from lockstep_amd import workloads as WL
    say("route + row quant", dict(T=T, E=E, k=k, H=H, I=I))
    x, experts, logits = WL.moe_inputs(T, E, k, H, I, seed=T + E)
    idx, w = routing_from_logits(logits, k)
    ref = C.moe_forward(x, oracle_experts(experts), idx, w, act=C.act_silu)
    dx, dexp, g = bf16_dev(x), device_experts(experts), bf16_dev(logits)
    for fuse in (1, 0):
        L.call("lsk_moe_fuse_route", fuse)
        try:
            y, di, dw = MR.moe_forward(dx, None, dexp, k, True, _tab(), 0, MR.act_silu, logits=g)
        finally:
            L.call("lsk_moe_fuse_route", 1)
        assert np.array_equal(u16(y), ref), fuse
        assert np.array_equal(di.cpu().numpy(), idx), fuse
        assert np.array_equal(u16(dw), w), fuse


@pytest.mark.parametrize("T", [1, 6, 40])
@pytest.mark.parametrize("wfmt", [1, 2])
def test_moe_mx_forward_from_logits(T, wfmt):
    """MXFP4 experts (per-row and block-scaled activations) with the routing computed inside the
    layer: the same bits as router_from_logits followed by the layer with routing=(idx, w)."""
    from lockstep_amd import moe_ref as MR
    from lockstep_amd import workloads as WL
    say("moe mx from logits", T, wfmt)
    x, experts, logits = WL.moe_mx_inputs(T, 8, 2, 256, 128, seed=120 + T, bias=True)
    dexp = MR.ExpertTablesMX([((to_dev(p13), to_dev(s13)), (to_dev(p2), to_dev(s2)), to_dev(b13), to_dev(b2))
                              for (p13, s13, p2, s2, b13, b2) in experts], packed=True)
    dx, g = bf16_dev(x), bf16_dev(logits)
    fwd = MR.moe_forward_mx if wfmt == 1 else MR.moe_forward_mx2
    ri, rw, _ = MR.router_from_logits(g, 2, True, _tab())
    y0, _, _ = fwd(dx, None, dexp, 2, True, _tab(), 0, MR.act_swigluoai, routing=(ri, rw))
    y1, di, dw = fwd(dx, None, dexp, 2, True, _tab(), 0, MR.act_swigluoai, logits=g)
    assert torch.equal(y1.view(torch.int16), y0.view(torch.int16))
    assert torch.equal(di, ri) and torch.equal(dw.view(torch.int16), rw.view(torch.int16))


@pytest.mark.parametrize("E,k,H,I,gdt,renorm,big_exp", [(32, 4, 2880, 2880, "bf16", True, False),
                                                       (128, 4, 2880, 2880, "f32", False, True),
                                                       (160, 8, 576, 1344, "bf16", True, False)])
def test_moe_mx_one_token_routed_in_gate_up_launch(E, k, H, I, gdt, renorm, big_exp):
    """One MXFP4 token routed from its logits inside the skinny gate/up launch (every wave runs the
    router's selection, each block quantises x itself, block 0 writes the dispatch): the same bits
    as router_from_logits followed by the layer, and the oracle's y; one, two and four experts per
    router lane (E = 32, 128, 160), f32 and bf16 logits, with and without renormalisation, and the
    multiply-then-add update."""
    from lockstep_amd import moe_ref as MR
    from lockstep_amd import workloads as WL
    say("moe mx token routed in the gate/up launch", dict(E=E, k=k, H=H, I=I, gdt=gdt, renorm=renorm))
    x, experts, logits = WL.moe_mx_inputs(1, E, k, H, I, seed=150 + E, bias=True)
    if big_exp:
        p13, s13, p2, s2, b13, b2 = experts[3]
        s2 = s2.copy()
        s2[::6, 2] = 245
        experts[3] = (p13, s13, p2, s2, b13, b2)
    dexp = MR.ExpertTablesMX([((to_dev(p13), to_dev(s13)), (to_dev(p2), to_dev(s2)), to_dev(b13), to_dev(b2))
                              for (p13, s13, p2, s2, b13, b2) in experts], packed=True)
    dx = bf16_dev(x)
    g = bf16_dev(logits) if gdt == "bf16" else torch.from_numpy(logits.astype(F32)).to(dev())
    ri, rw, _ = MR.router_from_logits(g, k, renorm, _tab())
    y0, _, _ = MR.moe_forward_mx(dx, None, dexp, k, renorm, _tab(), 0, MR.act_swigluoai, routing=(ri, rw))
    y1, di, dw = MR.moe_forward_mx(dx, None, dexp, k, renorm, _tab(), 0, MR.act_swigluoai, logits=g)
    assert torch.equal(di, ri) and torch.equal(dw.view(torch.int16), rw.view(torch.int16))
    assert torch.equal(y1.view(torch.int16), y0.view(torch.int16))
    oexp = []
    for (p13, s13, p2, s2, b13, b2) in experts:
        m13, _ = C.mx_to_m2(p13, s13)
        m2_, _ = C.mx_to_m2(p2, s2)
        oexp.append(((m13, s13), (m2_, s2), b13, b2))
    with np.errstate(over="ignore", invalid="ignore"):
        ref = C.moe_forward_mx(x, oexp, di.cpu().numpy(), dw.view(torch.int16).cpu().numpy().view(np.uint16),
                               C.act_swigluoai)
    assert np.array_equal(y1.view(torch.int16).cpu().numpy().view(np.uint16), ref)


@pytest.mark.parametrize("k,I,extra", [(8, 768, None), (4, 1024, "shared"), (6, 2048, "bias"), (3, 512, "skip"),
                                       (8, 1536, "skip_all"), (1, 256, None)])
def test_moe_one_token_down_and_combine(k, I, extra):
    """One token (the down projection and the combine in one launch): k experts of 1 to 8, I up to
    2048 (one and two 1 KB chunks), with a shared expert, with biases (SwiGLU-OAI), with some or
    all routing entries outside [0, E) (skipped: the token's output is then the shared part or
    zero), against the oracle."""
    E, H = 32, 512
    if extra == "skip":
        idx = np.array([[40, 3, 17]], np.int64)
        w = C.bf16_bits(np.array([[0.5, 0.25, 0.125]], F32))
        _run_case(1, E, k, H, I, seed=130, routing_override=(idx, w))
    elif extra == "skip_all":
        idx = np.arange(E, E + k, dtype=np.int64)[None, :]
        w = C.bf16_bits(np.full((1, k), 0.125, F32))
        _run_case(1, E, k, H, I, seed=131, routing_override=(idx, w))
    else:
        _run_case(1, E, k, H, I, seed=132 + k, bias=extra == "bias", act="swigluoai" if extra == "bias" else "silu",
                  shared=extra == "shared")


@pytest.mark.parametrize("E,k,H,I,bias,act,renorm", [(16, 4, 256, 128, False, "silu", True),
                                                     (128, 8, 2048, 768, False, "silu", True),
                                                     (200, 6, 1040, 320, True, "swigluoai", False),
                                                     (64, 1, 4096, 2048, True, "silu", True)])
def test_moe_one_token_fused_route(E, k, H, I, bias, act, renorm):
    """A one-token int8 layer routed from its logits runs the router, the row quant of x and the
    gate/up GEMV in one launch: y, idx and w equal the oracle's and the three-launch path's
    (lsk_moe_fuse_route(0)), logits as binary32 and bf16, with biases, SwiGLU-OAI, no
    renormalisation, one expert and E above 128."""
    from lockstep_amd import _lib as L
    from lockstep_amd import moe_ref as MR
    from lockstep_amd import workloads as WL
    say("one-token fused route", dict(E=E, k=k, H=H, I=I, bias=bias, act=act, renorm=renorm))
    x, experts, logits = WL.moe_inputs(1, E, k, H, I, seed=E + k + H, bias=bias)
    idx, w, _ = C.router_from_logits(logits, k, renorm)
    oact = C.act_silu if act == "silu" else C.act_swigluoai
    dact = MR.act_silu if act == "silu" else MR.act_swigluoai
    if bias or act != "silu":
        ref = C.moe_forward_b(x, oracle_experts(experts, True), idx, w, oact, rot_blk=0)
    else:
        ref = C.moe_forward(x, oracle_experts(experts), idx, w, act=oact)
    dx, dexp = bf16_dev(x), device_experts(experts)
    for g in (to_dev(logits), bf16_dev(logits)):
        outs = []
        for fuse in (1, 0):
            L.call("lsk_moe_fuse_route", fuse)
            try:
                y, di, dw = MR.moe_forward(dx, None, dexp, k, renorm, _tab(), 0, dact, logits=g)
            finally:
                L.call("lsk_moe_fuse_route", 1)
            assert np.array_equal(u16(y), ref), fuse
            assert np.array_equal(di.cpu().numpy(), idx), fuse
            assert np.array_equal(u16(dw), w), fuse
            outs.append(u16(y))
        assert np.array_equal(outs[0], outs[1])
