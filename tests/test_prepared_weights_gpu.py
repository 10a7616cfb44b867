"""Prepared weights on the GPU: the row-pair copies held by the weights, graph capture reading the
weight itself (replays follow in-place updates), and expert lists re-packing nothing when their
tables are rebuilt."""
import numpy as np
import pytest
import torch

from gpu_util import bf16_dev, dev, say, to_dev
from moe_util import device_experts, routing_device, routing_from_logits, u16
from oracle import contract as C

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _capture(fn):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fn()
    return graph, out


def test_captured_dense_linears_follow_in_place_weight_updates():
    """A w8a8_matmul and a linear_dyn at prefill rows (the eager calls read the weights' row-pair
    copies) captured into graphs, the weights then overwritten in place: every replay equals the
    eager result on the current weights, bit for bit."""
    from lockstep_amd import _lib as L
    from lockstep_amd import lockstep_fullstack as FS
    from lockstep_amd import ops
    from lockstep_amd import ref_block_v1 as RB
    g = np.random.default_rng(11)
    M, N, K = 512, 768, 512
    assert L.load().lsk_gemm_reads_row_pairs(M, N, K) == 1
    x = to_dev(g.standard_normal((M, K)).astype(np.float32))
    W = to_dev(g.integers(-127, 128, (N, K), dtype=np.int8))
    ws = to_dev(g.uniform(1e-3, 1e-2, N).astype(np.float32))
    packs = ops.row_pair_packs
    eager = FS.w8a8_matmul(x, W, ws, out_dtype=torch.bfloat16)
    assert ops.row_pair_packs == packs + 1
    g1, out1 = _capture(lambda: FS.w8a8_matmul(x, W, ws, out_dtype=torch.bfloat16))
    g2, out2 = _capture(lambda: RB.linear_dyn(x, W.t(), 7)[0])
    for step in range(3):
        say("replay", step)
        if step:
            W.copy_(to_dev(g.integers(-127, 128, (N, K), dtype=np.int8)))   # in place
        e1 = FS.w8a8_matmul(x, W, ws, out_dtype=torch.bfloat16)
        e2, _ = RB.linear_dyn(x, W.t(), 7)
        if step == 0:
            assert torch.equal(e1.view(torch.int16), eager.view(torch.int16))
        g1.replay()
        g2.replay()
        torch.cuda.synchronize()
        assert torch.equal(out1.view(torch.int16), e1.view(torch.int16)), step
        assert torch.equal(out2.view(torch.int32), e2.view(torch.int32)), step
    # one fresh copy per update for the eager calls (the two sites share it)
    assert ops.row_pair_packs == packs + 3


def test_fifty_expert_lists_pack_once(monkeypatch):
    """50 expert lists (int8 experts, as the reference passes them) through moe_forward at a token
    count whose grouped GEMMs read the experts' row-pair copies, twice, with the table cache bound
    at 4 lists so every second-pass call rebuilds its tables: the copies are made on the first pass
    only, and the second pass gives the same bits."""
    from lockstep_amd import _lib as L
    from lockstep_amd import contract_common as CC
    from lockstep_amd import moe_ref as MR
    from lockstep_amd import ops
    from lockstep_amd import workloads as WL
    monkeypatch.setattr(MR, "TABLES_MAX", 4)
    T, E, k, H, I = 128, 4, 2, 256, 128
    assert L.load().lsk_moe_reads_row_pairs(T, k, E, H, I, 0, 0) == 1
    tab = CC.table_on(dev())
    lists, runs = [], []
    for s in range(50):
        x, experts, logits = WL.moe_inputs(T, E, k, H, I, seed=100 + s)
        idx, w = routing_from_logits(logits, k)
        lists.append(device_experts(experts))
        runs.append((bf16_dev(x), routing_device(idx, w), (x, experts, idx, w)))
    packs = ops.row_pair_packs
    first = []
    for dexp, (dx, rt, _) in zip(lists, runs):
        y, _, _ = MR.moe_forward(dx, None, dexp, k, True, tab, 0, MR.act_silu, routing=rt)
        first.append(u16(y))
    assert ops.row_pair_packs == packs + 50 * 2 * E
    for i, (dexp, (dx, rt, _)) in enumerate(zip(lists, runs)):
        y, _, _ = MR.moe_forward(dx, None, dexp, k, True, tab, 0, MR.act_silu, routing=rt)
        assert np.array_equal(u16(y), first[i]), i
    assert ops.row_pair_packs == packs + 50 * 2 * E
    for i in (0, 49):
        x, experts, idx, w = runs[i][2]
        ref = C.moe_forward(x, [(w13.T, ws13, w2.T, ws2) for (w13, ws13, w2, ws2, _, _) in experts], idx, w)
        assert np.array_equal(first[i], ref), i
