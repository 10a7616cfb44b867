"""The weights' row-pair copies are prepared weights: made once per weight, held by the weight
tensor itself, made only where the GEMM reads them.  CPU-side: the C queries (no device work) and
the caching logic with the pack counted (pack_row_pairs replaced by a counting stand-in)."""
import pytest
import torch

from lockstep_amd import _lib as L
from lockstep_amd import ops


def test_gemm_row_pair_query():
    lib = L.load()
    # one activation row streams W8 whole rows; mid row counts use the register-staged tile: no copy
    for M in (1, 4, 64, 128):
        assert lib.lsk_gemm_reads_row_pairs(M, 28672, 4096) == 0, M
    # decode rows of wide weights whose activations fit in LDS: the skinny GEMV streams the copy
    for M, N, K in ((8, 28672, 4096), (32, 28672, 4096), (16, 14336, 4096)):
        assert lib.lsk_gemm_reads_row_pairs(M, N, K) == 1, (M, N, K)
    # narrow weights stream whole rows through LDS; 32 rows of K = 14336 exceed the LDS
    for M, N, K in ((16, 3584, 3584), (8, 4096, 14336), (32, 16384, 14336)):
        assert lib.lsk_gemm_reads_row_pairs(M, N, K) == 0, (M, N, K)
    # prefill row counts on the ping-pong tiles read it
    for M, N, K in ((2048, 28672, 4096), (2048, 4096, 14336), (8192, 37888, 3584), (8192, 3584, 18944)):
        assert lib.lsk_gemm_reads_row_pairs(M, N, K) == 1, (M, N, K)
    assert lib.lsk_gemm_reads_row_pairs(2048, 4096, 100) == 0        # K % 16 != 0
    assert lib.lsk_gemm_reads_row_pairs(0, 4096, 4096) == 0


def test_moe_row_pair_query():
    lib = L.load()
    E, k, H, I = 128, 8, 2048, 768
    assert lib.lsk_moe_reads_row_pairs(1, k, E, H, I, 0, 0) == 0       # the grouped GEMV
    for T in (2, 32, 192):                                                 # the skinny grouped GEMM
        assert lib.lsk_moe_reads_row_pairs(T, k, E, H, I, 0, 0) == 1, T
    assert lib.lsk_moe_reads_row_pairs(4096, k, E, H, I, 0, 0) == 1    # the ping-pong tiles
    assert lib.lsk_moe_reads_row_pairs(32, k, E, H, I, 8, 0) == 0      # rotated layers: the tiles
    # a per-call choice of the register-staged tile or the GEMV (select = variant + 2) reads none
    assert lib.lsk_moe_reads_row_pairs(4096, k, E, H, I, 0, 2) == 0
    assert lib.lsk_moe_reads_row_pairs(32, k, E, H, I, 0, 4) == 0
    # the thread's own setting is left as it was
    assert lib.lsk_moe_reads_row_pairs(4096, k, E, H, I, 0, 0) == 1


def test_moe_mx_skinny_query():
    """MXFP4 layers (GPT-OSS-20B: E 32, top 4, H = I = 2880, 90 E8M0 bytes a row) read the codes'
    skinny-layout copies from 1 to 256 tokens (one token only when k * 2I / 64 >= 320: with top 2
    the MX GEMV keeps it); under lsk_moe_mx_select(3) from one token; forced kernel families read
    none."""
    lib = L.load()
    E, k, H, I, lds = 32, 4, 2880, 2880, 90
    assert lib.lsk_moe_mx_reads_skinny(1, 2, E, H, I, lds, lds, 0, 0) == 0            # the MX GEMV
    assert lib.lsk_moe_mx_reads_skinny(1, 2, E, H, I, lds, lds, 0, 4) == 1            # mx_select 3
    for T in (1, 2, 24, 25, 128, 256):
        assert lib.lsk_moe_mx_reads_skinny(T, k, E, H, I, lds, lds, 0, 0) == 1, T
    for T in (257, 4096):                                                             # the tiles
        assert lib.lsk_moe_mx_reads_skinny(T, k, E, H, I, lds, lds, 0, 0) == 0, T
    assert lib.lsk_moe_mx_reads_skinny(1, k, E, H, I, lds, lds, 0, 4) == 1            # mx_select 3
    assert lib.lsk_moe_mx_reads_skinny(200, k, E, H, I, lds, lds, 2, 4) == 1          # ... over the tiles
    # a forced kernel family (select = variant + 2) reads none; the thread's settings stay as they were
    assert lib.lsk_moe_mx_reads_skinny(32, k, E, H, I, lds, lds, 2, 0) == 0
    assert lib.lsk_moe_mx_reads_skinny(32, k, E, H, I, lds, lds, 4, 4) == 0           # the GEMV forced
    assert lib.lsk_moe_mx_reads_skinny(32, k, E, H, I, lds, lds, 0, 2) == 0           # mx_select 1
    assert lib.lsk_moe_mx_reads_skinny(32, k, E, H, I, lds, lds, 0, 0) == 1
    # the chunk's rows and the E8M0 rows must fit the LDS: K = 16384 does not
    assert lib.lsk_moe_mx_reads_skinny(32, k, E, 16384, I, 512, lds, 0, 0) == 0
    assert lib.lsk_moe_mx_reads_skinny(32, k, E, H, I, lds, lds, 0, 10) == 0          # out of range
    # the grouped linear alone: experts averaging at most 32 rows
    assert lib.lsk_grouped_mx_reads_skinny(256, E, H, lds) == 1
    assert lib.lsk_grouped_mx_reads_skinny(32 * E, E, H, lds) == 1
    assert lib.lsk_grouped_mx_reads_skinny(32 * E + 1, E, H, lds) == 0
    assert lib.lsk_grouped_mx_reads_skinny(256, E, 16384, 512) == 0
    assert lib.lsk_grouped_mx_reads_skinny(256, E, 100, 4) == 0                        # K % 32 != 0


def test_mx_skinny_copy_size_and_argument_checks():
    """lsk_mx_skinny_bytes: 1 KB per group of 16 rows and step of 4 blocks (partial ones whole); the
    pack refuses K % 32 != 0, a row stride below K / 2 or not a multiple of 4, and null pointers,
    before any device work."""
    lib = L.load()
    assert lib.lsk_mx_skinny_bytes(16, 128) == 1024
    assert lib.lsk_mx_skinny_bytes(17, 128) == 2048
    assert lib.lsk_mx_skinny_bytes(16, 160) == 2048            # 5 blocks: two steps
    assert lib.lsk_mx_skinny_bytes(5760, 2880) == 360 * 23 * 1024
    for args in ((64, 16, 40), (16, 16, 64), (34, 16, 64)):     # (ldw, rows, K)
        ldw, rows, K = args
        assert lib.lsk_mx_skinny_pack(16, ldw, rows, K, 4096, None) != 0, args
    assert lib.lsk_mx_skinny_pack(None, 64, 16, 64, 4096, None) != 0
    assert "lsk_mx_skinny_pack" in L.last_error()


@pytest.fixture
def counting_pack(monkeypatch):
    made = []

    def fake_pack(w):
        made.append((w.data_ptr(), tuple(w.shape)))
        return torch.empty((L.load().lsk_row_pairs_bytes(*w.shape),), dtype=torch.int8)
    monkeypatch.setattr(ops, "pack_row_pairs", fake_pack)
    return made


def test_130_dense_weights_pack_once(counting_pack):
    """A model's worth of distinct dense weights (130) cycled twice through the prefill path: each
    copy is made on the first pass and reused on the second (decode rows that read it share the same
    copy); one activation row makes none."""
    ws = [torch.zeros((8192, 64), dtype=torch.int8) for _ in range(130)]
    for w in ws:
        assert ops.row_pairs_of(w, 1) is None
    assert counting_pack == []
    first = [ops.row_pairs_of(w, 2048) for w in ws]
    assert len(counting_pack) == 130 and all(p is not None for p in first)
    second = [ops.row_pairs_of(w, 2048) for w in ws]
    assert len(counting_pack) == 130
    assert all(a is b for a, b in zip(first, second))
    assert all(ops.row_pairs_of(w, 32) is p for w, p in zip(ws, first)) and len(counting_pack) == 130
    # views of the same storage (the reference's b8 = W8.t() turned back) share the copy
    assert ops.row_pairs_of(ws[0].t().t(), 2048) is first[0]
    # an in-place update re-makes that weight's copy only
    ws[7].add_(1)
    assert ops.row_pairs_of(ws[7], 2048) is not first[7]
    assert len(counting_pack) == 131
    assert ops.row_pairs_of(ws[8], 2048) is first[8] and len(counting_pack) == 131


def test_copy_lives_with_the_weight(counting_pack):
    import gc
    import weakref
    w = torch.zeros((64, 64), dtype=torch.int8)
    p = ops.row_pairs_of(w, 4096)
    ref = weakref.ref(p)
    del p
    assert ref() is not None                 # held by the weight
    ops.release_row_pairs(w)
    gc.collect()
    assert ref() is None
    p = ops.row_pairs_of(w, 4096)
    ref = weakref.ref(p)
    del p, w
    gc.collect()
    assert ref() is None                     # freed with the weight


def test_copies_can_be_turned_off(counting_pack, monkeypatch):
    monkeypatch.setattr(ops, "ROW_PAIR_COPIES", False)
    assert ops.row_pairs_of(torch.zeros((64, 64), dtype=torch.int8), 4096) is None
    assert counting_pack == []
