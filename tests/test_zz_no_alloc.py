"""The allocation-free dense contract linear (lsk_w8a8_matmul_noalloc) against the workspace entry
point (lsk_w8a8_matmul), both called through the C ABI: bit-equal outputs on two calls in a row,
the second smaller than the first (the shared scratch keeps the first call's contents), and the
size limit reported as an argument error."""
import ctypes

import numpy as np
import pytest
import torch

from gpu_util import bits, dev

pytestmark = pytest.mark.gpu

SCRATCH = 16 << 20


def _call_pair(L, x, W, ws, bias, order, out_code, out_t):
    M, K = x.shape
    N = W.shape[0]
    lib = L.load()
    ref = torch.empty((M, N), dtype=out_t, device=x.device)
    got = torch.full((M, N), float("nan"), dtype=out_t, device=x.device)
    nbytes = lib.lsk_w8a8_matmul_workspace(M, K)
    work = torch.empty((nbytes,), dtype=torch.uint8, device=x.device)
    s = L.stream_of(x)
    L.call("lsk_w8a8_matmul", L.ptr(x), L.dtype_code(x.dtype), K, M, K, L.ptr(W), K, N, L.ptr(ws), L.ptr(bias), order,
           L.ptr(ref), out_code, N, L.ptr(work), nbytes, s)
    L.call("lsk_w8a8_matmul_noalloc", L.ptr(x), L.dtype_code(x.dtype), K, M, K, L.ptr(W), K, N, L.ptr(ws),
           L.ptr(bias), order, L.ptr(got), out_code, N, s)
    torch.cuda.synchronize()
    return ref, got


@pytest.mark.parametrize("order", [0, 1])
def test_noalloc_matches_workspace_entry_point(order):
    from lockstep_amd import _lib as L
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    g = np.random.default_rng(21 + order)
    # first call near the scratch maximum, second smaller (stale contents must not leak through),
    # third a decode row with a bias
    cases = [(2048, 4096, 512, torch.float32, False), (37, 1000, 300, torch.bfloat16, False),
             (1, 14336, 4096, torch.float32, True)]
    for M, K, N, xt, with_bias in cases:
        x = torch.from_numpy(g.standard_normal((M, K)).astype(np.float32)).to(dev()).to(xt)
        W = torch.from_numpy(g.integers(-127, 128, (N, K), dtype=np.int8)).to(dev())
        ws = torch.from_numpy(g.uniform(1e-3, 1e-2, N).astype(np.float32)).to(dev())
        bias = torch.from_numpy(g.standard_normal(N).astype(np.float32)).to(dev()) if with_bias else None
        assert L.load().lsk_w8a8_matmul_workspace(M, K) <= SCRATCH
        ref, got = _call_pair(L, x, W, ws, bias, order, L.LSK_BF16, torch.bfloat16)
        assert np.array_equal(bits(ref), bits(got)), (M, K, N)


def test_noalloc_rejects_sizes_beyond_its_scratch():
    from lockstep_amd import _lib as L
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    lib = L.load()
    M, K, N = 4096, 8192, 64
    assert lib.lsk_w8a8_matmul_workspace(M, K) > SCRATCH
    rc = lib.lsk_w8a8_matmul_noalloc(None, 0, K, M, K, None, K, N, None, None, 0, None, 1, N, None)
    assert rc == 1 and b"maximum" in lib.lsk_last_error()
