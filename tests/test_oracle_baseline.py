"""The CPU-baseline restatement (torch on the host) computes the same bits as the numpy oracle,
so the baseline bench.py times is the same function the GPU path is checked against."""
import numpy as np
import torch

from oracle import contract as C
from oracle import cpu_baseline as B


def test_dense_baseline_matches_oracle():
    g = np.random.default_rng(0)
    x = g.standard_normal((5, 512)).astype(np.float32)
    W8 = g.integers(-127, 128, (96, 512), dtype=np.int8)
    ws = g.uniform(1e-3, 1e-2, 96).astype(np.float32)
    bias = g.standard_normal(96).astype(np.float32)
    for b in (None, bias):
        y = B.dense_w8a8(torch.from_numpy(x), torch.from_numpy(W8), torch.from_numpy(ws),
                         None if b is None else torch.from_numpy(b))
        ref = C.w8a8_matmul(x, W8, ws, b, "bf16")
        assert np.array_equal(y.view(torch.int16).numpy().view(np.uint16), ref)


def test_moe_baseline_matches_oracle():
    g = np.random.default_rng(1)
    T, H, I, E, k = 10, 64, 32, 5, 2
    x = C.bfr(g.standard_normal((T, H)).astype(np.float32))
    ex_np, ex_t = [], []
    for e in range(E):
        w13 = g.integers(-127, 128, (2 * I, H), dtype=np.int8)
        w2 = g.integers(-127, 128, (H, I), dtype=np.int8)
        ws13 = g.uniform(1e-3, 1e-2, 2 * I).astype(np.float32)
        ws2 = g.uniform(1e-3, 1e-2, H).astype(np.float32)
        ex_np.append((w13.T, ws13, w2.T, ws2))
        ex_t.append((torch.from_numpy(w13).t(), torch.from_numpy(ws13), torch.from_numpy(w2).t(), torch.from_numpy(ws2)))
    idx, w, _ = C.router_from_logits(C.bfr(g.standard_normal((T, E)).astype(np.float32)), k, True)
    y = B.moe_int8(torch.from_numpy(x).to(torch.bfloat16), ex_t, torch.from_numpy(idx),
                   torch.from_numpy(C.bf16_to_f32(w)).to(torch.bfloat16))
    ref = C.moe_forward(x, ex_np, idx, w)
    assert np.array_equal(y.view(torch.int16).numpy().view(np.uint16), ref)
