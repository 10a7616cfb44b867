"""Synthetic inputs of the named workloads, drawn from numpy's PCG64 stream (stable across
numpy versions and platforms), so the same seed gives the same bits on every machine.

Dense: x N(0,1) binary32 (optionally with 0.1% outliers at +-20), W8 uniform int8 on
[-127, 127], per-output-channel ws U(1e-3, 1e-2).
"""
from __future__ import annotations

import numpy as np

F32 = np.float32

# (N, K) of the dense projections
QWEN25_7B_O = (3584, 3584)                       # o_proj, hidden 3584
LLAMA8B = {"gate_up": (28672, 4096), "down": (4096, 14336)}   # hidden 4096, intermediate 14336
QWEN25_7B = {"qkv": (4608, 3584), "o": (3584, 3584), "gate_up": (37888, 3584), "down": (3584, 18944)}


def rng(seed):
    return np.random.Generator(np.random.PCG64(int(seed)))


def activations(g, M, K, outliers=False):
    x = g.standard_normal((M, K), dtype=np.float64).astype(F32)
    if outliers:
        mask = g.random((M, K)) < 0.001
        sign = g.integers(0, 2, (M, K), dtype=np.int8).astype(F32) * F32(2) - F32(1)
        x = np.where(mask, F32(20.0) * sign, x).astype(F32)
    return x


def int8_weight(g, N, K):
    W8 = g.integers(-127, 128, (N, K), dtype=np.int8)
    ws = g.uniform(1e-3, 1e-2, N).astype(F32)
    return W8, ws


def dense_inputs(M, N, K, seed=0, outliers=False):
    """(x f32 [M, K], W8 int8 [N, K], ws f32 [N])."""
    g = rng(seed)
    x = activations(g, M, K, outliers)
    W8, ws = int8_weight(g, N, K)
    return x, W8, ws
