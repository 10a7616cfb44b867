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


# ---------------------------------------------------------------- MoE
QWEN3_30B_A3B = dict(E=128, k=8, H=2048, I=768)     # per-expert SwiGLU
GPT_OSS_20B = dict(E=32, k=4, H=2880, I=2880)


def _bf16_round(x):
    u = np.ascontiguousarray(x, dtype=F32).view(np.uint32).astype(np.uint64)
    b = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32)
    return (b << 16).view(F32)


def zipf_logits(g, T, E, s=1.1):
    """Router logits N(0,1) plus an expert-popularity bias -s * ln(1 + rank_e) over a random
    rank permutation: routing probabilities follow a Zipf(s) law, so loads are skewed."""
    rank = g.permutation(E)
    bias = (-s * np.log1p(rank)).astype(F32)
    return _bf16_round(g.standard_normal((T, E), dtype=np.float64).astype(F32) + bias[None, :])


def moe_int8_experts(g, E, H, I, bias=False):
    """experts[e] = (w13 [2I, H] int8, ws13 [2I], w2 [H, I] int8, ws2 [H], b13 | None, b2 | None)."""
    out = []
    for _ in range(E):
        w13, ws13 = int8_weight(g, 2 * I, H)
        w2, ws2 = int8_weight(g, H, I)
        b13 = (g.standard_normal(2 * I) * 0.1).astype(F32) if bias else None
        b2 = (g.standard_normal(H) * 0.1).astype(F32) if bias else None
        out.append((w13, ws13, w2, ws2, b13, b2))
    return out


def moe_inputs(T, E, k, H, I, seed=0, bias=False, zipf=True):
    """x [T, H] (bf16 values as f32), experts (moe_int8_experts), logits [T, E] (bf16 values)."""
    g = rng(seed)
    x = _bf16_round(g.standard_normal((T, H), dtype=np.float64).astype(F32))
    logits = zipf_logits(g, T, E) if zipf else _bf16_round(g.standard_normal((T, E), dtype=np.float64).astype(F32))
    experts = moe_int8_experts(g, E, H, I, bias)
    return x, experts, logits


def mx_expert_weights(g, N, K):
    """Packed E2M1 codes [N, K/2] (uniform over all 16 codes) and E8M0 bytes [N, K/32] with
    exponents uniform in [-8, 2] (127 + U{-8..2})."""
    packed = g.integers(0, 256, (N, K // 2), dtype=np.uint8)
    scale = (127 + g.integers(-8, 3, (N, K // 32))).astype(np.uint8)
    return packed, scale


def moe_mx_inputs(T, E, k, H, I, seed=0, bias=False):
    """x [T, H] (bf16 values as f32), experts [(packed13, scale13, packed2, scale2, b13, b2)],
    logits [T, E] N(0,1) (bf16 values)."""
    g = rng(seed)
    x = _bf16_round(g.standard_normal((T, H), dtype=np.float64).astype(F32))
    logits = _bf16_round(g.standard_normal((T, E), dtype=np.float64).astype(F32))
    experts = []
    for _ in range(E):
        p13, s13 = mx_expert_weights(g, 2 * I, H)
        p2, s2 = mx_expert_weights(g, H, I)
        b13 = (g.standard_normal(2 * I) * 0.1).astype(F32) if bias else None
        b2 = (g.standard_normal(H) * 0.1).astype(F32) if bias else None
        experts.append((p13, s13, p2, s2, b13, b2))
    return x, experts, logits
