"""Regenerates the inputs of the reference's published contract vectors
(conformance/contract_vectors.json, copied here as contract_vectors.json).

The reference draws every input from numpy's PCG64 stream (tools/contract_vectors.py:22-31):
standard_normal(float64) narrowed to float32, then scaled and rounded in binary32 / bf16.
The draws below are taken in the same order from the same seeds
(tools/contract_vectors.py:60-80 for the linear, :82-98 for the outlier cases,
:106-144 for the norm / rope draws that precede the SiLU and R4 inputs), so the numpy
arrays returned are bit-identical to the reference's torch tensors.
"""
from __future__ import annotations

import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
F32 = np.float32


def _bf16(x):
    u = np.ascontiguousarray(x, dtype=F32).view(np.uint32).astype(np.uint64)
    b = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32)
    return (b << 16).view(F32)


class _Gen:
    def __init__(self, seed):
        self.g = np.random.Generator(np.random.PCG64(int(seed)))

    def randn(self, *shape):
        return self.g.standard_normal(size=shape, dtype=np.float64).astype(F32)


def load_vectors():
    with open(os.path.join(HERE, "contract_vectors.json")) as f:
        return json.load(f)["vectors"]


def linear_inputs():
    """x bf16 [5,512] (as float32 values), W bf16 [96,512], bias fp32 [96]."""
    g = _Gen(20260906)
    x = _bf16(g.randn(5, 512) * F32(3))
    W = _bf16(g.randn(96, 512) * F32(0.05))
    bias = (g.randn(96) * F32(0.1)).astype(F32)
    return g, x, W, bias


def silu_r4_inputs():
    """The SiLU gate/up (tools/contract_vectors.py:126-131) and the R4 rows (:133)."""
    g, _, _, _ = linear_inputs()
    for N in (512, 128):                    # rmsnorm draws (:106-111)
        g.randn(7, N)
        g.randn(N)
    g.randn(6, 256)                          # rope qh, kh (:119-120)
    g.randn(6, 128)
    a = g.randn(4, 256) * F32(4)
    b = (np.rint(g.randn(2, 256) * F32(2)) / F32(2)).astype(F32)
    c = np.array([[-40.0, 40.0, 0.0, 1e-30, -1e-30, 0.5, -0.5, 30.0] + [0.25] * 248], dtype=F32)
    xs = _bf16(np.concatenate([a.astype(F32), b, c], 0))
    gate = xs
    up = xs[:, ::-1].copy()
    v = _bf16(g.randn(3, 256))
    return gate, up, v


def outlier_inputs():
    """tools/contract_vectors.py:82-87: x5 bf16 [5,512] with two massive channels, W5 bf16 [96,512]."""
    g5 = _Gen(25)
    x5 = _bf16(g5.randn(5, 512) * F32(3))
    x5[:, 17] = _bf16(x5[:, 17] * F32(400))
    x5[:, 300] = _bf16(x5[:, 300] * F32(150))
    W5 = _bf16(g5.randn(96, 512) * F32(0.05))
    oidx = np.array([17, 300, 511], dtype=np.int32)
    return x5, W5, oidx


def norm_float_inputs():
    """tools/contract_vectors.py:155-164 (contract 2.6 float norm, its own stream): for N, eps in
    (4096, 1e-6), (3072, 1e-5), (128, 1e-6): x bf16 [6, N] = randn * 2 with row 1 zero, x[2, 7] = 3
    and row 3 = bf16(randn(N) * 1e-19); gain ones, or bf16(1 + 0.1 randn(N)) at N = 128."""
    g3 = _Gen(2026_09_10)
    out = []
    for N, eps in ((4096, 1e-6), (3072, 1e-5), (128, 1e-6)):
        xn = _bf16(g3.randn(6, N) * F32(2))
        xn[1] = 0
        xn[2, 7] = 3.0
        xn[3] = _bf16(g3.randn(N) * F32(1e-19))
        wn = np.ones(N, F32) if N != 128 else _bf16((F32(1.0) + F32(0.1) * g3.randn(N)).astype(F32))
        out.append((N, eps, xn, wn))
    return out
