"""Drop-in for reference/moe_ref.py (contract v3 MoE and its dense pieces), on MI355X.

Same names and signatures; GPU tensors only; results bit-identical to the reference.

    bfr                                   moe_ref.py:22-24
    rowquant(x)                           moe_ref.py:27-37
    lin_epilogue(acc, ws, asc)            moe_ref.py:40-42
    int_mm(a8, b8)                        moe_ref.py:48-55
    lin_epilogue_b(acc, ws, asc, bias)    moe_ref.py:164-169
"""
from __future__ import annotations

import torch

from . import _lib as L
from . import ops

BF = torch.bfloat16
F32 = torch.float32
INT8_MIN_ROWS = 17   # API compatibility only: the kernels take any row count


def bfr(x: torch.Tensor) -> torch.Tensor:
    """fl32 -> bf16 -> fl32 (torch's own RNE conversion, which the kernels reproduce)."""
    return x.to(BF).to(F32)


def rowquant(x: torch.Tensor):
    """asc = max(|x|, 1e-8) / 127 (a true division), q = clamp(rint(x / asc), +-127) per row.
    x [..., K] -> (q int8 [..., K], asc f32 [...])."""
    return ops.rowquant(x)


def lin_epilogue(acc: torch.Tensor, ws: torch.Tensor, asc: torch.Tensor) -> torch.Tensor:
    """y8 = bf16((fl32(acc) * ws[n]) * asc[m]), returned in binary32."""
    return ops.epilogue(acc, L.EPI_V21, L.LSK_BF16_AS_F32, asc=asc, ws=ws)


def lin_epilogue_b(acc: torch.Tensor, ws: torch.Tensor, asc: torch.Tensor, bias=None) -> torch.Tensor:
    """bfr(bfr(fl32(acc) * ws * asc) + b)."""
    return ops.epilogue(acc, L.EPI_V21, L.LSK_BF16_AS_F32, asc=asc, ws=ws, bias=bias)


def int_mm(a8: torch.Tensor, b8: torch.Tensor) -> torch.Tensor:
    """int8 [M, K] x int8 [K, N] -> int32 [M, N], exact, any M >= 0."""
    return ops.gemm(a8, ops.weight_nk(b8), L.EPI_RAW, L.LSK_I32)


def linear(q: torch.Tensor, asc: torch.Tensor, b8: torch.Tensor, ws: torch.Tensor, bias=None) -> torch.Tensor:
    """lin_epilogue_b(int_mm(q, b8), ws, asc, bias) in one launch (the fused form)."""
    return ops.gemm(q, ops.weight_nk(b8), L.EPI_V21, L.LSK_BF16_AS_F32, asc=asc, ws=ws, bias=bias)
