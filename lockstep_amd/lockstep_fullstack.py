"""Drop-in for the dense contract linear of reference/lockstep_fullstack.py, on MI355X.

Same names, signatures, dtypes and error behaviour as the reference functions below; the
arithmetic runs in the HIP kernels of liblockstep_amd.so (GPU tensors only).

    quantize_rows_int8(x2)                      lockstep_fullstack.py:476-481
    _int_mm_exact(a8, b8)                       lockstep_fullstack.py:484-500
    w8a8_matmul(x, W8, ws, bias, out_dtype, rowchunk)   lockstep_fullstack.py:503-530
    quantize_weight_int8(W)                     lockstep_fullstack.py:581-587
    silu_contract(x), fwht_blocks(x2, blk, scale), pow2_f32(e)   :590-604, :533-546, :280-284
    outlier_side(ho, wo)                        lockstep_fullstack.py:549-557
    w8a8_outlier_linear(x, oidx, wo, W8, ws, bias, out_dtype, rot)   lockstep_fullstack.py:560-578
"""
from __future__ import annotations

import torch

from . import _lib as L
from . import ops

INT8_MIN_ROWS = 17               # kept for API compatibility: the kernels take any M >= 0
SILU_C = -1.4426950216293335     # 0xBFB8AA3B, binary32 nearest -log2(e)
F32_MIN_NORMAL = 1.1754943508222875e-38
ROWCHUNK = 1024                  # schedule only in the reference; bit-invisible, unused here

_OUT = {torch.float32: L.LSK_F32, torch.bfloat16: L.LSK_BF16, torch.float16: L.LSK_F16}


def quantize_rows_int8(x2: torch.Tensor):
    """Per-token int8 quant: asc = max(|x|, 1e-8) / 127 (true division), q = clamp(rint(x / asc)).
    x2 [M, K] -> (x8 int8 [M, K], asc f32 [M])."""
    q, asc = ops.rowquant(x2)
    return q, asc


def _int_mm_exact(a8: torch.Tensor, b8: torch.Tensor) -> torch.Tensor:
    """int8 [M, K] x int8 [K, N] -> int32 [M, N], exact (any M >= 0; no row padding needed)."""
    return ops.gemm(a8, ops.weight_nk(b8), L.EPI_RAW, L.LSK_I32)


def w8a8_matmul(x, W8, ws, bias=None, out_dtype=None, rowchunk: int = 0):
    """The v2.1 W8A8 linear: x [..., K] float; W8 [N, K] int8; ws [N] f32; bias [N] or None.
    y = out(fl32(fl32(acc) * ws[n]) * asc[m]); with a bias out(fl32(y) + b[n]).  Row chunking
    is bit-invisible, so `rowchunk` is accepted and ignored."""
    L.require_cuda(x, W8, ws, bias, what="w8a8_matmul")
    shp = x.shape
    odt = out_dtype or x.dtype
    N = W8.shape[0]
    want64 = odt == torch.float64
    if not want64 and odt not in _OUT:
        raise TypeError("w8a8_matmul: out_dtype %s not supported" % odt)
    x2 = x.reshape(-1, shp[-1])
    if x2.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        x2 = x2.float()
    if x2.shape[0] == 0:
        return torch.zeros(*shp[:-1], N, dtype=odt, device=x.device)
    w = W8 if W8.stride(-1) == 1 else W8.contiguous()
    # prefill row counts run the GEMM on tiles that read the weight's row-pair copy (made once per
    # weight and held by it while it is unchanged, only when the GEMM at this row count reads it),
    # and so do 5..32 rows of a wide weight (the skinny decode GEMV); other decode rows stream W8
    wp = ops.row_pairs_of(w, x2.shape[0]) if w.dtype == torch.int8 else None
    y = ops.w8a8_matmul(x2, w, ws, bias, L.EPI_V21, L.LSK_F32 if want64 else _OUT[odt], w_pairs=wp)
    if want64:
        y = y.to(torch.float64)       # exact widening of the binary32 result
    return y.reshape(*shp[:-1], N)


def outlier_side(ho, wo):
    """Contract v2.5 side path: side[m, n] = sum_k fl32(ho[m, k]) * fl32(wo[n, k]), the sum sequential
    in k from +0 with binary32 adds.  ho [M, k], wo [N, k] -> f32 [M, N]."""
    L.require_cuda(ho, wo, what="outlier_side")
    return ops.outlier_side(ho, wo)


def w8a8_outlier_linear(x, oidx, wo, W8, ws, bias=None, out_dtype=None, rot=True):
    """The v2.5 norm-fed linear under R1 online: the declared channels oidx leave the row as ho,
    the masked row takes the 256-block butterfly / 16 (rot; rot=False is the v2.5.1 o_proj form)
    and the row quant, then y = bf16(fl32(bf16((fl32(acc) * ws[n]) * asc[m])) + side[m, n]), the
    bias as a further bf16 rounding, and the result cast to out_dtype (default x.dtype)."""
    L.require_cuda(x, oidx, wo, W8, ws, bias, what="w8a8_outlier_linear")
    shp = x.shape
    odt = out_dtype or x.dtype
    N = W8.shape[0]
    want64 = odt == torch.float64
    if not want64 and odt not in _OUT:
        raise TypeError("w8a8_outlier_linear: out_dtype %s not supported" % odt)
    x2 = x.reshape(-1, shp[-1])
    if rot and shp[-1] % 256:
        raise RuntimeError("w8a8_outlier_linear: width %d is not a multiple of the 256-wide rotation block"
                           % shp[-1])
    w = W8 if W8.stride(-1) == 1 else W8.contiguous()
    y = ops.w8a8_outlier_linear(x2, oidx, wo, w, ws, bias, rot, L.LSK_F32 if want64 else _OUT[odt])
    if want64:
        y = y.to(torch.float64)       # exact widening of the bf16-valued result
    return y.reshape(*shp[:-1], N)


def quantize_weight_int8(W):
    """Per-out-channel int8 weight (the row quant applied to W [N, K]) -> (W8, ws)."""
    W8, ws = ops.rowquant(W.detach())
    return W8.contiguous(), ws.contiguous()


def silu_contract(x):
    """The invariant SiLU: ten declared binary32 steps with the 8192-entry FRAC table."""
    return ops.act(x, None, ops.OP_SILU)


def fwht_blocks(x2, blk=256, scale=1.0 / 16.0):
    """The R4 / online-R1 butterfly on every blk-wide block of the last dim, then * scale."""
    return ops.fwht_blocks(x2, blk, scale)


def pow2_f32(e):
    """Exact 2^e as float32 from the exponent field, e in [-126, 127]."""
    return ((e.to(torch.int32) + 127) << 23).view(torch.float32)
