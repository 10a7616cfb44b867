"""Drop-in for the contract 2.6 float norm of reference/t16n_ref.py, on MI355X.

Same names, signatures and results as the reference (device tensors only; the arithmetic runs in
the HIP kernels of liblockstep_amd.so):

    sqrt_n(N)                               t16n_ref.py:38-39    the width constant fl32(sqrt N) (host)
    tree_sum(v)                             :42-50               the pinned adjacent-pairs tree
    row_sum_float(x2)                       :53-62               chains of 8, then the tree
    eps_term(N, eps)                        :65-67               fl32(fl64(N) * fl64(eps)) (host)
    rmsnorm_float(x, weight, sN, out_dtype, eps)   :70-92        the float RMSNorm, bf16 out

and the prologue of the contract linears that consume the norm (no counterpart function in the
reference; it is rmsnorm_float followed by lockstep_fullstack.quantize_rows_int8 of its output,
in one kernel):

    rmsnorm_float_rowquant(x, weight, sN, eps, want_out)  -> (q int8, asc f32, out bf16 or None)
"""
from __future__ import annotations

import math

import numpy as np
import torch

from . import _lib as L

FLT_MIN = 2.0 ** -126


def sqrt_n(N):
    """The published width constant fl32(sqrt(N)) (binary64 sqrt, one rounding)."""
    return float(np.float32(math.sqrt(N)))


def eps_term(N, eps):
    """ne = fl32(fl64(N) * fl64(eps))."""
    return float(np.float32(float(N) * float(eps or 0.0)))


def _float_rows(x):
    x2 = x.reshape(-1, x.shape[-1])
    if x2.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        x2 = x2.float()
    if x2.shape[-1] and x2.stride(-1) != 1:
        x2 = x2.contiguous()
    return x2


def tree_sum(v):
    """v: [R, n] float32 partial sums -> [R] by the pinned tree (largest power of two below n)."""
    L.require_cuda(v, what="tree_sum")
    v2 = v.to(torch.float32)
    v2 = v2 if v2.is_contiguous() else v2.contiguous()
    R, n = v2.shape
    out = torch.empty((R,), dtype=torch.float32, device=v.device)
    L.call("lsk_tree_sum", L.ptr(v2), max(n, 1), R, n, L.ptr(out), L.stream_of(v))
    return out


def row_sum_float(x2):
    """x2: [R, N] float32 -> S [R]: sq = fl32(x * x), chains of 8 in index order, then the tree."""
    L.require_cuda(x2, what="row_sum_float")
    x2 = _float_rows(x2)
    R, N = x2.shape
    if N % 8:
        raise AssertionError("row_sum_float: N=%d is not a multiple of 8" % N)
    S = torch.empty((R,), dtype=torch.float32, device=x2.device)
    L.call("lsk_rmsnorm_float", L.ptr(x2), L.dtype_code(x2.dtype), x2.stride(0) if R > 1 else max(N, 1), R, N, None,
           0, 0.0, 0.0, None, L.LSK_BF16, N, None, N, None, L.ptr(S), L.stream_of(x2))
    return S


def _gain(weight, N, dev):
    g = weight.detach().reshape(-1)
    if g.numel() != N:
        raise ValueError("rmsnorm_float: gain has %d entries for width %d" % (g.numel(), N))
    if g.device != dev:
        g = g.to(dev)
    if g.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        g = g.float()
    return g.contiguous()


_ODT = {torch.bfloat16: L.LSK_BF16, torch.float32: L.LSK_F32, torch.float16: L.LSK_F16}


def rmsnorm_float(x, weight, sN=None, out_dtype=None, eps=0.0):
    """x: [..., N] (bf16 or fp32), weight: [N] gain (folded norms pass ones).  Returns the bf16
    output (out_dtype=None -> bf16; another out_dtype is the bf16 value cast)."""
    L.require_cuda(x, what="rmsnorm_float")
    shp = x.shape
    N = shp[-1]
    x2 = _float_rows(x)
    R = x2.shape[0]
    odt = out_dtype or torch.bfloat16
    if odt not in _ODT:
        raise TypeError("rmsnorm_float: out_dtype %s not supported" % odt)
    if N % 8:
        raise AssertionError("rmsnorm_float: N=%d is not a multiple of 8" % N)
    g = _gain(weight, N, x.device)
    out = torch.empty((R, N), dtype=odt, device=x.device)
    L.call("lsk_rmsnorm_float", L.ptr(x2), L.dtype_code(x2.dtype), x2.stride(0) if R > 1 else max(N, 1), R, N,
           L.ptr(g), L.dtype_code(g.dtype), float(sqrt_n(N) if sN is None else sN), float(eps or 0.0), L.ptr(out),
           _ODT[odt], N, None, N, None, None, L.stream_of(x))
    return out.reshape(shp)


def rmsnorm_float_rowquant(x, weight, sN=None, eps=0.0, want_out=False):
    """The norm and the contract row quant of its bf16 output in one pass:
    (q int8 [..., N], asc f32 [...], out bf16 [..., N] when want_out else None)."""
    L.require_cuda(x, what="rmsnorm_float_rowquant")
    shp = x.shape
    N = shp[-1]
    x2 = _float_rows(x)
    R = x2.shape[0]
    if N % 8:
        raise AssertionError("rmsnorm_float_rowquant: N=%d is not a multiple of 8" % N)
    g = _gain(weight, N, x.device)
    q = torch.empty((R, N), dtype=torch.int8, device=x.device)
    asc = torch.empty((R,), dtype=torch.float32, device=x.device)
    out = torch.empty((R, N), dtype=torch.bfloat16, device=x.device) if want_out else None
    L.call("lsk_rmsnorm_float", L.ptr(x2), L.dtype_code(x2.dtype), x2.stride(0) if R > 1 else max(N, 1), R, N,
           L.ptr(g), L.dtype_code(g.dtype), float(sqrt_n(N) if sN is None else sN), float(eps or 0.0), L.ptr(out),
           L.LSK_BF16, N, L.ptr(q), N, L.ptr(asc), None, L.stream_of(x))
    return q.reshape(shp), asc.reshape(shp[:-1]), (None if out is None else out.reshape(shp))
