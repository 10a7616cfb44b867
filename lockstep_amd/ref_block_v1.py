"""Drop-in for the GEMM primitives of reference/ref_block_v1.py (the golden training block), on MI355X.

    _e_from_max(m)      ref_block_v1.py:56-62
    quant8_rows(x)      ref_block_v1.py:64-67
    quant8_cols(w)      ref_block_v1.py:69-72
    quant8_dyn(x)       ref_block_v1.py:122-130
    gemm_int(a, b)      ref_block_v1.py:132-133
    gemm_pow2(q8, e_a, w8, e_w)   the pow2 dequant sites :167, 193, 198, 218 fused into the GEMM
    linear_dyn(x, W8, ew)         a whole GEMM site (quant8_dyn, gemm_int, pow2 dequant), the
                                  activation exponent kept on the device

The reference works on numpy arrays; these functions take numpy arrays or GPU tensors and
return the same kind.  numpy inputs are uploaded to the current GPU and the results copied
back (the arithmetic is always the HIP kernels').  gemm_int's operands must be integers in
[-127, 127] (the quantisers' range), which makes the int32 accumulation exact.
"""
from __future__ import annotations

import numpy as np
import torch

from . import _lib as L
from . import ops


def _to_dev(x, dtype):
    if isinstance(x, torch.Tensor):
        L.require_cuda(x, what="ref_block_v1")
        return x.to(dtype), False
    return torch.from_numpy(np.ascontiguousarray(np.asarray(x))).to(device="cuda", dtype=dtype), True


def _back(t, was_np, np_dtype):
    return t.cpu().numpy().astype(np_dtype) if was_np else t


def _e_from_max(m):
    """Per-entry pow2 exponent of a vector of maxima (any non-negative binary32 values)."""
    t, was_np = _to_dev(m, torch.float32)
    t = t.reshape(1, -1)
    _, e = ops.quant8_pow2(t, 2)            # per column of a one-row matrix: e = rule(m)
    return _back(e.to(torch.int64), was_np, np.int64)


def quant8_rows(x):
    """Per-row pow2 scales: q [T, D] (int64 values in [-127, 127]), e [T]."""
    t, was_np = _to_dev(x, torch.float32)
    q, e = ops.quant8_pow2(t, 1)
    if was_np:
        return q.cpu().numpy().astype(np.int64), e.cpu().numpy().astype(np.int64)
    return q, e.to(torch.int64)


def quant8_cols(w):
    """Per-column pow2 scales: q [D, N], e [N]."""
    t, was_np = _to_dev(w, torch.float32)
    q, e = ops.quant8_pow2(t, 2)
    if was_np:
        return q.cpu().numpy().astype(np.int64), e.cpu().numpy().astype(np.int64)
    return q, e.to(torch.int64)


def quant8_dyn(x):
    """Per-tensor pow2 quant: (q, e) with e a Python int (0 and q = 0 for an all-zero tensor).
    The exponent is computed on the device; returning it as an int (as the reference does)
    synchronises with the device once.  linear_dyn keeps it on the device."""
    t, was_np = _to_dev(x, torch.float32)
    shp = t.shape
    t2 = t.reshape(-1, shp[-1]) if t.dim() >= 2 else t.reshape(1, -1)
    q, e = ops.quant8_dyn(t2)
    q = q.reshape(shp)
    e = int(e[0].item())
    if was_np:
        return q.cpu().numpy().astype(np.int64), e
    return q, e


def linear_dyn(x, W8, ew):
    """One GEMM site of the block, fused: (gemm_int(q8, W8).astype(F) * F(2.0**(-ex-ew))).astype(F)
    with (q8, ex) = quant8_dyn(x) -- ref_block_v1.py:166-167 (qkv), :191-193 (o), :196-198 (up),
    :216-218 (down, per-tensor form).  x [T, K] binary32 tensor; W8 the reference's right
    operand [K, N] of int8 values (a transposed view of a row-major [N, K] int8 weight is used in
    place); ew the weight's exponent from quant8_dyn at arm time.  The activation exponent stays on
    the device (no host synchronisation).  Returns (y binary32 [T, N], ex int32 [1] on the device)."""
    L.require_cuda(x, W8, what="linear_dyn")
    if x.dim() != 2:
        raise ValueError("linear_dyn: x must be [T, K], got %s" % (tuple(x.shape),))
    w_nk = ops.weight_nk(_as_int8(W8))
    return ops.linear_dyn(x, w_nk, int(ew), w_pairs=row_pairs_of(w_nk, x.shape[0]))


# the weights' row-pair copies (ops.row_pairs_of: one per weight, held by the weight while it is
# unchanged, made only when the GEMM at that row count reads it)
row_pairs_of = ops.row_pairs_of


def _as_int8(t):
    if t.dtype == torch.int8:
        return t
    if t.numel() and (t.max() > 127 or t.min() < -127):
        raise ValueError("gemm_int: operands must be quantised int8 values in [-127, 127]")
    return t.to(torch.int8)


def gemm_int(a, b):
    """Exact integer GEMM a [M, K] @ b [K, N] (int64 result, as the reference's numpy int64)."""
    ta, wa = _to_dev(a, torch.int64) if not isinstance(a, torch.Tensor) else (a, False)
    tb, wb = _to_dev(b, torch.int64) if not isinstance(b, torch.Tensor) else (b, False)
    L.require_cuda(ta, tb, what="gemm_int")
    acc = ops.gemm(_as_int8(ta), ops.weight_nk(_as_int8(tb)), L.EPI_RAW, L.LSK_I32)
    out = acc.to(torch.int64)
    return out.cpu().numpy() if (wa or wb) else out


def gemm_pow2(q8, e_a, w8, e_w):
    """fl32(gemm_int(q8, w8)) * 2^-(e_a + e_w) in one launch: the block's dequant sites
    (ref_block_v1.py:167,193,198,218).  e_a / e_w are Python ints (per tensor) or integer
    vectors (per row of q8 / per column of w8, as ref_block_v1.py:213-214)."""
    ta = q8 if isinstance(q8, torch.Tensor) else _to_dev(q8, torch.int64)[0]
    tb = w8 if isinstance(w8, torch.Tensor) else _to_dev(w8, torch.int64)[0]
    was_np = not isinstance(q8, torch.Tensor)
    shift = 0
    erow = ecol = None
    if np.ndim(e_a) == 0 and not (isinstance(e_a, torch.Tensor) and e_a.dim() > 0):
        shift += int(e_a)
    elif isinstance(e_a, torch.Tensor) and e_a.numel() == 1 and ta.shape[0] != 1:
        erow = e_a.reshape(1).to(torch.int32).expand(ta.shape[0])   # a per-tensor exponent on the device
    else:
        erow = _to_dev(e_a, torch.int32)[0] if not isinstance(e_a, torch.Tensor) else e_a
    if np.ndim(e_w) == 0 and not (isinstance(e_w, torch.Tensor) and e_w.dim() > 0):
        shift += int(e_w)
    else:
        ecol = _to_dev(e_w, torch.int32)[0] if not isinstance(e_w, torch.Tensor) else e_w
    y = ops.gemm(_as_int8(ta), ops.weight_nk(_as_int8(tb)), L.EPI_POW2, L.LSK_F32, erow=erow, ecol=ecol,
                 shift=shift)
    return y.cpu().numpy() if was_np else y
