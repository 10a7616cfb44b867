"""Drop-in for the linear-path pieces of reference/contract_common.py, on MI355X.

    FRAC_DIGEST, COEFFS, VERIFIED_NW, build_table, table_np, table_on, frac_on   :12-60
    w8a8_linear(lin)     :151-175  (the legacy E-v2 epilogue order, kept for the HF arm)
    apply_w8a8(model)    :177-185

The FRAC table is built in exact Python integers on the host (8192 entries, once) and cached
per device; every other computation runs in the HIP kernels.
"""
from __future__ import annotations

import hashlib

import numpy as np
import torch

from . import _lib as L
from . import ops

FRAC_DIGEST = "f472476ccea65299feb63f1ff863714a35910d2099470bafb5d3be0e92a598cd"
COEFFS = [1073741823, -744260975, 257938938, -59583045, 10286509, -1369790, 117454]
VERIFIED_NW = {(13, 15), (12, 14), (12, 15), (13, 14), (13, 16), (14, 16), (11, 15), (15, 16)}

_tables = {}
_frac_t = {}


def build_table(n, w):
    """FRAC_{n,w}[k] = (Horner(t = k << (20 - n)) + 2^(29 - w)) >> (30 - w), exact integers."""
    assert (n, w) in VERIFIED_NW, "(n,w)=(%d,%d) is not a verified point" % (n, w)
    tab = []
    for k in range(1 << n):
        t = k << (20 - n)
        p = COEFFS[6]
        for c in COEFFS[5::-1]:
            p = c + ((p * t) // (1 << 20))
        tab.append((p + (1 << (29 - w))) >> (30 - w))
    return np.asarray(tab, dtype=np.int64)


def table_np(n, w):
    if (n, w) not in _tables:
        t = build_table(n, w)
        if (n, w) == (13, 15):
            d = hashlib.sha256(np.asarray(t, dtype="<u2").tobytes()).hexdigest()
            assert d == FRAC_DIGEST, "FRAC digest mismatch: " + d
        _tables[(n, w)] = t
    return _tables[(n, w)]


def table_on(dev, n=13, w=15):
    k = (str(dev), n, w)
    if k not in _frac_t:
        _frac_t[k] = torch.tensor(table_np(n, w), dtype=torch.int64, device=dev)
    return _frac_t[k]


def frac_on(dev):
    return table_on(dev, 13, 15)


_frac_i32 = {}


def table_i32_on(dev, n=13, w=15):
    """The table as int32 (every entry is below 2^16), the form the kernels read."""
    k = (str(dev), n, w)
    if k not in _frac_i32:
        _frac_i32[k] = torch.tensor(table_np(n, w).astype(np.int32), dtype=torch.int32, device=dev)
    return _frac_i32[k]


def frac_check():
    d = hashlib.sha256(np.asarray(table_np(13, 15), dtype="<u2").tobytes()).hexdigest()
    assert d == FRAC_DIGEST, "FRAC digest mismatch: " + d
    return d


_OUT = {torch.float32: L.LSK_F32, torch.bfloat16: L.LSK_BF16, torch.float16: L.LSK_F16}


def w8a8_linear(lin):
    """Per-out-channel int8 W (true-division scale), per-token int8 A, exact GEMM, and the
    legacy epilogue y = fl32(fl32(acc) * asc[m]) * ws[n] (+ bias in binary32), one cast to
    x.dtype.  Replaces lin.forward in place, as the reference does."""
    W = lin.weight.data
    L.require_cuda(W, what="w8a8_linear")
    W8, ws = ops.rowquant(W.float())
    W8 = W8.contiguous()
    bias = lin.bias.data.clone().float() if lin.bias is not None else None

    def fwd(x):
        sh = x.shape
        x2 = x.reshape(-1, sh[-1])
        odt = _OUT.get(x.dtype, L.LSK_F32)
        y = ops.w8a8_matmul(x2.float() if x2.dtype not in _OUT else x2, W8, ws, bias, L.EPI_V2, odt)
        y = y.reshape(*sh[:-1], W8.shape[0])
        return y if y.dtype == x.dtype else y.to(x.dtype)

    lin.forward = fwd
    lin._ls_w8, lin._ls_ws = W8, ws
    return lin


def apply_w8a8(model):
    """Arm every nn.Linear under model.model except MoE routers ('.gate'); lm_head is outside
    model.model and stays as it is, as in the reference."""
    nrep, nskip = 0, 0
    for name, mod in model.model.named_modules():
        if isinstance(mod, torch.nn.Linear):
            if name.split(".")[-1] == "gate":
                nskip += 1
                continue
            w8a8_linear(mod)
            nrep += 1
    print("W8A8 linears replaced: %d (lm_head excluded, %d MoE routers skipped)" % (nrep, nskip), flush=True)
    return nrep, nskip
