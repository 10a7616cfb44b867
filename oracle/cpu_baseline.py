"""The reference's CPU op sequences, restated in torch on the host, for bench.py's cpu_baseline leg.

TEST INFRASTRUCTURE ONLY (timed as the CPU baseline, never shipped).  These follow the
reference's CPU code paths op for op, so their cost is the reference's cost:

  dense_w8a8: lockstep_fullstack.w8a8_matmul (reference/lockstep_fullstack.py:503-530):
      x.float(); quantize_rows_int8 with a tensor divisor (:476-481); _int_mm_exact (:484-500),
      which on CPU calls torch._int_mm with the rows zero-padded to 17; the v2.1 epilogue (:524-527).
  moe_int8:   moe_ref.moe_forward (reference/moe_ref.py:117-140) with routing injected: the per-expert
      Python loop, rowquant, int64 matmul (int_mm's CPU branch, :55), lin_epilogue, act_silu, combine.
Their results are checked against the numpy oracle in tests/test_oracle_baseline.py.
"""
from __future__ import annotations

import torch

from . import contract as C

BF = torch.bfloat16
F32 = torch.float32


def _quant_rows(x2):
    asc = x2.abs().amax(dim=1).clamp(min=1e-8) / torch.tensor(127.0, dtype=F32)
    x8 = torch.clamp(torch.round(x2 / asc[:, None]), -127, 127).to(torch.int8)
    return x8, asc


def _int_mm_exact(a8, b8):
    n = a8.shape[0]
    if n < 17:
        a8 = torch.cat([a8, torch.zeros(17 - n, a8.shape[1], dtype=torch.int8)])
    try:
        y = torch._int_mm(a8, b8)
    except RuntimeError:
        y = torch.matmul(a8.to(torch.int64), b8.to(torch.int64)).to(torch.int32)
    return y[:n]


def dense_w8a8(x, W8, ws, bias=None, out_dtype=BF):
    x2 = x.reshape(-1, x.shape[-1]).float()
    x8, asc = _quant_rows(x2)
    y = (_int_mm_exact(x8, W8.t()).float() * ws[None, :]) * asc[:, None]
    y = y.to(out_dtype)
    if bias is not None:
        y = (y.float() + bias.float()).to(out_dtype)
    return y


def _bfr(x):
    return x.to(BF).to(F32)


def _silu(x):
    frac = torch.from_numpy(C.frac_table())
    xc = torch.where(x.abs() < 1.1754943508222875e-38, torch.zeros_like(x), x)
    t = torch.clamp(xc * -1.4426950216293335, -30.0, 30.0)
    i = torch.ceil(t)
    g = i - t
    k = torch.clamp(torch.trunc(g * 8192.0), max=8191.0).to(torch.int64)
    f = frac[k].to(F32) * (2.0 ** -15)
    e2 = f * ((i.to(torch.int32) + 127) << 23).view(F32)
    return xc * (1.0 / (1.0 + e2))


def _rowquant(x):
    xf = x.to(F32)
    am = xf.abs().amax(dim=-1, keepdim=True).clamp(min=1e-8)
    asc = am / torch.tensor(127.0, dtype=F32)
    q = torch.clamp(torch.round(xf / asc), -127, 127).to(torch.int8)
    return q, asc.squeeze(-1)


def _lin(acc, ws, asc):
    return _bfr((acc.to(F32) * ws[None, :]) * asc[:, None])


def _int_mm64(a8, b8):
    return (a8.to(torch.int64) @ b8.to(torch.int64)).to(torch.int32)


def moe_int8(x, experts, idx, w):
    """x bf16 [T, H]; experts[e] = (w13col [H, 2I], ws13, w2col [I, H], ws2); idx int64 [T, k]; w bf16."""
    T, H = x.shape
    acc = torch.zeros(T, H, dtype=F32)
    for e in range(len(experts)):
        hit = idx == e
        if not hit.any():
            continue
        tok = hit.any(dim=-1).nonzero(as_tuple=True)[0]
        we = w[tok][hit[tok]].to(F32)
        w13, ws13, w2, ws2 = experts[e]
        q, asc = _rowquant(x[tok])
        y = _lin(_int_mm64(q, w13), ws13, asc)
        I = y.shape[-1] // 2
        h = _bfr(_silu(y[:, :I]) * y[:, I:])
        q2, asc2 = _rowquant(h)
        out = _lin(_int_mm64(q2, w2), ws2, asc2)
        acc[tok] += _bfr(we[:, None] * out)
    return acc.to(BF)
