"""Drop-in for reference/moe_mxfp4.py (exact MXFP4 dequantisation), on MI355X.

    fp4_values(codes)                               moe_mxfp4.py:13-16
    unpack_fp4(packed)                              moe_mxfp4.py:19-23
    dequant_mxfp4(packed, scale_e8m0, out_dtype, block)   moe_mxfp4.py:26-35
    self_test(device)                               moe_mxfp4.py:38-48

Layout (the checkpoint's): packed uint8 [..., K/2], element 2i in the low nibble; scale uint8
[..., K/32], one E8M0 exponent per block.  Every value fp4 * 2^(e - 127) is exact in bf16.
"""
from __future__ import annotations

import torch

from . import _lib as L
from . import ops


def unpack_fp4(packed: torch.Tensor) -> torch.Tensor:
    """uint8 [..., K/2] -> uint8 codes [..., K], low nibble first (a bit unpack, no arithmetic)."""
    L.require_cuda(packed, what="unpack_fp4")
    lo = packed & 0x0F
    hi = (packed >> 4) & 0x0F
    return torch.stack((lo, hi), dim=-1).reshape(*packed.shape[:-1], packed.shape[-1] * 2)


def fp4_values(codes: torch.Tensor) -> torch.Tensor:
    """uint8 codes 0..15 -> binary32 values (code 8 is -0.0), through the dequant kernel with a
    unit scale."""
    L.require_cuda(codes, what="fp4_values")
    shp = codes.shape
    c = codes.to(torch.uint8).reshape(-1)
    n = c.numel()
    if n == 0:
        return torch.empty(shp, dtype=torch.float32, device=codes.device)
    if n % 2:
        c = torch.cat([c, c.new_zeros(1)])
    packed = (c[0::2] | (c[1::2] << 4)).reshape(1, -1)
    scale = torch.full((1, 1), 127, dtype=torch.uint8, device=codes.device)
    vals = ops.dequant_mxfp4(packed, scale, torch.float32, block=c.numel())
    return vals.reshape(-1)[:n].reshape(shp)


def dequant_mxfp4(packed: torch.Tensor, scale_e8m0: torch.Tensor, out_dtype=torch.bfloat16, block: int = 32):
    """packed uint8 [..., K/2], scale uint8 [..., K/block] -> [..., K] in out_dtype, exact."""
    return ops.dequant_mxfp4(packed, scale_e8m0, out_dtype, block)


def self_test(device="cuda"):
    """The reference's closed-form self test, on the device."""
    g = torch.Generator(device="cpu").manual_seed(0)
    E, N, K = 3, 8, 128
    codes = torch.randint(0, 16, (E, N, K), dtype=torch.uint8, generator=g).to(device)
    packed = (codes[..., 0::2] | (codes[..., 1::2] << 4)).to(torch.uint8)
    scale = torch.randint(100, 140, (E, N, K // 32), dtype=torch.uint8, generator=g).to(device)
    y = dequant_mxfp4(packed, scale)
    ref = fp4_values(codes) * torch.pow(2.0, (scale.to(torch.float32) - 127.0)).repeat_interleave(32, dim=-1)
    assert torch.equal(y.to(torch.float32), ref), "mxfp4 dequant self-test failed"
    assert torch.equal(y.to(torch.float32).to(torch.bfloat16).to(torch.float32), ref), "not bf16-exact"
    return True
