"""Shared helpers of the GPU tests: device tensors from numpy and back, bit views."""
import numpy as np
import torch


def dev():
    return torch.device("cuda", 0)


def to_dev(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.to(dev())


def bf16_dev(f32_vals):
    """A bf16 device tensor holding the given (already bf16-representable) binary32 values."""
    return torch.from_numpy(np.ascontiguousarray(f32_vals, dtype=np.float32)).to(torch.bfloat16).to(dev())


def bits(t):
    """Host numpy view of a tensor's bits: bf16 -> uint16, f16 -> uint16, f32 -> uint32, ints as is."""
    t = t.detach().cpu().contiguous()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.float32:
        return t.numpy().view(np.uint32)
    return t.numpy()


def f32_bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def f16_bits(a):
    return np.ascontiguousarray(a, dtype=np.float16).view(np.uint16)


def say(*a):
    print(*a, flush=True)
