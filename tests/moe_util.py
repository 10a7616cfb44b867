"""Helpers of the MoE tests: device copies of a seeded case in the reference's layouts."""
import numpy as np
import torch

from gpu_util import bf16_dev, dev, to_dev
from oracle import contract as C


def device_experts(experts):
    """experts[e] -> (w13col [H, 2I], ws13, w2col [I, H], ws2, b13, b2) as the reference passes them:
    the int8 weights as transpose views of row-major [N, K] device matrices."""
    out = []
    for (w13, ws13, w2, ws2, b13, b2) in experts:
        out.append((to_dev(w13).t(), to_dev(ws13), to_dev(w2).t(), to_dev(ws2),
                    None if b13 is None else to_dev(b13), None if b2 is None else to_dev(b2)))
    return out


def oracle_experts(experts, with_bias=False):
    if with_bias:
        return [(w13.T, ws13, w2.T, ws2, b13, b2) for (w13, ws13, w2, ws2, b13, b2) in experts]
    return [(w13.T, ws13, w2.T, ws2) for (w13, ws13, w2, ws2, b13, b2) in experts]


def routing_from_logits(logits, k, renorm=True):
    idx, w, _ = C.router_from_logits(logits, k, renorm)
    return idx, w


def routing_device(idx, w_bits):
    return to_dev(idx), torch.from_numpy(C.bf16_to_f32(w_bits)).to(torch.bfloat16).to(dev())


def u16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)
