"""ctypes bindings of liblockstep_amd.so (the C ABI declared in include/lockstep_amd.h).

The library is loaded from this package directory; if it is missing the first call raises,
naming the build command.  There is no CPU fallback anywhere in this package: every entry
point runs the HIP kernels or raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liblockstep_amd.so")

LSK_F32, LSK_BF16, LSK_F16, LSK_I32, LSK_I8, LSK_BF16_AS_F32 = 0, 1, 2, 3, 4, 5
EPI_V21, EPI_V2, EPI_POW2, EPI_RAW, EPI_V25 = 0, 1, 2, 3, 4
LSK_ACT_SILU, LSK_ACT_SWIGLUOAI = 0, 1

_DTYPE = {torch.float32: LSK_F32, torch.bfloat16: LSK_BF16, torch.float16: LSK_F16,
          torch.int32: LSK_I32, torch.int8: LSK_I8}

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int

# name -> (restype, argtypes); kept in the order of include/lockstep_amd.h
SIGNATURES = {
    "lsk_last_error": (ctypes.c_char_p, []),
    "lsk_version": (ctypes.c_char_p, []),
    "lsk_rowquant": (_I, [_P, _I, _I64, _I64, _I64, _P, _I64, _P, _P]),
    "lsk_gemm_w8a8": (_I, [_P, _I64, _P, _I64, _I64, _I64, _I64, _I, _P, _P, _P, _P, _P, _I, _P, _I, _I64, _P]),
    "lsk_epilogue_apply": (_I, [_P, _I64, _I64, _I64, _I, _P, _P, _P, _P, _P, _I, _P, _I, _I64, _P]),
    "lsk_w8a8_matmul_workspace": (_I64, [_I64, _I64]),
    "lsk_w8a8_matmul": (_I, [_P, _I, _I64, _I64, _I64, _P, _I64, _I64, _P, _P, _I, _P, _I, _I64, _P, _I64, _P]),
    "lsk_w8a8_matmul_pairs": (_I, [_P, _I, _I64, _I64, _I64, _P, _I64, _P, _I64, _P, _P, _I, _P, _I, _I64, _P, _I64, _P]),
    "lsk_w8a8_matmul_noalloc": (_I, [_P, _I, _I64, _I64, _I64, _P, _I64, _I64, _P, _P, _I, _P, _I, _I64, _P]),
    "lsk_outlier_side": (_I, [_P, _I, _I64, _I64, _P, _I, _I64, _P, _P]),
    "lsk_outlier_split": (_I, [_P, _I, _I64, _I64, _I64, _P, _I64, _P, _I64, _P, _P]),
    "lsk_gemm_w8a8_outlier": (_I, [_P, _I64, _P, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _I64, _P, _I, _P, _I, _I64,
                                   _P]),
    "lsk_w8a8_outlier_linear_workspace": (_I64, [_I64, _I64, _I64]),
    "lsk_w8a8_outlier_linear": (_I, [_P, _I, _I64, _I64, _I64, _P, _I64, _P, _I, _P, _I64, _I64, _P, _P, _I, _P, _I,
                                     _I64, _P, _I64, _P]),
    "lsk_quant_planes": (_I, [_P, _I, _I64, _I64, _I64, _I, _P, _I, _P, _I64, _P, _P, _P]),
    "lsk_split_planes": (_I, [_P, _I64, _I, _P, _P, _P]),
    "lsk_planes_combine": (_I, [_P, _I64, _I64, _I64, _I, _I, _P, _P, _P, _P, _I, _I64, _P]),
    "lsk_planes_linear_workspace": (_I64, [_I64, _I64, _I64, _I, _I]),
    "lsk_planes_linear": (_I, [_P, _I, _I64, _I64, _I64, _I, _P, _P, _I64, _I64, _I, _P, _P, _P, _I, _I64, _P, _I64,
                               _P]),
    "lsk_rmsnorm_float": (_I, [_P, _I, _I64, _I64, _I64, _P, _I, ctypes.c_float, ctypes.c_double, _P, _I, _I64, _P,
                               _I64, _P, _P, _P]),
    "lsk_tree_sum": (_I, [_P, _I64, _I64, _I64, _P, _P]),
    "lsk_gemm_select": (_I, [_I]),
    "lsk_gemm_skinny_shape": (_I, [_I, _I, _I]),
    "lsk_moe_skinny_shape": (_I, [_I, _I]),
    "lsk_moe_pp_skinny_rows": (_I, [_I]),
    "lsk_gemm_fuse_rowquant": (_I, [_I]),
    "lsk_quant8_dyn_single_pass": (_I, [_I]),
    "lsk_quant8_dyn_variant": (_I, [_I]),
    "lsk_moe_fuse_route": (_I, [_I]),
    "lsk_gemm_persist": (_I, [_I]),
    "lsk_quant8_pow2": (_I, [_P, _I64, _I64, _I64, _I, _P, _I64, _P, _P, _P]),
    "lsk_quant8_dyn_workspace": (_I64, []),
    "lsk_quant8_dyn": (_I, [_P, _I64, _I64, _I64, _P, _I64, _P, _P, _P, _I64, _P]),
    "lsk_linear_dyn_workspace": (_I64, [_I64, _I64]),
    "lsk_linear_dyn": (_I, [_P, _I64, _I64, _I64, _P, _I64, _P, _I64, _I, _P, _I64, _P, _I, _P, _I64, _P]),
    "lsk_row_pairs_bytes": (_I64, [_I64, _I64]),
    "lsk_pack_row_pairs": (_I, [_P, _I64, _I64, _I64, _P, _P]),
    "lsk_gemm_reads_row_pairs": (_I, [_I64, _I64, _I64]),
    "lsk_moe_reads_row_pairs": (_I, [_I64, _I, _I64, _I64, _I64, _I, _I]),
    "lsk_router_topk": (_I, [_P, _I, _I64, _I64, _I64, _I, _I, _P, _P, _P, _P]),
    "lsk_act_elementwise": (_I, [_P, _P, _I64, _I, _P, _P, _P]),
    "lsk_table_scores": (_I, [_P, _I64, _P, _P, _P]),
    "lsk_fwht_blocks": (_I, [_P, _I64, _I64, _I64, _I, ctypes.c_float, _P, _I64, _P]),
    "lsk_gemm_mx": (_I, [_P, _I64, _P, _I, _I64, _P, _I64, _I64, _I64, _I64, _I, _P, _P, _P, _I64, _P]),
    "lsk_mx_epilogue": (_I, [_P, _I64, _I64, _P, _P, _P, _P]),
    "lsk_dequant_mxfp4": (_I, [_P, _P, _I64, _I64, _I, _P, _I, _P]),
    "lsk_blockquant": (_I, [_P, _I, _I64, _I64, _I64, _P, _I64, _P, _I64, _P]),
    "lsk_act_table": (_I, [_P, _I, _P, _P]),
    "lsk_gemm_mx2": (_I, [_P, _I64, _P, _I64, _P, _I, _I64, _P, _I64, _I64, _I64, _I64, _I, _P, _P, _I64, _P]),
    "lsk_mx_pack_m2": (_I, [_P, _I64, _P, _P, _P]),
    "lsk_mx_skinny_bytes": (_I64, [_I64, _I64]),
    "lsk_mx_skinny_pack": (_I, [_P, _I64, _I64, _I64, _P, _P]),
    "lsk_moe_workspace": (_I64, [_I64, _I, _I64, _I64, _I64, _I, _I]),
    "lsk_moe_forward": (_I, [_P, _P]),
    "lsk_moe_mx_reads_skinny": (_I, [_I64, _I, _I64, _I64, _I64, _I64, _I64, _I, _I]),
    "lsk_grouped_gemm_workspace": (_I64, [_I64, _I64]),
    "lsk_grouped_gemm_w8a8": (_I, [_P, _I64, _P, _P, _I64, _I64, _P, _I64, _P, _P, _I64, _I64, _P, _P, _I64, _P]),
    "lsk_grouped_gemm_w8a8_pairs": (_I, [_P, _I64, _P, _P, _I64, _I64, _P, _I64, _P, _P, _P, _I64, _I64, _P, _P, _I64,
                                         _P]),
    "lsk_grouped_gemm_mx": (_I, [_P, _I64, _P, _P, _I64, _I64, _P, _I64, _P, _I64, _P, _I64, _I64, _I, _P, _P, _I64,
                                 _P]),
    "lsk_grouped_gemm_mx_skinny": (_I, [_P, _I64, _P, _P, _I64, _I64, _P, _I64, _P, _P, _I64, _P, _I64, _I64, _I,
                                        _P, _P, _I64, _P]),
    "lsk_grouped_mx_reads_skinny": (_I, [_I64, _I64, _I64, _I64]),
    "lsk_moe_select": (_I, [_I]),
    "lsk_mfma_bf16_acc_probe": (_I, [_P, _P, _P, _P, _I, _P]),
    "lsk_mfma_probe": (_I, [_P, _I64, _I64, _I, _P, _P]),
    "lsk_bf16_cvt_check": (_I, [ctypes.c_uint64, ctypes.c_uint64, _P, _P, _P]),
    "lsk_moe_mx_select": (_I, [_I]),
}


class MoeArgs(ctypes.Structure):
    """Mirror of lsk_moe_args (include/lockstep_amd.h)."""
    _fields_ = [("T", _I64), ("H", _I64), ("I", _I64), ("E", _I64), ("k", _I), ("act", _I),
                ("wfmt", _I), ("mx_safe", _I), ("lds13", _I64), ("lds2", _I64),
                ("x", _P), ("idx", _P), ("w", _P), ("w13_ptrs", _P), ("ldw13", _I64), ("ws13_ptrs", _P),
                ("b13_ptrs", _P), ("w2_ptrs", _P), ("ldw2", _I64), ("ws2_ptrs", _P), ("b2_ptrs", _P),
                ("frac", _P), ("rot_blk", _I), ("rot_scale", ctypes.c_float), ("shared", _P), ("y", _P), ("workspace", _P), ("workspace_bytes", _I64),
                ("kw13_min", _I), ("kw13_max", _I), ("kw2_min", _I), ("kw2_max", _I), ("act_tab", _P),
                ("logits", _P), ("logits_dtype", _I), ("renormalize", _I), ("ld_logits", _I64), ("router_tab", _P),
                ("idx_out", _P), ("w_out", _P), ("select", _I), ("mx_select", _I),
                ("w13_pair_ptrs", _P), ("w2_pair_ptrs", _P)]

_lock = threading.Lock()
_lib = None


class LockstepError(RuntimeError):
    pass


def load(path: str = LIB_PATH):
    """Load the shared library (once) and bind every exported symbol."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(path):
            raise LockstepError("%s is not built: run `python -m lockstep_amd.build` (hipcc, gfx950)" % path)
        lib = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def last_error() -> str:
    return load().lsk_last_error().decode(errors="replace")


def call(name: str, *args):
    rc = getattr(load(), name)(*args)
    if rc != 0:
        raise LockstepError("%s failed (code %d): %s" % (name, rc, last_error()))
    return rc


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPE[dt]
    except KeyError:
        raise TypeError("unsupported dtype %s" % dt) from None


def ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(t: torch.Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def require_cuda(*ts, what: str = "lockstep_amd"):
    """Every tensor argument must live on one ROCm device; CPU tensors are refused (this
    package has no CPU path; the reference's own functions are the CPU path)."""
    dev = None
    for t in ts:
        if t is None:
            continue
        if not isinstance(t, torch.Tensor) or not t.is_cuda:
            raise ValueError("%s: expected a GPU tensor, got %s" % (what, type(t).__name__ if not isinstance(t, torch.Tensor) else t.device))
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError("%s: tensors on %s and %s" % (what, dev, t.device))
    return dev
