"""lockstep_amd: the Lockstep contract matrix-multiply path on MI355X (gfx950).

Drop-in modules with the reference's names and signatures:
    lockstep_amd.lockstep_fullstack   dense W8A8 linear (v2.1 epilogue)
    lockstep_amd.contract_common      legacy W8A8 linear (v2 epilogue), FRAC table
    lockstep_amd.ref_block_v1         pow2 quantisers and the exact integer GEMM
    lockstep_amd.moe_ref              contract v3 MoE (int8 and MXFP4 operands)
    lockstep_amd.moe_mxfp4            exact MXFP4 dequant
All arithmetic runs in the HIP kernels of liblockstep_amd.so; GPU tensors only.
"""
from . import _lib

__all__ = ["_lib"]
__version__ = "0.1"
