"""Builds liblockstep_amd.so from csrc/*.hip with hipcc for gfx950 only.

    python -m lockstep_amd.build          # or lockstep_amd.build.build()
    python -m lockstep_amd.build --incremental   # recompile only sources older than their inputs

Floating-point flags are part of the contract: no contraction into FMA, correctly rounded
binary32 division, denormals kept, no packed-fp32 instructions.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import re
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIB = os.path.join(HERE, "liblockstep_amd.so")
OBJDIR = os.path.join(HERE, "_build")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-ffp-contract=off", "-fno-fast-math",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
    "-I", INCLUDE, "-I", CSRC,
]


# Per-file code generation options.  mx.hip: the MX block update consumes every MFMA result
# with VALU FMAs, so MFMA results go straight to VGPRs (no accumulation-register copies between
# an MFMA and its FMAs).
FILE_FLAGS = {
    "mx.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _includes(path: str, seen: set) -> set:
    """path and the local headers it includes, transitively (#include "..." in csrc/ or include/)."""
    if path in seen or not os.path.exists(path):
        return seen
    seen.add(path)
    with open(path) as f:
        for line in f:
            m = re.match(r'\s*#\s*include\s+"([^"]+)"', line)
            if m:
                for d in (CSRC, INCLUDE):
                    _includes(os.path.join(d, m.group(1)), seen)
    return seen


def _stale(src: str, obj: str) -> bool:
    """Whether obj is missing or older than src, a header it includes, or this file."""
    if not os.path.exists(obj):
        return True
    deps = _includes(src, set()) | {__file__}
    return os.path.getmtime(obj) < max(os.path.getmtime(d) for d in deps)


def _compile(src: str, incremental: bool = False) -> str:
    obj = os.path.join(OBJDIR, os.path.basename(src) + ".o")
    if incremental and not _stale(src, obj):
        return obj
    cmd = [HIPCC, *FLAGS, *FILE_FLAGS.get(os.path.basename(src), []), "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("hipcc failed for %s:\n%s\n%s" % (src, " ".join(cmd), r.stderr))
    return obj


def build(verbose: bool = False, incremental: bool = False) -> str:
    """Compile every csrc/*.hip (all of them unless incremental) and link the library."""
    os.makedirs(OBJDIR, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda f: _compile(f, incremental), srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n%s\n%s" % (" ".join(cmd), r.stderr))
    os.replace(tmp, LIB)
    if verbose:
        print("built", LIB)
    return LIB


if __name__ == "__main__":
    build(verbose=True, incremental="--incremental" in sys.argv[1:])
    sys.exit(0)
