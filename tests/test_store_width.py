"""No global or buffer store in the built device code is wider than 8 bytes.

On MI355X a 16-byte global / buffer store followed a few instructions later by VALU writes to
its data registers was measured to store the newer values; the compiler leaves only one wait
state between them.  Every kernel therefore stores at most 8 bytes per instruction
(`store16_split` in csrc/lsk_common.h).  This test disassembles the gfx950 code objects of the
in-tree library and fails on any 12- or 16-byte global, buffer, flat or scratch store (register
spills included)."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "lockstep_amd", "liblockstep_amd.so")
OBJDUMP = "/opt/rocm/llvm/bin/llvm-objdump"
WIDE = re.compile(r"\b(global|buffer|flat|scratch)_store_(dwordx[34]|b96|b128)\b")


@pytest.mark.skipif(not (os.path.exists(LIB) and os.path.exists(OBJDUMP)),
                    reason="needs the built library and ROCm's llvm-objdump")
def test_no_wide_vector_stores(tmp_path):
    lib = tmp_path / "lib.so"
    shutil.copy(LIB, lib)
    subprocess.run([OBJDUMP, "--offloading", str(lib)], cwd=tmp_path, check=True, capture_output=True)
    objs = sorted(p for p in tmp_path.iterdir() if p.name.endswith("gfx950"))
    assert objs, "no gfx950 code object in the library"
    bad = []
    for p in objs:
        dis = subprocess.run([OBJDUMP, "-d", str(p)], check=True, capture_output=True, text=True).stdout
        fn = "?"
        for line in dis.splitlines():
            if line.endswith(">:"):
                fn = line.split("<", 1)[-1][:-2]
            elif WIDE.search(line):
                bad.append((fn, line.strip()))
    assert not bad, "%d wide stores, first in %s: %s" % (len(bad), bad[0][0], bad[0][1])
