"""The ctypes mirror of lsk_moe_args (lockstep_amd/_lib.py) against the C declaration in
include/lockstep_amd.h: a small C program compiled with the host compiler prints the size and
every field's offset, which must equal ctypes' (a field added on one side only would shift every
later field and pass garbage pointers to the layer)."""
import os
import shutil
import subprocess

import pytest

from lockstep_amd import _lib as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="no host C compiler")
def test_moe_args_layout_matches_header(tmp_path):
    names = [f[0] for f in L.MoeArgs._fields_]
    src = tmp_path / "layout.c"
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "lockstep_amd.h"', "int main(void) {",
             '  printf("size %zu\\n", sizeof(lsk_moe_args));']
    lines += ['  printf("%s %%zu\\n", offsetof(lsk_moe_args, %s));' % (n, n) for n in names]
    lines += ["  return 0;", "}"]
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    got = dict(line.split() for line in out if line.strip())
    assert int(got["size"]) == __import__("ctypes").sizeof(L.MoeArgs)
    for n in names:
        assert int(got[n]) == getattr(L.MoeArgs, n).offset, n
