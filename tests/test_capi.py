"""CPU-side checks of the C ABI: the library loads and exports every function the header
declares, with the Python bindings covering each one (no compute calls without a GPU)."""
import ctypes
import os
import re

from lockstep_amd import _lib as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = []
    for fn in os.listdir(os.path.join(ROOT, "include")):
        if fn.endswith(".h"):
            src = open(os.path.join(ROOT, "include", fn)).read()
            src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
            names += re.findall(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(lsk_\w+)\s*\(", src, flags=re.M)
    return sorted(set(names))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(L.LIB_PATH)
    names = declared_functions()
    assert len(names) >= 6, names
    for n in names:
        assert hasattr(lib, n), n


def test_bindings_cover_the_header():
    assert set(declared_functions()) == set(L.SIGNATURES), set(declared_functions()) ^ set(L.SIGNATURES)


def test_version_and_error_string_without_gpu():
    lib = L.load()
    assert b"gfx950" in lib.lsk_version()
    assert isinstance(lib.lsk_last_error(), bytes)


def test_argument_errors_are_reported_without_touching_the_gpu():
    lib = L.load()
    # negative sizes are refused before any HIP call
    rc = lib.lsk_gemm_w8a8(None, 0, None, 0, -1, 1, 1, 0, None, None, None, None, None, 0, None, 0, 0, None)
    assert rc == 1 and b"negative" in lib.lsk_last_error()
    rc = lib.lsk_gemm_w8a8(None, 0, None, 0, 1, 1, 200000, 0, None, None, None, None, None, 0, None, 0, 0, None)
    assert rc == 1 and b"133144" in lib.lsk_last_error()
    rc = lib.lsk_gemm_w8a8(None, 0, None, 0, 1, 1, 16, 3, None, None, None, None, None, 0, None, 0, 1, None)
    assert rc == 1 and b"int32" in lib.lsk_last_error()
    rc = lib.lsk_rowquant(None, 7, 1, 1, 1, None, 1, None, None)
    assert rc == 1
    # M == 0 is legal and a no-op
    assert lib.lsk_rowquant(None, 0, 0, 16, 16, None, 16, None, None) == 0


def test_outlier_entry_points_refuse_bad_arguments_without_touching_the_gpu():
    lib = L.load()
    # V25 needs its side inputs: the plain GEMM refuses it
    rc = lib.lsk_gemm_w8a8(None, 16, None, 16, 1, 1, 16, 4, None, None, None, None, None, 0, None, 1, 1, None)
    assert rc == 1 and b"V25" in lib.lsk_last_error()
    # the rotation needs whole 256-wide blocks
    rc = lib.lsk_w8a8_outlier_linear(None, 1, 300, 1, 300, None, 0, None, 1, None, 300, 8, None, None, 1, None, 1, 8,
                                     None, 0, None)
    assert rc == 1 and b"256" in lib.lsk_last_error()
    rc = lib.lsk_gemm_w8a8_outlier(None, 16, None, 16, 1, 1, 16, None, None, None, None, 0, None, 7, None, 1, 1, None)
    assert rc == 1 and b"wo" in lib.lsk_last_error()
    # zero rows: a no-op
    assert lib.lsk_w8a8_outlier_linear(None, 1, 256, 0, 256, None, 3, None, 1, None, 256, 8, None, None, 1, None, 1, 8,
                                       None, 0, None) == 0
    assert lib.lsk_w8a8_outlier_linear_workspace(4, 256, 3) >= 4 * 256 * 5 + 4 * 3 * 4 + 16
