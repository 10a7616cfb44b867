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


def test_block_scaled_and_router_entry_points_without_touching_the_gpu():
    """lsk_blockquant / lsk_gemm_mx2 / lsk_router_topk / lsk_act_table: zero rows are a no-op that
    needs no pointer; bad sizes, formats and activation codes are refused before any HIP call."""
    lib = L.load()
    # lsk_blockquant(x, x_dtype, ldx, M, K, q, ldq, ka, ldka, stream)
    assert lib.lsk_blockquant(None, L.LSK_BF16, 64, 0, 64, None, 64, None, 2, None) == 0
    assert lib.lsk_blockquant(None, L.LSK_F32, 48, 3, 48, None, 48, None, 1, None) == 1
    assert b"multiple of the 32-element block" in lib.lsk_last_error()
    assert lib.lsk_blockquant(None, L.LSK_F32, 64, -1, 64, None, 64, None, 2, None) == 1
    assert b"negative" in lib.lsk_last_error()
    # lsk_gemm_mx2(q, ldq, ka, ldka, b, b_fmt, ldb, kexp, lds, M, N, K, epilogue, bias, out, ldo, stream)
    assert lib.lsk_gemm_mx2(None, 64, None, 2, None, 1, 32, None, 2, 0, 16, 64, 0, None, None, 16, None) == 0
    assert lib.lsk_gemm_mx2(None, 64, None, 2, None, 1, 32, None, 2, 5, 0, 64, 0, None, None, 16, None) == 0
    assert lib.lsk_gemm_mx2(None, 64, None, 2, None, 2, 32, None, 2, 1, 16, 64, 0, None, None, 16, None) == 1
    assert b"b_fmt" in lib.lsk_last_error()
    assert lib.lsk_gemm_mx2(None, 64, None, 2, None, 1, 32, None, 2, 1, 16, 64, 3, None, None, 16, None) == 1
    assert b"epilogue" in lib.lsk_last_error()
    # lsk_router_topk(g, g_dtype, ldg, T, E, k, renormalize, tab, idx, w, stream)
    assert lib.lsk_router_topk(None, L.LSK_F32, 8, 0, 8, 2, 1, None, None, None, None) == 0
    assert lib.lsk_router_topk(None, L.LSK_F32, 8, 4, 8, 9, 1, None, None, None, None) == 1
    assert b"k=9" in lib.lsk_last_error()
    # lsk_act_table(frac, act, table, stream): an unknown activation code, then null tables
    assert lib.lsk_act_table(None, 7, None, None) == 1
    assert b"unknown act 7" in lib.lsk_last_error()
    assert lib.lsk_act_table(None, L.LSK_ACT_SILU, None, None) == 1
    assert b"null pointer" in lib.lsk_last_error()


def test_noalloc_entry_point_refuses_sizes_beyond_its_scratch_without_touching_the_gpu():
    lib = L.load()
    M, K = 4096, 8192                      # 32 MiB of quantised rows: above the 16 MiB scratch
    rc = lib.lsk_w8a8_matmul_noalloc(None, 0, K, M, K, None, K, 64, None, None, 0, None, 1, 64, None)
    assert rc == 1 and b"maximum" in lib.lsk_last_error()
    # M == 0 is a no-op, as for lsk_w8a8_matmul
    assert lib.lsk_w8a8_matmul_noalloc(None, 0, K, 0, K, None, K, 64, None, None, 0, None, 1, 64, None) == 0


def test_moe_forward_rejects_bad_kernel_choice():
    """lsk_moe_args.select / mx_select outside their ranges are rejected before any device work."""
    import ctypes
    from lockstep_amd import _lib as L
    lib = L.load()
    for sel, mxsel in ((10, 0), (0, 5), (-1, 0)):
        a = L.MoeArgs(T=1, H=16, I=16, E=1, k=1, select=sel, mx_select=mxsel)
        assert lib.lsk_moe_forward(ctypes.addressof(a), None) != 0
        assert b"select" in lib.lsk_last_error()
