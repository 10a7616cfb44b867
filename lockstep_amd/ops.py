"""Torch-level wrappers over the C ABI: shape / dtype / stride handling, output allocation.

These are the building blocks of the drop-in modules (`lockstep_fullstack`, `moe_ref`,
`contract_common`, `ref_block_v1`, `moe_mxfp4`), which keep the reference's signatures.
"""
from __future__ import annotations


import torch

from . import _lib as L


def _rows(x: torch.Tensor) -> torch.Tensor:
    """x [..., K] -> a 2-D view/copy [rows, K] with unit stride along K."""
    x2 = x.reshape(-1, x.shape[-1])
    if x2.shape[-1] > 0 and x2.stride(-1) != 1:
        x2 = x2.contiguous()
    return x2


def weight_nk(b8: torch.Tensor) -> torch.Tensor:
    """The reference passes weights as b8 [K, N] = W8.t() of a row-major W8 [N, K].  Return
    W8 [N, K] with unit stride along K: a free view when b8 is that transpose, else a copy."""
    w = b8.t()
    if w.shape[-1] > 0 and w.stride(-1) != 1:
        w = w.contiguous()
    return w


def _f32(t):
    if t is None:
        return None
    t = t.to(torch.float32)
    return t if t.is_contiguous() else t.contiguous()


def rowquant(x: torch.Tensor):
    """Per-row int8 quant of x [..., K] (f32 / bf16 / f16; other float dtypes go through f32).
    Returns (q int8 [..., K], asc f32 [...])."""
    L.require_cuda(x, what="rowquant")
    if x.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        x = x.to(torch.float32)
    lead = x.shape[:-1]
    K = x.shape[-1]
    x2 = _rows(x)
    M = x2.shape[0]
    q = torch.empty((M, K), dtype=torch.int8, device=x.device)
    asc = torch.empty((M,), dtype=torch.float32, device=x.device)
    L.call("lsk_rowquant", L.ptr(x2), L.dtype_code(x2.dtype), M, K, x2.stride(0) if M else K,
           L.ptr(q), K, L.ptr(asc), L.stream_of(x))
    return q.reshape(*lead, K), asc.reshape(lead)


def gemm(a8: torch.Tensor, w_nk: torch.Tensor, order: int, out_dtype: int, asc=None, ws=None, bias=None,
         erow=None, ecol=None, shift: int = 0, out: torch.Tensor = None) -> torch.Tensor:
    """Exact GEMM a8 [M, K] x w_nk [N, K]^T with the given epilogue, out [M, N]."""
    L.require_cuda(a8, w_nk, asc, ws, bias, erow, ecol, what="gemm")
    if a8.dtype != torch.int8 or w_nk.dtype != torch.int8:
        raise TypeError("gemm: int8 operands required, got %s x %s" % (a8.dtype, w_nk.dtype))
    M, K = a8.shape
    N, K2 = w_nk.shape
    if K != K2:
        raise ValueError("gemm: K mismatch %d vs %d" % (K, K2))
    a8 = a8 if (K == 0 or a8.stride(-1) == 1) else a8.contiguous()
    tdt = {L.LSK_F32: torch.float32, L.LSK_BF16: torch.bfloat16, L.LSK_F16: torch.float16,
           L.LSK_I32: torch.int32, L.LSK_BF16_AS_F32: torch.float32}[out_dtype]
    if out is None:
        out = torch.empty((M, N), dtype=tdt, device=a8.device)
    asc, ws, bias = _f32(asc), _f32(ws), _f32(bias)
    erow = None if erow is None else erow.to(torch.int32).contiguous()
    ecol = None if ecol is None else ecol.to(torch.int32).contiguous()
    if M and N:
        L.call("lsk_gemm_w8a8", L.ptr(a8), a8.stride(0) if M > 1 else max(K, 1), L.ptr(w_nk),
               w_nk.stride(0) if N > 1 else max(K, 1), M, N, K, order, L.ptr(asc), L.ptr(ws), L.ptr(bias),
               L.ptr(erow), L.ptr(ecol), int(shift), L.ptr(out), out_dtype, out.stride(0), L.stream_of(a8))
    return out


def epilogue(acc: torch.Tensor, order: int, out_dtype: int, asc=None, ws=None, bias=None,
             erow=None, ecol=None, shift: int = 0) -> torch.Tensor:
    """The contract epilogue over an existing int32 accumulator [M, N]."""
    L.require_cuda(acc, asc, ws, bias, erow, ecol, what="epilogue")
    if acc.dtype != torch.int32:
        acc = acc.to(torch.int32)
    acc = acc if acc.is_contiguous() else acc.contiguous()
    M, N = acc.shape
    tdt = {L.LSK_F32: torch.float32, L.LSK_BF16: torch.bfloat16, L.LSK_F16: torch.float16,
           L.LSK_BF16_AS_F32: torch.float32}[out_dtype]
    out = torch.empty((M, N), dtype=tdt, device=acc.device)
    asc, ws, bias = _f32(asc), _f32(ws), _f32(bias)
    erow = None if erow is None else erow.to(torch.int32).contiguous()
    ecol = None if ecol is None else ecol.to(torch.int32).contiguous()
    if M and N:
        L.call("lsk_epilogue_apply", L.ptr(acc), N, M, N, order, L.ptr(asc), L.ptr(ws), L.ptr(bias),
               L.ptr(erow), L.ptr(ecol), int(shift), L.ptr(out), out_dtype, N, L.stream_of(acc))
    return out


def w8a8_matmul(x2: torch.Tensor, w_nk: torch.Tensor, ws: torch.Tensor, bias, order: int,
                out_dtype: int, w_pairs=None) -> torch.Tensor:
    """Row quant + exact GEMM + epilogue in two launches, x2 [M, K] -> [M, N]; w_pairs: None or
    pack_row_pairs(w_nk), read when the GEMM takes the quantised rows in the row-pair layout."""
    L.require_cuda(x2, w_nk, ws, bias, what="w8a8_matmul")
    if x2.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        x2 = x2.to(torch.float32)
    x2 = _rows(x2)
    M, K = x2.shape
    N = w_nk.shape[0]
    tdt = {L.LSK_F32: torch.float32, L.LSK_BF16: torch.bfloat16, L.LSK_F16: torch.float16,
           L.LSK_BF16_AS_F32: torch.float32}[out_dtype]
    out = torch.empty((M, N), dtype=tdt, device=x2.device)
    if M == 0 or N == 0:
        return out
    nbytes = L.load().lsk_w8a8_matmul_workspace(M, K)
    ws_buf = torch.empty((nbytes,), dtype=torch.uint8, device=x2.device)
    ws, bias = _f32(ws), _f32(bias)
    L.call("lsk_w8a8_matmul_pairs", L.ptr(x2), L.dtype_code(x2.dtype), x2.stride(0) if M > 1 else max(K, 1), M, K,
           L.ptr(w_nk), w_nk.stride(0) if N > 1 else max(K, 1), L.ptr(w_pairs), N, L.ptr(ws), L.ptr(bias), order,
           L.ptr(out), out_dtype, N, L.ptr(ws_buf), nbytes, L.stream_of(x2))
    return out


_OUT_T = {L.LSK_F32: torch.float32, L.LSK_BF16: torch.bfloat16, L.LSK_F16: torch.float16,
          L.LSK_BF16_AS_F32: torch.float32}


def _float_code(t: torch.Tensor):
    """A float tensor as (contiguous tensor, dtype code): f32 / bf16 / f16 kept, others to f32."""
    if t.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        t = t.to(torch.float32)
    return (t if t.is_contiguous() else t.contiguous()), L.dtype_code(t.dtype)


def outlier_side(ho: torch.Tensor, wo: torch.Tensor) -> torch.Tensor:
    """side [M, N] binary32 = sum_j fl32(ho[m, j] * wo[n, j]), sequential in j from +0."""
    L.require_cuda(ho, wo, what="outlier_side")
    M, ko = ho.shape
    N, ko2 = wo.shape
    if ko != ko2:
        raise ValueError("outlier_side: ho has %d channels, wo %d" % (ko, ko2))
    h, hc = _float_code(ho)
    w, wc = _float_code(wo)
    side = torch.empty((M, N), dtype=torch.float32, device=ho.device)
    L.call("lsk_outlier_side", L.ptr(h), hc, M, ko, L.ptr(w), wc, N, L.ptr(side), L.stream_of(ho))
    return side


def w8a8_outlier_linear(x2: torch.Tensor, oidx: torch.Tensor, wo: torch.Tensor, w_nk: torch.Tensor,
                        ws: torch.Tensor, bias, rot: bool, out_dtype: int) -> torch.Tensor:
    """The v2.5 outlier linear of rows x2 [M, K] -> [M, N] of out_dtype (one C-ABI call)."""
    L.require_cuda(x2, oidx, wo, w_nk, ws, bias, what="w8a8_outlier_linear")
    x2, xc = _float_code(_rows(x2))
    M, K = x2.shape
    N = w_nk.shape[0]
    oi = oidx.reshape(-1).to(torch.int32).contiguous()
    ko = oi.numel()
    if wo.shape != (N, ko):
        raise ValueError("w8a8_outlier_linear: wo shape %s, expected [%d, %d]" % (tuple(wo.shape), N, ko))
    if wo.dtype == torch.bfloat16:
        wod, woc = (wo if wo.is_contiguous() else wo.contiguous()), L.LSK_BF16
    else:
        wod, woc = wo.to(torch.float32).contiguous(), L.LSK_F32
    out = torch.empty((M, N), dtype=_OUT_T[out_dtype], device=x2.device)
    if M == 0 or N == 0:
        return out
    nbytes = L.load().lsk_w8a8_outlier_linear_workspace(M, K, ko)
    work = torch.empty((nbytes,), dtype=torch.uint8, device=x2.device)
    ws, bias = _f32(ws), _f32(bias)
    L.call("lsk_w8a8_outlier_linear", L.ptr(x2), xc, x2.stride(0) if M > 1 else max(K, 1), M, K, L.ptr(oi), ko,
           L.ptr(wod), woc, L.ptr(w_nk), w_nk.stride(0) if N > 1 else max(K, 1), N, L.ptr(ws), L.ptr(bias),
           1 if rot else 0, L.ptr(out), out_dtype, N, L.ptr(work), nbytes, L.stream_of(x2))
    return out


def _bits_ok(bits):
    if bits not in (8, 11, 15):
        raise ValueError("width %d not supported (8, 11, 15)" % bits)


def quant_bits(x2: torch.Tensor, bits: int):
    """Per-row <bits> quant of x2 [M, K]: (a int32 [M, K], asc f32 [M])."""
    L.require_cuda(x2, what="quant_bits")
    _bits_ok(bits)
    x2, xc = _float_code(_rows(x2))
    M, K = x2.shape
    a = torch.empty((M, K), dtype=torch.int32, device=x2.device)
    asc = torch.empty((M,), dtype=torch.float32, device=x2.device)
    L.call("lsk_quant_planes", L.ptr(x2), xc, x2.stride(0) if M > 1 else max(K, 1), M, K, int(bits), None, 0, None,
           max(K, 1), L.ptr(a), L.ptr(asc), L.stream_of(x2))
    return a, asc


def quant_planes(W: torch.Tensor, bits: int, sdiv=None, sdiv_op: int = 0):
    """Per-row <bits> quant of W [N, K] (times / divided by sdiv per column) as stacked int8 planes
    [P * N, K] (hi plane rows first) and the f32 scales [N]."""
    L.require_cuda(W, sdiv, what="quant_planes")
    _bits_ok(bits)
    W2, wc = _float_code(_rows(W))
    N, K = W2.shape
    P = 1 if bits == 8 else 2
    q = torch.empty((P * N, K), dtype=torch.int8, device=W.device)
    ws = torch.empty((N,), dtype=torch.float32, device=W.device)
    sd = _f32(sdiv) if sdiv_op else None
    L.call("lsk_quant_planes", L.ptr(W2), wc, W2.stride(0) if N > 1 else max(K, 1), N, K, int(bits), L.ptr(sd),
           int(sdiv_op), L.ptr(q), max(K, 1), None, L.ptr(ws), L.stream_of(W))
    return q, ws


def split_planes(a: torch.Tensor, sh: int):
    """[(sh, hi int8), (0, lo int8)] of int32 values a (sh = 0: [(0, a as int8)])."""
    L.require_cuda(a, what="split_planes")
    a = a.to(torch.int32).contiguous()
    hi = torch.empty(a.shape, dtype=torch.int8, device=a.device)
    lo = torch.empty(a.shape, dtype=torch.int8, device=a.device) if sh else None
    L.call("lsk_split_planes", L.ptr(a), a.numel(), int(sh), L.ptr(hi), L.ptr(lo), L.stream_of(a))
    return [(0, hi)] if sh == 0 else [(int(sh), hi), (0, lo)]


def planes_linear(x2: torch.Tensor, w2: torch.Tensor, wbits: int, ws: torch.Tensor, abits: int, sdiv=None,
                  bias=None, out_dtype: int = L.LSK_F32) -> torch.Tensor:
    """The a<abits>w<wbits> linear of rows x2 [M, K] against stacked weight planes w2 [P * N, K]."""
    L.require_cuda(x2, w2, ws, sdiv, bias, what="planes_linear")
    _bits_ok(abits)
    _bits_ok(wbits)
    x2, xc = _float_code(_rows(x2))
    M, K = x2.shape
    P = 1 if wbits == 8 else 2
    if w2.shape[0] % P or w2.shape[1] != K:
        raise ValueError("planes_linear: weight planes %s do not fit K=%d and %d planes" % (tuple(w2.shape), K, P))
    if w2.stride(-1) != 1:
        w2 = w2.contiguous()
    N = w2.shape[0] // P
    out = torch.empty((M, N), dtype=_OUT_T[out_dtype], device=x2.device)
    if M == 0 or N == 0:
        return out
    nbytes = L.load().lsk_planes_linear_workspace(M, K, N, int(abits), int(wbits))
    work = torch.empty((nbytes,), dtype=torch.uint8, device=x2.device)
    ws, sdiv, bias = _f32(ws), _f32(sdiv), _f32(bias)
    L.call("lsk_planes_linear", L.ptr(x2), xc, x2.stride(0) if M > 1 else max(K, 1), M, K, int(abits), L.ptr(sdiv),
           L.ptr(w2), w2.stride(0) if w2.shape[0] > 1 else max(K, 1), N, int(wbits), L.ptr(ws), L.ptr(bias),
           L.ptr(out), out_dtype, N, L.ptr(work), nbytes, L.stream_of(x2))
    return out


def quant8_pow2(x: torch.Tensor, mode: int):
    """Power-of-two quant of x [M, K] binary32: mode 0 tensor, 1 rows, 2 columns.
    Returns (q int8 [M, K], e int32 [1] / [M] / [K])."""
    L.require_cuda(x, what="quant8_pow2")
    x = x.to(torch.float32)
    x = x if x.is_contiguous() else x.contiguous()
    M, K = x.shape
    q = torch.empty((M, K), dtype=torch.int8, device=x.device)
    ne = {0: 1, 1: M, 2: K}[mode]
    e = torch.zeros((max(ne, 1),), dtype=torch.int32, device=x.device)
    work = torch.empty((4 * (M + K + 64),), dtype=torch.uint8, device=x.device)
    L.call("lsk_quant8_pow2", L.ptr(x), M, K, max(K, 1), mode, L.ptr(q), max(K, 1), L.ptr(e), L.ptr(work),
           L.stream_of(x))
    return q, e[:ne]


def quant8_dyn(x: torch.Tensor, erow: bool = False):
    """Per-tensor power-of-two quant of x [..., K] binary32 on the device (lsk_quant8_dyn).
    Returns (q int8 [..., K], e int32 [1]) and, with erow, also the exponent repeated per row
    ([rows] int32, the POW2 epilogue's row operand); the exponent stays on the device."""
    L.require_cuda(x, what="quant8_dyn")
    x = x.to(torch.float32)
    lead, K = x.shape[:-1], x.shape[-1]
    x2 = _rows(x)
    M = x2.shape[0]
    q = torch.empty((M, K), dtype=torch.int8, device=x.device)
    e = torch.empty((1,), dtype=torch.int32, device=x.device)
    er = torch.empty((M,), dtype=torch.int32, device=x.device) if erow else None
    nbytes = L.load().lsk_quant8_dyn_workspace()
    work = torch.empty((nbytes,), dtype=torch.uint8, device=x.device)
    L.call("lsk_quant8_dyn", L.ptr(x2), M, K, x2.stride(0) if M > 1 else max(K, 1), L.ptr(q), max(K, 1), L.ptr(e),
           L.ptr(er), L.ptr(work), nbytes, L.stream_of(x))
    q = q.reshape(*lead, K)
    return (q, e, er) if erow else (q, e)


def pack_row_pairs(w_nk: torch.Tensor) -> torch.Tensor:
    """w_nk [N, K] int8 (K % 16 == 0) copied into the row-pair layout of the GEMM tiles
    (lsk_pack_row_pairs): a flat int8 tensor of lsk_row_pairs_bytes(N, K) bytes."""
    L.require_cuda(w_nk, what="pack_row_pairs")
    if w_nk.dim() != 2 or w_nk.dtype != torch.int8:
        raise ValueError("pack_row_pairs: w [N, K] int8 expected, got %s %s" % (tuple(w_nk.shape), w_nk.dtype))
    if w_nk.shape[1] > 0 and (w_nk.stride(1) != 1 or w_nk.stride(0) % 16 != 0):
        w_nk = w_nk.contiguous()
    N, K = w_nk.shape
    out = torch.empty((L.load().lsk_row_pairs_bytes(N, K),), dtype=torch.int8, device=w_nk.device)
    L.call("lsk_pack_row_pairs", L.ptr(w_nk), N, K, w_nk.stride(0) if N > 1 else max(K, 16), L.ptr(out),
           L.stream_of(w_nk))
    return out


# Row-pair copies of weights (the GEMM tiles read them in whole 128-byte lines): a prepared weight,
# like the reference's arm-time W8 / ws on the module (lockstep_fullstack.py:1010-1011).  The copy is
# held by the tensor that owns the weight's storage (an attribute of that tensor object), so it lives
# exactly as long as the weight, with no cap and no eviction: one more copy of each such weight in HBM
# (lsk_row_pairs_bytes(N, K), about N * K bytes).  Each entry records the owner's version counter,
# which every in-place write through the weight or a view of it advances; a stale copy is remade.
# ROW_PAIR_COPIES = False turns the copies off (the GEMMs then read the weights themselves);
# release_row_pairs(w) frees a weight's copies.  row_pair_packs counts the copies made.
ROW_PAIR_COPIES = True
row_pair_packs = 0
_ATTR = "_lsk_row_pairs"


def _pair_key(w_nk):
    owner = w_nk._base if w_nk._base is not None else w_nk
    return owner, (w_nk.data_ptr(), int(w_nk.shape[0]), int(w_nk.shape[1]), int(w_nk.stride(0)))


def row_pair_copy(w_nk):
    """pack_row_pairs(w_nk), made once per weight and kept on the tensor owning its storage while
    that tensor is unchanged; None where the layout does not apply (K % 16 != 0, a strided or
    unaligned weight), while a graph is being captured (the graph then reads the weight itself, so
    replays follow later in-place updates of it), or with ROW_PAIR_COPIES off."""
    global row_pair_packs
    if not ROW_PAIR_COPIES or w_nk.dim() != 2 or w_nk.dtype != torch.int8:
        return None
    N, K = w_nk.shape
    if K == 0 or N == 0 or K % 16 != 0 or w_nk.stride(1) != 1 or w_nk.stride(0) % 16 != 0 \
            or w_nk.data_ptr() % 16 != 0:
        return None
    if w_nk.is_cuda and torch.cuda.is_current_stream_capturing():
        return None
    owner, key = _pair_key(w_nk)
    held = owner.__dict__.get(_ATTR)
    if held is None:
        held = {}
        setattr(owner, _ATTR, held)
    hit = held.get(key)
    if hit is not None and hit[0] == owner._version:
        return hit[1]
    held.pop(key, None)                      # stale: free it before the new copy is made
    packed = pack_row_pairs(w_nk)
    row_pair_packs += 1
    held[key] = (owner._version, packed)
    return packed


def row_pairs_of(w_nk, rows):
    """The weight's row-pair copy when a GEMM of `rows` activation rows against w_nk [N, K] reads one
    (lsk_gemm_reads_row_pairs under the calling thread's tile selection), else None."""
    if w_nk.dim() != 2 or not int(rows) > 0:
        return None
    N, K = w_nk.shape
    if K % 16 != 0 or not L.load().lsk_gemm_reads_row_pairs(int(rows), int(N), int(K)):
        return None
    return row_pair_copy(w_nk)


def release_row_pairs(w_nk):
    """Free every row-pair copy held for the weight's storage."""
    owner, _ = _pair_key(w_nk)
    owner.__dict__.pop(_ATTR, None)


def linear_dyn(x: torch.Tensor, w_nk: torch.Tensor, ew: int, stages: int = 3, work=None, y=None, ex=None,
               w_pairs=None):
    """quant8_dyn of x [T, K] binary32 and the exact GEMM with w_nk [N, K] int8 under the POW2
    dequant 2^-(ex + ew), in one call (lsk_linear_dyn).  Returns (y binary32 [T, N], ex int32 [1]
    on the device).  stages 1 / 2 run only the quant / only the GEMM (the same work buffer
    carries q between them), for timing the GEMM alone.  w_pairs: pack_row_pairs(w_nk) or None."""
    L.require_cuda(x, w_nk, what="linear_dyn")
    x = x.to(torch.float32)
    if x.dim() != 2 or w_nk.dim() != 2 or w_nk.dtype != torch.int8 or w_nk.shape[1] != x.shape[1]:
        raise ValueError("linear_dyn: x [T, K] binary32 and w [N, K] int8 expected, got %s and %s %s"
                         % (tuple(x.shape), tuple(w_nk.shape), w_nk.dtype))
    if x.shape[1] > 0 and x.stride(1) != 1:
        x = x.contiguous()
    if w_nk.shape[1] > 0 and w_nk.stride(1) != 1:
        w_nk = w_nk.contiguous()
    M, K = x.shape
    N = w_nk.shape[0]
    if y is None:
        y = torch.empty((M, N), dtype=torch.float32, device=x.device)
    if ex is None:
        ex = torch.empty((1,), dtype=torch.int32, device=x.device)
    nbytes = L.load().lsk_linear_dyn_workspace(M, K)
    if work is None:
        work = torch.empty((nbytes,), dtype=torch.uint8, device=x.device)
    elif work.numel() < nbytes:
        raise ValueError("linear_dyn: work buffer of %d bytes, %d needed" % (work.numel(), nbytes))
    if w_pairs is not None and (w_pairs.dtype != torch.int8 or w_pairs.device != x.device
                                or w_pairs.numel() < L.load().lsk_row_pairs_bytes(N, K)):
        raise ValueError("linear_dyn: w_pairs is not pack_row_pairs of a [%d, %d] weight" % (N, K))
    L.call("lsk_linear_dyn", L.ptr(x), M, K, x.stride(0) if M > 1 else max(K, 1), L.ptr(w_nk),
           w_nk.stride(0) if N > 1 else max(K, 1), L.ptr(w_pairs), N, int(ew), L.ptr(y),
           y.stride(0) if M > 1 else max(N, 1),
           L.ptr(ex), int(stages), L.ptr(work), work.numel(), L.stream_of(x))
    return y, ex


OP_SILU, OP_SIGMOID, OP_ACT_SILU, OP_ACT_SWIGLUOAI = 0, 1, 2, 3


def frac_i32(dev) -> torch.Tensor:
    """The FRAC (13, 15) table as int32 on `dev` (values < 2^16), built once per device."""
    from . import contract_common as CC
    return CC.table_i32_on(dev)


_ACT_TABLES = {}


def act_table(dev, act: int) -> torch.Tensor:
    """The activation's gate table over the 65536 bf16 bit patterns (lsk_act_table), built once per
    device and activation."""
    dev = torch.device(dev)
    key = (str(dev), int(act))
    t = _ACT_TABLES.get(key)
    if t is None:
        t = torch.empty(65536, dtype=torch.float32, device=dev)
        L.call("lsk_act_table", L.ptr(frac_i32(dev)), int(act), L.ptr(t), L.stream_of(t))
        _ACT_TABLES[key] = t
    return t


def tab_i32(tab: torch.Tensor) -> torch.Tensor:
    """A caller's router table (int64 in the reference) as the int32 table the kernels read."""
    L.require_cuda(tab, what="table")
    if tab.numel() != 8192:
        raise ValueError("the router table must have 8192 entries (TAB_N = 13), got %d" % tab.numel())
    return tab.to(torch.int32).contiguous()


def act(g: torch.Tensor, u, op: int) -> torch.Tensor:
    """Elementwise table activation in binary32 (shape of g)."""
    L.require_cuda(g, u, what="activation")
    gf = g.to(torch.float32).contiguous()
    uf = None
    if u is not None:
        uf = u.to(torch.float32)
        if uf.shape != gf.shape:
            uf = uf.expand(gf.shape)
        uf = uf.contiguous()
    out = torch.empty_like(gf)
    L.call("lsk_act_elementwise", L.ptr(gf), L.ptr(uf), gf.numel(), op, L.ptr(frac_i32(g.device)), L.ptr(out),
           L.stream_of(g))
    return out


def table_scores(dgap: torch.Tensor, tab: torch.Tensor) -> torch.Tensor:
    L.require_cuda(dgap, tab, what="table_scores")
    d = dgap.to(torch.float32).contiguous()
    out = torch.empty(d.shape, dtype=torch.int64, device=d.device)
    L.call("lsk_table_scores", L.ptr(d), d.numel(), L.ptr(tab_i32(tab)), L.ptr(out), L.stream_of(d))
    return out


def fwht_blocks(x: torch.Tensor, blk: int = 256, scale: float = 1.0 / 16.0) -> torch.Tensor:
    L.require_cuda(x, what="fwht_blocks")
    sh = x.shape
    x2 = x.to(torch.float32).reshape(-1, sh[-1]).contiguous()
    y = torch.empty_like(x2)
    L.call("lsk_fwht_blocks", L.ptr(x2), x2.shape[0], x2.shape[1], x2.shape[1], int(blk), float(scale), L.ptr(y),
           x2.shape[1], L.stream_of(x))
    return y.reshape(sh)


def router_topk(g: torch.Tensor, k: int, renormalize: bool, tab: torch.Tensor):
    """Top-k routing from logits g [T, E] (bf16 values): (idx int64 [T, k], w bf16 [T, k])."""
    L.require_cuda(g, tab, what="router")
    T, E = g.shape
    if g.dtype == torch.bfloat16:
        gd, code = g.contiguous(), L.LSK_BF16
    else:
        gd, code = g.to(torch.float32).contiguous(), L.LSK_F32
    idx = torch.empty((T, k), dtype=torch.int64, device=g.device)
    w = torch.empty((T, k), dtype=torch.bfloat16, device=g.device)
    if T:
        L.call("lsk_router_topk", L.ptr(gd), code, E, T, E, int(k), 1 if renormalize else 0, L.ptr(tab_i32(tab)),
               L.ptr(idx), L.ptr(w), L.stream_of(g))
    return idx, w


def gemm_mx(a8: torch.Tensor, b: torch.Tensor, kexp: torch.Tensor, b_fmt: int, asc=None, bias=None,
            epilogue: int = 0) -> torch.Tensor:
    """MX-operand GEMM: a8 int8 [M, K] with m2 int8 [N, K] (b_fmt 0) or packed E2M1 [N, K/2]
    (b_fmt 1) and E8M0 kexp [N, K/32] -> binary32 [M, N] (epilogue 1: bfr(acc * asc) + bias)."""
    L.require_cuda(a8, b, kexp, asc, bias, what="gemm_mx")
    if a8.dtype != torch.int8:
        raise TypeError("gemm_mx: a8 must be int8")
    a8 = a8 if (a8.stride(-1) == 1 and a8.stride(0) % 16 == 0) else a8.contiguous()
    b = b.contiguous()
    kexp = kexp.to(torch.uint8).contiguous()
    M, K = a8.shape
    N = b.shape[0]
    out = torch.empty((M, N), dtype=torch.float32, device=a8.device)
    if M and N:
        ld_a = a8.stride(0) if M > 1 else K
        asc, bias = _f32(asc), _f32(bias)
        L.call("lsk_gemm_mx", L.ptr(a8), ld_a, L.ptr(b), int(b_fmt), b.stride(0), L.ptr(kexp), kexp.stride(0),
               M, N, K, int(epilogue), L.ptr(asc), L.ptr(bias), L.ptr(out), N, L.stream_of(a8))
    return out


def blockquant(x: torch.Tensor):
    """Per-32-block int8 quant with power-of-two block exponents: x [T, K] (bf16 / f32; other float
    dtypes go through f32), K % 32 == 0 -> (q int8 [T, K], ka int32 [T, K/32])."""
    L.require_cuda(x, what="blockquant")
    if x.dim() != 2:
        raise ValueError("blockquant: x must be [T, K]")
    if x.dtype not in (torch.float32, torch.bfloat16):
        x = x.to(torch.float32)
    T, K = x.shape
    if K % 32:
        raise ValueError("blockquant: K=%d not a multiple of 32" % K)
    x = x.contiguous()
    q = torch.empty((T, K), dtype=torch.int8, device=x.device)
    ka = torch.empty((T, K // 32), dtype=torch.int32, device=x.device)
    if T and K:
        L.call("lsk_blockquant", L.ptr(x), L.dtype_code(x.dtype), K, T, K, L.ptr(q), K, L.ptr(ka), K // 32,
               L.stream_of(x))
    return q, ka


def gemm_mx2(q: torch.Tensor, ka: torch.Tensor, b: torch.Tensor, kexp: torch.Tensor, b_fmt: int, bias=None,
             epilogue: int = 0) -> torch.Tensor:
    """MX operand with block-scaled activations: q int8 [M, K] and ka int32 [M, K/32] with m2 int8
    [N, K] (b_fmt 0) or packed E2M1 [N, K/2] (b_fmt 1) and E8M0 kexp [N, K/32] -> binary32 [M, N]
    (epilogue 1: bfr(acc), then bfr(+ bias))."""
    L.require_cuda(q, ka, b, kexp, bias, what="gemm_mx2")
    if q.dtype != torch.int8:
        raise TypeError("gemm_mx2: q must be int8")
    M, K = q.shape
    if tuple(ka.shape) != (M, K // 32):
        raise ValueError("gemm_mx2: ka %s does not match q %s" % (tuple(ka.shape), tuple(q.shape)))
    q = q if (q.stride(-1) == 1 and q.stride(0) % 16 == 0) else q.contiguous()
    ka = ka.to(torch.int32).contiguous()
    b = b.contiguous()
    kexp = kexp.to(torch.uint8).contiguous()
    N = b.shape[0]
    out = torch.empty((M, N), dtype=torch.float32, device=q.device)
    if M and N:
        ld_q = q.stride(0) if M > 1 else K
        L.call("lsk_gemm_mx2", L.ptr(q), ld_q, L.ptr(ka), K // 32, L.ptr(b), int(b_fmt), b.stride(0), L.ptr(kexp),
               kexp.stride(0), M, N, K, int(epilogue), L.ptr(_f32(bias)), L.ptr(out), N, L.stream_of(q))
    return out


def mx_epilogue(acc: torch.Tensor, asc: torch.Tensor, bias=None) -> torch.Tensor:
    L.require_cuda(acc, asc, bias, what="lin_epilogue_mx")
    acc = acc.to(torch.float32).contiguous()
    M, N = acc.shape
    out = torch.empty_like(acc)
    L.call("lsk_mx_epilogue", L.ptr(acc), M, N, L.ptr(_f32(asc)), L.ptr(_f32(bias)), L.ptr(out), L.stream_of(acc))
    return out


def dequant_mxfp4(packed: torch.Tensor, scale: torch.Tensor, out_dtype=torch.bfloat16, block: int = 32):
    L.require_cuda(packed, scale, what="dequant_mxfp4")
    lead = packed.shape[:-1]
    K = packed.shape[-1] * 2
    if scale.shape[-1] * block != K:
        raise AssertionError((tuple(scale.shape), K))
    p2 = packed.to(torch.uint8).reshape(-1, K // 2).contiguous()
    s2 = scale.to(torch.uint8).reshape(-1, K // block).contiguous()
    code = L.LSK_BF16 if out_dtype == torch.bfloat16 else L.LSK_F32
    out = torch.empty((p2.shape[0], K), dtype=torch.bfloat16 if code == L.LSK_BF16 else torch.float32,
                      device=packed.device)
    L.call("lsk_dequant_mxfp4", L.ptr(p2), L.ptr(s2), p2.shape[0], K, int(block), L.ptr(out), code,
           L.stream_of(packed))
    out = out.reshape(*lead, K)
    return out if out.dtype == out_dtype else out.to(out_dtype)


def pack_m2(m2: torch.Tensor):
    """Doubled mantissas m2 int8 [..., K] -> packed E2M1 codes uint8 [..., K/2]; raises if some
    value is not twice an E2M1 value (one host synchronisation)."""
    L.require_cuda(m2, what="pack_m2")
    m = m2.to(torch.int8).contiguous()
    packed = torch.empty((*m.shape[:-1], m.shape[-1] // 2), dtype=torch.uint8, device=m.device)
    bad = torch.zeros((1,), dtype=torch.int32, device=m.device)
    L.call("lsk_mx_pack_m2", L.ptr(m), m.numel(), L.ptr(packed), L.ptr(bad), L.stream_of(m))
    if int(bad.item()):
        raise ValueError("m2 holds a value that is not 2 * an E2M1 value {0, +-1, +-2, +-3, +-4, +-6, +-8, +-12}")
    return packed
