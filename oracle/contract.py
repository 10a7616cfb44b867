"""CPU oracle: a numpy restatement of the reference's contract matrix-multiply path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package (`lockstep_amd`) may import,
call or link anything under `oracle/`; only the tests, `__graft_entry__.smoke()` and the
`cpu_baseline` leg of `bench.py` use it, and only as the checker.

Every function restates one reference function (file:line cited in its docstring) with
numpy float32 / integer arithmetic.  numpy float32 `+ - * /` are single IEEE binary32
operations rounded to nearest-even, `np.rint` rounds half to even, and int -> float32
casts round to nearest-even, so each torch op of the reference maps to one numpy op here.

Pinning (how each function is checked, see tests/test_oracle_*.py):
  rowquant / quantize_rows_int8 / quantize_weight_int8 / lin_epilogue / w8a8_matmul:
      the committed conformance digests act_quant.*, weight_quant.*, linear.v2_1.*
  silu_contract / act_silu: the silu / silu_mul digests
  fwht_blocks: the r4.block256 digest and the Hadamard closed form
  frac table: FRAC_DIGEST (sha256 of the 8192 uint16 entries)
  int_mm: two independent exact methods (int64 and float64-BLAS) against each other
  quant8_* (pow2): brute force over exponents and closed-form edge cases; the quantised values
      of quant8_rows / quant8_cols by round-half-even of the exact rational x * 2^e in Python
      integers, with a truncation slip that must differ
  fp4 / dequant_mxfp4: the closed form fp4 * 2^(e-127) over all codes and exponents
  int_mm_mx: one-block closed form, equal-exponent integer identity, scalar brute force,
      and a negative control (reversed block order differs)
  lin_epilogue_mx: rational brute force of bfr(fl32(acc * asc)) then bfr(fl32(y + b)), with two
      slips that must differ (bias before the first bf16 rounding; one merged rounding)
  router / combine / moe_forward*: scalar brute force in Python ints and numpy float32
  blockquant (MX2): the exact exponent min{k : 127 * 2^k >= am} clamped to [-126, 127] from the
      binary32 bits, round-half-even halves, the reconstruction bound, negative controls
  int_mm_mx2: equals int_mm_mx with kexp + c when every ka is c (row by row), the one-block
      closed form fl32(s * fl32(2^e)) from binary64 including underflow to 0 / overflow to inf,
      a negative control (the fused block update differs below 2^-149)
  expert_block_mx2 / moe_forward_mx2: compositions of the pinned pieces in moe_ref.py's order
  row_sum_float / rmsnorm_float (contract 2.6 float norm): the digests norm_float.*, a
      rational brute force of the tree, the zero-padded balanced tree identity
  outlier_side / w8a8_outlier_linear: the digests outlier.*, linear.v2_5.*, linear.v2_5_1.*
  quant_rows_bits / planes / quantize_weight_bits / mm_planes: rowquant at 8 bits (digest-pinned),
      rational brute force of the quant at 11 / 15 bits, the plane identity (hi << sh) + lo = a,
      the int64 combine equal to the direct exact product, an RNE brute force of fl32(s)
  w8a8_linear (E-v2 order), sigmoid_contract, act_swigluoai, mm_planes' epilogue order:
      parity unpinned by any reference-held vector; checked by scalar brute force of the
      written rule only.  smooth_scales (binary32 pow): parity unpinned.
"""
from __future__ import annotations

import hashlib

import numpy as np

F32 = np.float32
MX_BLOCK = 32
INT8_LIM = 127
RNE_MIN_AMAX = F32(1e-8)          # torch clamp(min=1e-8) casts the scalar to binary32
SILU_C = F32(-1.4426950216293335)  # lockstep_fullstack.py:175, 0xBFB8AA3B
F32_MIN_NORMAL = F32(1.1754943508222875e-38)
SWIGLU_ALPHA = F32(1.702)          # moe_ref.py:146
SWIGLU_LIMIT = F32(7.0)            # moe_ref.py:147
BHI, TAB_N, TAB_W = 26, 13, 15     # moe_ref.py:60
# moe_ref.py:61: 2^26 / ln 2 in binary64, then rounded once to binary32 (moe_ref.py:68)
ROUTER_C = F32(float(2.0 ** BHI) / 0.6931471805599453)
FRAC_DIGEST = "f472476ccea65299feb63f1ff863714a35910d2099470bafb5d3be0e92a598cd"  # contract_common.py:12
FRAC_COEFFS = [1073741823, -744260975, 257938938, -59583045, 10286509, -1369790, 117454]  # contract_common.py:29


# ----------------------------------------------------------------------------- bf16 helpers
def bf16_bits(x) -> np.ndarray:
    """binary32 -> bf16 bit pattern, round to nearest even; NaN -> 0x7FC0 (torch's c10::BFloat16
    conversion; the same method as reference/t16n_ref.py:95-100)."""
    u = np.ascontiguousarray(x, dtype=F32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(np.asarray(x, dtype=F32))
    return np.where(nan, np.uint16(0x7FC0), r).astype(np.uint16)


def bf16_to_f32(bits) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(F32)


def bfr(x) -> np.ndarray:
    """fl32 -> bf16 -> fl32 (moe_ref.py:22-24)."""
    return bf16_to_f32(bf16_bits(x))


def cast_out(y: np.ndarray, out: str) -> np.ndarray:
    """Round a binary32 array to the named output type, returned as that type's numpy
    carrier: 'f32' -> float32, 'bf16' -> uint16 bits, 'f16' -> float16 (RNE)."""
    if out == "f32":
        return y.astype(F32)
    if out == "bf16":
        return bf16_bits(y)
    if out == "f16":
        return y.astype(F32).astype(np.float16)
    raise ValueError(out)


def out_to_f32(y: np.ndarray, out: str) -> np.ndarray:
    return bf16_to_f32(y) if out == "bf16" else y.astype(F32)


# ----------------------------------------------------------------------------- A1 row quant
def rowquant(x):
    """moe_ref.py:27-37 (== lockstep_fullstack.quantize_rows_int8 :476-481 and the inline
    quant of contract_common.w8a8_linear :168-169): am = max(max_k |x|, fl32(1e-8));
    asc = fl32(am / 127) (a true division); q = clamp(rint_even(fl32(x / asc)), +-127)."""
    xf = np.asarray(x, dtype=F32)
    if xf.shape[-1] == 0:
        am = np.zeros(xf.shape[:-1] + (1,), dtype=F32)
    else:
        am = np.abs(xf).max(axis=-1, keepdims=True)
    am = np.maximum(am, RNE_MIN_AMAX)
    asc = (am / F32(127.0)).astype(F32)
    with np.errstate(invalid="ignore", divide="ignore"):
        q = np.clip(np.rint((xf / asc).astype(F32)), -127, 127).astype(np.int8)
    return q, asc[..., 0]


quantize_rows_int8 = rowquant


def quantize_weight_int8(W):
    """lockstep_fullstack.py:581-587: per-output-channel rowquant of the weight [N, K]."""
    return rowquant(W)


# ----------------------------------------------------------------------------- A2 exact int GEMM
def int_mm(a8, b8, method: str = "f64"):
    """moe_ref.py:48-55 / lockstep_fullstack.py:484-500 / ref_block_v1.py:132-133:
    acc[m, n] = sum_k a8[m, k] * b8[k, n], exact.  b8 is [K, N] (the reference's W8.t()).

    method 'i64' is the reference's own op sequence (int64 matmul, then narrowed);
    method 'f64' uses binary64 BLAS, exact because every partial sum is an integer of
    magnitude <= K * 127 * 127 < 2^53 (asserted)."""
    a = np.asarray(a8)
    b = np.asarray(b8)
    K = a.shape[-1]
    if method == "i64":
        return (a.astype(np.int64) @ b.astype(np.int64)).astype(np.int32)
    amax = int(np.abs(a.astype(np.int64)).max()) if a.size else 0
    bmax = int(np.abs(b.astype(np.int64)).max()) if b.size else 0
    assert K * amax * bmax < 2 ** 53, "float64 path not exact at this K"
    return (a.astype(np.float64) @ b.astype(np.float64)).astype(np.int64).astype(np.int32)


# ----------------------------------------------------------------------------- A3 epilogues
def lin_epilogue(acc, ws, asc):
    """moe_ref.py:40-42 (E-v2.1): bfr( fl32( fl32(fl32(acc) * ws[n]) * asc[m] ) )."""
    y = (np.asarray(acc).astype(F32) * np.asarray(ws, F32)[None, :]).astype(F32)
    y = (y * np.asarray(asc, F32)[:, None]).astype(F32)
    return bfr(y)


def lin_epilogue_b(acc, ws, asc, bias=None):
    """moe_ref.py:164-169: the E-v2.1 epilogue, then bfr(y + b[n]) as a second rounding."""
    y = lin_epilogue(acc, ws, asc)
    if bias is not None:
        y = bfr((y + np.asarray(bias, F32)[None, :]).astype(F32))
    return y


def epilogue_v21(acc, ws, asc, bias=None, out="bf16"):
    """lockstep_fullstack.py:524-527 (the w8a8_matmul order): y = fl32(fl32(acc)*ws)*asc,
    cast to `out`; with a bias, cast(fl32(y_out) + bias)."""
    y = (np.asarray(acc).astype(F32) * np.asarray(ws, F32)[None, :]).astype(F32)
    y = (y * np.asarray(asc, F32)[:, None]).astype(F32)
    yo = cast_out(y, out)
    if bias is not None:
        yo = cast_out((out_to_f32(yo, out) + np.asarray(bias, F32)[None, :]).astype(F32), out)
    return yo


def epilogue_v2(acc, ws, asc, bias=None, out="bf16"):
    """contract_common.py:172-174 (E-v2, legacy): y = fl32(fl32(acc)*asc)*ws; with a bias
    y = fl32(y + bias) before the single cast to the output type."""
    y = (np.asarray(acc).astype(F32) * np.asarray(asc, F32)[:, None]).astype(F32)
    y = (y * np.asarray(ws, F32)[None, :]).astype(F32)
    if bias is not None:
        y = (y + np.asarray(bias, F32)[None, :]).astype(F32)
    return cast_out(y, out)


# ----------------------------------------------------------------------------- A4 / A5 dense linears
def w8a8_matmul(x, W8, ws, bias=None, out="bf16"):
    """lockstep_fullstack.py:503-530.  x [rows, K] (binary32 values), W8 [N, K] int8,
    ws [N] fp32 -> [rows, N] in `out`.  Row chunking is bit-invisible, so none here."""
    x2 = np.asarray(x, F32).reshape(-1, np.shape(x)[-1])
    N = W8.shape[0]
    if x2.shape[0] == 0:
        return cast_out(np.zeros((0, N), F32), out)
    q, asc = quantize_rows_int8(x2)
    acc = int_mm(q, np.asarray(W8).T)
    return epilogue_v21(acc, ws, asc, bias, out)


def w8a8_linear_prepare(W):
    """contract_common.py:161-164: the arm-time weight quant (same rule as rowquant)."""
    return quantize_weight_int8(W)


def w8a8_linear_fwd(x, W8, ws, bias=None, out="f32"):
    """contract_common.py:166-174: rowquant, exact GEMM, E-v2 epilogue, one cast."""
    x2 = np.asarray(x, F32).reshape(-1, np.shape(x)[-1])
    q, asc = rowquant(x2)
    acc = int_mm(q, np.asarray(W8).T)
    return epilogue_v2(acc, ws, asc, bias, out)


# ----------------------------------------------------------------------------- A6 pow2 (ref_block_v1)
def _e_from_max(m):
    """ref_block_v1.py:56-62: e = 6 - (biased_exp(m) - 127); e = 0 where m == 0;
    e -= 1 where fl32(m * 2^e) > 127; clip to [-32, 40]."""
    m = np.asarray(m, F32)
    e = 6 - ((m.view(np.uint32).astype(np.int64) >> 23) - 127)
    e = np.where(m == 0, 0, e)
    with np.errstate(over="ignore"):
        over = (m * np.ldexp(F32(1.0), e).astype(F32)).astype(F32) > F32(127.0)
    e = np.where(over, e - 1, e)
    return np.clip(e, -32, 40)


def quant8_rows(x):
    """ref_block_v1.py:64-67: per-row pow2 quant; q int64 [T, D], e int64 [T]."""
    x = np.asarray(x, F32)
    e = _e_from_max(np.max(np.abs(x), axis=1))
    q = np.clip(np.rint((x * np.ldexp(F32(1.0), e)[:, None].astype(F32)).astype(F32)), -127, 127).astype(np.int64)
    return q, e


def quant8_cols(w):
    """ref_block_v1.py:69-72: per-column pow2 quant; q int64 [D, N], e int64 [N]."""
    w = np.asarray(w, F32)
    e = _e_from_max(np.max(np.abs(w), axis=0))
    q = np.clip(np.rint((w * np.ldexp(F32(1.0), e)[None, :].astype(F32)).astype(F32)), -127, 127).astype(np.int64)
    return q, e


def quant8_dyn(x):
    """ref_block_v1.py:122-130: per-tensor pow2 quant; returns (q int64, e int)."""
    x = np.asarray(x, F32)
    m = F32(np.max(np.abs(x))) if x.size else F32(0)
    if m == 0:
        return np.zeros_like(x, dtype=np.int64), 0
    e = 6 - ((np.float32(m).view(np.uint32) >> 23).astype(np.int64) - 127)
    if F32(m * F32(2.0 ** int(e))) > F32(127.0):
        e -= 1
    e = int(max(-32, min(40, int(e))))
    return np.clip(np.rint((x * F32(2.0 ** e)).astype(F32)), -127, 127).astype(np.int64), e


def gemm_int(a, b):
    """ref_block_v1.py:132-133: exact integer GEMM a [M, K] @ b [K, N] (int64 out)."""
    return np.asarray(a).astype(np.int64) @ np.asarray(b).astype(np.int64)


def dequant_pow2(acc, shift):
    """ref_block_v1.py:167,193,198,218: fl32(acc) * fl32(2^-shift), shift = ea + eb
    (an integer, or an array broadcast against acc as in the per-row/column form :213-214)."""
    sc = np.ldexp(F32(1.0), -np.asarray(shift, dtype=np.int64)).astype(F32)
    return (np.asarray(acc).astype(F32) * sc).astype(F32)


# ----------------------------------------------------------------------------- FRAC table, SiLU, sigmoid
def build_table(n=13, w=15):
    """contract_common.py:33-41: FRAC_{n,w}[k] = (Horner(t = k << (20-n)) + 2^(29-w)) >> (30-w),
    each Horner step p = c + floor(p * t / 2^20) in exact integers."""
    tab = []
    for k in range(1 << n):
        t = k << (20 - n)
        p = FRAC_COEFFS[6]
        for c in FRAC_COEFFS[5::-1]:
            p = c + ((p * t) // (1 << 20))
        tab.append((p + (1 << (29 - w))) >> (30 - w))
    return np.asarray(tab, dtype=np.int64)


_FRAC = None


def frac_table():
    global _FRAC
    if _FRAC is None:
        t = build_table(13, 15)
        d = hashlib.sha256(np.asarray(t, dtype="<u2").tobytes()).hexdigest()
        assert d == FRAC_DIGEST, "FRAC digest mismatch"
        _FRAC = t
    return _FRAC


def pow2_f32(e):
    """lockstep_fullstack.py:280-284: exact 2^e from the exponent field, e in [-126, 127]."""
    return ((np.asarray(e, np.int64) + 127).astype(np.int32) << 23).view(F32)


def _sigmoid_steps(x):
    """Steps (1)-(9) shared by silu_contract (lockstep_fullstack.py:590-604) and
    sigmoid_contract (moe_ref.py:150-161).  Returns (xc, sig)."""
    x = np.asarray(x, F32)
    frac = frac_table()
    xc = np.where(np.abs(x) < F32_MIN_NORMAL, F32(0.0), x).astype(F32)
    t = np.clip((xc * SILU_C).astype(F32), F32(-30.0), F32(30.0))
    i = np.ceil(t).astype(F32)
    g = (i - t).astype(F32)
    k = np.minimum(np.trunc((g * F32(8192.0)).astype(F32)), F32(8191.0)).astype(np.int64)
    f = (frac[k].astype(F32) * F32(2.0 ** -15)).astype(F32)
    e2 = (f * pow2_f32(i.astype(np.int64))).astype(F32)
    den = (F32(1.0) + e2).astype(F32)
    sig = (F32(1.0) / den).astype(F32)
    return xc, sig


def silu_contract(x):
    """lockstep_fullstack.py:590-604: the ten declared binary32 steps."""
    xc, sig = _sigmoid_steps(x)
    return (xc * sig).astype(F32)


def sigmoid_contract(x):
    """moe_ref.py:150-161: silu_contract without its final multiply."""
    return _sigmoid_steps(x)[1]


def act_silu(gate, up):
    """moe_ref.py:183-186: bfr( fl32(silu(g)) * u )."""
    return bfr((silu_contract(gate) * np.asarray(up, F32)).astype(F32))


def act_swigluoai(gate, up):
    """moe_ref.py:172-180: gc = min(g, 7); uc = clamp(u, -7, 7); arg = bfr(gc * 1.702);
    glu = bfr(gc * sig(arg)); h = bfr((uc + 1) * glu)."""
    g = np.asarray(gate, F32)
    u = np.asarray(up, F32)
    gc = np.minimum(g, SWIGLU_LIMIT)
    uc = np.clip(u, -SWIGLU_LIMIT, SWIGLU_LIMIT)
    arg = bfr((gc * SWIGLU_ALPHA).astype(F32))
    glu = bfr((gc * sigmoid_contract(arg)).astype(F32))
    return bfr(((uc + F32(1.0)).astype(F32) * glu).astype(F32))


# ----------------------------------------------------------------------------- two-plane wide-integer linears
def quant_rows_bits(x2, abits, sdiv=None, sdiv_op=0):
    """t16h_lmvariants.py:80-84 (_quant_rows) and :95-103 (quantize_weight's quant): amax_q =
    2^(bits-1) - 1; asc = fl32(max(max_k |v|, fl32(1e-8)) / amax_q); a = clamp(rint(fl32(v / asc)),
    +-amax_q) as int64.  v = x, or fl32(x / sdiv) (sdiv_op 1, Variant.logits :154), or
    fl32(x * sdiv) (sdiv_op 2, the fold of Variant.prepare :145)."""
    v = np.asarray(x2, F32)
    if sdiv_op == 1:
        v = (v / np.asarray(sdiv, F32)[None, :]).astype(F32)
    elif sdiv_op == 2:
        v = (v * np.asarray(sdiv, F32)[None, :]).astype(F32)
    qmax = F32((1 << (abits - 1)) - 1)
    am = np.abs(v).max(axis=1) if v.shape[1] else np.zeros(v.shape[0], F32)
    asc = (np.maximum(am, RNE_MIN_AMAX) / qmax).astype(F32)
    with np.errstate(invalid="ignore", divide="ignore"):
        a = np.clip(np.rint((v / asc[:, None]).astype(F32)), -qmax, qmax).astype(np.int64)
    return a, asc


def planes(a, sh):
    """t16h_lmvariants.py:71-77: a = (hi << sh) + lo, hi = a >> sh (floor), lo in [0, 2^sh - 1];
    sh = 0 is one plane.  Returns [(shift, int8 plane)], the hi plane first."""
    a = np.asarray(a, np.int64)
    if sh == 0:
        return [(0, a.astype(np.int8))]
    hi = a >> sh
    lo = a - (hi << sh)
    return [(sh, hi.astype(np.int8)), (0, lo.astype(np.int8))]


def quantize_weight_bits(W, wbits, sdiv=None):
    """t16h_lmvariants.py:95-103 with the prepare-time fold :137-148: per-out-channel <wbits>
    quant of W [N, K] (times sdiv per column when given) carried by int8 planes [N, K]."""
    a, ws = quant_rows_bits(W, wbits, sdiv, 2 if sdiv is not None else 0)
    return planes(a, wbits - 8), ws


def mm_planes(x2, wplanes, ws, abits, sdiv=None):
    """t16h_lmvariants.py:115-125 (_mm_planes, with Variant.logits' divide :150-155): the plane
    products as exact integer GEMMs, combined in int64 (activation planes outer, weight planes
    inner), then fl32(fl32(fl32(s) * asc[m]) * ws[n]) with fl32(s) rounded to nearest even."""
    a, asc = quant_rows_bits(x2, abits, sdiv, 1 if sdiv is not None else 0)
    ap = planes(a, abits - 8)
    if len(ap) == 1 and len(wplanes) == 1:
        acc = int_mm(ap[0][1], np.asarray(wplanes[0][1]).T).astype(F32)
    else:
        s = np.zeros((a.shape[0], np.asarray(wplanes[0][1]).shape[0]), np.int64)
        for ash, p in ap:
            for wsh, w in wplanes:
                s = s + (int_mm(p, np.asarray(w).T).astype(np.int64) << (ash + wsh))
        acc = s.astype(F32)                       # int64 -> binary32, round to nearest even
    return ((acc * asc[:, None]).astype(F32) * np.asarray(ws, F32)[None, :]).astype(F32)


def smooth_scales(act_amax, W, alpha):
    """t16h_lmvariants.py:106-112: s = max(a_amax^alpha / w_amax^(1-alpha), 1e-5) per input channel,
    w_amax / a_amax clamped below at 1e-5, in binary32 (pow is not correctly rounded: a prepare-time
    artifact, parity unpinned beyond the tolerance its tests state)."""
    w_amax = np.maximum(np.abs(np.asarray(W, F32)).max(axis=0), F32(1e-5))
    a_amax = np.maximum(np.asarray(act_amax, F32), F32(1e-5))
    s = (np.power(a_amax, F32(alpha)) / np.power(w_amax, F32(1.0 - alpha))).astype(F32)
    return np.maximum(s, F32(1e-5)).astype(F32)


# ----------------------------------------------------------------------------- contract 2.6 float norm
FLT_MIN_NORMAL = F32(2.0 ** -126)


def sqrt_n(N):
    """t16n_ref.py:38-39: the published width constant fl32(sqrt(N)) (binary64 sqrt, one rounding)."""
    return F32(np.sqrt(np.float64(N)))


def tree_sum(v):
    """t16n_ref.py:42-50: T(one value) = the value; T(v) = fl32(T(v[:P]) + T(v[P:])) with P the
    largest power of two below n (a power-of-two count is halved).  v [R, n] -> [R]."""
    v = np.asarray(v, F32)
    n = v.shape[1]
    if n == 1:
        return v[:, 0].copy()
    P = 1 << (n.bit_length() - 1)
    if P == n:
        P = n // 2
    return (tree_sum(v[:, :P]) + tree_sum(v[:, P:])).astype(F32)


def row_sum_float(x2):
    """t16n_ref.py:53-62: sq = fl32(x * x); chains of 8 in index order; then tree_sum over groups."""
    x = np.asarray(x2, F32)
    R, N = x.shape
    assert N % 8 == 0
    sq = (x * x).astype(F32).reshape(R, N // 8, 8)
    a = sq[:, :, 0].copy()
    for i in range(1, 8):
        a = (a + sq[:, :, i]).astype(F32)
    return tree_sum(a)


def eps_term(N, eps):
    """t16n_ref.py:65-67: ne = fl32(fl64(N) * fl64(eps))."""
    return F32(np.float64(N) * np.float64(eps or 0.0))


def rmsnorm_float(x, weight, sN=None, eps=0.0):
    """t16n_ref.py:70-92: S = row_sum_float, + ne when eps, max(S, 2^-126); rs = fl32(sN / fl32(sqrt S))
    (IEEE sqrt and division); out = bf16(fl32(fl32(x * rs) * g)).  x [..., N] binary32 values; returns
    bf16 bits of the input shape."""
    x = np.asarray(x, F32)
    shp = x.shape
    N = shp[-1]
    x2 = x.reshape(-1, N)
    sN = sqrt_n(N) if sN is None else F32(sN)
    S = row_sum_float(x2)
    if eps:
        S = (S + eps_term(N, eps)).astype(F32)
    S = np.maximum(S, FLT_MIN_NORMAL).astype(F32)
    rs = (sN / np.sqrt(S).astype(F32)).astype(F32)
    y = (x2 * rs[:, None]).astype(F32)
    g = np.asarray(weight, F32).reshape(-1)
    if not np.all(g == 1.0):
        y = (y * g[None, :]).astype(F32)
    return bf16_bits(y).reshape(shp)


# ----------------------------------------------------------------------------- rotation
def fwht_blocks(x2, blk=256, scale=1.0 / 16.0):
    """lockstep_fullstack.py:533-546: on every blk-wide block, pairs (i, i+h) -> (a+b, a-b)
    for h = 1, 2, ..., blk/2 (binary32 adds), then one multiply by `scale` (a power of two)."""
    x = np.asarray(x2, F32)
    sh = x.shape
    D = sh[-1]
    nb = D // blk
    v = x.reshape(-1, nb, blk).copy()
    h = 1
    while h < blk:
        v = v.reshape(-1, nb, blk // (2 * h), 2, h)
        a = v[..., 0, :]
        b = v[..., 1, :]
        v = np.stack(((a + b).astype(F32), (a - b).astype(F32)), axis=-2).reshape(-1, nb, blk)
        h *= 2
    return (v * F32(scale)).astype(F32).reshape(sh)


# ----------------------------------------------------------------------------- v2.5 outlier side path
def outlier_side(ho, wo):
    """lockstep_fullstack.py:549-557: side[m, n] = sum_k fl32(ho[m, k]) * fl32(wo[n, k]), the sum
    sequential in k from +0 with binary32 adds (each add rounds).  ho [M, k], wo [N, k] binary32
    values (bf16-valued in the contract, so every product is exact)."""
    h = np.asarray(ho, F32)
    w = np.asarray(wo, F32)
    side = np.zeros((h.shape[0], w.shape[0]), F32)
    for k in range(h.shape[1]):
        side = (side + (h[:, k:k + 1] * w[None, :, k]).astype(F32)).astype(F32)
    return side


def w8a8_outlier_linear(x, oidx, wo, W8, ws, bias=None, out="bf16", rot=True):
    """lockstep_fullstack.py:560-578 (contract v2.5 / v2.5.1): the declared channels oidx leave the
    row as ho (exact), the masked row takes the 256-block butterfly / 16 (rot) and the row quant,
        y8 = bf16((fl32(acc) * ws[n]) * asc[m]);  y = bf16(fl32(y8) + side[m, n]);
        with a bias y = bf16(fl32(y) + bias[n]);  then cast to `out` (from the bf16 value).
    x [rows, K] binary32 values; oidx int [k]; wo [N, k]; W8 [N, K] int8; ws [N] fp32."""
    x2 = np.asarray(x, F32).reshape(-1, np.shape(x)[-1])
    idx = np.asarray(oidx).astype(np.int64)
    ho = x2[:, idx]
    xm = x2.copy()
    xm[:, idx] = F32(0.0)
    xr = fwht_blocks(xm) if rot else xm
    q, asc = quantize_rows_int8(xr)
    acc = int_mm(q, np.asarray(W8).T)
    y = bfr(((acc.astype(F32) * np.asarray(ws, F32)[None, :]).astype(F32) * asc[:, None]).astype(F32))
    y = bfr((y + outlier_side(ho, wo)).astype(F32))
    if bias is not None:
        y = bfr((y + np.asarray(bias, F32)[None, :]).astype(F32))
    return cast_out(y, out)


# ----------------------------------------------------------------------------- A12 router
def table_scores(dgap, tab=None):
    """moe_ref.py:64-74: d = max(rint(fl32(dgap * C)), 0); s = tab[(d >> 13) & 8191] >> min(d >> 26, 63);
    0 where d >= 16 << 26."""
    tab = frac_table() if tab is None else np.asarray(tab, np.int64)
    d = np.rint((np.asarray(dgap, F32) * ROUTER_C).astype(F32)).astype(np.int64)
    d = np.maximum(d, 0)
    win = (TAB_W + 1) << BHI
    idx = (d >> (BHI - TAB_N)) & ((1 << TAB_N) - 1)
    sh = np.minimum(d >> BHI, 63)
    s = tab[idx] >> sh
    return np.where(d < win, s, 0)


def router_from_logits(g, k, renormalize=True, tab=None):
    """moe_ref.py:85-97: scores from the max gap, top-k by key = s*E + (E-1-e) (ties -> lower
    index), w = bf16(fl32(s_sel) / fl32(S)), S clamped >= 1.  Returns (idx int64 [T,k] by
    rank, w as bf16 bits [T,k], g as bf16 bits)."""
    g = np.asarray(g, F32)
    T, E = g.shape
    m = g.max(axis=-1, keepdims=True)
    s = table_scores((m - g).astype(F32), tab)
    key = s * E + (E - 1 - np.arange(E, dtype=np.int64))[None, :]
    order = np.argsort(-key, axis=-1, kind="stable")[:, :k]
    s_sel = np.take_along_axis(s, order, axis=1)
    S = s_sel.sum(axis=-1, keepdims=True) if renormalize else s.sum(axis=-1, keepdims=True)
    S = np.maximum(S, 1)
    w = bf16_bits((s_sel.astype(F32) / S.astype(F32)).astype(F32))
    return order.astype(np.int64), w, bf16_bits(g)


def router(x, gate_w8col, gate_ws, k, renormalize=True, tab=None, gate_bias=None):
    """moe_ref.py:77-82 and router_b :203-210: rowquant, exact GEMM, the (biased) E-v2.1
    epilogue, then router_from_logits.  gate_w8col is [H, E]."""
    q, asc = rowquant(x)
    g = lin_epilogue_b(int_mm(q, gate_w8col), gate_ws, asc, gate_bias)
    return router_from_logits(g, k, renormalize, tab)


# ----------------------------------------------------------------------------- A7 MXFP4
_FP4_MAG = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], dtype=F32)


def fp4_values(codes):
    """moe_mxfp4.py:13-16: code c -> +-mag[c & 7], negative when c & 8 (code 8 -> -0.0)."""
    c = np.asarray(codes).astype(np.int64)
    mag = _FP4_MAG[c & 7]
    return np.where((c & 8) != 0, -mag, mag).astype(F32)


def unpack_fp4(packed):
    """moe_mxfp4.py:19-23: element 2i is the low nibble, 2i+1 the high nibble."""
    p = np.asarray(packed, np.uint8)
    lo = p & 0x0F
    hi = (p >> 4) & 0x0F
    return np.stack((lo, hi), axis=-1).reshape(*p.shape[:-1], p.shape[-1] * 2)


def dequant_mxfp4(packed, scale_e8m0, out="bf16", block=32):
    """moe_mxfp4.py:26-35: fp4_value * 2^(e - 127), exact; returns bf16 bits or float32."""
    vals = fp4_values(unpack_fp4(packed))
    K = vals.shape[-1]
    sc = np.asarray(scale_e8m0).astype(np.int64)
    assert sc.shape[-1] * block == K
    p2 = np.ldexp(np.ones(sc.shape, F32), (sc - 127).astype(np.int32)).astype(F32)
    p2 = np.repeat(p2, block, axis=-1)
    y = (vals * p2).astype(F32)
    return bf16_bits(y) if out == "bf16" else y


def mx_to_m2(packed, scale_e8m0):
    """The MX operand form of moe_ref.py:233-238: doubled mantissas m2 = 2 * fp4 value
    (int8 in {0, +-1, +-2, +-3, +-4, +-6, +-8, +-12}) and kexp = the E8M0 byte, so that
    m2 * 2^(kexp - 128) == fp4 * 2^(e - 127)."""
    m2 = (fp4_values(unpack_fp4(packed)) * F32(2.0)).astype(np.int8)
    return m2, np.asarray(scale_e8m0, np.uint8)


def int_mm_mx(a8, m2, kexp):
    """moe_ref.py:243-255: for blocks b = 0 .. K/32-1 ascending,
    acc = fl32(acc + fl32(s_b) * 2^(kexp[n,b] - 128)) with s_b the exact int block sum."""
    a = np.asarray(a8).astype(np.int64)
    m = np.asarray(m2).astype(np.int64)
    T, K = a.shape
    N = m.shape[0]
    nb = K // MX_BLOCK
    scale = np.ldexp(np.ones((N, nb), F32), np.asarray(kexp).astype(np.int32) - 128).astype(F32)
    acc = np.zeros((T, N), F32)
    for b in range(nb):
        sl = slice(b * MX_BLOCK, (b + 1) * MX_BLOCK)
        s = (a[:, sl] @ m[:, sl].T).astype(F32)
        acc = (acc + (s * scale[:, b][None, :]).astype(F32)).astype(F32)
    return acc


def lin_epilogue_mx(acc, asc, bias=None):
    """moe_ref.py:258-261: bfr(acc * asc[m]), then bfr(y + b)."""
    y = bfr((np.asarray(acc, F32) * np.asarray(asc, F32)[:, None]).astype(F32))
    if bias is not None:
        y = bfr((y + np.asarray(bias, F32)[None, :]).astype(F32))
    return y


# ----------------------------------------------------------------------------- A13 MX2 block-scaled activations
KA_MIN, KA_MAX = -126, 127


def blockquant(x):
    """moe_ref.py:299-314: per 32-wide block of each row, am = max |x|; ka = ceil(log2(fl32(am / 127)))
    (-126 for an all-zero block), clamped to [-126, 127], raised by one where fl32(127 * 2^ka) < am;
    q = clamp(rint(x / 2^ka), +-127).  x [T, K] binary32 values -> (q int8 [T, K], ka int32 [T, K/32])."""
    xf = np.asarray(x, F32)
    T, K = xf.shape
    nb = K // MX_BLOCK
    xb = xf.reshape(T, nb, MX_BLOCK)
    am = np.abs(xb).max(axis=-1).astype(F32)
    with np.errstate(divide="ignore"):
        l2 = np.log2((am / F32(127.0)).astype(F32)).astype(F32)
    ka = np.where(am > 0, np.ceil(l2), F32(KA_MIN)).astype(F32)
    ka = np.clip(ka, KA_MIN, KA_MAX).astype(F32)
    with np.errstate(over="ignore"):
        bad = (F32(127.0) * np.ldexp(np.ones_like(ka), ka.astype(np.int32))).astype(F32) < am
    ka = np.where(bad, ka + F32(1.0), ka).astype(np.int32)
    sc = np.ldexp(np.ones(ka.shape, F32), ka).astype(F32)
    with np.errstate(invalid="ignore"):
        q = np.clip(np.rint((xb / sc[..., None]).astype(F32)), -INT8_LIM, INT8_LIM).astype(np.int8)
    return q.reshape(T, K), ka


def int_mm_mx2(q, ka, m2, kexp):
    """moe_ref.py:317-326: for blocks b ascending, p = fl32(2^(ka[m,b] + kexp[n,b] - 128)) (0 below
    2^-149, inf from 2^128) and acc = fl32(acc + fl32(s_b * p)), s_b the exact int block sum."""
    a = np.asarray(q).astype(np.int64)
    m = np.asarray(m2).astype(np.int64)
    kaa = np.asarray(ka).astype(np.int64)
    kw = np.asarray(kexp).astype(np.int64)
    T, K = a.shape
    N = m.shape[0]
    acc = np.zeros((T, N), F32)
    with np.errstate(over="ignore", invalid="ignore"):
        for b in range(K // MX_BLOCK):
            sl = slice(b * MX_BLOCK, (b + 1) * MX_BLOCK)
            s = (a[:, sl] @ m[:, sl].T).astype(F32)
            e = kaa[:, b][:, None] + (kw[:, b] - 128)[None, :]
            p = np.ldexp(np.ones(e.shape, F32), np.clip(e, -400, 400).astype(np.int32)).astype(F32)
            acc = (acc + (s * p).astype(F32)).astype(F32)
    return acc


def expert_block_mx2(x_rows, w13, w2, act, b13=None, b2=None):
    """moe_ref.py:329-339: blockquant -> int_mm_mx2 -> bfr (+ bfr(+ b13)) -> act -> blockquant of
    the bf16-rounded h -> int_mm_mx2 -> bfr (+ bfr(+ b2)); no per-row scale."""
    q, ka = blockquant(x_rows)
    y = bfr(int_mm_mx2(q, ka, w13[0], w13[1]))
    if b13 is not None:
        y = bfr((y + np.asarray(b13, F32)[None, :]).astype(F32))
    I = y.shape[-1] // 2
    h = act(y[:, :I], y[:, I:])
    q2, ka2 = blockquant(bfr(h))
    o = bfr(int_mm_mx2(q2, ka2, w2[0], w2[1]))
    if b2 is not None:
        o = bfr((o + np.asarray(b2, F32)[None, :]).astype(F32))
    return o


# ----------------------------------------------------------------------------- A10 expert blocks
def expert_swiglu(x_rows, w13col, ws13, w2col, ws2, act=act_silu, rot=False):
    """moe_ref.py:100-114 (w13col [H, 2I], w2col [I, H])."""
    xin = fwht_blocks(np.asarray(x_rows, F32)) if rot else np.asarray(x_rows, F32)
    q, asc = rowquant(xin)
    y = lin_epilogue(int_mm(q, w13col), ws13, asc)
    I = y.shape[-1] // 2
    h = act(y[:, :I], y[:, I:])
    hin = fwht_blocks(h) if rot else h
    q2, asc2 = rowquant(hin)
    return lin_epilogue(int_mm(q2, w2col), ws2, asc2)


def expert_block(x_rows, w13col, ws13, w2col, ws2, act, b13=None, b2=None, rot_blk=256):
    """moe_ref.py:189-200: biased epilogues and a parametrised R1 / R4 block (0 = none)."""
    def rot(v):
        if not rot_blk:
            return np.asarray(v, F32)
        return fwht_blocks(v, blk=rot_blk, scale=1.0 / (rot_blk ** 0.5))
    q, asc = rowquant(rot(x_rows))
    y = lin_epilogue_b(int_mm(q, w13col), ws13, asc, b13)
    I = y.shape[-1] // 2
    h = act(y[:, :I], y[:, I:])
    q2, asc2 = rowquant(rot(h))
    return lin_epilogue_b(int_mm(q2, w2col), ws2, asc2, b2)


def expert_block_mx(x_rows, w13, w2, act, b13=None, b2=None):
    """moe_ref.py:264-271: w13 = (m2 [2I, H], kexp [2I, H/32]), w2 = (m2 [H, I], kexp)."""
    q, asc = rowquant(x_rows)
    y = lin_epilogue_mx(int_mm_mx(q, w13[0], w13[1]), asc, b13)
    I = y.shape[-1] // 2
    h = act(y[:, :I], y[:, I:])
    q2, asc2 = rowquant(h)
    return lin_epilogue_mx(int_mm_mx(q2, w2[0], w2[1]), asc2, b2)


# ----------------------------------------------------------------------------- A11 MoE layers
def _combine(T, H, idx, w, expert_out, E):
    """moe_ref.py:127-140: for e in range(E) ascending, acc[tok] += bfr(w_e * out) in binary32
    from +0 (routing entries outside [0, E) are never visited)."""
    idx = np.asarray(idx, np.int64)
    wf = bf16_to_f32(w)
    acc = np.zeros((T, H), F32)
    for e in range(E):
        hit = idx == e
        if not hit.any():
            continue
        tok = np.nonzero(hit.any(axis=-1))[0]
        we = wf[tok][hit[tok]]
        out = expert_out(e, tok)
        acc[tok] = (acc[tok] + bfr((we[:, None] * out).astype(F32))).astype(F32)
    return acc


def moe_forward(x, experts, idx, w, act=act_silu, rot=False, shared_out=None):
    """moe_ref.py:117-140 with routing=(idx, w) injected; x [T, H] binary32 values (bf16 in
    the reference); experts[e] = (w13col, ws13, w2col, ws2); shared_out: the shared expert's
    output [T, H] (added as bfr(shared) after every routed expert).  Returns y as bf16 bits."""
    x = np.asarray(x, F32)
    T, H = x.shape
    acc = _combine(T, H, idx, w, lambda e, tok: expert_swiglu(x[tok], *experts[e][:4], act=act, rot=rot),
                   len(experts))
    if shared_out is not None:
        acc = (acc + bfr(np.asarray(shared_out, F32))).astype(F32)
    return bf16_bits(acc)


def moe_forward_b(x, experts, idx, w, act, rot_blk=256):
    """moe_ref.py:213-230 with routing injected; experts[e] = (w13col, ws13, w2col, ws2, b13, b2)."""
    x = np.asarray(x, F32)
    T, H = x.shape

    def run(e, tok):
        ex = experts[e]
        return expert_block(x[tok], ex[0], ex[1], ex[2], ex[3], act,
                            ex[4] if len(ex) > 4 else None, ex[5] if len(ex) > 5 else None, rot_blk)
    return bf16_bits(_combine(T, H, idx, w, run, len(experts)))


def moe_forward_mx(x, experts, idx, w, act):
    """moe_ref.py:274-290 with routing injected; experts[e] = ((m2_13, kexp_13), (m2_2, kexp_2), b13, b2)."""
    x = np.asarray(x, F32)
    T, H = x.shape

    def run(e, tok):
        ex = experts[e]
        return expert_block_mx(x[tok], ex[0], ex[1], act,
                               ex[2] if len(ex) > 2 else None, ex[3] if len(ex) > 3 else None)
    return bf16_bits(_combine(T, H, idx, w, run, len(experts)))


def moe_forward_mx2(x, experts, idx, w, act):
    """moe_ref.py:342-352 with routing injected; experts[e] as moe_forward_mx."""
    x = np.asarray(x, F32)
    T, H = x.shape

    def run(e, tok):
        ex = experts[e]
        return expert_block_mx2(x[tok], ex[0], ex[1], act,
                                ex[2] if len(ex) > 2 else None, ex[3] if len(ex) > 3 else None)
    return bf16_bits(_combine(T, H, idx, w, run, len(experts)))


# ----------------------------------------------------------------------------- digest (tools/contract_vectors.py:40-49)
def digest(arr: np.ndarray, dtype_name: str) -> str:
    """sha256 of b'lockstep-tensor-v1|' + dtype + '|' + 'x'.join(shape) + '|' + raw bytes."""
    a = np.ascontiguousarray(arr)
    h = hashlib.sha256()
    h.update(b"lockstep-tensor-v1|")
    h.update(dtype_name.encode())
    h.update(b"|")
    h.update("x".join(str(int(d)) for d in a.shape).encode())
    h.update(b"|")
    if a.size:
        h.update(a.reshape(-1).view(np.uint8).tobytes())
    return h.hexdigest()
