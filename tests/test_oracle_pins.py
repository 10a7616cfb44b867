"""Pins for the oracle functions that no reference-held vector covers: closed forms,
invariants and brute force written independently of the oracle's own formulas, each chosen
so that a plausible slip (dropped term, wrong sign / index / shift, swapped operand) fails."""
import math
from fractions import Fraction

import numpy as np
import pytest

from oracle import contract as C

F32 = np.float32


def f32_round(fr: Fraction) -> float:
    """Round an exact rational to the nearest binary32 (ties to even), independently of
    numpy: scale into [2^23, 2^24) and round the integer significand."""
    if fr == 0:
        return 0.0
    s = -1 if fr < 0 else 1
    a = abs(fr)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, -126)                       # subnormals share the 2^-149 quantum
    q = a / Fraction(2) ** (e - 23)
    n = q.numerator // q.denominator
    r = q - n
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return s * float(Fraction(n) * Fraction(2) ** (e - 23))


def bf16_round(v: float) -> float:
    """Round a binary32 value to bf16 (8 significant bits, ties to even) by rationals."""
    if v == 0:
        return v
    fr = Fraction(v)
    s = -1 if fr < 0 else 1
    a = abs(fr)
    e = math.floor(math.log2(a))
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, -126)
    q = a / Fraction(2) ** (e - 7)
    n = q.numerator // q.denominator
    r = q - n
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return s * float(Fraction(n) * Fraction(2) ** (e - 7))


# ------------------------------------------------------------------ bf16 rounding helper
def test_bf16_bits_matches_rational_rounding():
    rng = np.random.default_rng(1)
    vals = np.concatenate([rng.standard_normal(2000).astype(F32) * F32(1e3),
                           np.array([1.0, 1.00390625, 1.005859375, -3.0, 65504.0, 1e-39, -1e-40], F32)])
    got = C.bfr(vals)
    for v, g in zip(vals, got):
        assert float(g) == bf16_round(float(v)), v


# ------------------------------------------------------------------ A1 row quant
def test_rowquant_brute_force():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((6, 37)) * 5).astype(F32)
    x[3] = 0.0                                 # an all-zero row takes the 1e-8 floor
    x[4, 5] = 127.0 * 0.5 + 0.25
    q, asc = C.rowquant(x)
    for m in range(x.shape[0]):
        am = max(max(abs(float(v)) for v in x[m]), float(F32(1e-8)))
        a = f32_round(Fraction(am) / 127)
        assert float(asc[m]) == a
        for k in range(x.shape[1]):
            quo = f32_round(Fraction(float(x[m, k])) / Fraction(a))
            qq = round(quo)                    # Python round: half to even
            qq = max(-127, min(127, qq))
            assert q[m, k] == qq, (m, k)
    assert np.all(q[3] == 0)


# ------------------------------------------------------------------ A2 exact GEMM
def test_int_mm_methods_agree_and_bound():
    rng = np.random.default_rng(3)
    for (M, N, K) in [(1, 1, 1), (3, 5, 64), (17, 9, 300), (4, 7, 4096)]:
        a = rng.integers(-127, 128, (M, K), dtype=np.int8)
        b = rng.integers(-127, 128, (K, N), dtype=np.int8)
        r1 = C.int_mm(a, b, "i64")
        r2 = C.int_mm(a, b, "f64")
        assert np.array_equal(r1, r2)
        # brute force one element
        assert int(r1[M - 1, N - 1]) == sum(int(a[M - 1, k]) * int(b[k, N - 1]) for k in range(K))
    # extreme operands: |acc| reaches K * 127^2 exactly
    K = 18944
    a = np.full((1, K), -127, np.int8)
    b = np.full((K, 1), 127, np.int8)
    assert int(C.int_mm(a, b)[0, 0]) == -K * 127 * 127
    assert K * 127 * 127 < 2 ** 31 - 1


# ------------------------------------------------------------------ A3 epilogue order
def test_epilogue_v21_brute_force_and_order():
    rng = np.random.default_rng(4)
    acc = rng.integers(-(2 ** 28), 2 ** 28, (4, 6)).astype(np.int32)
    ws = rng.uniform(1e-3, 1e-2, 6).astype(F32)
    asc = rng.uniform(1e-3, 1e-1, 4).astype(F32)
    bias = rng.standard_normal(6).astype(F32)
    y = C.bf16_to_f32(C.epilogue_v21(acc, ws, asc, bias, "bf16"))
    y2 = C.bf16_to_f32(C.epilogue_v2(acc, ws, asc, None, "bf16"))
    for m in range(4):
        for n in range(6):
            a = f32_round(Fraction(int(acc[m, n])))
            t = f32_round(Fraction(a) * Fraction(float(ws[n])))
            t = f32_round(Fraction(t) * Fraction(float(asc[m])))
            t = bf16_round(t)
            t = bf16_round(f32_round(Fraction(t) + Fraction(float(bias[n]))))
            assert float(y[m, n]) == t
            u = f32_round(Fraction(a) * Fraction(float(asc[m])))
            u = bf16_round(f32_round(Fraction(u) * Fraction(float(ws[n]))))
            assert float(y2[m, n]) == u


# ------------------------------------------------------------------ A6 pow2 exponents
def _e_brute(m: float) -> int:
    if m == 0:
        return 0
    best = None
    for e in range(-200, 200):
        if Fraction(m) * Fraction(2) ** e <= 127:              # exact: a power-of-two scaling
            best = e
    return max(-32, min(40, best))


def test_pow2_exponent_brute_force():
    rng = np.random.default_rng(5)
    ms = list((rng.standard_normal(200) ** 2 * 10.0 ** rng.integers(-12, 12, 200)).astype(F32))
    ms += [F32(0), F32(127.0), F32(127.5), F32(127.99), F32(128.0), F32(63.9), F32(64.0),
           F32(1e-30), F32(3e38), F32(1e-40), F32(2.0 ** -33)]
    e = C._e_from_max(np.array(ms, F32))
    for m, ee in zip(ms, e):
        assert int(ee) == _e_brute(float(m)), m


def test_quant8_dyn_rows_cols_consistent():
    rng = np.random.default_rng(6)
    x = (rng.standard_normal((9, 33)) * 3).astype(F32)
    q, e = C.quant8_dyn(x)
    assert e == _e_brute(float(np.abs(x).max()))
    assert np.abs(q).max() <= 127
    qr, er = C.quant8_rows(x)
    for i in range(9):
        assert er[i] == _e_brute(float(np.abs(x[i]).max()))
    qc, ec = C.quant8_cols(x)
    assert np.array_equal(qc.T, C.quant8_rows(x.T.copy())[0])
    # the pow2 dequant is exact: it equals the rational value
    acc = np.array([[12345, -7], [2 ** 30, 1]], np.int64)
    d = C.dequant_pow2(acc, 17)
    assert float(d[0, 0]) == float(f32_round(Fraction(12345) / 2 ** 17))
    assert float(d[1, 0]) == 2.0 ** 13


# ------------------------------------------------------------------ A7 MXFP4
def _e2m1(c: int) -> float:
    """OCP E2M1: sign | 2-bit exponent (bias 1) | 1-bit mantissa; exponent 0 is subnormal."""
    s = -1.0 if c & 8 else 1.0
    ex = (c >> 1) & 3
    man = c & 1
    v = man * 0.5 if ex == 0 else 2.0 ** (ex - 1) * (1 + man / 2)
    return math.copysign(v, s)


def test_fp4_closed_form_all_codes():
    vals = C.fp4_values(np.arange(16))
    for c in range(16):
        assert float(vals[c]) == _e2m1(c)
        assert math.copysign(1.0, float(vals[c])) == math.copysign(1.0, _e2m1(c))
    assert math.copysign(1.0, float(vals[8])) == -1.0        # code 8 is -0.0


def test_dequant_mxfp4_closed_form():
    rng = np.random.default_rng(7)
    codes = rng.integers(0, 16, (3, 4, 128), dtype=np.uint8)
    packed = (codes[..., 0::2] | (codes[..., 1::2] << 4)).astype(np.uint8)
    scale = rng.integers(100, 140, (3, 4, 4), dtype=np.uint8)
    y = C.bf16_to_f32(C.dequant_mxfp4(packed, scale))
    for idx in np.ndindex(codes.shape):
        e = int(scale[idx[0], idx[1], idx[2] // 32]) - 127
        assert float(y[idx]) == _e2m1(int(codes[idx])) * 2.0 ** e
    # every e8m0 byte that yields a normal binary32 power of two
    sc = np.arange(1, 255, dtype=np.uint8).reshape(1, -1)
    pk = np.full((1, 254 * 16), 0x22, np.uint8)               # codes 2, 2 -> value 1.0
    y = C.dequant_mxfp4(pk, sc, out="f32")
    for j in range(254):
        assert float(y[0, j * 32]) == 2.0 ** (j + 1 - 127)


def test_m2_form_matches_dequant():
    rng = np.random.default_rng(8)
    codes = rng.integers(0, 16, (5, 64), dtype=np.uint8)
    packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8)
    scale = rng.integers(118, 130, (5, 2), dtype=np.uint8)
    m2, kexp = C.mx_to_m2(packed, scale)
    assert set(np.unique(np.abs(m2.astype(np.int64)))) <= {0, 1, 2, 3, 4, 6, 8, 12}
    deq = C.dequant_mxfp4(packed, scale, out="f32")
    for n in range(5):
        for k in range(64):
            assert float(deq[n, k]) == float(m2[n, k]) * 2.0 ** (int(kexp[n, k // 32]) - 128)


# ------------------------------------------------------------------ A8 int_mm_mx
def test_int_mm_mx_one_block_closed_form():
    rng = np.random.default_rng(9)
    a = rng.integers(-127, 128, (3, 32), dtype=np.int8)
    m2 = rng.choice(np.array([0, 1, 2, 3, 4, 6, 8, 12, -1, -2, -3, -4, -6, -8, -12], np.int8), (4, 32))
    k = rng.integers(110, 140, (4, 1), dtype=np.uint8)
    acc = C.int_mm_mx(a, m2, k)
    for t in range(3):
        for n in range(4):
            s = sum(int(a[t, j]) * int(m2[n, j]) for j in range(32))
            assert float(acc[t, n]) == s * 2.0 ** (int(k[n, 0]) - 128)


def test_int_mm_mx_equal_exponent_identity():
    """With one exponent per row and small values nothing rounds: acc = exact GEMM * 2^(k-128)."""
    rng = np.random.default_rng(10)
    a = rng.integers(-3, 4, (5, 256), dtype=np.int8)
    m2 = rng.choice(np.array([0, 1, -1, 2, -2], np.int8), (6, 256))
    k = np.full((6, 8), 125, np.uint8)
    acc = C.int_mm_mx(a, m2, k)
    ref = (a.astype(np.int64) @ m2.astype(np.int64).T).astype(np.float64) * 2.0 ** -3
    assert np.array_equal(acc.astype(np.float64), ref)


def test_int_mm_mx_scalar_brute_force_and_negative_control():
    rng = np.random.default_rng(11)
    T, N, K = 3, 8, 64 * 2
    a = rng.integers(-127, 128, (T, K), dtype=np.int8)
    m2 = rng.choice(np.array([0, 1, 2, 3, 4, 6, 8, 12, -1, -2, -3, -4, -6, -8, -12], np.int8), (N, K))
    k = rng.integers(100, 160, (N, K // 32), dtype=np.uint8)
    acc = C.int_mm_mx(a, m2, k)
    for t in range(T):
        for n in range(N):
            r = 0.0
            for b in range(K // 32):
                s = sum(int(a[t, b * 32 + j]) * int(m2[n, b * 32 + j]) for j in range(32))
                r = f32_round(Fraction(r) + Fraction(s) * Fraction(2) ** (int(k[n, b]) - 128))
            assert float(acc[t, n]) == r
    # negative control: a crafted row whose result depends on the block order
    a1 = np.zeros((1, 96), np.int8)
    a1[0, 0] = 1; a1[0, 32] = 1; a1[0, 64] = 1
    m21 = np.zeros((1, 96), np.int8)
    m21[0, 0] = 1; m21[0, 32] = 1; m21[0, 64] = -1
    kk = np.array([[128 + 24, 128, 128 + 24]], np.uint8)        # +2^24, +1, -2^24
    fwd = C.int_mm_mx(a1, m21, kk)[0, 0]                        # 2^24 + 1 rounds to 2^24
    rev = C.int_mm_mx(a1[:, ::-1].copy(), m21[:, ::-1].copy(), kk[:, ::-1].copy())[0, 0]
    assert float(fwd) == 0.0 and float(rev) == 1.0


# ------------------------------------------------------------------ FRAC, router
def test_frac_and_table_scores_approximate_exp():
    """s = 2^15 * exp(-dgap) to within the table's quantisation, and 0 past 16 doublings."""
    tab = C.frac_table()
    k = np.arange(8192)
    assert np.max(np.abs(tab / 2.0 ** 15 - 2.0 ** (-k / 8192.0))) < 2.0 ** -14
    assert float(C.ROUTER_C) == float(F32(2.0 ** 26 / math.log(2)))
    dg = np.linspace(0, 12, 997).astype(F32)
    s = C.table_scores(dg)
    ref = 2.0 ** 15 * np.exp(-dg.astype(np.float64))
    assert np.all(np.abs(s - ref) <= ref * 2.0 ** -11 + 1.0)
    assert int(C.table_scores(np.array([0.0], F32))[0]) == int(tab[0])
    assert int(C.table_scores(np.array([11.5], F32))[0]) == 0                # 16.6 doublings
    assert int(C.table_scores(np.array([-1.0], F32))[0]) == int(tab[0])      # d clamped at 0


def test_router_brute_force_ties():
    rng = np.random.default_rng(12)
    T, E, k = 40, 16, 4
    g = C.bfr((rng.integers(-8, 8, (T, E)) / 4.0).astype(F32))   # tie-dense logits
    for renorm in (True, False):
        idx, w, gb = C.router_from_logits(g, k, renorm)
        s = C.table_scores((g.max(axis=-1, keepdims=True) - g).astype(F32))
        for t in range(T):
            order = sorted(range(E), key=lambda e: (-int(s[t, e]), e))[:k]
            assert list(idx[t]) == order
            S = sum(int(s[t, e]) for e in order) if renorm else sum(int(v) for v in s[t])
            S = max(S, 1)
            for j, e in enumerate(order):
                ref = bf16_round(f32_round(Fraction(int(s[t, e]), S)))
                assert float(C.bf16_to_f32(w[t, j])) == ref


# ------------------------------------------------------------------ SwiGLU-OAI / sigmoid
def test_sigmoid_contract_against_logistic():
    x = np.linspace(-20, 20, 4001).astype(F32)
    sg = C.sigmoid_contract(x).astype(np.float64)
    ref = 1.0 / (1.0 + np.exp(-x.astype(np.float64)))
    assert np.max(np.abs(sg - ref)) < 2e-4
    assert np.array_equal(C.silu_contract(x), (C.sigmoid_contract(x) * x).astype(F32))


def test_act_swigluoai_brute_force():
    rng = np.random.default_rng(13)
    g = C.bfr((rng.standard_normal(300) * 6).astype(F32))
    u = C.bfr((rng.standard_normal(300) * 6).astype(F32))
    h = C.act_swigluoai(g, u)
    for i in range(300):
        gc = min(float(g[i]), 7.0)
        uc = min(max(float(u[i]), -7.0), 7.0)
        arg = bf16_round(f32_round(Fraction(gc) * Fraction(float(F32(1.702)))))
        sg = float(C.sigmoid_contract(np.array([arg], F32))[0])
        glu = bf16_round(f32_round(Fraction(gc) * Fraction(sg)))
        ref = bf16_round(f32_round(Fraction(f32_round(Fraction(uc) + 1)) * Fraction(glu)))
        assert float(h[i]) == ref


# ------------------------------------------------------------------ combine and the MoE layer
def test_moe_combine_per_token_brute_force():
    """moe_forward seen per token: sum over the token's experts in ascending index of
    bf16(w * out), binary32 adds from +0, then bf16.  The oracle walks experts instead."""
    rng = np.random.default_rng(14)
    T, H, I, E, k = 12, 64, 32, 6, 3
    x = C.bfr(rng.standard_normal((T, H)).astype(F32))
    experts = []
    for e in range(E):
        w13 = rng.integers(-127, 128, (2 * I, H), dtype=np.int8)
        w2 = rng.integers(-127, 128, (H, I), dtype=np.int8)
        experts.append((w13.T, rng.uniform(1e-3, 1e-2, 2 * I).astype(F32), w2.T,
                        rng.uniform(1e-3, 1e-2, H).astype(F32)))
    logits = C.bfr(rng.standard_normal((T, E)).astype(F32))
    idx, w, _ = C.router_from_logits(logits, k, True)
    y = C.bf16_to_f32(C.moe_forward(x, experts, idx, w))
    wf = C.bf16_to_f32(w)
    for t in range(T):
        pairs = sorted(zip(idx[t], wf[t]))
        acc = np.zeros(H, F32)
        for e, we in pairs:
            out = C.expert_swiglu(x[t:t + 1], *experts[e])[0]
            acc = (acc + C.bfr((F32(we) * out).astype(F32))).astype(F32)
        assert np.array_equal(C.bfr(acc), y[t])


def test_expert_rows_are_independent():
    """Per-row quant and exact GEMMs: an expert's output row does not depend on the other
    rows routed to it (what lets the device permute rows freely)."""
    rng = np.random.default_rng(15)
    H, I = 64, 32
    x = C.bfr(rng.standard_normal((7, H)).astype(F32))
    w13 = rng.integers(-127, 128, (2 * I, H), dtype=np.int8)
    w2 = rng.integers(-127, 128, (H, I), dtype=np.int8)
    ex = (w13.T, rng.uniform(1e-3, 1e-2, 2 * I).astype(F32), w2.T, rng.uniform(1e-3, 1e-2, H).astype(F32))
    full = C.expert_swiglu(x, *ex)
    for r in range(7):
        assert np.array_equal(C.expert_swiglu(x[r:r + 1], *ex)[0], full[r])


# ------------------------------------------------------------------ table_scores, exactly
def _router_c() -> float:
    """moe_ref.py:61,68: 2^26 / ln 2 divided in binary64, then rounded once to binary32."""
    return f32_round(Fraction(float(2 ** 26) / 0.6931471805599453))


def _table_scores_rule(dgap: float, tab) -> int:
    """moe_ref.py:64-74 in Python integers and rationals: d = rint_even(fl32(dgap * C)) clamped at
    0; 0 when d >= 16 << 26; else tab[(d >> 13) & 8191] >> min(d >> 26, 63)."""
    p = f32_round(Fraction(float(dgap)) * Fraction(_router_c()))
    d = max(round(Fraction(p)), 0)            # round() of a Fraction: nearest, ties to even
    if d >= 16 << 26:
        return 0
    return int(tab[(d >> 13) & 8191]) >> min(d >> 26, 63)


def _straddling_gaps():
    """Gaps whose binary32 product fl32(dgap * C) lies in [8192 j - 0.5, 8192 j): rounding to the
    nearest integer gives d = 8192 j (table index j), truncation d = 8192 j - 1 (index j - 1)."""
    c = _router_c()
    out = []
    for j in list(range(1, 40)) + list(range(40, 1024, 37)):
        target = Fraction(8192 * j) - Fraction(1, 4)
        x = F32(float(target) / c)
        for _ in range(64):
            p = Fraction(f32_round(Fraction(float(x)) * Fraction(c)))
            if 8192 * j - Fraction(1, 2) <= p < 8192 * j:
                out.append(float(x))
                break
            x = np.nextafter(x, F32(np.inf)) if p < target else np.nextafter(x, F32(0))
    return out


def test_table_scores_exact_rule_and_rounding_negative_control():
    tab = C.frac_table()
    c = _router_c()
    assert float(C.ROUTER_C) == c
    gaps = _straddling_gaps()
    assert len(gaps) >= 60
    # the window edge: the largest gap whose product stays below 16 << 26 = 2^30 and the next one
    # up (products near 2^30 step by more than their 64-unit spacing), and far beyond it
    x = F32(2 ** 30 / c)
    while f32_round(Fraction(float(x)) * Fraction(c)) >= 2 ** 30:
        x = np.nextafter(x, F32(0))
    while f32_round(Fraction(float(np.nextafter(x, F32(np.inf)))) * Fraction(c)) < 2 ** 30:
        x = np.nextafter(x, F32(np.inf))
    edge = [float(x), float(np.nextafter(x, F32(np.inf))), float(F32(2 ** 33 / c))]
    allg = np.array(gaps + edge + [0.0, 1e-30, 3.5, 11.0], F32)
    got = C.table_scores(allg)
    ref = [_table_scores_rule(float(v), tab) for v in allg]
    assert [int(v) for v in got] == ref
    d_in = round(Fraction(f32_round(Fraction(edge[0]) * Fraction(c))))
    assert d_in < 2 ** 30 and ref[len(gaps)] == int(tab[(d_in >> 13) & 8191]) >> 15   # tab < 2^16
    assert ref[len(gaps) + 1] == 0 and ref[len(gaps) + 2] == 0
    # planted slip: truncating instead of rounding moves every straddling gap one table entry
    def floor_variant(dg):
        d = np.floor((np.asarray(dg, F32) * C.ROUTER_C).astype(F32)).astype(np.int64)
        d = np.maximum(d, 0)
        s = tab[(d >> 13) & 8191] >> np.minimum(d >> 26, 63)
        return np.where(d < (16 << 26), s, 0)
    slipped = floor_variant(np.array(gaps, F32))
    assert np.all(slipped != np.array(ref[:len(gaps)]))


# ------------------------------------------------------------------ E-v2 with a bias
def test_epilogue_v2_bias_brute_force_and_negative_control():
    """contract_common.py:172-174: y = fl32(fl32(fl32(acc) * asc) * ws); the bias is added in
    binary32 before the single cast to the output type (y + bias.float(), then .to(x.dtype))."""
    rng = np.random.default_rng(41)
    M, N = 5, 40
    acc = rng.integers(-(2 ** 27), 2 ** 27, (M, N)).astype(np.int32)
    asc = rng.uniform(1e-3, 1e-1, M).astype(F32)
    ws = rng.uniform(1e-3, 1e-2, N).astype(F32)
    bias = (rng.standard_normal(N) * 3).astype(F32)
    for out in ("bf16", "f32"):
        y = C.out_to_f32(C.epilogue_v2(acc, ws, asc, bias, out), out)
        slip = 0
        for m in range(M):
            for n in range(N):
                a = f32_round(Fraction(int(acc[m, n])))
                t = f32_round(Fraction(a) * Fraction(float(asc[m])))
                t = f32_round(Fraction(t) * Fraction(float(ws[n])))
                ref = f32_round(Fraction(t) + Fraction(float(bias[n])))
                if out == "bf16":
                    ref = bf16_round(ref)
                    # the planted slip: cast first, add the bias after, cast again
                    wrong = bf16_round(f32_round(Fraction(bf16_round(t)) + Fraction(float(bias[n]))))
                    slip += wrong != ref
                assert float(y[m, n]) == ref, (out, m, n)
        if out == "bf16":
            assert slip > 0


# ------------------------------------------------------------------ A9 MX epilogue
def test_lin_epilogue_mx_brute_force_and_negative_controls():
    """moe_ref.py:258-261: y = bfr(fl32(acc * asc[m])); with a bias y = bfr(fl32(y + b[n])).
    Each step is evaluated on exact rationals and rounded by f32_round / bf16_round; two
    planted slips must differ somewhere: the bias added before the first bf16 rounding, and
    the two bf16 roundings merged into one after the bias."""
    rng = np.random.default_rng(58)
    T, N = 6, 48
    # accumulators of the size the MX block chain produces: sums of s * 2^(k-128), k in [119, 130]
    acc = (rng.standard_normal((T, N)) * 2.0 ** rng.integers(-20, 12, (T, N))).astype(F32)
    acc[0, :4] = [0.0, -0.0, 1.0, -3.0]
    asc = rng.uniform(1e-3, 1e-1, T).astype(F32)
    bias = (rng.standard_normal(N) * 0.5).astype(F32)
    y0 = C.lin_epilogue_mx(acc, asc)
    y1 = C.lin_epilogue_mx(acc, asc, bias)
    assert y0.dtype == F32 and y1.dtype == F32
    early = merged = 0
    for m in range(T):
        for n in range(N):
            p = f32_round(Fraction(float(acc[m, n])) * Fraction(float(asc[m])))
            t = bf16_round(p)
            assert float(y0[m, n]) == t, (m, n)
            ref = bf16_round(f32_round(Fraction(t) + Fraction(float(bias[n]))))
            assert float(y1[m, n]) == ref, (m, n)
            early += bf16_round(bf16_round(f32_round(Fraction(p) + Fraction(float(bias[n]))))) != ref
            merged += bf16_round(f32_round(Fraction(p) + Fraction(float(bias[n])))) != ref
    assert early > 0 and merged > 0


# ------------------------------------------------------------------ A6 pow2 quantised values
def _rne_int(fr: Fraction) -> int:
    """Round an exact rational to the nearest integer, ties to even, in Python integers."""
    n = fr.numerator // fr.denominator
    r = fr - n
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return n


def test_quant8_rows_cols_values_brute_force_and_truncation_control():
    """ref_block_v1.py:64-72: q = clip(rint(fl32(x * 2^e)), -127, 127) with e from the row (or
    column) maximum.  The scaling by a power of two is exact, so q equals round-half-even of the
    exact rational x * 2^e clamped to +-127, computed here in Python integers with the exponent
    from the independent brute-force search.  A truncating rint must differ somewhere."""
    rng = np.random.default_rng(64)
    x = (rng.standard_normal((7, 40)) * 2.0 ** rng.integers(-6, 6, (7, 1))).astype(F32)
    x[1, :] = 0.0                                  # an all-zero row: e = 0, q = 0
    x[2, 5] = F32(127.0 / 64.0)                    # the maximum lands exactly on 127 after scaling
    # exact half-integers after scaling put the ties-to-even rule to work
    e3 = _e_brute(float(np.abs(x[3]).max()))
    x[3, :8] = (np.array([0.5, 1.5, 2.5, -0.5, -2.5, 3.5, 126.5, -125.5]) * 2.0 ** -e3).astype(F32)
    for fn, xx in ((C.quant8_rows, x), (C.quant8_cols, x.T.copy())):
        q, e = fn(xx)
        q = np.asarray(q)
        rows = xx if fn is C.quant8_rows else xx.T
        qq = q if fn is C.quant8_rows else q.T
        ee = np.asarray(e)
        trunc_slips = 0
        for i in range(rows.shape[0]):
            m = float(np.abs(rows[i]).max())
            ei = _e_brute(m)
            assert int(ee[i]) == ei
            for j in range(rows.shape[1]):
                v = Fraction(float(rows[i, j])) * Fraction(2) ** ei
                ref = max(-127, min(127, _rne_int(v)))
                assert int(qq[i, j]) == ref, (fn.__name__, i, j)
                tr = max(-127, min(127, int(v)))      # the planted slip: truncation toward zero
                trunc_slips += tr != ref
        assert trunc_slips > 0
