"""Pins the oracle's two-plane wide-integer linears (t16h_lmvariants.py:71-125) by what the
mathematics fixes: the 8-bit quant is the digest-pinned row quant, the wider quants match a
rational brute force, the plane split is an exact identity, the int64 plane combine equals the
direct exact product, and fl32(s) is the correctly rounded value of s."""
from fractions import Fraction

import numpy as np
import pytest

from oracle import contract as C
from test_oracle_pins import f32_round

F32 = np.float32


def test_quant_rows_bits_at_8_is_the_row_quant():
    r = np.random.default_rng(1)
    x = (r.standard_normal((9, 300)) * 4).astype(F32)
    x[3] = 0
    a, asc = C.quant_rows_bits(x, 8)
    q, asc8 = C.rowquant(x)
    assert np.array_equal(a, q.astype(np.int64)) and np.array_equal(asc, asc8)


@pytest.mark.parametrize("bits", [11, 15])
def test_quant_rows_bits_brute_force(bits):
    r = np.random.default_rng(bits)
    x = (r.standard_normal((4, 40)) * 3).astype(F32)
    x[1, :5] = [0.5, -0.5, 1e-30, 0.0, -2.0]
    x[2] = 0.0
    qmax = (1 << (bits - 1)) - 1
    a, asc = C.quant_rows_bits(x, bits)
    for m in range(x.shape[0]):
        am = max(max(abs(float(v)) for v in x[m]), float(F32(1e-8)))
        s = f32_round(Fraction(am) / qmax)
        assert float(asc[m]) == s
        for k in range(x.shape[1]):
            quo = f32_round(Fraction(float(x[m, k])) / Fraction(s))
            fr = Fraction(quo)
            n = fr.numerator // fr.denominator
            rem = fr - n
            if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
                n += 1
            assert int(a[m, k]) == max(-qmax, min(qmax, n)), (m, k)


@pytest.mark.parametrize("bits", [8, 11, 15])
def test_plane_identity(bits):
    qmax = (1 << (bits - 1)) - 1
    a = np.arange(-qmax, qmax + 1, dtype=np.int64)
    ps = C.planes(a, bits - 8)
    rebuilt = sum(p.astype(np.int64) << sh for sh, p in ps)
    assert np.array_equal(rebuilt, a)
    if bits > 8:
        (sh, hi), (_, lo) = ps
        assert sh == bits - 8 and hi.min() >= -128 and hi.max() <= 127
        assert lo.min() == 0 and lo.max() == (1 << sh) - 1
        assert np.array_equal(hi.astype(np.int64), np.floor_divide(a, 1 << sh))


@pytest.mark.parametrize("abits,wbits", [(8, 8), (15, 8), (8, 15), (11, 11), (15, 15)])
def test_mm_planes_equals_direct_exact_product(abits, wbits):
    r = np.random.default_rng(abits * 100 + wbits)
    M, N, K = 5, 33, 700
    x = (r.standard_normal((M, K)) * 2).astype(F32)
    W = (r.standard_normal((N, K)) * 0.05).astype(F32)
    wp, ws = C.quantize_weight_bits(W, wbits)
    y = C.mm_planes(x, wp, ws, abits)
    a, asc = C.quant_rows_bits(x, abits)
    wq, _ = C.quant_rows_bits(W, wbits)
    s = a @ wq.T                                           # exact: |s| < 2^53
    for m in range(M):
        for n in range(N):
            v = f32_round(Fraction(int(s[m, n])))
            v = f32_round(Fraction(v) * Fraction(float(asc[m])))
            v = f32_round(Fraction(v) * Fraction(float(ws[n])))
            assert float(y[m, n]) == v, (m, n)


def test_mm_planes_a8w8_is_the_e_v2_linear():
    r = np.random.default_rng(7)
    x = (r.standard_normal((6, 256)) * 3).astype(F32)
    W = (r.standard_normal((40, 256)) * 0.05).astype(F32)
    wp, ws = C.quantize_weight_bits(W, 8)
    W8, ws8 = C.quantize_weight_int8(W)
    assert np.array_equal(wp[0][1], W8) and np.array_equal(ws, ws8)
    assert np.array_equal(C.mm_planes(x, wp, ws, 8), C.w8a8_linear_fwd(x, W8, ws8, None, "f32"))


def test_int64_to_f32_is_round_to_nearest_even():
    """numpy's int64 -> float32 cast rounds to nearest even at every halfway case the combine can
    produce (|s| < 2^41 for K <= 3584 at 15 x 15 bits)."""
    vals = []
    for e in range(24, 41):
        base = 1 << e
        ulp = 1 << (e - 23)
        for k in (0, 1, 2, 3, 7):
            for d in (-1, 0, 1):
                vals.append(base + k * ulp + ulp // 2 + d)
    vals = np.array(vals + [-v for v in vals], np.int64)
    got = vals.astype(F32)
    for v, g in zip(vals.tolist(), got.tolist()):
        assert g == f32_round(Fraction(v)), v


def test_smooth_scales_is_the_textbook_formula():
    r = np.random.default_rng(3)
    W = (r.standard_normal((20, 16)) * 0.1).astype(F32)
    act = np.abs(r.standard_normal(16) * 5).astype(F32)
    s = C.smooth_scales(act, W, 0.5)
    ref = np.sqrt(np.maximum(act.astype(np.float64), 1e-5)) / np.sqrt(np.maximum(np.abs(W).max(0), 1e-5))
    assert np.allclose(s, ref, rtol=1e-6)
