"""Pins the oracle's MX2 functions (block-scaled activations, reference/moe_ref.py:293-352).

The reference holds no vectors for this path, so each function is checked against what the
mathematics fixes:
  blockquant: the exponent is the least k with 127 * 2^k >= am (exact, from Python integers and
  binary64), clamped to [-126, 127]; q rounds half to even and reconstructs x within half a step;
  int_mm_mx2: with one exponent per row it is int_mm_mx with shifted weight exponents; a single
  block is fl32(s * fl32(2^e)) computed through binary64; plausible slips fail these checks.
"""
import math

import numpy as np
import pytest

from oracle import contract as C

F32 = np.float32


def exact_ka(am: float) -> int:
    """least k with 127 * 2^k >= am (am > 0 finite), in binary64 (exact for these operands)"""
    k = math.frexp(am)[1] - 8
    while 127.0 * math.ldexp(1.0, k) < am:
        k += 1
    while k > -400 and 127.0 * math.ldexp(1.0, k - 1) >= am:
        k -= 1
    return k


def expected_ka(am):
    am = float(am)
    if am == 0.0:
        return -126
    if math.isinf(am):
        return 127
    return min(127, max(-126, exact_ka(am)))


def adversarial_maxima():
    vals = [0.0, 1.0, 127.0, 63.5, 63.5000038, 128.0, 3.0e38, float(np.finfo(F32).max), 1e-45, 1e-40, 1.17e-38,
            127.0 * 2.0 ** -126, 127.0 * 2.0 ** -127, float("inf")]
    for j in range(-130, 122, 3):
        b = F32(127.0 * 2.0 ** j) if j > -140 else F32(0)
        vals += [float(b), float(np.nextafter(b, F32(np.inf))), float(np.nextafter(b, F32(0)))]
    r = np.random.default_rng(1)
    vals += list((r.standard_normal(200) * np.exp2(r.integers(-120, 120, 200))).astype(F32).astype(float))
    return np.abs(np.array(vals, dtype=F32))


def blocks_with_maxima(am):
    """one 32-wide block per maximum: the maximum at a varying lane (sign alternating), the rest
    smaller values of both signs"""
    n = am.shape[0]
    r = np.random.default_rng(2)
    x = (r.uniform(-1, 1, (n, 32)).astype(F32) * np.where(np.isinf(am), F32(1e30), am)[:, None]).astype(F32)
    lane = np.arange(n) % 32
    x[np.arange(n), lane] = np.where(np.arange(n) % 2 == 0, am, -am)
    return x


def test_blockquant_exponent_is_exact():
    am = adversarial_maxima()
    x = blocks_with_maxima(am)
    q, ka = C.blockquant(x)
    want = np.array([expected_ka(a) for a in am], np.int32)
    assert np.array_equal(ka[:, 0], want), np.nonzero(ka[:, 0] != want)


def test_blockquant_values():
    am = adversarial_maxima()
    finite = np.isfinite(am)
    x = blocks_with_maxima(am[finite])
    q, ka = C.blockquant(x)
    q64 = q.astype(np.float64)
    step = np.ldexp(1.0, ka[:, 0].astype(np.int64))[:, None]
    err = np.abs(x.astype(np.float64) - q64 * step)
    assert (np.abs(q64) <= 127).all()
    assert (err <= step / 2).all()
    # the block maximum lands in [64, 127] whenever the exponent is not clamped at -126
    big = (ka[:, 0] > -126) & (am[finite] > 0)
    assert (np.abs(q64[big]).max(axis=1) >= 64).all()
    # exact halves round to even
    h = np.zeros((1, 32), F32)
    h[0, :6] = [127.0, 0.5, 1.5, 2.5, -2.5, -0.5]
    qh, kh = C.blockquant(h)
    assert kh[0, 0] == 0 and qh[0, :6].tolist() == [127, 0, 2, 2, -2, 0]
    # infinities saturate at +-127 with the exponent clamped at 127
    qi, ki = C.blockquant(np.array([[np.inf] + [1.0] * 31], F32))
    assert ki[0, 0] == 127 and qi[0, 0] == 127


def test_blockquant_negative_controls():
    """floor instead of ceil, a 128 divisor, or no guard each miss the exact exponent somewhere"""
    am = adversarial_maxima()
    am = am[np.isfinite(am) & (am > 0)]
    want = np.array([expected_ka(a) for a in am])
    with np.errstate(divide="ignore"):
        l2 = np.log2((am / F32(127.0)).astype(F32))
        l2b = np.log2((am / F32(128.0)).astype(F32))
    floor = np.clip(np.floor(l2), -126, 127)
    d128 = np.clip(np.ceil(l2b), -126, 127)
    assert (floor != want).any() and (d128 != want).any()
    # the guard matters where fl32(am / 127) rounds down onto a power of two
    j = -10
    b = np.nextafter(F32(127.0 * 2.0 ** j), F32(np.inf))
    unguarded = int(np.ceil(np.log2((b / F32(127.0)).astype(F32))))
    assert expected_ka(b) == j + 1
    assert C.blockquant(np.full((1, 32), b, F32))[1][0, 0] == j + 1
    if unguarded == j:  # this host's log2f lands on the integer: the guard is what fixes it
        assert unguarded != expected_ka(b)


def _m2(r, shape):
    vals = np.array([0, 1, 2, 3, 4, 6, 8, 12], np.int64)
    return (vals[r.integers(0, 8, shape)] * r.choice([-1, 1], shape)).astype(np.int8)


def test_int_mm_mx2_equals_mx_with_shifted_exponents():
    r = np.random.default_rng(3)
    T, N, K = 5, 7, 96
    q = r.integers(-127, 128, (T, K)).astype(np.int8)
    m2 = _m2(r, (N, K))
    kexp = r.integers(100, 150, (N, K // 32)).astype(np.int64)
    c = r.integers(-40, 40, T)
    ka = np.repeat(c[:, None], K // 32, axis=1).astype(np.int32)
    got = C.int_mm_mx2(q, ka, m2, kexp)
    for m in range(T):
        ref = C.int_mm_mx(q[m:m + 1], m2, (kexp + c[m]).astype(np.uint8))
        assert np.array_equal(got[m:m + 1].view(np.uint32), ref.view(np.uint32)), m


@pytest.mark.parametrize("ka", [-126, -60, -21, 0, 57, 111, 127])
def test_int_mm_mx2_one_block_closed_form(ka):
    r = np.random.default_rng(200 + ka)
    N = 24
    q = r.integers(-127, 128, (3, 32)).astype(np.int8)
    q[2] = 0
    m2 = _m2(r, (N, 32))
    kexp = np.array([0, 1, 2, 20, 100, 127, 128, 129, 200, 239, 240, 255] * 2, np.int64)[:, None]
    got = C.int_mm_mx2(q, np.full((3, 1), ka, np.int32), m2, kexp)
    s = q.astype(np.int64) @ m2.astype(np.int64).T
    for m in range(3):
        for n in range(N):
            e = ka + int(kexp[n, 0]) - 128
            p = F32(math.ldexp(1.0, e)) if e < 1000 else F32(np.inf)  # binary64 -> binary32, RNE
            prod = float(s[m, n]) * float(p)                         # exact in binary64
            want = F32(prod) if not math.isnan(prod) else F32(np.nan)
            g = got[m, n]
            assert (np.isnan(g) and np.isnan(want)) or g.view(np.uint32) == (F32(0) + want).view(np.uint32), (m, n, e)


def test_int_mm_mx2_negative_controls():
    # the fused update fl32(s * 2^e) keeps a contribution that fl32(2^e) = 0 drops (e = -150)
    q = np.zeros((1, 32), np.int8)
    q[0, 0] = 3
    m2 = np.zeros((1, 32), np.int8)
    m2[0, 0] = 1
    got = C.int_mm_mx2(q, np.array([[-126]], np.int32), m2, np.array([[104]]))
    assert got[0, 0] == 0
    assert F32(3.0 * 2.0 ** -150) != 0
    # ascending block order is observable: 1 + 1 + 2^24 is exact, 2^24 + 1 + 1 rounds twice
    q4 = np.zeros((1, 96), np.int8)
    m4 = np.zeros((1, 96), np.int8)
    q4[0, [0, 32, 64]] = 1
    m4[0, [0, 32, 64]] = 1
    kw = np.array([[128, 128, 128]])
    asc = C.int_mm_mx2(q4, np.array([[0, 0, 24]], np.int32), m4, kw)
    dsc = C.int_mm_mx2(q4, np.array([[24, 0, 0]], np.int32), m4, kw)
    assert asc[0, 0] == F32(2.0 ** 24 + 2) and dsc[0, 0] == F32(2.0 ** 24)


def test_expert_block_mx2_composition():
    """expert_block_mx2 on rows whose block exponents are all equal reduces to the MX operand with
    shifted exponents and no row scale (y = bfr(acc))"""
    r = np.random.default_rng(5)
    H, I = 64, 32
    x = np.zeros((2, H), F32)
    x[:, :] = r.integers(-127, 128, (2, H)).astype(F32) * F32(2.0 ** -3)
    x[:, ::32] = F32(127 * 2.0 ** -3)       # every block's maximum pins ka = -3
    m13, k13 = _m2(r, (2 * I, H)), r.integers(118, 126, (2 * I, H // 32))
    m2, k2 = _m2(r, (H, I)), r.integers(118, 126, (H, I // 32))
    q, ka = C.blockquant(x)
    assert (ka == -3).all()
    y = C.bfr(C.int_mm_mx(q, m13, (k13 - 3).astype(np.uint8)))
    h = C.act_silu(y[:, :I], y[:, I:])
    q2, ka2 = C.blockquant(C.bfr(h))
    want = C.bfr(C.int_mm_mx2(q2, ka2, m2, k2))
    got = C.expert_block_mx2(x, (m13, k13), (m2, k2), C.act_silu)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
