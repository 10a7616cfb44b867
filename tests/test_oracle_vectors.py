"""Pins the oracle against the reference's committed conformance digests
(conformance/contract_vectors.json, tools/contract_vectors.py:59-144)."""
import numpy as np
import pytest

from oracle import contract as C
from vector_inputs import linear_inputs, load_vectors, outlier_inputs, silu_r4_inputs

V = load_vectors()


def _check(name, arr, dtype):
    got = C.digest(arr, dtype)
    assert got == V[name]["sha256"], (name, np.asarray(arr).reshape(-1)[:6], V[name]["head"])


def test_act_quant_digests():
    _, x, _, _ = linear_inputs()
    q, asc = C.quantize_rows_int8(x)
    _check("act_quant.q", q, "int8")
    _check("act_quant.asc", asc.astype(np.float32), "float32")


def test_weight_quant_digests():
    _, _, W, _ = linear_inputs()
    W8, ws = C.quantize_weight_int8(W)
    _check("weight_quant.w8", W8, "int8")
    _check("weight_quant.ws", ws.astype(np.float32), "float32")


@pytest.mark.parametrize("method", ["i64", "f64"])
def test_linear_v21_digests(method):
    _, x, W, bias = linear_inputs()
    W8, ws = C.quantize_weight_int8(W)
    q, asc = C.rowquant(x)
    acc = C.int_mm(q, W8.T, method=method)
    y = C.epilogue_v21(acc, ws, asc, None, "bf16")
    _check("linear.v2_1.no_bias", y, "bfloat16")
    yb = C.epilogue_v21(acc, ws, asc, bias, "bf16")
    _check("linear.v2_1.bias", yb, "bfloat16")
    # the composite form and moe_ref's lin_epilogue agree with the same digests
    _check("linear.v2_1.no_bias", C.w8a8_matmul(x, W8, ws, None, "bf16"), "bfloat16")
    _check("linear.v2_1.bias", C.w8a8_matmul(x, W8, ws, bias, "bf16"), "bfloat16")
    _check("linear.v2_1.no_bias", C.bf16_bits(C.lin_epilogue(acc, ws, asc)), "bfloat16")
    _check("linear.v2_1.bias", C.bf16_bits(C.lin_epilogue_b(acc, ws, asc, bias)), "bfloat16")


def test_linear_negative_control_v2_order_differs_or_matches_v21_rarely():
    """E-v2 multiplies asc first; on these vectors it must not reproduce the v2.1 digest
    unless every element happens to agree (it does not, on the bias case, by rounding)."""
    _, x, W, bias = linear_inputs()
    W8, ws = C.quantize_weight_int8(W)
    q, asc = C.rowquant(x)
    acc = C.int_mm(q, W8.T)
    v21 = C.epilogue_v21(acc, ws, asc, bias, "bf16")
    v2 = C.epilogue_v2(acc, ws, asc, bias, "bf16")
    # E-v2 adds the bias before the single bf16 rounding: it is a different function
    assert not np.array_equal(v21, v2)


def test_silu_digests():
    gate, up, _ = silu_r4_inputs()
    s = C.silu_contract(gate)
    _check("silu", s, "float32")
    _check("silu_mul", C.bf16_bits((s * up).astype(np.float32)), "bfloat16")
    # moe_ref.act_silu is the same function, kept in binary32
    _check("silu_mul", C.bf16_bits(C.act_silu(gate, up)), "bfloat16")


def test_r4_digest():
    _, _, v = silu_r4_inputs()
    _check("r4.block256", C.fwht_blocks(v), "float32")


def test_outlier_inputs_regenerate():
    """The outlier case draws from its own stream; its published inputs pin the generator."""
    x5, W5, oidx = outlier_inputs()
    _check("outlier.oidx", oidx, "int32")
    _check("outlier.ho", C.bf16_bits(x5[:, oidx]), "bfloat16")
    W64 = W5.astype(np.float64)
    wo = C.bf16_bits(W64[:, oidx].astype(np.float32))
    _check("outlier.wo", wo, "bfloat16")
    W64[:, oidx] = 0.0
    W8n, _ = C.quantize_weight_int8(C.bfr(W64.astype(np.float32)))
    _check("outlier.norot.w8", W8n, "int8")


def outlier_weights(rot=True):
    """The published outlier weights (tools/contract_vectors.py:88-99): wo from the bf16 weight's
    oidx columns; W8 from the weight with those columns zeroed, block-rotated in binary32 when
    `rot`, rounded to bf16 and quantised per output channel."""
    x5, W5, oidx = outlier_inputs()
    W64 = W5.astype(np.float64)
    wo = C.bfr(W64[:, oidx].astype(np.float32))
    W64[:, oidx] = 0.0
    Wz = W64.astype(np.float32)
    Wr = C.bfr(C.fwht_blocks(Wz) if rot else Wz)
    W8, ws = C.quantize_weight_int8(Wr)
    return x5, oidx, wo, W8, ws


def test_outlier_side_and_linear_digests():
    x5, oidx, wo, W8o, wso = outlier_weights(rot=True)
    _check("outlier.w8", W8o, "int8")
    _check("outlier.side", C.outlier_side(x5[:, oidx], wo), "float32")
    _, _, _, bias = linear_inputs()
    _check("linear.v2_5.outliers.no_bias", C.w8a8_outlier_linear(x5, oidx, wo, W8o, wso, None, "bf16"), "bfloat16")
    _check("linear.v2_5.outliers.bias", C.w8a8_outlier_linear(x5, oidx, wo, W8o, wso, bias, "bf16"), "bfloat16")
    x5, oidx, won, W8n, wsn = outlier_weights(rot=False)
    _check("outlier.norot.w8", W8n, "int8")
    _check("linear.v2_5_1.outliers_norot.no_bias",
           C.w8a8_outlier_linear(x5, oidx, won, W8n, wsn, None, "bf16", rot=False), "bfloat16")


def test_outlier_negative_controls():
    """A plausible slip fails a digest: the side added before the y8 rounding, the side summed
    in reverse order, or the rotation left out of the rotated case."""
    x5, oidx, wo, W8o, wso = outlier_weights(rot=True)
    ref = V["linear.v2_5.outliers.no_bias"]["sha256"]
    xr = C.fwht_blocks(np.where(np.isin(np.arange(512), oidx)[None, :], np.float32(0), x5))
    q, asc = C.rowquant(xr)
    acc = C.int_mm(q, W8o.T)
    y = ((acc.astype(np.float32) * wso[None, :]).astype(np.float32) * asc[:, None]).astype(np.float32)
    fused = C.bf16_bits((y + C.outlier_side(x5[:, oidx], wo)).astype(np.float32))
    assert C.digest(fused, "bfloat16") != ref
    rev = C.outlier_side(x5[:, oidx][:, ::-1], wo[:, ::-1])
    assert C.digest(rev, "float32") != V["outlier.side"]["sha256"]
    norot = C.w8a8_outlier_linear(x5, oidx, wo, W8o, wso, None, "bf16", rot=False)
    assert C.digest(norot, "bfloat16") != ref


def test_frac_table_digest():
    t = C.frac_table()
    assert t.shape == (8192,)
    assert t.min() >= 1 << 14 and t.max() <= 1 << 15


def test_norm_float_digests():
    from vector_inputs import norm_float_inputs
    for N, eps, xn, wn in norm_float_inputs():
        _check("norm_float.N%d.out" % N, C.rmsnorm_float(xn, wn, eps=eps), "bfloat16")
        _check("norm_float.N%d.S" % N, C.row_sum_float(xn), "float32")


def test_tree_equals_negzero_padded_perfect_tree():
    """The kernels evaluate the pinned tree as a perfect pairwise tree over leaves padded with -0
    to a power of two; the two are the same function (x + (-0) == x in binary32), including
    signed zeros, while +0 padding is not (a negative control)."""
    r = np.random.default_rng(0)

    def perfect(v, pad):
        n = v.shape[1]
        P = 1 << max(0, (n - 1).bit_length())
        w = np.full((v.shape[0], P), pad, np.float32)
        w[:, :n] = v
        h = 1
        while h < P:
            w[:, 0::2 * h] = (w[:, 0::2 * h] + w[:, h::2 * h]).astype(np.float32)
            h *= 2
        return w[:, 0]

    for n in (1, 2, 3, 5, 6, 7, 9, 100, 384, 448, 1000):
        v = (r.standard_normal((6, n)) * np.exp2(r.integers(-30, 30, (6, n)))).astype(np.float32)
        v[0] = -0.0
        v[1, ::2] = -0.0
        assert np.array_equal(C.tree_sum(v).view(np.uint32), perfect(v, -0.0).view(np.uint32)), n
    v = np.full((1, 3), -0.0, np.float32)
    assert C.tree_sum(v).view(np.uint32)[0] != perfect(v, 0.0).view(np.uint32)[0]
