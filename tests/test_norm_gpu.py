"""GPU parity of the contract 2.6 float norm (t16n_ref.py:38-92): the published norm_float digests,
then bit equality with the oracle over widths (power-of-two and not, one to sixteen waves per row),
input / gain / output dtypes, eps, special rows, the tree over given leaves, and the fused row
quant that feeds the contract GEMM."""
import numpy as np
import pytest
import torch

from gpu_util import bits, dev, f16_bits, f32_bits, say, to_dev
from oracle import contract as C
from vector_inputs import load_vectors, norm_float_inputs

pytestmark = pytest.mark.gpu

F32 = np.float32


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import lockstep_amd._lib as L
    L.load()


def test_norm_float_vectors_on_gpu():
    from lockstep_amd import t16n_ref as N_
    V = load_vectors()
    for N, eps, xn, wn in norm_float_inputs():
        xd = torch.from_numpy(xn).to(torch.bfloat16).to(dev())
        wd = torch.from_numpy(wn).to(torch.bfloat16).to(dev())
        out = N_.rmsnorm_float(xd, wd, eps=eps)
        assert C.digest(bits(out), "bfloat16") == V["norm_float.N%d.out" % N]["sha256"], N
        S = N_.row_sum_float(xd.float())
        assert C.digest(bits(S).view(F32), "float32") == V["norm_float.N%d.S" % N]["sha256"], N


WIDTHS = [8, 24, 128, 1000, 3072, 3584, 4096, 5120, 8192, 14336, 65536]


@pytest.mark.parametrize("N", WIDTHS)
@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float32])
def test_rmsnorm_parity(N, xdt):
    from lockstep_amd import t16n_ref as N_
    say("rmsnorm", N, xdt)
    r = np.random.default_rng(N)
    R = 5 if N <= 16384 else 2
    x = (r.standard_normal((R, N)) * 2).astype(F32)
    x[1] = 0.0
    if R > 2:
        x[2] = (r.standard_normal(N) * 1e-19).astype(F32)
        x[3, 0] = 3e4
    xt = torch.from_numpy(x).to(xdt)
    xr = xt.float().numpy()
    g = C.bfr((1.0 + 0.1 * r.standard_normal(N)).astype(F32))
    for eps, gain in ((0.0, None), (1e-5, g), (1e-6, np.ones(N, F32))):
        gd = torch.from_numpy(gain if gain is not None else np.ones(N, F32)).to(torch.bfloat16).to(dev())
        out = N_.rmsnorm_float(xt.to(dev()), gd, eps=eps)
        ref = C.rmsnorm_float(xr, gain if gain is not None else np.ones(N, F32), eps=eps)
        assert np.array_equal(bits(out), ref), (N, eps, int((bits(out) != ref).sum()))
    S = N_.row_sum_float(xt.to(dev()))
    assert np.array_equal(bits(S), f32_bits(C.row_sum_float(xr)))


@pytest.mark.parametrize("N", [128, 3584, 8192])
def test_fused_norm_rowquant_feeds_the_linear(N):
    """q, asc of the fused kernel equal the row quant of the bf16 norm output; the whole prologue +
    contract linear equals the oracle's rmsnorm_float -> w8a8_matmul."""
    from lockstep_amd import lockstep_fullstack as FS
    from lockstep_amd import ops
    from lockstep_amd import t16n_ref as N_
    import lockstep_amd._lib as L
    r = np.random.default_rng(N + 1)
    R, Nout = 33, 256
    x = C.bfr((r.standard_normal((R, N)) * 2).astype(F32))
    g = C.bfr((1.0 + 0.1 * r.standard_normal(N)).astype(F32))
    xd = torch.from_numpy(x).to(torch.bfloat16).to(dev())
    gd = torch.from_numpy(g).to(torch.bfloat16).to(dev())
    q, asc, out = N_.rmsnorm_float_rowquant(xd, gd, eps=1e-6, want_out=True)
    ob = C.rmsnorm_float(x, g, eps=1e-6)
    assert np.array_equal(bits(out), ob)
    qo, asco = C.rowquant(C.bf16_to_f32(ob))
    assert np.array_equal(bits(q), qo) and np.array_equal(bits(asc), f32_bits(asco))
    W8 = r.integers(-127, 128, (Nout, N), dtype=np.int8)
    ws = r.uniform(1e-3, 1e-2, Nout).astype(F32)
    y = ops.gemm(q, to_dev(W8), L.EPI_V21, L.LSK_BF16, asc=asc, ws=to_dev(ws))
    ref = C.w8a8_matmul(C.bf16_to_f32(ob), W8, ws, None, "bf16")
    assert np.array_equal(bits(y), ref)
    y2 = FS.w8a8_matmul(out, to_dev(W8), to_dev(ws), out_dtype=torch.bfloat16)
    assert np.array_equal(bits(y2), ref)


def test_out_dtypes_and_f32_gain():
    from lockstep_amd import t16n_ref as N_
    r = np.random.default_rng(9)
    N = 1024
    x = (r.standard_normal((3, N)) * 2).astype(F32)
    g = (1.0 + 0.1 * r.standard_normal(N)).astype(F32)                 # a binary32 gain (not bf16-valued)
    ob = C.rmsnorm_float(x, g, eps=1e-5)
    xd, gd = to_dev(x), to_dev(g)
    assert np.array_equal(bits(N_.rmsnorm_float(xd, gd, eps=1e-5)), ob)
    o32 = N_.rmsnorm_float(xd, gd, out_dtype=torch.float32, eps=1e-5)
    assert np.array_equal(bits(o32), f32_bits(C.bf16_to_f32(ob)))
    o16 = N_.rmsnorm_float(xd, gd, out_dtype=torch.float16, eps=1e-5)
    assert np.array_equal(bits(o16), f16_bits(C.bf16_to_f32(ob).astype(np.float16)))
    # an explicit sN, and leading dimensions
    o = N_.rmsnorm_float(xd.reshape(1, 3, N), gd, sN=32.0)
    assert np.array_equal(bits(o).reshape(3, N), C.rmsnorm_float(x, g, sN=32.0))


@pytest.mark.parametrize("n", [1, 2, 3, 7, 64, 65, 384, 1000, 4096, 5000])
def test_tree_sum_parity(n):
    """Arbitrary-sign leaves, -0 included: the -0 padding keeps every subtree exact."""
    from lockstep_amd import t16n_ref as N_
    r = np.random.default_rng(n)
    v = (r.standard_normal((4, n)) * np.exp2(r.integers(-20, 20, (4, n)))).astype(F32)
    v[1] = -0.0
    v[2, ::3] = -0.0
    out = N_.tree_sum(to_dev(v))
    assert np.array_equal(bits(out), f32_bits(C.tree_sum(v)))
