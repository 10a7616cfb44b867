"""GPU parity of the contract v2.5 outlier side path (lockstep_fullstack.py:549-578): the
published vectors, then bit equality with the oracle over every dense kernel family
(whole-row / streaming GEMV, 128x128 tile, ping-pong tiles), channel counts, dtypes and biases."""
import numpy as np
import pytest
import torch

from gpu_util import bf16_dev, bits, dev, f16_bits, f32_bits, say, to_dev
from oracle import contract as C
from test_oracle_vectors import outlier_weights
from vector_inputs import linear_inputs, load_vectors

pytestmark = pytest.mark.gpu

F32 = np.float32


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import lockstep_amd._lib as L
    L.load()


def test_outlier_vectors_on_gpu():
    from lockstep_amd import lockstep_fullstack as FS
    V = load_vectors()
    _, _, _, bias = linear_inputs()
    x5, oidx, wo, W8o, wso = outlier_weights(rot=True)
    xd = bf16_dev(x5)
    od = to_dev(oidx)
    wod = bf16_dev(wo)
    side = FS.outlier_side(xd[:, od.long()], wod)
    assert C.digest(bits(side).view(F32), "float32") == V["outlier.side"]["sha256"]
    y = FS.w8a8_outlier_linear(xd, od, wod, to_dev(W8o), to_dev(wso), out_dtype=torch.bfloat16)
    assert C.digest(bits(y), "bfloat16") == V["linear.v2_5.outliers.no_bias"]["sha256"]
    yb = FS.w8a8_outlier_linear(xd, od, wod, to_dev(W8o), to_dev(wso), to_dev(bias), out_dtype=torch.bfloat16)
    assert C.digest(bits(yb), "bfloat16") == V["linear.v2_5.outliers.bias"]["sha256"]
    # default out_dtype is x.dtype (bf16 here)
    assert C.digest(bits(FS.w8a8_outlier_linear(xd, od, wod, to_dev(W8o), to_dev(wso))), "bfloat16") == \
        V["linear.v2_5.outliers.no_bias"]["sha256"]
    x5, oidx, won, W8n, wsn = outlier_weights(rot=False)
    yn = FS.w8a8_outlier_linear(xd, od, bf16_dev(won), to_dev(W8n), to_dev(wsn), out_dtype=torch.bfloat16,
                                rot=False)
    assert C.digest(bits(yn), "bfloat16") == V["linear.v2_5_1.outliers_norot.no_bias"]["sha256"]


def _case(M, N, K, ko, seed, massive=True):
    r = np.random.default_rng(seed)
    x = C.bfr((r.standard_normal((M, K)) * 3).astype(F32))
    oidx = np.sort(r.choice(K, size=ko, replace=False)).astype(np.int32)
    if massive and ko:
        x[:, oidx[0]] = C.bfr((x[:, oidx[0]] * F32(400)).astype(F32))
    W8 = r.integers(-127, 128, (N, K), dtype=np.int8)
    ws = r.uniform(1e-3, 1e-2, N).astype(F32)
    wo = C.bfr((r.standard_normal((N, ko)) * 0.05).astype(F32))
    bias = (r.standard_normal(N) * 0.1).astype(F32)
    return x, oidx, wo, W8, ws, bias


# M picks the kernel family: <= 4 whole-row GEMV, <= 32 streaming GEMV, <= 128 the 128x128 tile,
# above that the ping-pong tiles (256x256 / 256x128)
SHAPES = [(1, 96, 512), (3, 1000, 256), (8, 4096, 4096), (32, 520, 1024), (33, 130, 512), (128, 256, 768),
          (300, 1000, 512), (512, 2048, 1024)]


@pytest.mark.parametrize("M,N,K", SHAPES)
@pytest.mark.parametrize("ko", [0, 1, 3, 8, 32])
def test_outlier_linear_parity(M, N, K, ko):
    from lockstep_amd import lockstep_fullstack as FS
    say("outlier_linear", M, N, K, ko)
    x, oidx, wo, W8, ws, bias = _case(M, N, K, ko, seed=M * 7919 + N * 31 + K + ko)
    use_bias = ko % 2 == 1
    rot = (M + ko) % 3 != 0
    y = FS.w8a8_outlier_linear(bf16_dev(x), to_dev(oidx), bf16_dev(wo), to_dev(W8), to_dev(ws),
                               to_dev(bias) if use_bias else None, out_dtype=torch.bfloat16, rot=rot)
    ref = C.w8a8_outlier_linear(x, oidx, wo, W8, ws, bias if use_bias else None, "bf16", rot=rot)
    assert np.array_equal(bits(y), ref), (M, N, K, ko, rot, int((bits(y) != ref).sum()))


@pytest.mark.parametrize("out", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("M", [2, 20, 200])
def test_outlier_linear_dtypes(out, xdt, M):
    """f32 rows (not bf16-valued), f32 wo, and each output type (the bf16 result cast like the
    reference's final .to(out_dtype))."""
    from lockstep_amd import lockstep_fullstack as FS
    say("outlier dtypes", out, xdt, M)
    N, K, ko = 264, 512, 5
    x, oidx, wo, W8, ws, bias = _case(M, N, K, ko, seed=11 + M)
    r = np.random.default_rng(5 + M)
    if xdt == torch.float32:
        x = (r.standard_normal((M, K)) * 3).astype(F32)
        x[:, oidx[1]] *= F32(-250)
        wo = (r.standard_normal((N, ko)) * 0.05).astype(F32)
        wod = to_dev(wo)
    else:
        wod = bf16_dev(wo)
    odt = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[out]
    xd = to_dev(x).to(xdt)
    y = FS.w8a8_outlier_linear(xd, to_dev(oidx), wod, to_dev(W8), to_dev(ws), to_dev(bias), out_dtype=odt)
    ybf = C.w8a8_outlier_linear(xd.float().cpu().numpy(), oidx, wo, W8, ws, bias, "bf16")
    yv = C.bf16_to_f32(ybf)
    want = {"f32": f32_bits(yv), "bf16": ybf, "f16": f16_bits(yv.astype(np.float16))}[out]
    assert np.array_equal(bits(y), want)


def test_outlier_side_parity_and_edges():
    from lockstep_amd import lockstep_fullstack as FS
    r = np.random.default_rng(3)
    for M, N, ko in [(1, 1, 1), (7, 300, 32), (65, 33, 4), (4, 5, 0)]:
        ho = C.bfr((r.standard_normal((M, ko)) * 100).astype(F32))
        wo = C.bfr((r.standard_normal((N, ko)) * 0.05).astype(F32))
        if ko:
            ho[0, 0] = -0.0
        side = FS.outlier_side(bf16_dev(ho), bf16_dev(wo))
        assert np.array_equal(bits(side), f32_bits(C.outlier_side(ho, wo))), (M, N, ko)
        # binary32 operands (products then round) take the same sequential rule
        hf = (r.standard_normal((M, ko)) * 100).astype(F32)
        wf = (r.standard_normal((N, ko)) * 0.05).astype(F32)
        side = FS.outlier_side(to_dev(hf), to_dev(wf))
        assert np.array_equal(bits(side), f32_bits(C.outlier_side(hf, wf))), (M, N, ko)


def test_outlier_linear_negative_index_and_empty():
    """torch indexing counts negative channels from the end; zero rows give an empty result."""
    from lockstep_amd import lockstep_fullstack as FS
    x, oidx, wo, W8, ws, bias = _case(6, 128, 512, 3, seed=99)
    neg = oidx.copy()
    neg[2] = neg[2] - 512
    y = FS.w8a8_outlier_linear(bf16_dev(x), to_dev(neg), bf16_dev(wo), to_dev(W8), to_dev(ws),
                               out_dtype=torch.bfloat16)
    assert np.array_equal(bits(y), C.w8a8_outlier_linear(x, oidx, wo, W8, ws, None, "bf16"))
    y0 = FS.w8a8_outlier_linear(torch.zeros((0, 512), dtype=torch.bfloat16, device=dev()), to_dev(oidx),
                                bf16_dev(wo), to_dev(W8), to_dev(ws))
    assert y0.shape == (0, 128)
    x3 = bf16_dev(x).reshape(2, 3, 512)
    y3 = FS.w8a8_outlier_linear(x3, to_dev(oidx), bf16_dev(wo), to_dev(W8), to_dev(ws))
    assert y3.shape == (2, 3, 128)
    assert np.array_equal(bits(y3).reshape(6, 128), C.w8a8_outlier_linear(x, oidx, wo, W8, ws, None, "bf16"))
