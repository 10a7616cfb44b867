"""GPU parity of the two-plane wide-integer linears (t16h_lmvariants.py:71-201): the <bits> row
quant, the plane split, the weight planes, and the a<A>w<W> logits against the oracle, bit for bit,
over every kernel family the stacked plane GEMM lands on; the int64 -> binary32 rounding at
constructed halfway cases."""
import numpy as np
import pytest
import torch

from gpu_util import bits, dev, f32_bits, say, to_dev
from oracle import contract as C

pytestmark = pytest.mark.gpu

F32 = np.float32


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import lockstep_amd._lib as L
    L.load()


@pytest.mark.parametrize("nbits", [8, 11, 15])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_quant_rows_and_planes(nbits, dtype):
    from lockstep_amd import t16h_lmvariants as T
    say("quant_rows", nbits, dtype)
    r = np.random.default_rng(nbits)
    x = (r.standard_normal((37, 777)) * 3).astype(F32)
    x[4] = 0
    x[5, :3] = [1e-30, 60000.0, -0.5]
    xt = torch.from_numpy(x).to(dtype)
    xr = xt.float().numpy()
    a, asc = T._quant_rows(xt.to(dev()), nbits)
    ao, asco = C.quant_rows_bits(xr, nbits)
    assert np.array_equal(bits(a), ao.astype(np.int32))
    assert np.array_equal(bits(asc), f32_bits(asco))
    got = T._planes(a, nbits - 8)
    ref = C.planes(ao, nbits - 8)
    assert [s for s, _ in got] == [s for s, _ in ref]
    for (_, g), (_, o) in zip(got, ref):
        assert np.array_equal(bits(g), o)


@pytest.mark.parametrize("wbits", [8, 11, 15])
def test_quantize_weight_planes(wbits):
    from lockstep_amd import t16h_lmvariants as T
    r = np.random.default_rng(40 + wbits)
    W = C.bfr((r.standard_normal((300, 512)) * 0.05).astype(F32))
    planes, ws = T.quantize_weight(torch.from_numpy(W).to(torch.bfloat16).to(dev()), wbits)
    ref, wso = C.quantize_weight_bits(W, wbits)
    assert np.array_equal(bits(ws), f32_bits(wso))
    assert [s for s, _ in planes] == [s for s, _ in ref]
    for (_, p), (_, o) in zip(planes, ref):
        assert p.shape == (512, 300) and p.stride() == (1, 512)     # [K, N] views, as the reference returns
        assert np.array_equal(bits(p.t()), o)


# rows x activation planes decide the kernel: <= 4 whole-row GEMV, <= 32 streaming GEMV,
# <= 128 the 128x128 tile, above that the ping-pong tiles
@pytest.mark.parametrize("spec", ["a8", "a15", "a11", "w15", "a15w15", "a11w11"])
@pytest.mark.parametrize("M,N,K", [(1, 1000, 512), (2, 4096, 3584), (9, 520, 1024), (40, 260, 768),
                                   (100, 2048, 512)])
def test_variant_logits_parity(spec, M, N, K):
    from lockstep_amd import t16h_lmvariants as T
    say("variant", spec, M, N, K)
    r = np.random.default_rng(M * 131 + N + K)
    W = C.bfr((r.standard_normal((N, K)) * 0.05).astype(F32))
    x = (r.standard_normal((M, K)) * 2).astype(F32)
    x[0, 3] = 40.0                                  # an outlier channel sets the row scale
    v = T.build(spec).prepare(torch.from_numpy(W).to(torch.bfloat16).to(dev()))
    y = v.logits(to_dev(x))
    wp, ws = C.quantize_weight_bits(W, v.wbits)
    ref = C.mm_planes(x, wp, ws, v.abits)
    assert np.array_equal(bits(y), f32_bits(ref)), (spec, M, N, K, int((bits(y) != f32_bits(ref)).sum()))
    # the free function over the reference-shaped planes list gives the same bits
    y2 = T._mm_planes(to_dev(x), v.wplanes, v.ws, v.abits)
    assert np.array_equal(bits(y2), f32_bits(ref))
    assert v.gemms() == (2 if v.abits > 8 else 1) * (2 if v.wbits > 8 else 1)


def test_smoothquant_variant_parity():
    """sq<AA>: the smoothing vector is a prepare-time artifact (binary32 pow); given the same
    vector, the fold (W * s), the runtime divide (x / s) and the planes are bit-exact."""
    from lockstep_amd import t16h_lmvariants as T
    r = np.random.default_rng(77)
    N, K, M = 640, 512, 6
    W = C.bfr((r.standard_normal((N, K)) * 0.05).astype(F32))
    act = np.abs(r.standard_normal(K) * 4).astype(F32) + F32(0.01)
    x = (r.standard_normal((M, K)) * 2).astype(F32)
    for spec in ("sq50", "sq80a15w15", "sq50a15"):
        v = T.build(spec).prepare(torch.from_numpy(W).to(torch.bfloat16).to(dev()), to_dev(act))
        sd = v.sdiv.cpu().numpy()
        assert np.allclose(sd, C.smooth_scales(act, W, v.alpha), rtol=2e-6)
        y = v.logits(to_dev(x))
        wp, ws = C.quantize_weight_bits(W, v.wbits, sdiv=sd)
        ref = C.mm_planes(x, wp, ws, v.abits, sdiv=sd)
        assert np.array_equal(bits(y), f32_bits(ref)), spec


def test_bias_and_bf16_logits():
    """get_logits_contract's tail: y + embedding_bias in binary32, then the cast to bf16."""
    from lockstep_amd import ops
    from lockstep_amd import t16h_lmvariants as T
    import lockstep_amd._lib as L
    r = np.random.default_rng(5)
    N, K, M = 1000, 1024, 3
    W = C.bfr((r.standard_normal((N, K)) * 0.05).astype(F32))
    x = (r.standard_normal((M, K)) * 2).astype(F32)
    b = (r.standard_normal(N) * 0.1).astype(F32)
    v = T.build("a15w15").prepare(torch.from_numpy(W).to(torch.bfloat16).to(dev()))
    y = ops.planes_linear(to_dev(x), v._w2, 15, v.ws, 15, bias=to_dev(b), out_dtype=L.LSK_BF16)
    wp, ws = C.quantize_weight_bits(W, 15)
    ref = C.bf16_bits((C.mm_planes(x, wp, ws, 15) + b[None, :]).astype(F32))
    assert np.array_equal(bits(y), ref)


def test_int64_rounding_at_halfway_cases():
    """Rows and weights that quantise to themselves (amax 16383, so every scale is exactly 1) make
    the logits fl32(s) of chosen integers s: each rounding case of int64 -> binary32 (ties to even,
    one above / below a tie, carries into the next binade) from 2^25 to 2^34, both signs."""
    from lockstep_amd import t16h_lmvariants as T
    Q = 16383
    targets = []
    for e in range(25, 34):
        ulp = 1 << (e - 23)
        for base in ((1 << e), (1 << e) + 3 * ulp, (2 << e) - ulp):
            for d in (ulp // 2, ulp // 2 - 1, ulp // 2 + 1, -(ulp // 2)):
                targets.append(base + d)
    targets += [-t for t in targets]
    N, K = len(targets), 160
    x = np.full((1, K), Q, F32)
    x[0, K - 1] = 1.0                         # the last column carries the remainder below Q
    W = np.zeros((N, K), np.int64)
    for n, t in enumerate(targets):
        q, rem = divmod(abs(t), Q * Q)
        a2, b2 = divmod(rem, Q)
        W[n, :q] = Q                          # q * Q^2
        W[n, q] = a2                          # a2 * Q
        W[n, K - 3], W[n, K - 2] = Q, -Q      # the row amax is Q (scale 1); the pair cancels
        W[n, K - 1] = b2                      # b2 * 1
        if t < 0:
            W[n] = -W[n]
    s = (x[0].astype(np.int64)[None, :] * W).sum(1)
    assert s.tolist() == targets
    v = T.build("a15w15").prepare(torch.from_numpy(W.astype(F32)).to(dev()))
    assert np.all(v.ws.cpu().numpy() == 1.0)
    y = v.logits(to_dev(x))
    want = np.array(targets, np.int64).astype(F32)[None, :]
    assert np.array_equal(bits(y), f32_bits(want))
