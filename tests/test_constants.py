"""The constants loader (tools/lockstep_manifest.py:132-285): the tensor digest is the published
preimage (checked against the conformance digests), a saved file round-trips, and a tampered,
reshaped, retyped, missing or extra tensor is refused before anything reaches a device."""
import numpy as np
import pytest
import torch

from lockstep_amd import constants as K
from oracle import contract as C
from vector_inputs import linear_inputs, load_vectors


def _manifest(tensors, fname="constants.safetensors"):
    return {"constants": {"file": fname, "sha256": "", "count": len(tensors), "tensors": K.tensor_entries(tensors),
                          "export_meta": {}}}


def test_digest_is_the_published_preimage():
    V = load_vectors()
    _, x, W, bias = linear_inputs()
    W8, ws = C.quantize_weight_int8(W)
    assert K.sha256_tensor(torch.from_numpy(W8)) == V["weight_quant.w8"]["sha256"]
    assert K.sha256_tensor(torch.from_numpy(ws)) == V["weight_quant.ws"]["sha256"]
    y = C.w8a8_matmul(x, W8, ws, None, "bf16")
    assert K.sha256_tensor(torch.from_numpy(y.view(np.int16)).view(torch.bfloat16)) == \
        V["linear.v2_1.no_bias"]["sha256"]


def _consts():
    r = np.random.default_rng(0)
    return {"model.layers.0.mlp.down_proj.w8": torch.from_numpy(r.integers(-127, 128, (64, 256), dtype=np.int8)),
            "model.layers.0.mlp.down_proj.ws": torch.from_numpy(r.uniform(1e-3, 1e-2, 64).astype(np.float32)),
            "lm_head.plane0": torch.from_numpy(r.integers(-128, 128, (32, 256), dtype=np.int8)),
            "lm_head.plane1": torch.from_numpy(r.integers(0, 128, (32, 256), dtype=np.int8)),
            "lm_head.ws": torch.from_numpy(r.uniform(1e-5, 1e-4, 32).astype(np.float32)),
            "model.layers.0.mlp.experts.down_proj_blocks": torch.from_numpy(
                r.integers(0, 256, (2, 16, 4, 16), dtype=np.uint8)),
            "model.layers.0.mlp.experts.down_proj_scales": torch.from_numpy(
                r.integers(119, 130, (2, 16, 4), dtype=np.uint8)),
            "model.norm.G": torch.zeros(4, dtype=torch.int32).bfloat16()}


def test_round_trip_and_consumer_views(tmp_path):
    t = _consts()
    K.save_constants(str(tmp_path / "constants.safetensors"), t)
    got = K.load_constants(str(tmp_path), _manifest(t), "cpu")
    assert set(got) == set(t) and all(torch.equal(got[n], t[n]) for n in t)
    W8, ws, b = K.linear(got, "model.layers.0.mlp.down_proj")
    assert W8.shape == (64, 256) and ws.shape == (64,) and b is None
    w2, hws = K.lm_head_planes(got, "lm_head", 15)
    assert w2.shape == (64, 256) and torch.equal(w2[32:], t["lm_head.plane1"])
    codes, sc = K.mx_expert(got, "model.layers.0.mlp.experts.down_proj", 1)
    assert codes.shape == (16, 64) and sc.shape == (16, 4)
    assert torch.equal(codes[3, 16:32], t["model.layers.0.mlp.experts.down_proj_blocks"][1, 3, 1])


@pytest.mark.parametrize("fault", ["byte", "shape", "dtype", "missing", "extra", "count"])
def test_tampered_constants_are_refused(tmp_path, fault):
    t = _consts()
    m = _manifest(t)
    bad = dict(t)
    if fault == "byte":
        w = bad["lm_head.plane1"].clone()
        w[3, 7] += 1
        bad["lm_head.plane1"] = w
    elif fault == "shape":
        bad["lm_head.ws"] = bad["lm_head.ws"][:31]
    elif fault == "dtype":
        bad["lm_head.ws"] = bad["lm_head.ws"].double()
    elif fault == "missing":
        del bad["lm_head.plane0"]
    elif fault == "extra":
        bad["lm_head.extra"] = torch.zeros(2)
    elif fault == "count":
        m["constants"]["count"] += 1
    K.save_constants(str(tmp_path / "constants.safetensors"), bad)
    with pytest.raises(K.ManifestError):
        K.load_constants(str(tmp_path), m, "cpu")


def test_rank_blocks():
    m = {"constants": {"file": "a"}, "constants_ranks": [{"file": "a"}, {"file": "b"}]}
    assert K.constants_block(m, 1)["file"] == "b"
    with pytest.raises(K.ManifestError):
        K.constants_block(m, 2)
    with pytest.raises(K.ManifestError):
        K.constants_block({"constants": {"file": "a"}}, 1)


@pytest.mark.gpu
def test_loaded_constants_feed_the_device_linears(tmp_path):
    """Constants verified on load go straight to HBM and reproduce the published linear digest
    and the oracle's a15w15 logits."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from lockstep_amd import lockstep_fullstack as FS
    from lockstep_amd import ops
    V = load_vectors()
    _, x, W, _ = linear_inputs()
    W8, ws = C.quantize_weight_int8(W)
    wp, hws = C.quantize_weight_bits(W, 15)
    t = {"q_proj.w8": torch.from_numpy(W8), "q_proj.ws": torch.from_numpy(ws),
         "lm_head.plane0": torch.from_numpy(wp[0][1]), "lm_head.plane1": torch.from_numpy(wp[1][1]),
         "lm_head.ws": torch.from_numpy(hws)}
    K.save_constants(str(tmp_path / "constants.safetensors"), t)
    got = K.load_constants(str(tmp_path), _manifest(t), torch.device("cuda", 0))
    W8d, wsd, bd = K.linear(got, "q_proj")
    xd = torch.from_numpy(x).to(torch.bfloat16).cuda()
    y = FS.w8a8_matmul(xd, W8d, wsd, bd, out_dtype=torch.bfloat16)
    assert K.sha256_tensor(y) == V["linear.v2_1.no_bias"]["sha256"]
    w2, hwsd = K.lm_head_planes(got, "lm_head", 15)
    logits = ops.planes_linear(xd.float(), w2, 15, hwsd, 15)
    ref = C.mm_planes(x, wp, hws, 15)
    assert np.array_equal(logits.cpu().numpy().view(np.uint32), ref.view(np.uint32))


def test_every_problem_is_reported(tmp_path):
    """A file with several faults is refused once, with one record per fault (digest faults are
    reported only after the structural checks pass)."""
    t = _consts()
    m = _manifest(t)
    bad = dict(t)
    bad["lm_head.ws"] = bad["lm_head.ws"][:31]          # shape
    del bad["model.norm.G"]                              # absent
    bad["stray"] = torch.ones(3)                         # unlisted
    K.save_constants(str(tmp_path / "constants.safetensors"), bad)
    with pytest.raises(K.ConstantsRejected) as ei:
        K.load_constants(str(tmp_path), m, "cpu")
    kinds = sorted((p.kind, p.tensor) for p in ei.value.problems)
    assert kinds == [("absent", "model.norm.G"), ("shape", "lm_head.ws"), ("unlisted", "stray")]
    bad = dict(t)
    for n in ("lm_head.plane0", "model.layers.0.mlp.down_proj.ws"):
        w = bad[n].clone()
        w.view(torch.uint8).view(-1)[5] ^= 1
        bad[n] = w
    K.save_constants(str(tmp_path / "constants.safetensors"), bad)
    with pytest.raises(K.ConstantsRejected) as ei:
        K.load_constants(str(tmp_path), m, "cpu")
    assert sorted(p.tensor for p in ei.value.problems if p.kind == "digest") == \
        ["lm_head.plane0", "model.layers.0.mlp.down_proj.ws"]
