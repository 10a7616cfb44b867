"""Published constants on disk -> HBM, verified (the on-disk side of tools/lockstep_manifest.py).

The reference's deployment unit is a manifest directory whose `constants.safetensors` holds the
armed constants (`<module>.w8` int8 [N, K], `<module>.ws` f32 [N], `<module>.bias`, the lm_head
planes `<lm_head>.plane0` / `.plane1` int8 [N, K] + `.ws`, ...) and whose manifest lists every
tensor's shape, dtype and `lockstep-tensor-v1` digest (tools/lockstep_manifest.py:132-145, 224-285).
This module reads such a file and moves the tensors the contract GEMMs consume into device memory,
refusing to return anything when a tensor's shape, dtype or digest differs from the manifest:

    sha256_tensor(t)                         lockstep_manifest.py:132-145 (same preimage)
    tensor_entries(tensors)                  :147-155
    save_constants(path, tensors, metadata)  :183-196 (safetensors)
    constants_block(manifest, rank)          :209-221
    load_constants(mdir, manifest, device, rank)   :224-285
    linear(consts, name) / lm_head_planes(consts, name) / mx_expert(consts, name)
        the consumers' views: (W8, ws, bias) for w8a8_matmul, the stacked planes for
        t16h_lmvariants, (codes, scales) for the MXFP4 experts

Reading is memory-mapped (safetensors), the digests run in a thread pool on the host cores
(hashlib releases the GIL), and each verified tensor is copied to the device once; on a 288 GB
MI355X every constant of a model stays resident.  Only safetensors containers are read (no
pickle-based loader).
"""
from __future__ import annotations

import hashlib
import json
import os
import sys
from concurrent.futures import ThreadPoolExecutor
from typing import Any, Dict, List, Optional

import torch

TENSOR_DIGEST_TAG = b"lockstep-tensor-v1|"
MANIFEST_FILE = "lockstep.manifest.json"


class ManifestError(RuntimeError):
    """A manifest, a file or a tensor failed validation; nothing is returned."""


def dtype_name(dtype: torch.dtype) -> str:
    return str(dtype).replace("torch.", "")


def _host_bytes(t: torch.Tensor):
    if sys.byteorder != "little":
        raise ManifestError("tensor digests are defined on little-endian hosts only")
    c = t.detach().to("cpu").contiguous().reshape(-1)
    return memoryview(c.view(torch.uint8).numpy()) if c.numel() else b""


def sha256_tensor(t: torch.Tensor) -> str:
    """sha256 of 'lockstep-tensor-v1|<dtype>|<d0>x<d1>...|' followed by the raw little-endian bytes."""
    h = hashlib.sha256(TENSOR_DIGEST_TAG)
    h.update(("%s|%s|" % (dtype_name(t.dtype), "x".join(str(int(d)) for d in t.shape))).encode("ascii"))
    h.update(_host_bytes(t))
    return h.hexdigest()


def tensor_entries(tensors: Dict[str, torch.Tensor]) -> Dict[str, Dict[str, Any]]:
    """{name: {shape, dtype, sha256}} for every tensor, names sorted."""
    return {n: {"shape": [int(d) for d in tensors[n].shape], "dtype": dtype_name(tensors[n].dtype),
                "sha256": sha256_tensor(tensors[n])} for n in sorted(tensors)}


def save_constants(path: str, tensors: Dict[str, torch.Tensor], metadata: Optional[Dict[str, str]] = None) -> str:
    """Write {name: tensor} as safetensors (contiguous host copies); returns the file's sha256."""
    from safetensors.torch import save_file
    save_file({k: v.detach().to("cpu").contiguous() for k, v in tensors.items()}, path, metadata=metadata or {})
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 20), b""):
            h.update(chunk)
    return h.hexdigest()


def read_manifest(mdir: str) -> Dict[str, Any]:
    with open(os.path.join(mdir, MANIFEST_FILE)) as f:
        return json.load(f)


def constants_block(manifest: Dict[str, Any], rank: int = 0) -> Dict[str, Any]:
    """The rank's constants block: manifest['constants_ranks'][rank] when present, else
    manifest['constants'] (rank 0 only)."""
    ranks = manifest.get("constants_ranks")
    if ranks:
        if not 0 <= rank < len(ranks):
            raise ManifestError("no constants block for tp rank %d (manifest has %d)" % (rank, len(ranks)))
        return ranks[rank]
    if rank != 0:
        raise ManifestError("manifest carries a single constants block but tp rank %d asked" % rank)
    return manifest["constants"]


def load_constants(mdir: str, manifest: Dict[str, Any], device, rank: int = 0,
                   threads: Optional[int] = None) -> Dict[str, torch.Tensor]:
    """Verify every tensor of the rank's constants file against the manifest (presence, count,
    shape, dtype, digest) and return {name: tensor on `device`}.  Raises ManifestError naming up to
    eight problems; nothing is moved to the device unless all pass."""
    from safetensors import safe_open
    blk = constants_block(manifest, rank)
    path = os.path.join(mdir, blk["file"])
    if not os.path.isfile(path):
        raise ManifestError("constants file missing: %s" % path)
    want = blk["tensors"]
    with safe_open(path, framework="pt", device="cpu") as f:
        cpu = {k: f.get_tensor(k) for k in f.keys()}
    bad: List[str] = ["%s: missing from file" % n for n in sorted(set(want) - set(cpu))]
    bad += ["%s: not in manifest" % n for n in sorted(set(cpu) - set(want))]
    if not (len(cpu) == len(want) == int(blk["count"])):
        bad.append("count: manifest %s, tensors listed %d, in file %d" % (blk["count"], len(want), len(cpu)))
    names = []
    for n in sorted(set(want) & set(cpu)):
        t, e = cpu[n], want[n]
        if [int(d) for d in t.shape] != [int(d) for d in e["shape"]]:
            bad.append("%s: shape %s != manifest %s" % (n, list(t.shape), e["shape"]))
        elif dtype_name(t.dtype) != e["dtype"]:
            bad.append("%s: dtype %s != manifest %s" % (n, dtype_name(t.dtype), e["dtype"]))
        else:
            names.append(n)
    if not bad:
        nthreads = threads or max(1, min(16, os.cpu_count() or 8))
        with ThreadPoolExecutor(max_workers=nthreads) as ex:
            digests = list(ex.map(lambda n: sha256_tensor(cpu[n]), names))
        bad += ["%s: sha256 %s != manifest %s" % (n, h[:16], want[n]["sha256"][:16])
                for n, h in zip(names, digests) if h != want[n]["sha256"]]
    if bad:
        raise ManifestError("constants verification FAILED (%s, rank %d): %s" % (blk["file"], rank, "; ".join(bad[:8])))
    return {k: v.to(device) for k, v in cpu.items()}


def linear(consts: Dict[str, torch.Tensor], name: str):
    """(W8 int8 [N, K], ws f32 [N], bias f32 [N] or None) of a contract linear: the operands of
    lockstep_fullstack.w8a8_matmul."""
    try:
        W8, ws = consts[name + ".w8"], consts[name + ".ws"]
    except KeyError as e:
        raise ManifestError("linear %s: constant %s missing" % (name, e.args[0])) from None
    if W8.dtype != torch.int8 or W8.dim() != 2 or ws.shape != (W8.shape[0],):
        raise ManifestError("linear %s: w8 %s %s / ws %s do not form a [N, K] int8 weight and [N] scales"
                            % (name, W8.dtype, tuple(W8.shape), tuple(ws.shape)))
    return W8, ws, consts.get(name + ".bias")


def lm_head_planes(consts: Dict[str, torch.Tensor], name: str, wbits: int = 15):
    """The lm_head weight planes stacked as one [P * N, K] buffer (hi plane rows first) and ws [N]:
    the operands of the a<A>w<wbits> planes linear."""
    p0 = consts.get(name + ".plane0")
    if p0 is None:
        raise ManifestError("lm_head %s: plane0 missing" % name)
    planes = [p0] + ([consts[name + ".plane1"]] if wbits > 8 else [])
    return (planes[0] if len(planes) == 1 else torch.cat(planes, 0)).contiguous(), consts[name + ".ws"]


def mx_expert(consts: Dict[str, torch.Tensor], name: str, expert: Optional[int] = None):
    """(packed E2M1 codes uint8 [N, K/2], E8M0 scales uint8 [N, K/32]) of an MXFP4 weight stored as
    the checkpoint's `<name>_blocks` [E, N, K/32, 16] and `<name>_scales` [E, N, K/32] (one expert
    when `expert` is given)."""
    codes, scales = consts.get(name + "_blocks"), consts.get(name + "_scales")
    if codes is None or scales is None:
        raise ManifestError("MXFP4 weight %s: _blocks / _scales missing" % name)
    if expert is not None:
        codes, scales = codes[expert], scales[expert]
    if codes.dtype != torch.uint8 or scales.dtype != torch.uint8 or codes.shape[-1] != 16 \
            or tuple(codes.shape[:-1]) != tuple(scales.shape):
        raise ManifestError("MXFP4 weight %s: blocks %s %s do not match scales %s %s"
                            % (name, codes.dtype, tuple(codes.shape), scales.dtype, tuple(scales.shape)))
    return codes.reshape(*codes.shape[:-2], -1).contiguous(), scales.contiguous()
