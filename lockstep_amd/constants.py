"""Published constants on disk -> HBM, verified before any byte reaches the device.

The reference deploys a model as a manifest directory: `constants.safetensors` holds the armed
constants (`<module>.w8` int8 [N, K], `<module>.ws` f32 [N], `<module>.bias`, the lm_head planes
`<lm_head>.plane0` / `.plane1` + `.ws`, the MXFP4 `_blocks` / `_scales`), and the manifest lists
each tensor's shape, dtype and `lockstep-tensor-v1` digest (reference/tools/lockstep_manifest.py:
132-145 the digest preimage, :183-196 the container, :209-285 the per-rank block and its check).
The manifest schema and the digest preimage are the interface kept here; the loader is this
module's own:

    sha256_tensor(t)                 the lockstep-tensor-v1 digest of a tensor
    tensor_entries(tensors)          {name: {shape, dtype, sha256}}, names sorted
    save_constants(path, tensors)    a safetensors container; returns the file's sha256
    constants_block(manifest, rank)  the rank's block of the manifest
    load_constants(mdir, manifest, device, rank)
    linear / lm_head_planes / mx_expert   the consumers' views of loaded constants

How loading works: the container's own header (an 8-byte little-endian length, then JSON with
every tensor's dtype, shape and byte range) is parsed first, so names, shapes and dtypes are
checked against the manifest before any tensor data is read.  The file is then memory-mapped
once and every digest is computed over its byte range in the map (no host copy; hashlib drops
the GIL, so the digests of a model run on all host cores).  Only when every tensor passes are
the byte ranges viewed as tensors and copied to the device, one transfer per tensor: on a 288 GB
MI355X every constant of a model stays resident.  A file that fails raises ConstantsRejected
carrying every problem found, and nothing is returned.  No pickle-based container is read.
"""
from __future__ import annotations

import hashlib
import json
import mmap
import os
import struct
import sys
from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass
from typing import Any, Dict, List, Optional, Tuple

import numpy as np
import torch

TENSOR_DIGEST_TAG = b"lockstep-tensor-v1|"
MANIFEST_FILE = "lockstep.manifest.json"

# safetensors dtype codes -> (torch dtype, bytes per element)
_ST_DTYPES = {
    "BOOL": (torch.bool, 1), "U8": (torch.uint8, 1), "I8": (torch.int8, 1), "I16": (torch.int16, 2),
    "I32": (torch.int32, 4), "I64": (torch.int64, 8), "F16": (torch.float16, 2), "BF16": (torch.bfloat16, 2),
    "F32": (torch.float32, 4), "F64": (torch.float64, 8),
}


class ManifestError(RuntimeError):
    """A manifest or a constants file is unusable; nothing is returned."""


@dataclass(frozen=True)
class Problem:
    """One reason a constants file is refused: `kind` is one of absent (listed, not in the file),
    unlisted (in the file, not listed), shape, dtype, digest, count or layout."""
    tensor: str
    kind: str
    detail: str

    def __str__(self):
        return "[%s] %s: %s" % (self.kind, self.tensor, self.detail)


class ConstantsRejected(ManifestError):
    """Raised with every Problem of a refused file (`.problems`)."""

    def __init__(self, path: str, rank: int, problems: List[Problem]):
        self.path, self.rank, self.problems = path, rank, list(problems)
        shown = "\n  ".join(str(p) for p in self.problems[:12])
        more = "" if len(self.problems) <= 12 else "\n  ... and %d more" % (len(self.problems) - 12)
        super().__init__("%s (rank %d) refused, %d problem(s):\n  %s%s"
                         % (os.path.basename(path), rank, len(self.problems), shown, more))


def dtype_name(dtype: torch.dtype) -> str:
    return str(dtype).replace("torch.", "")


def _digest_header(dtype: str, shape) -> bytes:
    return TENSOR_DIGEST_TAG + ("%s|%s|" % (dtype, "x".join(str(int(d)) for d in shape))).encode("ascii")


def _digest(header: bytes, payload) -> str:
    h = hashlib.sha256(header)
    h.update(payload)
    return h.hexdigest()


def sha256_tensor(t: torch.Tensor) -> str:
    """The lockstep-tensor-v1 digest: sha256 of 'lockstep-tensor-v1|<dtype>|<d0>x<d1>...|' and the
    tensor's little-endian bytes in row-major order."""
    if sys.byteorder != "little":
        raise ManifestError("lockstep-tensor-v1 digests are defined over little-endian bytes")
    flat = t.detach().to("cpu").contiguous().reshape(-1)
    payload = flat.view(torch.uint8).numpy().data if flat.numel() else b""
    return _digest(_digest_header(dtype_name(t.dtype), t.shape), payload)


def tensor_entries(tensors: Dict[str, torch.Tensor]) -> Dict[str, Dict[str, Any]]:
    """The manifest's tensor table for `tensors`: {name: {shape, dtype, sha256}}, names sorted."""
    table = {}
    for name in sorted(tensors):
        t = tensors[name]
        table[name] = {"shape": list(map(int, t.shape)), "dtype": dtype_name(t.dtype), "sha256": sha256_tensor(t)}
    return table


def _file_sha256(path: str) -> str:
    with open(path, "rb") as f, mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ) as mm:
        return hashlib.sha256(mm).hexdigest()


def save_constants(path: str, tensors: Dict[str, torch.Tensor], metadata: Optional[Dict[str, str]] = None) -> str:
    """Write {name: tensor} as a safetensors container (host copies, contiguous, no shared
    storage) and return the sha256 of the written file."""
    from safetensors.torch import save_file
    save_file({n: t.detach().to("cpu").contiguous().clone() for n, t in tensors.items()}, path,
              metadata=dict(metadata or {}))
    return _file_sha256(path)


def read_manifest(mdir: str) -> Dict[str, Any]:
    with open(os.path.join(mdir, MANIFEST_FILE)) as f:
        return json.load(f)


def constants_block(manifest: Dict[str, Any], rank: int = 0) -> Dict[str, Any]:
    """The constants block that rank `rank` loads.  A manifest written for tensor parallelism
    carries one block per rank in `constants_ranks`; otherwise its single `constants` block
    serves rank 0 only."""
    per_rank = manifest.get("constants_ranks") or []
    if per_rank:
        if rank in range(len(per_rank)):
            return per_rank[rank]
        raise ManifestError("rank %d asked for constants; the manifest has blocks for ranks 0..%d"
                            % (rank, len(per_rank) - 1))
    if rank == 0:
        return manifest["constants"]
    raise ManifestError("rank %d asked for constants; the manifest is single-rank" % rank)


@dataclass
class _Entry:
    dtype: str           # torch dtype name
    torch_dtype: torch.dtype
    shape: Tuple[int, ...]
    begin: int           # absolute byte offsets in the file
    end: int


def _container_index(path: str) -> Tuple[Dict[str, _Entry], List[Problem]]:
    """Parse a safetensors header: {name: _Entry} with absolute byte ranges, and layout problems
    (an unknown dtype, a byte range that disagrees with shape x element size or leaves the file)."""
    size = os.path.getsize(path)
    with open(path, "rb") as f:
        head = f.read(8)
        if len(head) != 8:
            raise ManifestError("%s: not a safetensors container (%d bytes)" % (path, size))
        (hlen,) = struct.unpack("<Q", head)
        if hlen > size - 8:
            raise ManifestError("%s: header length %d past the end of the file" % (path, hlen))
        header = json.loads(f.read(hlen))
    base = 8 + hlen
    index, problems = {}, []
    for name, meta in header.items():
        if name == "__metadata__":
            continue
        code, shape = meta.get("dtype"), tuple(int(d) for d in meta.get("shape", ()))
        lo, hi = (int(v) for v in meta.get("data_offsets", (0, -1)))
        if code not in _ST_DTYPES:
            problems.append(Problem(name, "layout", "container dtype %r is not one this loader reads" % code))
            continue
        tdt, esz = _ST_DTYPES[code]
        if hi - lo != esz * int(np.prod(shape, dtype=np.int64)) or base + hi > size or lo < 0:
            problems.append(Problem(name, "layout", "byte range [%d, %d) does not hold %s %s" % (lo, hi, code, shape)))
            continue
        index[name] = _Entry(dtype_name(tdt), tdt, shape, base + lo, base + hi)
    return index, problems


def load_constants(mdir: str, manifest: Dict[str, Any], device, rank: int = 0,
                   threads: Optional[int] = None) -> Dict[str, torch.Tensor]:
    """Verify the rank's constants file against its manifest block and return {name: tensor on
    `device`}.  Checked, in this order: the file exists; the container's tensor set equals the
    manifest's list (and its declared count); every shape and dtype; every digest.  Any failure
    raises ConstantsRejected listing all problems; nothing reaches the device unless all pass."""
    blk = constants_block(manifest, rank)
    path = os.path.join(mdir, blk["file"])
    if not os.path.isfile(path):
        raise ManifestError("rank %d constants file %s does not exist" % (rank, path))
    listed: Dict[str, Dict[str, Any]] = blk["tensors"]
    index, problems = _container_index(path)

    for name in sorted(set(listed) | set(index)):
        if name not in index:
            if not any(p.tensor == name for p in problems):
                problems.append(Problem(name, "absent", "listed in the manifest, not in the file"))
            continue
        if name not in listed:
            problems.append(Problem(name, "unlisted", "in the file, not in the manifest"))
            continue
        e, want = index[name], listed[name]
        if list(e.shape) != [int(d) for d in want["shape"]]:
            problems.append(Problem(name, "shape", "file %s, manifest %s" % (list(e.shape), list(want["shape"]))))
        elif e.dtype != want["dtype"]:
            problems.append(Problem(name, "dtype", "file %s, manifest %s" % (e.dtype, want["dtype"])))
    declared = int(blk.get("count", len(listed)))
    if declared != len(listed):
        problems.append(Problem("*", "count", "block declares %d tensors, lists %d" % (declared, len(listed))))
    if problems:
        raise ConstantsRejected(path, rank, problems)

    with open(path, "rb") as f:
        mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
    try:
        names = sorted(index)
        workers = threads or max(1, min(len(names), os.cpu_count() or 1))
        with ThreadPoolExecutor(max_workers=workers) as pool:
            got = list(pool.map(lambda n: _range_digest(mm, index[n]), names))
        problems = [Problem(n, "digest", "file %s.., manifest %s.." % (g[:12], listed[n]["sha256"][:12]))
                    for n, g in zip(names, got) if g != listed[n]["sha256"]]
        if problems:
            raise ConstantsRejected(path, rank, problems)
        return {n: _range_tensor(mm, index[n]).to(device) for n in names}
    finally:
        mm.close()


def _range_digest(mm: mmap.mmap, e: _Entry) -> str:
    """The digest of one tensor, hashed straight from its byte range in the map."""
    raw = np.frombuffer(mm, dtype=np.uint8, count=e.end - e.begin, offset=e.begin)
    return _digest(_digest_header(e.dtype, e.shape), raw)


def _range_tensor(mm: mmap.mmap, e: _Entry) -> torch.Tensor:
    """A host tensor holding one verified byte range (copied out, so the map can close)."""
    raw = np.frombuffer(mm, dtype=np.uint8, count=e.end - e.begin, offset=e.begin).copy()
    return torch.from_numpy(raw).view(e.torch_dtype).reshape(e.shape)


def linear(consts: Dict[str, torch.Tensor], name: str):
    """(W8 int8 [N, K], ws f32 [N], bias f32 [N] or None) of a contract linear: the operands of
    lockstep_fullstack.w8a8_matmul."""
    W8, ws = consts.get(name + ".w8"), consts.get(name + ".ws")
    if W8 is None or ws is None:
        raise ManifestError("linear %s needs %s.w8 and %s.ws" % (name, name, name))
    if W8.dtype != torch.int8 or W8.dim() != 2 or tuple(ws.shape) != (W8.shape[0],):
        raise ManifestError("linear %s: %s %s weight with %s scales is not an int8 [N, K] / [N] pair"
                            % (name, W8.dtype, tuple(W8.shape), tuple(ws.shape)))
    return W8, ws, consts.get(name + ".bias")


def lm_head_planes(consts: Dict[str, torch.Tensor], name: str, wbits: int = 15):
    """The lm_head weight planes stacked as one [P * N, K] buffer (hi plane rows first) and ws [N]:
    the operands of the a<A>w<wbits> planes linear."""
    keys = [name + ".plane0"] + ([name + ".plane1"] if wbits > 8 else [])
    missing = [k for k in keys + [name + ".ws"] if k not in consts]
    if missing:
        raise ManifestError("lm_head %s: %s not loaded" % (name, ", ".join(missing)))
    planes = [consts[k] for k in keys]
    stacked = planes[0] if len(planes) == 1 else torch.cat(planes, 0)
    return stacked.contiguous(), consts[name + ".ws"]


def mx_expert(consts: Dict[str, torch.Tensor], name: str, expert: Optional[int] = None):
    """(packed E2M1 codes uint8 [N, K/2], E8M0 scales uint8 [N, K/32]) of an MXFP4 weight stored as
    the checkpoint's `<name>_blocks` [E, N, K/32, 16] and `<name>_scales` [E, N, K/32] (one expert
    when `expert` is given)."""
    codes, scales = consts.get(name + "_blocks"), consts.get(name + "_scales")
    if codes is None or scales is None:
        raise ManifestError("MXFP4 weight %s needs %s_blocks and %s_scales" % (name, name, name))
    if expert is not None:
        codes, scales = codes[expert], scales[expert]
    if codes.dtype != torch.uint8 or scales.dtype != torch.uint8 or codes.shape[-1] != 16 \
            or tuple(codes.shape[:-1]) != tuple(scales.shape):
        raise ManifestError("MXFP4 weight %s: blocks %s %s and scales %s %s do not pair up"
                            % (name, codes.dtype, tuple(codes.shape), scales.dtype, tuple(scales.shape)))
    return codes.reshape(*codes.shape[:-2], -1).contiguous(), scales.contiguous()
