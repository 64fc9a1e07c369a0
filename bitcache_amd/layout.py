"""Views of the dense planar blobs as semantic arrays, and conversion to the
reference's array-of-structs bytes.

Blob of capacity n (include/bitcache.h):
  binary:   sign bytes [n, d/8] | fp16 scale [n]  (n*36 bytes allocated)
  residual: code bytes [n, d/2] | fp16 scale [n]  (n*130 bytes allocated)
"""
from __future__ import annotations

import torch
from torch import Tensor

from bitcache_amd import _C, _require_extension

BINARY_VEC = 36
RESIDUAL_VEC = 130


def blob_bytes(blob: Tensor) -> int:
    """Bytes of the whole blob a tensor stands for, by the operators' rule: a
    tensor that starts at byte 0 of its storage and covers less of it is a
    prefix view of a whole blob (what BitCache.attend passes) and has the
    storage's size; any other tensor is a blob of its own."""
    stor = blob.untyped_storage().nbytes()
    prefix = blob.storage_offset() == 0 and blob.numel() < stor
    return stor if prefix else blob.numel()


def capacity(blob: Tensor, residual: bool) -> int:
    per = RESIDUAL_VEC if residual else BINARY_VEC
    size = blob_bytes(blob)
    assert size % per == 0, "blob size is not a multiple of the vector size"
    return size // per


def _whole(blob: Tensor, residual: bool) -> Tensor:
    """The whole blob a tensor stands for: itself, or for a prefix view the
    allocation it is a prefix of (its planes lie past the view's end)."""
    per = RESIDUAL_VEC if residual else BINARY_VEC
    n = capacity(blob, residual)
    if blob.numel() == n * per:
        return blob
    return blob.new_empty(0).set_(blob.untyped_storage(), 0, (n * per,))


def binary_planes(blob: Tensor, head_dim: int, n: int | None = None):
    """-> (sign words int32 view [n, d/32] of little-endian uint32, scale fp16 [n]).
    A prefix view of a larger blob (BitCache's) reads that blob's planes."""
    if n is None:
        n = capacity(blob, False)
        blob = _whole(blob, False)
    sb = n * (head_dim // 8)
    signs = blob[:sb].view(torch.int32).view(n, head_dim // 32)
    scale = blob[sb:sb + 2 * n].view(torch.float16)
    return signs, scale


def residual_planes(blob: Tensor, head_dim: int, n: int | None = None):
    """-> (code bytes uint8 [n, d/2], scale fp16 [n]).
    A prefix view of a larger blob (BitCache's) reads that blob's planes."""
    if n is None:
        n = capacity(blob, True)
        blob = _whole(blob, True)
    cb = n * (head_dim // 2)
    codes = blob[:cb].view(n, head_dim // 2)
    scale = blob[cb:cb + 2 * n].view(torch.float16)
    return codes, scale


def to_reference(blob: Tensor, head_dim: int, residual: bool) -> Tensor:
    """Dense planar blob -> the reference's BinaryVec/ResidualVec bytes (device kernel)."""
    _require_extension()
    return _C.convert(_whole(blob, residual), capacity(blob, residual), head_dim, residual, True)


def from_reference(ref_bytes: Tensor, head_dim: int, residual: bool) -> Tensor:
    """The reference's BinaryVec/ResidualVec bytes -> dense planar blob (device kernel)."""
    _require_extension()
    return _C.convert(ref_bytes, capacity(ref_bytes, residual), head_dim, residual, False)
