"""Low-level functional API (bitcache/functional.py of the reference).

Same functions, arguments and validation as the reference (ROCm tensors play
the reference's CUDA tensors: ``Tensor.is_cuda`` is True for them), plus
GQA/ring-stride keywords and the operators the reference lacks.  CPU tensors
are rejected, as in the reference: there is no CPU path.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
from torch import Tensor

from bitcache_amd import _C, _require_extension, default_top_k


def encode(src: Tensor) -> Tensor:
    """Sign bits + fp16 mean-|x| scale; [n, d] fp16 -> uint8 [n * 36]
    (bitcache/functional.py:17-35)."""
    _require_extension()
    assert src.is_cuda, "src must be on a ROCm device"
    assert src.is_contiguous(), "src must be contiguous"
    assert src.dtype == torch.float16, "src must be float16"
    assert src.dim() == 2, "src must be 2D [n_vecs, head_dim]"
    return _C.binary_encode(src)


def compute_residual(src: Tensor, binary_blob: Tensor) -> Tensor:
    """INT4 residual against the binary encoding; -> uint8 [n * 130]
    (bitcache/functional.py:38-56)."""
    _require_extension()
    assert src.is_cuda and binary_blob.is_cuda, "tensors must be on a ROCm device"
    assert src.is_contiguous() and binary_blob.is_contiguous(), "tensors must be contiguous"
    assert src.dtype == torch.float16, "src must be float16"
    return _C.residual_encode(src, binary_blob)


def encode_fused(src: Tensor, fp32_scale: bool = False) -> Tuple[Tensor, Tensor]:
    """encode() and compute_residual() in one pass (fp32_scale=True: the
    online-encode residual math)."""
    _require_extension()
    assert src.is_cuda and src.is_contiguous() and src.dtype == torch.float16
    return _C.encode_fused(src, fp32_scale)


def _check_q(Q: Tensor) -> None:
    assert Q.is_cuda, "Q must be on a ROCm device"
    assert Q.is_contiguous(), "Q must be contiguous"
    assert Q.dtype == torch.float16, "Q must be float16"


def binary_attention(Q: Tensor, K_bin: Tensor, V_bin: Tensor, batch: int, n_heads: int,
                     seq_len: int, head_dim: int, *, n_kv_heads: Optional[int] = None,
                     kv_stride: Optional[int] = None) -> Tensor:
    """XNOR-popcount scores, sign*scale values (bitcache/functional.py:59-88)."""
    _require_extension()
    _check_q(Q)
    if n_kv_heads is None and kv_stride is None:
        return _C.binary_attention(Q, K_bin, V_bin, batch, n_heads, seq_len, head_dim)
    return _C.attention(Q, K_bin, None, V_bin, None, batch, n_heads,
                        n_heads if n_kv_heads is None else n_kv_heads, seq_len,
                        seq_len if kv_stride is None else kv_stride, head_dim)


def compensated_attention(Q: Tensor, K_bin: Tensor, K_res: Tensor, V_bin: Tensor,
                          V_res: Tensor, batch: int, n_heads: int, seq_len: int, head_dim: int,
                          *, n_kv_heads: Optional[int] = None,
                          kv_stride: Optional[int] = None) -> Tensor:
    """Binary score + INT4 residual dot, binary + residual values
    (bitcache/functional.py:91-127)."""
    _require_extension()
    _check_q(Q)
    if n_kv_heads is None and kv_stride is None:
        return _C.compensated_attention(Q, K_bin, K_res, V_bin, V_res, batch, n_heads, seq_len,
                                        head_dim)
    return _C.attention(Q, K_bin, K_res, V_bin, V_res, batch, n_heads,
                        n_heads if n_kv_heads is None else n_kv_heads, seq_len,
                        seq_len if kv_stride is None else kv_stride, head_dim)


def adaptive_attention(Q: Tensor, K_bin: Tensor, K_res: Tensor, V_bin: Tensor, V_res: Tensor,
                       batch: int, n_heads: int, seq_len: int, head_dim: int, *,
                       n_kv_heads: Optional[int] = None, kv_stride: Optional[int] = None,
                       frac: float = 0.10, top_k: Optional[int] = None,
                       return_selected: bool = False):
    """Residual correction on the top-k keys per (batch, query head) by the
    exact binary key scale_k*(2*popcount-d), ties to the lowest index."""
    _require_extension()
    _check_q(Q)
    k = default_top_k(seq_len, frac) if top_k is None else top_k
    out, sel = _C.adaptive_attention(Q, K_bin, K_res, V_bin, V_res, batch, n_heads,
                                     n_heads if n_kv_heads is None else n_kv_heads, seq_len,
                                     seq_len if kv_stride is None else kv_stride, head_dim, k,
                                     return_selected)
    return (out, sel) if return_selected else out


def binary_scores(Q: Tensor, K_bin: Tensor, batch: int, n_heads: int, seq_len: int,
                  head_dim: int, *, n_kv_heads: Optional[int] = None,
                  kv_stride: Optional[int] = None) -> Tuple[Tensor, Tensor]:
    """Exact per-key binary scores (xnor_dot/sqrt(d), fp32) and popcounts (int32)."""
    _require_extension()
    _check_q(Q)
    return _C.binary_scores(Q, K_bin, batch, n_heads, n_heads if n_kv_heads is None else n_kv_heads,
                            seq_len, seq_len if kv_stride is None else kv_stride, head_dim)


def compute_head_entropy(Q: Tensor, K_bin: Tensor, batch: int, n_heads: int, seq_len: int,
                         head_dim: int, *, n_kv_heads: Optional[int] = None,
                         kv_stride: Optional[int] = None) -> Tensor:
    """Per-(b,h) entropy of the binary-score softmax (src/adaptive_precision.cu:13-130),
    float32 [batch, n_heads].  n_kv_heads / kv_stride: GQA and ring-stride caches."""
    _require_extension()
    _check_q(Q)
    if n_kv_heads is None and kv_stride is None:
        return _C.compute_head_entropy(Q, K_bin, batch, n_heads, seq_len, head_dim)
    return _C.head_entropy(Q, K_bin, batch, n_heads, n_heads if n_kv_heads is None else n_kv_heads,
                           seq_len, seq_len if kv_stride is None else kv_stride, head_dim)


def adaptive_select(entropy: Tensor, threshold: float) -> Tensor:
    """uint8 mode per head: 0 = binary (entropy >= threshold), 1 = compensated."""
    _require_extension()
    return _C.adaptive_select(entropy, threshold)


def head_mode_attention(Q: Tensor, K_bin: Tensor, K_res: Tensor, V_bin: Tensor, V_res: Tensor,
                        modes: Tensor, batch: int, n_heads: int, seq_len: int, head_dim: int, *,
                        n_kv_heads: Optional[int] = None, kv_stride: Optional[int] = None) -> Tensor:
    """Binary attention for the heads with modes[b, h] == 0, compensated attention for the
    others, in one launch (the per-head intent of src/adaptive_precision.cuh:6-49).
    modes: uint8 [batch, n_heads], as adaptive_select returns it."""
    _require_extension()
    _check_q(Q)
    return _C.head_mode_attention(Q, K_bin, K_res, V_bin, V_res, modes.contiguous(), batch,
                                  n_heads, n_heads if n_kv_heads is None else n_kv_heads, seq_len,
                                  seq_len if kv_stride is None else kv_stride, head_dim)


def entropy_dispatch_attention(Q: Tensor, K_bin: Tensor, K_res: Tensor, V_bin: Tensor,
                               V_res: Tensor, batch: int, n_heads: int, seq_len: int,
                               head_dim: int, threshold: float, *,
                               n_kv_heads: Optional[int] = None,
                               kv_stride: Optional[int] = None) -> Tuple[Tensor, Tensor]:
    """The reference's adaptive precision end to end: per-head entropy of the binary
    scores (src/adaptive_precision.cu:13-130), mode = binary where entropy >= threshold
    (:133-144), then head_mode_attention.  Returns (out, modes)."""
    kw = dict(n_kv_heads=n_kv_heads, kv_stride=kv_stride)
    ent = compute_head_entropy(Q, K_bin, batch, n_heads, seq_len, head_dim, **kw)
    modes = adaptive_select(ent, threshold).view(batch, n_heads)
    hkv = n_heads if n_kv_heads is None else n_kv_heads
    if kv_stride is None:
        # the stride compute_head_entropy read with: the blob's capacity per kv row
        # (a prefix view of a ring reads the ring's own stride)
        kv_stride = _capacity(K_bin, _C.sizeof_binary_vec()) // max(batch * hkv, 1)
    out = head_mode_attention(Q, K_bin, K_res, V_bin, V_res, modes, batch, n_heads, seq_len,
                              head_dim, n_kv_heads=hkv, kv_stride=kv_stride)
    return out, modes


def _capacity(blob: Tensor, per: int) -> int:
    """Vectors a blob was laid out for: its storage's when it is a prefix view
    of a larger allocation, else its own (the operators' rule)."""
    from bitcache_amd.layout import blob_bytes
    return blob_bytes(blob) // per


def reference_attention(Q: Tensor, K: Tensor, V: Tensor, batch: int, n_heads: int, seq_len: int,
                        head_dim: int, *, n_kv_heads: Optional[int] = None) -> Tensor:
    """Exact fp16 attention, fp32 accumulation (src/reference_attention.cu)."""
    _require_extension()
    _check_q(Q)
    return _C.reference_attention(Q, K, V, batch, n_heads,
                                  n_heads if n_kv_heads is None else n_kv_heads, seq_len, head_dim)


def sizeof_binary_vec() -> int:
    _require_extension()
    return _C.sizeof_binary_vec()


def sizeof_residual_vec() -> int:
    _require_extension()
    return _C.sizeof_residual_vec()
