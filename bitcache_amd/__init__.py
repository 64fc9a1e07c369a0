"""bitcache_amd: binary KV-cache with XNOR-popcount scoring and INT4 residual
correction, as hand-written HIP kernels for AMD Instinct MI355X (gfx950).

Drop-in for the reference package ``bitcache`` (anishesg/bitcache):
``BitCache`` (ring buffer, bitcache/__init__.py:29-207), ``functional``
(bitcache/functional.py) and the operator module ``_C``
(src/torch_binding.cpp:168-177).  There is no CPU fallback: every entry point
needs the in-tree HIP build (``python -m bitcache_amd.build``) and ROCm
tensors, and raises if either is missing.
"""
from __future__ import annotations

from fractions import Fraction
from typing import Optional

import torch
from torch import Tensor

try:
    from bitcache_amd import _C  # noqa: F401  (loads libbitcache_hip.so)
    _HAS_EXTENSION = True
    _IMPORT_ERROR: Optional[BaseException] = None
except ImportError as e:  # pragma: no cover - depends on the build
    _HAS_EXTENSION = False
    _C = None  # type: ignore[assignment]
    _IMPORT_ERROR = e


def _require_extension() -> None:
    """Raise if the HIP extension is not built (bitcache/__init__.py:22-26)."""
    if not _HAS_EXTENSION:
        raise RuntimeError(
            "bitcache_amd HIP extension not found (" + str(_IMPORT_ERROR) + "). "
            "Build it with: python -m bitcache_amd.build"
        )


def default_top_k(seq_len: int, frac: float = 0.10) -> int:
    """ceil(frac * seq_len), computed exactly on the decimal value of frac."""
    f = Fraction(str(frac))
    return min(seq_len, -((-f.numerator * seq_len) // f.denominator))


class BitCache:
    """Binary KV-cache for one transformer layer with ring-buffer semantics.

    Same constructor, methods and properties as the reference
    (bitcache/__init__.py:29-207), plus GQA (``n_kv_heads``), a bulk
    ``prefill`` and ``attend_adaptive``.  Differences from the reference, all
    fixes: attention reads the ring with stride ``max_seq`` (the reference
    read with stride ``seq_len``), binary-only caches never write residuals
    (the reference aliased them into the binary buffer), one launch appends K
    and V, and ``compression_ratio`` counts every buffer.

    Args:
        batch, n_heads, head_dim, max_seq, device, compensated: as the reference.
        n_kv_heads: KV heads (GQA); defaults to n_heads.  append() takes K/V of
            shape [batch, n_kv_heads, head_dim]; attend() takes Q of shape
            [batch, n_heads, head_dim].
    """

    def __init__(self, batch: int, n_heads: int, head_dim: int, max_seq: int,
                 device: str = "cuda", compensated: bool = True,
                 n_kv_heads: Optional[int] = None) -> None:
        _require_extension()
        assert head_dim % 32 == 0, "head_dim must be a multiple of 32"
        assert head_dim <= 256, "head_dim must be <= 256"
        assert max_seq > 0, "max_seq must be > 0"
        self.batch = batch
        self.n_heads = n_heads
        self.n_kv_heads = n_heads if n_kv_heads is None else n_kv_heads
        assert self.n_kv_heads > 0 and n_heads % self.n_kv_heads == 0, \
            "n_heads must be a multiple of n_kv_heads"
        self.head_dim = head_dim
        self.max_seq = max_seq
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise RuntimeError("BitCache needs a ROCm device (got %s)" % self.device)
        self.compensated = compensated
        self._bv_size = _C.sizeof_binary_vec()
        self._rv_size = _C.sizeof_residual_vec()
        n_slots = batch * self.n_kv_heads * max_seq
        u8 = dict(dtype=torch.uint8, device=self.device)
        self._k_bin = torch.zeros(n_slots * self._bv_size, **u8)
        self._v_bin = torch.zeros(n_slots * self._bv_size, **u8)
        if compensated:
            self._k_res = torch.zeros(n_slots * self._rv_size, **u8)
            self._v_res = torch.zeros(n_slots * self._rv_size, **u8)
        else:
            self._k_res = None
            self._v_res = None
        self._write_pos = 0
        self._filled = 0

    # ------------------------------------------------------------------ core API
    def append(self, K: Tensor, V: Tensor) -> None:
        """Encode one token per (b, kv head) into the ring (bitcache/__init__.py:95-113)."""
        self._validate_kv(K, V)
        _C.online_encode_kv(K, V, self._k_bin, self._k_res, self._v_bin, self._v_res,
                            self.batch, self.n_kv_heads, self.head_dim, self._write_pos,
                            self.max_seq)
        self._write_pos = (self._write_pos + 1) % self.max_seq
        self._filled = min(self._filled + 1, self.max_seq)

    def prefill(self, K: Tensor, V: Tensor, layout: str = "bhsd") -> None:
        """Append S tokens at once: K/V [batch, n_kv_heads, S, head_dim] fp16
        (layout "bhsd") or [batch, S, n_kv_heads, head_dim] (layout "bshd").

        Produces the same bytes as S calls to append() (online-encode math,
        src/online_encode.cu:74,88).  The tokens must fit without wrapping."""
        B, H, d = self.batch, self.n_kv_heads, self.head_dim
        assert layout in ("bhsd", "bshd"), "layout must be 'bhsd' or 'bshd'"
        S = K.shape[2] if layout == "bhsd" else K.shape[1]
        shape = (B, H, S, d) if layout == "bhsd" else (B, S, H, d)
        assert K.shape == shape and V.shape == shape, f"K/V must be {layout} {shape}"
        assert K.dtype == torch.float16 and V.dtype == torch.float16
        assert K.is_contiguous() and V.is_contiguous()
        assert self._write_pos + S <= self.max_seq, "prefill would wrap the ring buffer"
        for src, bin_, res in ((K, self._k_bin, self._k_res), (V, self._v_bin, self._v_res)):
            if layout == "bhsd":
                _C.encode_into_cache(src, bin_, res, B * H, S, d, self._write_pos, self.max_seq, True)
            else:
                _C.encode_into_cache_bshd(src, bin_, res, B, S, H, d, self._write_pos,
                                          self.max_seq, True)
        self._write_pos = (self._write_pos + S) % self.max_seq
        self._filled = min(self._filled + S, self.max_seq)

    def attend(self, Q: Tensor) -> Tensor:
        """Attention over the cached tokens (bitcache/__init__.py:115-148)."""
        assert self._filled > 0, "cache is empty, call append() first"
        return _C.attention(Q, self._k_bin, self._k_res, self._v_bin, self._v_res,
                            self.batch, self.n_heads, self.n_kv_heads, self._filled,
                            self.max_seq, self.head_dim)

    def append_attend(self, K: Tensor, V: Tensor, Q: Tensor) -> Tensor:
        """One decode step: append(K, V) followed by attend(Q), with the same
        cache bytes and output, in one attention launch where the kernels allow
        it (the append of bitcache/__init__.py:95-113 and the attention of
        :115-148 fused)."""
        self._validate_kv(K, V)
        # tokens appended so far, as the kernels' ring rule reads it: slot =
        # current % max_seq, attended positions = min(current + 1, max_seq)
        current = self._write_pos if self._filled < self.max_seq else self._write_pos + self.max_seq
        out = _C.append_attention(Q, K, V, self._k_bin, self._k_res, self._v_bin, self._v_res,
                                  self.batch, self.n_heads, self.n_kv_heads, self.head_dim,
                                  current, self.max_seq)
        self._write_pos = (self._write_pos + 1) % self.max_seq
        self._filled = min(self._filled + 1, self.max_seq)
        return out

    def attend_adaptive(self, Q: Tensor, frac: float = 0.10, top_k: Optional[int] = None,
                        return_selected: bool = False):
        """Residual correction only on the top-k keys by binary score per
        (batch, query head); needs compensated=True."""
        assert self.compensated, "adaptive attention needs the residual buffers"
        assert self._filled > 0, "cache is empty, call append() first"
        k = default_top_k(self._filled, frac) if top_k is None else top_k
        out, sel = _C.adaptive_attention(Q, self._k_bin, self._k_res, self._v_bin, self._v_res,
                                         self.batch, self.n_heads, self.n_kv_heads,
                                         self._filled, self.max_seq, self.head_dim, k,
                                         return_selected)
        return (out, sel) if return_selected else out

    def attend_head_mode(self, Q: Tensor, threshold: Optional[float] = None,
                         modes: Optional[Tensor] = None, return_modes: bool = False):
        """Binary or compensated attention chosen per (batch, query head) in one
        launch: from ``modes`` (uint8 [batch, n_heads], 0 = binary) or, given a
        ``threshold``, from the entropy of each head's binary scores over the
        cached tokens (binary where entropy >= threshold): the reference's
        adaptive precision (src/adaptive_precision.cuh:6-49).  Needs
        compensated=True."""
        assert self.compensated, "per-head modes need the residual buffers"
        assert self._filled > 0, "cache is empty, call append() first"
        assert (threshold is None) != (modes is None), "give exactly one of threshold and modes"
        if modes is None:
            ent = _C.head_entropy(Q, self._k_bin, self.batch, self.n_heads, self.n_kv_heads,
                                  self._filled, self.max_seq, self.head_dim)
            modes = _C.adaptive_select(ent, threshold).view(self.batch, self.n_heads)
        out = _C.head_mode_attention(Q, self._k_bin, self._k_res, self._v_bin, self._v_res,
                                     modes.contiguous(), self.batch, self.n_heads,
                                     self.n_kv_heads, self._filled, self.max_seq, self.head_dim)
        return (out, modes) if return_modes else out

    def reset(self) -> None:
        """Clear the cache (bitcache/__init__.py:150-158)."""
        self._k_bin.zero_()
        self._v_bin.zero_()
        if self.compensated:
            self._k_res.zero_()
            self._v_res.zero_()
        self._write_pos = 0
        self._filled = 0

    # ------------------------------------------------------------------ properties
    @property
    def seq_len(self) -> int:
        return self._filled

    @property
    def memory_bytes(self) -> int:
        """Bytes allocated for the cache buffers (bitcache/__init__.py:169-175)."""
        total = self._k_bin.numel() + self._v_bin.numel()
        if self.compensated:
            total += self._k_res.numel() + self._v_res.numel()
        return total

    @property
    def payload_bytes(self) -> int:
        """Bytes that carry information: d/8+2 per vector (+ d/2+2 with residuals)."""
        per = self.head_dim // 8 + 2 + ((self.head_dim // 2 + 2) if self.compensated else 0)
        return 2 * self.batch * self.n_kv_heads * self.max_seq * per

    @property
    def compression_ratio(self) -> float:
        """fp16 KV bytes / allocated cache bytes, counting residual buffers too
        (the reference counted the binary buffers only, bitcache/__init__.py:177-185)."""
        fp16 = 2 * self.batch * self.n_kv_heads * self.max_seq * self.head_dim * 2
        return fp16 / self.memory_bytes

    # ------------------------------------------------------------------ helpers
    def _validate_kv(self, K: Tensor, V: Tensor) -> None:
        expected = (self.batch, self.n_kv_heads, self.head_dim)
        assert K.shape == torch.Size(expected), f"K shape {tuple(K.shape)} != {expected}"
        assert V.shape == torch.Size(expected), f"V shape {tuple(V.shape)} != {expected}"
        assert K.dtype == torch.float16, "K must be float16"
        assert V.dtype == torch.float16, "V must be float16"
        assert K.is_cuda and V.is_cuda, "K and V must be on a ROCm device"
        assert K.is_contiguous() and V.is_contiguous(), "K and V must be contiguous"

    def __repr__(self) -> str:
        mode = "compensated" if self.compensated else "binary"
        return (f"BitCache(batch={self.batch}, n_heads={self.n_heads}, "
                f"n_kv_heads={self.n_kv_heads}, head_dim={self.head_dim}, "
                f"max_seq={self.max_seq}, filled={self._filled}, mode={mode}, "
                f"mem={self.memory_bytes / 1024:.1f}KB)")


from bitcache_amd import functional  # noqa: E402,F401

__all__ = ["BitCache", "functional", "default_top_k"]
