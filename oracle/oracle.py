"""CPU oracle for the bitcache compressed-KV decode-attention path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker (or as the timed CPU baseline).  The product path (``bitcache_amd``)
never imports it and has no CPU fallback.

This module restates the reference algorithm (anishesg/bitcache, ``src/*.cu``)
in IEEE-754 float32 numpy / torch-CPU arithmetic.  Everything is expressed on
*semantic* arrays (sign words, fp16 scales, INT4 codes), never on device blob
layouts.  Each function cites the reference lines it follows.

Bit-exact parts (encode, popcounts, binary scores, top-k sets) reproduce the
reference's fp32 operation order exactly.  Softmax/attention parts follow the
reference formulas; their summation order is vectorised (the reference's own
order is restated by the slow ``*_exact_order`` helpers used on small inputs).

Pinning (what checks each function; see tests/test_oracle.py):
  binary_encode      brute-force bits, KATs, closed-form scale for constant |x|,
                     agreement with the independent scalar C oracle (oracle/bitcache_oracle.c)
  residual_encode    KATs at half-steps / absmax 0 / clamp, reconstruction bound,
                     agreement with the C oracle
  online_encode      same as residual_encode with the fp32-scale semantics; C oracle
  query_prep         closed form (sequential sum) + C oracle
  popcounts/scores   2*pc-d == sign(q).sign(k) (exact integer matmul); C oracle
  compensated scores matmul closed form over decoded K (float64)
  attention          S=1, equal-score mean, float64 softmax closed form, exact-order loop
  head_entropy       float64 -sum p log p closed form; C oracle
  topk_select        brute-force stable sort
  reference_attention  float64 softmax closed form
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from fractions import Fraction
from typing import Optional

import numpy as np

F32 = np.float32
MAX_HEAD_DIM = 256          # src/binary_encode.cuh:10
SIZEOF_BINARY_VEC = 36      # sizeof(BinaryVec): u32 words[8] + __half scale, padded (src/binary_encode.cuh:13-18)
SIZEOF_RESIDUAL_VEC = 130   # sizeof(ResidualVec): u8 nibbles[128] + __half scale (src/residual.cuh:11-16)


# ----------------------------------------------------------------------------
# semantic containers
# ----------------------------------------------------------------------------
@dataclass
class BinaryEnc:
    words: np.ndarray       # uint32 [n, d/32]; bit i of the vector is bit i%32 of words[i//32]
    scale: np.ndarray       # float16 [n]; mean |x| rounded to fp16
    mean32: np.ndarray      # float32 [n]; the same mean before fp16 rounding


@dataclass
class ResidualEnc:
    codes: np.ndarray       # int8 [n, d] in [-7, 7]
    scale: np.ndarray       # float16 [n]; absmax of the residual rounded to fp16

    @property
    def nibbles(self) -> np.ndarray:
        return pack_nibbles(self.codes)


def _check_x(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x)
    if x.dtype != np.float16:
        raise TypeError("oracle encode expects float16 input")
    if x.ndim != 2:
        raise ValueError("expected [n, head_dim]")
    d = x.shape[1]
    if d % 32 != 0 or d > MAX_HEAD_DIM or d == 0:
        raise ValueError("head_dim must be a positive multiple of 32 and <= 256")
    return x


# ----------------------------------------------------------------------------
# bit packing helpers (src/binary_encode.cu:36-38: bit i -> word i/32, bit i%32)
# ----------------------------------------------------------------------------
def pack_bits(bits: np.ndarray) -> np.ndarray:
    """bool [..., d] -> uint32 [..., d/32], little-endian bit order."""
    b = np.packbits(bits.astype(np.uint8), axis=-1, bitorder="little")
    b = np.ascontiguousarray(b)
    return b.view("<u4").astype(np.uint32)


def unpack_bits(words: np.ndarray, d: int) -> np.ndarray:
    w = np.ascontiguousarray(words.astype("<u4"))
    b = w.view(np.uint8)
    return np.unpackbits(b, axis=-1, bitorder="little")[..., :d].astype(bool)


def pack_nibbles(codes: np.ndarray) -> np.ndarray:
    """int8 codes [..., d] -> uint8 [..., d/2]; element 2j in the low nibble
    (src/residual.cu:75-76: (q0 & 0xF) | ((q1 & 0xF) << 4))."""
    c = codes.astype(np.int16)
    lo = c[..., 0::2] & 0xF
    hi = c[..., 1::2] & 0xF
    return (lo | (hi << 4)).astype(np.uint8)


def unpack_nibbles(nib: np.ndarray) -> np.ndarray:
    """uint8 [..., d/2] -> int8 [..., d]; 4-bit sign extension (src/residual.cuh:42-52)."""
    n = nib.astype(np.int16)
    lo = n & 0xF
    hi = (n >> 4) & 0xF
    lo = np.where(lo >= 8, lo - 16, lo)
    hi = np.where(hi >= 8, hi - 16, hi)
    out = np.empty(nib.shape[:-1] + (nib.shape[-1] * 2,), dtype=np.int8)
    out[..., 0::2] = lo
    out[..., 1::2] = hi
    return out


# ----------------------------------------------------------------------------
# encode
# ----------------------------------------------------------------------------
def _tree_abs_sum(x32: np.ndarray) -> np.ndarray:
    """Sum of |x| in the reference's 128-thread order.

    src/binary_encode.cu:31-53: thread t (blockDim 128) accumulates
    0.0f + |x_t| + |x_{t+128}| + ... sequentially, then a shared-memory tree
    p[t] += p[t+s] for s = 64, 32, ..., 1.  The same order is used by
    src/online_encode.cu:56-72 and src/adaptive_precision.cu:46-59.
    """
    n, d = x32.shape
    p = np.zeros((n, 128), dtype=F32)
    a = np.abs(x32)
    for k in range(0, d, 128):
        seg = a[:, k:k + 128]
        if seg.shape[1] < 128:
            seg = np.concatenate([seg, np.zeros((n, 128 - seg.shape[1]), F32)], axis=1)
        p = (p + seg).astype(F32)
    s = 64
    while s > 0:
        p[:, :s] = (p[:, :s] + p[:, s:2 * s]).astype(F32)
        s //= 2
    return p[:, 0]


def binary_encode(x: np.ndarray) -> BinaryEnc:
    """src/binary_encode.cu:8-60.

    bits: x >= 0.0f (so +-0 -> 1, NaN -> 0)  (:36)
    scale: fp16(tree_sum|x| / (float)d)       (:53-54), round-to-nearest-even.
    """
    x = _check_x(x)
    d = x.shape[1]
    x32 = x.astype(F32)
    with np.errstate(invalid="ignore"):
        bits = x32 >= F32(0.0)
    total = _tree_abs_sum(x32)
    mean32 = (total / F32(d)).astype(F32)
    with np.errstate(over="ignore", invalid="ignore"):
        scale = mean32.astype(np.float16)
    return BinaryEnc(words=pack_bits(bits), scale=scale, mean32=mean32)


def _quantize_residual(x32: np.ndarray, bits: np.ndarray, s: np.ndarray) -> ResidualEnc:
    """Shared body of src/residual.cu:28-77 and src/online_encode.cu:84-119.

    r_i = x_i - (bit_i ? s : -s)          (src/residual.cu:34-37)
    absmax = fmaxf over |r_i| from 0.0f   (src/residual.cu:31,39,44-53) -- NaN ignored
    inv = absmax > 0 ? 7.0f/absmax : 0    (src/residual.cu:54)
    q = clamp(rint_half_even(r * inv), -7, 7), NaN -> 0   (src/residual.cu:67-72)
    scale = fp16(absmax)                  (src/residual.cu:57)
    """
    s = s.astype(F32)[:, None]
    recon = np.where(bits, s, -s).astype(F32)
    with np.errstate(invalid="ignore", over="ignore"):
        r = (x32 - recon).astype(F32)
        absmax = np.fmax.reduce(np.abs(r), axis=1, initial=F32(0.0)).astype(F32)
        pos = absmax > F32(0.0)
        safe = np.where(pos, absmax, F32(1.0))
        inv = np.where(pos, (F32(7.0) / safe).astype(F32), F32(0.0)).astype(F32)
        v = (r * inv[:, None]).astype(F32)
        q = np.rint(v)
        q = np.where(np.isnan(q), 0.0, q)
        q = np.clip(q, -7.0, 7.0).astype(np.int8)
        scale = absmax.astype(np.float16)
    return ResidualEnc(codes=q, scale=scale)


def residual_encode(x: np.ndarray, binary: BinaryEnc) -> ResidualEnc:
    """Two-step residual: src/residual.cu:9-78.  Uses the *fp16-rounded*
    binary scale read back from the BinaryVec (:28) and the stored bits (:34)."""
    x = _check_x(x)
    d = x.shape[1]
    bits = unpack_bits(binary.words, d)
    s = binary.scale.astype(F32)
    return _quantize_residual(x.astype(F32), bits, s)


def online_encode(x: np.ndarray):
    """Fused single-token encode: src/online_encode.cu:17-120.

    Same bits and fp16 scale as binary_encode, but the residual is computed
    against the *fp32* mean before rounding (:74, :88)."""
    b = binary_encode(x)
    d = x.shape[1]
    bits = unpack_bits(b.words, d)
    r = _quantize_residual(x.astype(F32), bits, b.mean32)
    return b, r


def encode_fused(x: np.ndarray, fp32_scale: bool = False):
    """binary_encode followed by residual_encode (fp32_scale=False), or the
    online-encode math (fp32_scale=True)."""
    if fp32_scale:
        return online_encode(x)
    b = binary_encode(x)
    return b, residual_encode(x, b)


def dequant_binary(b: BinaryEnc, d: int) -> np.ndarray:
    """sign(x) * scale as float32 [n, d] (src/binary_attention.cu:67-73)."""
    bits = unpack_bits(b.words, d)
    s = b.scale.astype(F32)[:, None]
    return np.where(bits, s, -s).astype(F32)


def dequant_residual(r: ResidualEnc) -> np.ndarray:
    """(n / 7.0f) * scale as float32 (src/residual.cuh:37-39)."""
    return ((r.codes.astype(F32) / F32(7.0)) * r.scale.astype(F32)[:, None]).astype(F32)


# ----------------------------------------------------------------------------
# query preparation
# ----------------------------------------------------------------------------
def query_prep(q: np.ndarray):
    """src/compensated_attention.cu:56-69 / src/binary_attention.cu:24-39.

    q32 = float(Q); sign words via pack_sign_bits (src/xnor_dot.cuh:36-52, >= 0.0f);
    scale_q = (sequential fp32 sum_i |q_i|) / d  -- not rounded to fp16.
    """
    q = np.asarray(q)
    d = q.shape[-1]
    q32 = q.reshape(-1, d).astype(F32)
    with np.errstate(invalid="ignore"):
        bits = q32 >= F32(0.0)
    acc = np.zeros(q32.shape[0], dtype=F32)
    for i in range(d):
        acc = (acc + np.abs(q32[:, i])).astype(F32)
    scale_q = (acc / F32(d)).astype(F32)
    return pack_bits(bits), scale_q, q32


def query_prep_tree(q: np.ndarray):
    """src/adaptive_precision.cu:31-62: tree-order scale_q (same order as encode)."""
    q = np.asarray(q)
    d = q.shape[-1]
    q32 = q.reshape(-1, d).astype(F32)
    with np.errstate(invalid="ignore"):
        bits = q32 >= F32(0.0)
    total = _tree_abs_sum(q32)
    return pack_bits(bits), (total / F32(d)).astype(F32), q32


def inv_sqrt(d: int) -> np.float32:
    """1.0f / sqrtf((float)d)  (src/compensated_attention.cu:69), IEEE."""
    return F32(F32(1.0) / np.sqrt(F32(d)))


# ----------------------------------------------------------------------------
# scores
# ----------------------------------------------------------------------------
def popcounts(qwords: np.ndarray, kwords: np.ndarray) -> np.ndarray:
    """sum_w popc(~(q_w ^ k_w))  (src/xnor_dot.cuh:20-27).
    qwords [W], kwords [S, W] -> int32 [S]."""
    x = ~(kwords.astype(np.uint32) ^ qwords.astype(np.uint32)[None, :])
    return np.bitwise_count(x).astype(np.int32).sum(axis=-1).astype(np.int32)


def xnor_dot(scale_q: np.float32, pc: np.ndarray, kscale16: np.ndarray, d: int) -> np.ndarray:
    """(scale_q * scale_k) * (float)(2*pc - d)  (src/xnor_dot.cuh:28-30)."""
    sk = kscale16.astype(F32)
    return ((F32(scale_q) * sk).astype(F32) * (2 * pc - d).astype(F32)).astype(F32)


def residual_dot(q32: np.ndarray, r: ResidualEnc) -> np.ndarray:
    """src/compensated_attention.cu:23-37, sequential over element pairs:
    dot = dot + (q[2j]*r0 + q[2j+1]*r1) with r = (n/7.0f)*scale.  q32 [d] -> [S]."""
    deq = dequant_residual(r)               # [S, d]
    S, d = deq.shape
    dot = np.zeros(S, dtype=F32)
    for j in range(d // 2):
        t = (q32[2 * j] * deq[:, 2 * j]).astype(F32) + (q32[2 * j + 1] * deq[:, 2 * j + 1]).astype(F32)
        dot = (dot + t.astype(F32)).astype(F32)
    return dot


def binary_scores(Q: np.ndarray, K: BinaryEnc, batch: int, n_heads: int, seq_len: int,
                  n_kv_heads: Optional[int] = None) -> np.ndarray:
    """Per-key binary attention score xnor_dot * inv_sqrt_d, float32 [B, Hq, S]
    (src/binary_attention.cu:56, :63).  K holds B*Hkv*S vectors, head-major."""
    hkv = n_heads if n_kv_heads is None else n_kv_heads
    d = Q.shape[-1]
    qw, sq, _ = query_prep(Q.reshape(batch * n_heads, d))
    kw = K.words.reshape(batch, hkv, seq_len, -1)
    ks = K.scale.reshape(batch, hkv, seq_len)
    g = n_heads // hkv
    out = np.empty((batch, n_heads, seq_len), dtype=F32)
    isd = inv_sqrt(d)
    for b in range(batch):
        for h in range(n_heads):
            i = b * n_heads + h
            pc = popcounts(qw[i], kw[b, h // g])
            out[b, h] = (xnor_dot(sq[i], pc, ks[b, h // g], d) * isd).astype(F32)
    return out


def binary_popcounts(Q: np.ndarray, K: BinaryEnc, batch: int, n_heads: int, seq_len: int,
                     n_kv_heads: Optional[int] = None) -> np.ndarray:
    hkv = n_heads if n_kv_heads is None else n_kv_heads
    d = Q.shape[-1]
    qw, _, _ = query_prep(Q.reshape(batch * n_heads, d))
    kw = K.words.reshape(batch, hkv, seq_len, -1)
    g = n_heads // hkv
    out = np.empty((batch, n_heads, seq_len), dtype=np.int32)
    for b in range(batch):
        for h in range(n_heads):
            out[b, h] = popcounts(qw[b * n_heads + h], kw[b, h // g])
    return out


# ----------------------------------------------------------------------------
# attention
# ----------------------------------------------------------------------------
def _softmax_out(scores: np.ndarray, vrec: np.ndarray):
    """Two-pass softmax + weighted sum (src/compensated_attention.cu:76-108):
    m = max(-1e38f, scores); w = exp(s - m); out = fp16(acc * (l>0 ? 1/l : 0)).
    scores [S], vrec [S, d] (the per-key V reconstruction)."""
    d = vrec.shape[1]
    if scores.size == 0:
        return np.zeros(d, np.float16), np.zeros(d, F32)
    m = max(F32(-1e38), F32(np.max(scores)))
    w = np.exp((scores - m).astype(F32)).astype(F32)
    l = F32(np.sum(w, dtype=F32))
    acc = (w[None, :] @ vrec).astype(F32)[0]
    inv = F32(F32(1.0) / l) if l > 0 else F32(0.0)
    o32 = (acc * inv).astype(F32)
    with np.errstate(over="ignore", invalid="ignore"):
        return o32.astype(np.float16), o32


def _heads(batch, n_heads, n_kv_heads):
    hkv = n_heads if n_kv_heads is None else n_kv_heads
    if n_heads % hkv != 0:
        raise ValueError("n_heads must be a multiple of n_kv_heads")
    return hkv, n_heads // hkv


def compensated_attention(Q, Kb: BinaryEnc, Kr: ResidualEnc, Vb: BinaryEnc, Vr: ResidualEnc,
                          batch, n_heads, seq_len, n_kv_heads=None, return_f32=False):
    """src/compensated_attention.cu:42-109 with GQA (q head h -> kv head h // (Hq/Hkv)).

    score_s = (xnor_dot + residual_dot) * inv_sqrt_d   (:79-80)
    vrec_s  = (bit ? sv : -sv) + (n/7)*rs              (:93-101)
    """
    hkv, g = _heads(batch, n_heads, n_kv_heads)
    d = Q.shape[-1]
    qw, sq, q32 = query_prep(Q.reshape(batch * n_heads, d))
    isd = inv_sqrt(d)
    kb_rec = None
    out = np.empty((batch, n_heads, d), np.float16)
    o32 = np.empty((batch, n_heads, d), F32)
    kw = Kb.words.reshape(batch, hkv, seq_len, -1)
    ks = Kb.scale.reshape(batch, hkv, seq_len)
    kc = Kr.codes.reshape(batch, hkv, seq_len, d)
    krs = Kr.scale.reshape(batch, hkv, seq_len)
    vrec_all = (dequant_binary(Vb, d) + dequant_residual(Vr)).astype(F32).reshape(batch, hkv, seq_len, d)
    for b in range(batch):
        for kh in range(hkv):
            kres = ResidualEnc(codes=kc[b, kh], scale=krs[b, kh])
            deq = dequant_residual(kres)
            for h in range(kh * g, (kh + 1) * g):
                i = b * n_heads + h
                pc = popcounts(qw[i], kw[b, kh])
                xd = xnor_dot(sq[i], pc, ks[b, kh], d)
                rd = (deq @ q32[i]).astype(F32)
                sc = ((xd + rd).astype(F32) * isd).astype(F32)
                out[b, h], o32[b, h] = _softmax_out(sc, vrec_all[b, kh])
    return (out, o32) if return_f32 else out


def binary_attention(Q, Kb: BinaryEnc, Vb: BinaryEnc, batch, n_heads, seq_len,
                     n_kv_heads=None, return_f32=False):
    """src/binary_attention.cu:8-82: scores from xnor_dot only, V = sign*scale."""
    hkv, g = _heads(batch, n_heads, n_kv_heads)
    d = Q.shape[-1]
    sc_all = binary_scores(Q, Kb, batch, n_heads, seq_len, n_kv_heads)
    vrec = dequant_binary(Vb, d).reshape(batch, hkv, seq_len, d)
    out = np.empty((batch, n_heads, d), np.float16)
    o32 = np.empty((batch, n_heads, d), F32)
    for b in range(batch):
        for h in range(n_heads):
            out[b, h], o32[b, h] = _softmax_out(sc_all[b, h], vrec[b, h // g])
    return (out, o32) if return_f32 else out


def compensated_attention_exact_order(Q, Kb, Kr, Vb, Vr, seq_len):
    """Literal restatement of compensated_attention_kernel for ONE (b,h) with the
    reference's sequential loops (src/compensated_attention.cu:76-108).  Slow:
    used on small inputs to bound the effect of the vectorised summation order."""
    d = Q.shape[-1]
    qw, sq, q32 = query_prep(Q.reshape(1, d))
    qw, sq, q32 = qw[0], sq[0], q32[0]
    isd = inv_sqrt(d)
    bits_v = unpack_bits(Vb.words, d)
    scores = np.empty(seq_len, F32)
    for s in range(seq_len):
        pc = popcounts(qw, Kb.words[s:s + 1])[0]
        xd = xnor_dot(sq, np.array([pc]), Kb.scale[s:s + 1], d)[0]
        rd = residual_dot(q32, ResidualEnc(Kr.codes[s:s + 1], Kr.scale[s:s + 1]))[0]
        scores[s] = F32(F32(xd + rd) * isd)
    m = F32(-1e38)
    for s in range(seq_len):
        if scores[s] > m:
            m = scores[s]
    acc = np.zeros(d, F32)
    l = F32(0.0)
    for s in range(seq_len):
        w = F32(np.exp(F32(scores[s] - m)))
        l = F32(l + w)
        sv = F32(Vb.scale[s])
        acc = (acc + (w * np.where(bits_v[s], sv, -sv).astype(F32)).astype(F32)).astype(F32)
        rv = dequant_residual(ResidualEnc(Vr.codes[s:s + 1], Vr.scale[s:s + 1]))[0]
        acc = (acc + (w * rv).astype(F32)).astype(F32)
    inv = F32(F32(1.0) / l) if l > 0 else F32(0.0)
    return (acc * inv).astype(F32)


def head_entropy(Q, Kb: BinaryEnc, batch, n_heads, seq_len, n_kv_heads=None) -> np.ndarray:
    """src/adaptive_precision.cu:13-130.

    score = (scale_q * scale_k) * (2pc - d)  -- NO 1/sqrt(d) (:74-75)
    scale_q in tree order (:46-59)
    H = (logf(Z) + M) - W / fmaxf(Z, 1e-12)   (:126-127)
    """
    hkv, g = _heads(batch, n_heads, n_kv_heads)
    d = Q.shape[-1]
    qw, sq, _ = query_prep_tree(Q.reshape(batch * n_heads, d))
    kw = Kb.words.reshape(batch, hkv, seq_len, -1)
    ks = Kb.scale.reshape(batch, hkv, seq_len)
    out = np.empty((batch, n_heads), F32)
    for b in range(batch):
        for h in range(n_heads):
            i = b * n_heads + h
            pc = popcounts(qw[i], kw[b, h // g])
            s = xnor_dot(sq[i], pc, ks[b, h // g], d)
            M = F32(max(F32(-1e30), np.max(s))) if seq_len > 0 else F32(-1e30)
            e = np.exp((s - M).astype(F32)).astype(F32)
            Z = F32(np.sum(e, dtype=F32))
            W = F32(np.sum((e * s).astype(F32), dtype=F32))
            with np.errstate(divide="ignore"):
                out[b, h] = F32(F32(np.log(Z) + M) - F32(W / max(Z, F32(1e-12))))
    return out


def reference_attention(Q, K, V, batch, n_heads, seq_len, n_kv_heads=None, return_f32=False):
    """src/reference_attention.cu:6-69: exact attention with fp32 accumulation,
    1/sqrt(d) scaling, fp16 output.  Q [B,Hq,d], K/V [B,Hkv,S,d] fp16."""
    import torch
    hkv, g = _heads(batch, n_heads, n_kv_heads)
    d = Q.shape[-1]
    q = torch.from_numpy(np.asarray(Q, np.float16).astype(F32)).reshape(batch, n_heads, 1, d)
    k = torch.from_numpy(np.asarray(K, np.float16).astype(F32)).reshape(batch, hkv, seq_len, d)
    v = torch.from_numpy(np.asarray(V, np.float16).astype(F32)).reshape(batch, hkv, seq_len, d)
    if g > 1:
        k = k.repeat_interleave(g, dim=1)
        v = v.repeat_interleave(g, dim=1)
    s = (q @ k.transpose(-1, -2)) * float(inv_sqrt(d))
    w = torch.softmax(s, dim=-1)
    o = (w @ v).reshape(batch, n_heads, d)
    o32 = o.numpy().astype(F32)
    with np.errstate(over="ignore"):
        o16 = o32.astype(np.float16)
    return (o16, o32) if return_f32 else o16


# ----------------------------------------------------------------------------
# adaptive top-k residual selection (build-defined semantics; see topk_select)
# ----------------------------------------------------------------------------
def default_top_k(seq_len: int, frac: float = 0.10) -> int:
    """k = ceil(frac * S) computed exactly on the decimal value of frac."""
    f = Fraction(str(frac))
    return min(seq_len, -((-f.numerator * seq_len) // f.denominator))


def topk_key(kscale16: np.ndarray, pc: np.ndarray, d: int) -> np.ndarray:
    """Ranking key: float(scale_k) * (2pc - d), exact in fp32 (<= 19 significant
    bits), order-equivalent to the reference score (src/xnor_dot.cuh:30) since
    scale_q > 0.  -0 is canonicalised to +0; NaN ranks below every other key."""
    key = (kscale16.astype(F32) * (2 * pc - d).astype(F32)).astype(F32)
    key = (key + F32(0.0)).astype(F32)
    key = np.where(np.isnan(key), F32(-np.inf), key)
    return key


def topk_select(key: np.ndarray, k: int) -> np.ndarray:
    """Indices (ascending) of the k largest keys, ties broken by lowest index.
    Brute-force stable sort."""
    S = key.shape[0]
    k = min(k, S)
    order = np.lexsort((np.arange(S), -key.astype(np.float64)))
    return np.sort(order[:k])


def adaptive_attention(Q, Kb, Kr, Vb, Vr, batch, n_heads, seq_len, top_k,
                       n_kv_heads=None, return_f32=False, return_sets=False):
    """Adaptive precision (config c5 of bitcache_amd/workloads.py; not in the reference, whose intent is
    src/adaptive_precision.cuh:6-12,33-41):  per (b, query head) select the top_k
    keys by topk_key; selected keys use the compensated score and V (binary +
    residual), the rest use the binary score and binary V; one softmax over all S."""
    hkv, g = _heads(batch, n_heads, n_kv_heads)
    d = Q.shape[-1]
    qw, sq, q32 = query_prep(Q.reshape(batch * n_heads, d))
    isd = inv_sqrt(d)
    kw = Kb.words.reshape(batch, hkv, seq_len, -1)
    ks = Kb.scale.reshape(batch, hkv, seq_len)
    kc = Kr.codes.reshape(batch, hkv, seq_len, d)
    krs = Kr.scale.reshape(batch, hkv, seq_len)
    vbin = dequant_binary(Vb, d).reshape(batch, hkv, seq_len, d)
    vres = dequant_residual(Vr).reshape(batch, hkv, seq_len, d)
    out = np.empty((batch, n_heads, d), np.float16)
    o32 = np.empty((batch, n_heads, d), F32)
    sets = {}
    for b in range(batch):
        for kh in range(hkv):
            deq = dequant_residual(ResidualEnc(kc[b, kh], krs[b, kh]))
            for h in range(kh * g, (kh + 1) * g):
                i = b * n_heads + h
                pc = popcounts(qw[i], kw[b, kh])
                sel = topk_select(topk_key(ks[b, kh], pc, d), top_k)
                sets[(b, h)] = sel
                xd = xnor_dot(sq[i], pc, ks[b, kh], d)
                sc = (xd * isd).astype(F32)
                rd = (deq[sel] @ q32[i]).astype(F32)
                sc[sel] = ((xd[sel] + rd).astype(F32) * isd).astype(F32)
                vrec = vbin[b, kh].copy()
                vrec[sel] = (vrec[sel] + vres[b, kh][sel]).astype(F32)
                out[b, h], o32[b, h] = _softmax_out(sc, vrec)
    res = [out]
    if return_f32:
        res.append(o32)
    if return_sets:
        res.append(sets)
    return res[0] if len(res) == 1 else tuple(res)


# ----------------------------------------------------------------------------
# ring buffer (BitCache) state machine: bitcache/__init__.py:95-113
# ----------------------------------------------------------------------------
class RingState:
    """write_pos/filled bookkeeping of BitCache.append (bitcache/__init__.py:112-113)."""

    def __init__(self, max_seq: int):
        self.max_seq = max_seq
        self.write_pos = 0
        self.filled = 0

    def append(self) -> int:
        slot = self.write_pos
        self.write_pos = (self.write_pos + 1) % self.max_seq
        self.filled = min(self.filled + 1, self.max_seq)
        return slot


# ----------------------------------------------------------------------------
# torch-CPU fast path for the CPU baseline (same math, multi-threaded)
# ----------------------------------------------------------------------------
def _torch_sign_bytes(words):
    """int64 view of u32 sign words [S, d/32] -> uint8 [S, d/8] (little-endian)."""
    import torch
    sh = torch.tensor([0, 8, 16, 24], dtype=torch.int64)
    return ((words.unsqueeze(-1) >> sh) & 0xFF).to(torch.uint8).reshape(words.shape[0], -1)


_POPC8 = None


def _torch_popcounts(q32, kbytes):
    """XNOR popcounts (src/xnor_dot.cuh:20-27) of query rows q32 [G, d] against
    key sign bytes [S, d/8] -> int32 [G, S], by a 256-entry byte table."""
    import torch
    global _POPC8
    if _POPC8 is None:
        _POPC8 = torch.tensor([bin(i).count("1") for i in range(256)], dtype=torch.int32)
    G, d = q32.shape
    qbits = (q32 >= 0).to(torch.uint8).reshape(G, d // 8, 8)
    qbytes = (qbits << torch.arange(8, dtype=torch.uint8)).sum(-1).to(torch.uint8)   # [G, d/8]
    x = torch.bitwise_not(torch.bitwise_xor(kbytes.unsqueeze(0), qbytes.unsqueeze(1)))
    return _POPC8[x.long()].sum(-1, dtype=torch.int32)


def _torch_scale_q(q32):
    """scale_q per row: sequential fp32 sum of |q_i|, / d (src/compensated_attention.cu:65-67)."""
    import torch
    d = q32.shape[-1]
    sq = torch.zeros(q32.shape[0], dtype=torch.float32)
    for i in range(d):
        sq = sq + q32[:, i].abs()
    return sq / d


def _torch_vbin(vwords, vscale16, d):
    """+-scale_v per element from the V sign words [S, d]."""
    import torch
    vb = _torch_sign_bytes(vwords)
    bits = ((vb.unsqueeze(-1) >> torch.arange(8, dtype=torch.uint8)) & 1).reshape(vb.shape[0], d)
    sv = vscale16.float().unsqueeze(1)
    return torch.where(bits.bool(), sv, -sv)


def _torch_softmax_out(sc, vrec):
    """m = max(-1e38, s); w = exp(s - m); out = fp16((w @ vrec) / sum w), per row."""
    import torch
    m = torch.clamp(sc.max(dim=-1, keepdim=True).values, min=-1e38)
    w = torch.exp(sc - m)
    l = w.sum(-1, keepdim=True)
    return ((w @ vrec) * (1.0 / l)).half()


def binary_attention_torch_cpu(q16, kwords, kscale16, vwords, vscale16):
    """Query rows q16 [G, d] over one kv head's S keys, binary attention on torch
    CPU tensors (src/binary_attention.cu:24-81): score = (scale_q*scale_k) *
    (2pc - d) * inv_sqrt_d, V = +-scale_v.  Words: int64 view of the u32 sign
    words; scales fp16.  Returns fp16 [G, d]."""
    d = q16.shape[-1]
    q32 = q16.reshape(-1, d).float()
    pc = _torch_popcounts(q32, _torch_sign_bytes(kwords))
    xd = (_torch_scale_q(q32).unsqueeze(1) * kscale16.float().unsqueeze(0)) * (2 * pc - d).float()
    return _torch_softmax_out(xd * float(inv_sqrt(d)), _torch_vbin(vwords, vscale16, d))


def adaptive_attention_torch_cpu(q16, kwords, kscale16, kcodes, krscale16, vwords, vscale16,
                                 vcodes, vrscale16, top_k):
    """adaptive_attention for query rows q16 [G, d] sharing one kv head's S keys,
    on torch CPU tensors: per row the top_k keys by topk_key (a stable sort on
    -key: largest first, lowest index on ties; NaN last, -0 as +0) take the
    compensated score and V, the others the binary ones; one softmax.  Returns
    (fp16 [G, d], bool [G, S] selected)."""
    import torch
    d = q16.shape[-1]
    q32 = q16.reshape(-1, d).float()
    G, S = q32.shape[0], kwords.shape[0]
    pc = _torch_popcounts(q32, _torch_sign_bytes(kwords))
    n = (2 * pc - d).float()
    xd = (_torch_scale_q(q32).unsqueeze(1) * kscale16.float().unsqueeze(0)) * n
    key = kscale16.float().unsqueeze(0) * n + 0.0
    key = torch.where(torch.isnan(key), torch.tensor(-math.inf), key)
    k = min(top_k, S)
    order = torch.sort(-key, dim=-1, stable=True).indices[:, :k]
    sel = torch.zeros((G, S), dtype=torch.bool)
    sel.scatter_(1, order, True)
    isd = float(inv_sqrt(d))
    vbin = _torch_vbin(vwords, vscale16, d)
    out = torch.empty((G, d), dtype=torch.float16)
    for g in range(G):
        idx = order[g]
        kdeq = (kcodes[idx].float() / 7.0) * krscale16[idx].float().unsqueeze(1)
        sc = xd[g] * isd
        sc[idx] = (xd[g, idx] + kdeq @ q32[g]) * isd
        # softmax as _torch_softmax_out, with the V residual added on the
        # selected rows only: sum_s w_s vbin_s + sum_{s in sel} w_s vres_s
        m = torch.clamp(sc.max(), min=-1e38)
        w = torch.exp(sc - m)
        vdeq = (vcodes[idx].float() / 7.0) * vrscale16[idx].float().unsqueeze(1)
        acc = w @ vbin + w[idx] @ vdeq
        out[g] = (acc * (1.0 / w.sum())).half()
    return out, sel


def compensated_attention_torch_cpu(q16, kwords, kscale16, kcodes, krscale16,
                                    vwords, vscale16, vcodes, vrscale16):
    """One (b, head) of compensated attention on torch CPU tensors, vectorised.

    Same formulas as compensated_attention (src/compensated_attention.cu:56-108):
    scores from popcounts of the packed sign words and the INT4 residual dot,
    V from sign*scale + dequantised residual.  Inputs are torch CPU tensors
    (words int64 view of the u32 words, scales fp16, codes int8)."""
    import torch
    d = q16.shape[-1]
    q32 = q16.float()
    qbits = (q32 >= 0)
    sq = torch.zeros((), dtype=torch.float32)
    for i in range(d):
        sq = sq + q32[i].abs()
    sq = sq / d
    # popcount of XNOR == d - hamming; computed from unpacked sign bits
    shifts = torch.arange(32, dtype=torch.int64)
    kb = ((kwords.unsqueeze(-1) >> shifts) & 1).reshape(kwords.shape[0], d).bool()
    pc = (kb == qbits).sum(dim=1, dtype=torch.int32)
    xd = (sq * kscale16.float()) * (2 * pc - d).float()
    deq = (kcodes.float() / 7.0) * krscale16.float().unsqueeze(1)
    rd = deq @ q32
    sc = (xd + rd) * float(inv_sqrt(d))
    m = torch.clamp(sc.max(), min=-1e38)
    w = torch.exp(sc - m)
    l = w.sum()
    vb = ((vwords.unsqueeze(-1) >> shifts) & 1).reshape(vwords.shape[0], d).bool()
    vrec = torch.where(vb, vscale16.float().unsqueeze(1), -vscale16.float().unsqueeze(1))
    vrec = vrec + (vcodes.float() / 7.0) * vrscale16.float().unsqueeze(1)
    acc = w @ vrec
    return (acc * (1.0 / l)).half()
