"""Helpers shared by the GPU parity tests: blob -> oracle semantic arrays and
the output tolerance of the compressed path."""
from __future__ import annotations

import sys

import numpy as np
import torch

from oracle import oracle as O

# parity bar for fp16/fp32 outputs: max-abs error relative to the
# largest reference magnitude <= 2e-3 and cosine similarity >= 0.9999.
REL_TOL = 2e-3
COS_TOL = 0.9999


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()


def bin_from_blob(blob: torch.Tensor, n: int, d: int) -> O.BinaryEnc:
    b = to_np(blob)
    sb = n * d // 8
    words = b[:sb].view("<u4").reshape(n, d // 32).astype(np.uint32)
    scale = b[sb:sb + 2 * n].view(np.float16).copy()
    return O.BinaryEnc(words=words, scale=scale, mean32=scale.astype(np.float32))


def res_from_blob(blob: torch.Tensor, n: int, d: int) -> O.ResidualEnc:
    b = to_np(blob)
    cb = n * d // 2
    nib = b[:cb].reshape(n, d // 2)
    scale = b[cb:cb + 2 * n].view(np.float16).copy()
    return O.ResidualEnc(codes=O.unpack_nibbles(nib), scale=scale)


def slice_enc(e, lo, hi):
    if isinstance(e, O.BinaryEnc):
        return O.BinaryEnc(e.words[lo:hi], e.scale[lo:hi], e.mean32[lo:hi])
    return O.ResidualEnc(e.codes[lo:hi], e.scale[lo:hi])


def assert_same_bin(got: O.BinaryEnc, exp: O.BinaryEnc, what=""):
    assert np.array_equal(got.words, exp.words), f"sign words differ {what}"
    assert np.array_equal(got.scale.view(np.uint16), exp.scale.view(np.uint16)), f"scales differ {what}"


def assert_same_res(got: O.ResidualEnc, exp: O.ResidualEnc, what=""):
    assert np.array_equal(got.codes, exp.codes), f"codes differ {what}"
    assert np.array_equal(got.scale.view(np.uint16), exp.scale.view(np.uint16)), f"rscales differ {what}"


def close(got: np.ndarray, ref: np.ndarray, rel=REL_TOL, cos=COS_TOL, what=""):
    g = np.asarray(got, np.float64).reshape(-1)
    r = np.asarray(ref, np.float64).reshape(-1)
    assert np.all(np.isfinite(g)), f"non-finite output {what}"
    scale = max(np.max(np.abs(r)), 1e-30)
    err = np.max(np.abs(g - r)) / scale
    c = float(g @ r / (np.linalg.norm(g) * np.linalg.norm(r) + 1e-300))
    assert err <= rel, f"max-abs rel err {err:.3e} > {rel} {what}"
    assert c >= cos, f"cosine {c:.6f} < {cos} {what}"
    return err, c


def ring_oracle_attend(q, hist_k, hist_v, max_seq, B, Hq, Hkv, d, compensated=True):
    """Oracle attention over the tokens a ring of max_seq slots per row holds
    after appending hist_k / hist_v ([B, Hkv, d] per step, online-encode math):
    the last min(len, max_seq) tokens (slot order does not matter for softmax
    attention).  Returns the fp32 output [B, Hq, d]."""
    n = min(len(hist_k), max_seq)
    slots = {}
    for t, (k, v) in enumerate(zip(hist_k, hist_v)):
        slots[t % max_seq] = (k, v)
    ks = np.stack([slots[s][0] for s in range(n)], axis=2)  # [B, Hkv, n, d]
    vs = np.stack([slots[s][1] for s in range(n)], axis=2)
    Kb, Kr = O.online_encode(ks.reshape(-1, d))
    Vb, Vr = O.online_encode(vs.reshape(-1, d))
    if compensated:
        return O.compensated_attention(q, Kb, Kr, Vb, Vr, B, Hq, n, n_kv_heads=Hkv,
                                       return_f32=True)[1]
    return O.binary_attention(q, Kb, Vb, B, Hq, n, n_kv_heads=Hkv, return_f32=True)[1]


def ring_oracle_keys(hist_k, max_seq, B, Hkv, d):
    """Online-encoded K of the tokens a ring holds (as ring_oracle_attend)."""
    n = min(len(hist_k), max_seq)
    slots = {t % max_seq: k for t, k in enumerate(hist_k)}
    ks = np.stack([slots[s] for s in range(n)], axis=2)
    return O.online_encode(ks.reshape(-1, d))[0], n


def bin_head_tensors(bb, n, d, lo, S):
    """S vectors from cache vector lo of a binary blob (capacity n) as torch-CPU
    tensors: sign words (int64 view of the u32 words) and fp16 scales."""
    w = bb[lo * d // 8:(lo + S) * d // 8].cpu().view(torch.int32).view(S, d // 32)
    sc = bb[n * d // 8 + 2 * lo:n * d // 8 + 2 * (lo + S)].cpu().view(torch.float16)
    return w.to(torch.int64) & 0xFFFFFFFF, sc


def blob_head_tensors(kb, kr, vb, vr, n, d, lo, S):
    """One (b, head)'s S keys starting at cache vector lo, read from the
    device blobs (capacity n) as the torch-CPU tensors
    oracle.compensated_attention_torch_cpu takes: sign words (int64 view of
    the u32 words), fp16 scales, int8 codes, fp16 residual scales, for K then V."""
    def planes(bb, rb):
        w = bb[lo * d // 8:(lo + S) * d // 8].cpu().view(torch.int32).view(S, d // 32)
        sc = bb[n * d // 8 + 2 * lo:n * d // 8 + 2 * (lo + S)].cpu().view(torch.float16)
        c = rb[lo * d // 2:(lo + S) * d // 2].cpu().view(S, d // 2).to(torch.int16)
        lo_, hi_ = c & 0xF, (c >> 4) & 0xF
        lo_ = torch.where(lo_ >= 8, lo_ - 16, lo_)
        hi_ = torch.where(hi_ >= 8, hi_ - 16, hi_)
        codes = torch.stack([lo_, hi_], dim=-1).reshape(S, d).to(torch.int8)
        rs = rb[n * d // 2 + 2 * lo:n * d // 2 + 2 * (lo + S)].cpu().view(torch.float16)
        return w.to(torch.int64) & 0xFFFFFFFF, sc, codes, rs
    return planes(kb, kr) + planes(vb, vr)
