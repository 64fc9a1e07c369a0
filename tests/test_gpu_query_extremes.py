"""Queries far from the Gaussian draws of the other tests, against the
oracle within 2e-3 max-abs relative error and cosine 0.9999: a few channels scaled x10 and x100 (the
massive-activation channels of real decoder queries), fp16 extremes near
65504, fp16 subnormals, and signed zeros.

The matrix-core kernels take the INT4 residual dot q . dequant(K_res) on the
stored nibbles with the query as 24-bit fixed point (q_int = rint(q / step),
step = max|q| / 7,800,000), where the reference sums q * (n/7 * s) in fp32
(src/compensated_attention.cu:29-37).  A tile uses the top 16 bits unless a
key's residual scale lets that truncation move its score by more than 2^-11
nats, in which case it also adds the low 8 bits.  The rounding error per
element is then at most step/2, the same absolute bound on every element, so
elements far below max|q| keep fewer significant bits; these cases bound what
that costs on the outputs: compensated MHA and GQA, adaptive top-k (whose
selection uses only the exact binary key) and per-head modes, at d = 64, 128
and 256, plus the VALU kernel's head dims (fp32 residual dot)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.gpu_util import bin_from_blob, close, res_from_blob, say, to_np

pytestmark = pytest.mark.gpu

KINDS = ["x10", "x100", "fp16_extremes", "subnormal", "signed_zero"]


def make_query(B, Hq, d, kind, rng):
    q = rng.standard_normal((B, Hq, d)) * 0.09
    ch = rng.choice(d, size=4, replace=False)
    if kind == "x10":
        q[..., ch] *= 10.0
    elif kind == "x100":
        q[..., ch] *= 100.0
    elif kind == "fp16_extremes":
        # a few elements near the fp16 maximum, the rest ordinary: the
        # softmax is close to one-hot, the residual dot is dominated by them
        q[..., ch] = np.sign(q[..., ch]) * rng.uniform(3.0e4, 6.5e4, size=q[..., ch].shape)
    elif kind == "subnormal":
        # most elements below the fp16 normal range (< 6.1e-5), one head
        # entirely subnormal, the others with four ordinary channels
        q = q * 1e-4
        q[:, 1:, ch[:2]] = rng.standard_normal(q[:, 1:, ch[:2]].shape) * 0.09
    elif kind == "signed_zero":
        q[..., ch[:2]] = 0.0
        q[..., ch[2:]] = -0.0
    q16 = q.astype(np.float16)
    if kind == "signed_zero":
        q16[..., ch[2:]] = np.float16(-0.0)
    assert np.all(np.isfinite(q16))
    return q16


def make_kv(B, Hkv, S, d, rng):
    k = rng.standard_normal((B, Hkv, S, d)) * 0.09
    v = rng.standard_normal((B, Hkv, S, d)) * 0.09
    return k.astype(np.float16), v.astype(np.float16)


def encoded(F, x, n, d):
    xb, xr = F.encode_fused(torch.from_numpy(np.ascontiguousarray(x.reshape(-1, d))).cuda())
    return xb, xr, bin_from_blob(xb, n, d), res_from_blob(xr, n, d)


SHAPES = [
    # (B, Hq, Hkv, S, d)
    (1, 4, 4, 700, 64),
    (1, 4, 4, 900, 128),
    (1, 4, 4, 500, 256),
    (2, 8, 2, 333, 64),     # GQA 4
    (1, 8, 2, 700, 128),    # GQA 4
    (1, 8, 4, 600, 128),    # GQA 2
    (1, 16, 2, 300, 128),   # GQA 8
    (1, 8, 2, 400, 256),    # GQA 4
    (1, 4, 4, 300, 96),     # VALU kernel (fp32 residual dot)
    (1, 8, 2, 260, 160),
]


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("shape", SHAPES, ids=[str(s) for s in SHAPES])
def test_compensated_and_adaptive_with_extreme_queries(shape, kind):
    import bitcache_amd.functional as F
    B, Hq, Hkv, S, d = shape
    say(f"case query {kind} {shape}")
    rng = np.random.default_rng(S + d + KINDS.index(kind))
    q = make_query(B, Hq, d, kind, rng)
    k, v = make_kv(B, Hkv, S, d, rng)
    n = B * Hkv * S
    kb, kr, Kb, Kr = encoded(F, k, n, d)
    vb, vr, Vb, Vr = encoded(F, v, n, d)
    qt = torch.from_numpy(q).cuda()
    kw = dict(n_kv_heads=Hkv) if Hkv != Hq else {}
    out = F.compensated_attention(qt, kb, kr, vb, vr, B, Hq, S, d, **kw)
    _, ref = O.compensated_attention(q, Kb, Kr, Vb, Vr, B, Hq, S, n_kv_heads=Hkv, return_f32=True)
    close(to_np(out).astype(np.float32), ref, what=f"compensated {kind} {shape}")
    top_k = max(1, S // 10)
    aout, sel = F.adaptive_attention(qt, kb, kr, vb, vr, B, Hq, S, d, n_kv_heads=Hkv,
                                     top_k=top_k, return_selected=True)
    _, aref, sets = O.adaptive_attention(q, Kb, Kr, Vb, Vr, B, Hq, S, top_k, n_kv_heads=Hkv,
                                         return_f32=True, return_sets=True)
    sel = to_np(sel)
    for (b, h), idx in sets.items():
        assert np.array_equal(np.nonzero(sel[b, h])[0], idx), f"set differs at ({b}, {h})"
    close(to_np(aout).astype(np.float32), aref, what=f"adaptive {kind} {shape}")
    # per-head modes (the matrix-core kernel at 64/128/256, the VALU one otherwise)
    modes = torch.from_numpy((np.arange(B * Hq) % 2).astype(np.uint8).reshape(B, Hq)).cuda()
    mout = F.head_mode_attention(qt, kb, kr, vb, vr, modes, B, Hq, S, d, n_kv_heads=Hkv)
    _, bref = O.binary_attention(q, Kb, Vb, B, Hq, S, n_kv_heads=Hkv, return_f32=True)
    got = to_np(mout).astype(np.float32)
    m = to_np(modes)
    for b in range(B):
        for h in range(Hq):
            close(got[b, h], ref[b, h] if m[b, h] else bref[b, h],
                  what=f"head mode {kind} {shape} ({b},{h})")
