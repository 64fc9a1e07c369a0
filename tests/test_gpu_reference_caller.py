"""The reference's own caller on this build's operator module.

The reference's ``BitCache`` (bitcache/__init__.py:50-148) drives ``_C`` in a
fixed pattern: it allocates every buffer as exactly n_slots * sizeof bytes,
appends with two ``online_encode_token`` calls per step (a binary-mode cache
passes its binary buffer as the residual buffer, :104-111), and attends by
handing *prefix views* ``buf[: batch*n_heads*filled*sizeof]`` to
``compensated_attention`` / ``binary_attention`` (:131-148).
``ReferenceCaller`` below restates that pattern in this test's own code and
runs it against ``bitcache_amd._C`` -- the operator module a caller of the
reference imports in place of ``bitcache._C`` -- at B*H = 1 partly filled,
B*H > 1 partly filled, and a full ring that has wrapped.  Outputs are checked
against the oracle's attention over the tokens the ring holds (online-encode
math, read with the ring's own stride), within 2e-3 max-abs relative error
and cosine >= 0.9999; the reference's own
checkpoints of tests/test_python.py:75-158 are replayed with their cosine
bars against exact fp32 attention.
"""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.gpu_util import close, ring_oracle_attend, ring_oracle_keys, say, to_np

pytestmark = pytest.mark.gpu


class ReferenceCaller:
    """Restatement of the reference BitCache's calls into ``_C``
    (bitcache/__init__.py:50-158), with the operator module passed in."""

    def __init__(self, C, batch, n_heads, head_dim, max_seq, compensated=True):
        self.C, self.B, self.H, self.d, self.max_seq = C, batch, n_heads, head_dim, max_seq
        self.comp = compensated
        self.bv, self.rv = C.sizeof_binary_vec(), C.sizeof_residual_vec()
        n_slots = batch * n_heads * max_seq
        u8 = dict(dtype=torch.uint8, device="cuda")
        self.k_bin = torch.zeros(n_slots * self.bv, **u8)
        self.v_bin = torch.zeros(n_slots * self.bv, **u8)
        self.k_res = torch.zeros(n_slots * self.rv, **u8) if compensated else None
        self.v_res = torch.zeros(n_slots * self.rv, **u8) if compensated else None
        self.write_pos = 0
        self.filled = 0

    def append(self, K, V):
        # binary mode hands the binary buffer over as the residual buffer
        self.C.online_encode_token(K, self.k_bin, self.k_res if self.comp else self.k_bin,
                                   self.B, self.H, self.d, self.write_pos, self.max_seq)
        self.C.online_encode_token(V, self.v_bin, self.v_res if self.comp else self.v_bin,
                                   self.B, self.H, self.d, self.write_pos, self.max_seq)
        self.write_pos = (self.write_pos + 1) % self.max_seq
        self.filled = min(self.filled + 1, self.max_seq)

    def _prefix(self, buf, per):
        return buf[: self.B * self.H * self.filled * per]

    def attend(self, Q):
        kb, vb = self._prefix(self.k_bin, self.bv), self._prefix(self.v_bin, self.bv)
        if self.comp:
            kr, vr = self._prefix(self.k_res, self.rv), self._prefix(self.v_res, self.rv)
            return self.C.compensated_attention(Q, kb, kr, vb, vr, self.B, self.H, self.filled,
                                                self.d)
        return self.C.binary_attention(Q, kb, vb, self.B, self.H, self.filled, self.d)

    def entropy(self, Q):
        return self.C.compute_head_entropy(Q, self._prefix(self.k_bin, self.bv), self.B, self.H,
                                           self.filled, self.d)


def _tok(rng, shape, sigma=0.3):
    return (rng.standard_normal(shape) * sigma).astype(np.float16)


@pytest.mark.parametrize("B,H,d,max_seq,steps,comp", [
    (1, 1, 128, 64, 40, True),      # B*H = 1, partly filled
    (1, 1, 64, 32, 9, False),       # B*H = 1, partly filled, binary mode (aliased residual)
    (2, 4, 128, 64, 40, True),      # B*H > 1, partly filled
    (2, 3, 96, 48, 17, True),       # B*H > 1, head dim without the matrix-core kernel
    (1, 4, 256, 40, 23, False),     # B*H > 1, binary mode
    (2, 4, 64, 16, 37, True),       # full ring, wrapped twice
    (1, 2, 128, 32, 70, False),     # full ring, binary mode
])
def test_reference_call_sequence(B, H, d, max_seq, steps, comp):
    from bitcache_amd import _C
    say(f"case reference caller B={B} H={H} d={d} max_seq={max_seq} steps={steps} comp={comp}")
    rng = np.random.default_rng(1000 + steps + d)
    c = ReferenceCaller(_C, B, H, d, max_seq, comp)
    hk, hv = [], []
    for t in range(steps):
        k, v = _tok(rng, (B, H, d)), _tok(rng, (B, H, d))
        c.append(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
        hk.append(k)
        hv.append(v)
        if t in (0, steps // 3, steps - 1):
            q = _tok(rng, (B, H, d))
            qt = torch.from_numpy(q).cuda()
            out = c.attend(qt)
            ref = ring_oracle_attend(q, hk, hv, max_seq, B, H, H, d, comp)
            close(to_np(out).astype(np.float32), ref, what=f"step {t}")
            Kb, n = ring_oracle_keys(hk, max_seq, B, H, d)
            ent = to_np(c.entropy(qt))
            np.testing.assert_allclose(ent, O.head_entropy(q, Kb, B, H, n), rtol=2e-4, atol=2e-4)
    if not comp:
        # the aliased "residual" writes went nowhere: the binary planes hold
        # exactly the online-encoded sign bits and scales, the rest is zero
        cap = B * H * max_seq
        blob = to_np(c.k_bin)
        assert not blob[cap * (d // 8 + 2):].any()


def test_reference_entropy_dispatch_on_prefix_views():
    """functional.entropy_dispatch_attention on the reference caller's prefix
    views: every head matches the oracle's binary or compensated output,
    whichever its entropy selects."""
    import bitcache_amd.functional as F
    from bitcache_amd import _C
    say("case reference caller entropy dispatch")
    B, H, d, max_seq, steps = 2, 4, 128, 96, 50
    rng = np.random.default_rng(7)
    c = ReferenceCaller(_C, B, H, d, max_seq, True)
    hk, hv = [], []
    for t in range(steps):
        k, v = _tok(rng, (B, H, d)), _tok(rng, (B, H, d))
        c.append(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
        hk.append(k)
        hv.append(v)
    q = _tok(rng, (B, H, d))
    qt = torch.from_numpy(q).cuda()
    ent = to_np(c.entropy(qt))
    thr = float(np.median(ent))
    pre = lambda buf, per: c._prefix(buf, per)
    out, modes = F.entropy_dispatch_attention(qt, pre(c.k_bin, 36), pre(c.k_res, 130),
                                              pre(c.v_bin, 36), pre(c.v_res, 130), B, H,
                                              c.filled, d, thr)
    modes = to_np(modes).reshape(B, H)
    assert np.array_equal(modes, (ent < thr).astype(np.uint8))
    comp = ring_oracle_attend(q, hk, hv, max_seq, B, H, H, d, True)
    binr = ring_oracle_attend(q, hk, hv, max_seq, B, H, H, d, False)
    got = to_np(out).astype(np.float32)
    for b in range(B):
        for h in range(H):
            ref = comp[b, h] if modes[b, h] else binr[b, h]
            close(got[b, h], ref, what=f"head ({b},{h}) mode {modes[b, h]}")


def test_bitcache_head_mode_on_partly_filled_gqa_ring():
    """BitCache.attend_head_mode on a partly filled GQA ring: per head the
    oracle's binary or compensated output, modes from the ring's entropies."""
    from bitcache_amd import BitCache
    say("case bitcache head mode gqa ring")
    B, Hq, Hkv, d, max_seq, steps = 2, 8, 2, 128, 128, 77
    rng = np.random.default_rng(8)
    cache = BitCache(B, Hq, d, max_seq, n_kv_heads=Hkv)
    hk, hv = [], []
    for t in range(steps):
        k, v = _tok(rng, (B, Hkv, d)), _tok(rng, (B, Hkv, d))
        cache.append(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
        hk.append(k)
        hv.append(v)
    q = _tok(rng, (B, Hq, d))
    Kb, n = ring_oracle_keys(hk, max_seq, B, Hkv, d)
    ent = O.head_entropy(q, Kb, B, Hq, n, n_kv_heads=Hkv)
    thr = float(np.median(ent))
    out, modes = cache.attend_head_mode(torch.from_numpy(q).cuda(), threshold=thr,
                                        return_modes=True)
    modes = to_np(modes).reshape(B, Hq)
    # heads whose entropy sits within rounding of the threshold may go either way
    near = np.abs(ent - thr) <= 2e-4 * np.maximum(1.0, np.abs(ent))
    assert np.array_equal(modes[~near], (ent < thr).astype(np.uint8)[~near])
    comp = ring_oracle_attend(q, hk, hv, max_seq, B, Hq, Hkv, d, True)
    binr = ring_oracle_attend(q, hk, hv, max_seq, B, Hq, Hkv, d, False)
    got = to_np(out).astype(np.float32)
    for b in range(B):
        for h in range(Hq):
            close(got[b, h], comp[b, h] if modes[b, h] else binr[b, h], what=f"head ({b},{h})")


def test_reference_caller_rejects_views_it_cannot_place():
    """A blob view that is neither a whole blob nor a prefix of one of
    batch*n_heads*kv_stride vectors is an error, not a silent misread."""
    from bitcache_amd import _C
    say("case reference caller invalid views")
    B, H, d, S = 1, 2, 128, 16
    q = torch.zeros((B, H, d), dtype=torch.float16, device="cuda")
    kb = torch.zeros(B * H * S * 36 + 36, dtype=torch.uint8, device="cuda")   # 33 vectors
    with pytest.raises(RuntimeError, match="kv_stride"):
        _C.binary_attention(q, kb, kb, B, H, S, d)
    odd = torch.zeros(B * H * S * 36 + 5, dtype=torch.uint8, device="cuda")[: B * H * S * 36]
    with pytest.raises(RuntimeError, match="whole number"):
        _C.binary_attention(q, odd, odd, B, H, S, d)
    # a ring written for max_seq = 16 read through a prefix view of its K and a
    # whole V blob of another capacity
    k_ring = torch.zeros(B * H * 16 * 36, dtype=torch.uint8, device="cuda")
    v_other = torch.zeros(B * H * 8 * 36, dtype=torch.uint8, device="cuda")
    with pytest.raises(RuntimeError, match="exactly"):
        _C.binary_attention(q, k_ring[: B * H * 8 * 36], v_other, B, H, 8, d)


@pytest.mark.parametrize("batch,n_heads,head_dim,seq_len,comp", [
    (1, 1, 64, 128, False),
    (1, 1, 64, 128, True),
    (1, 1, 128, 256, True),
    (1, 4, 128, 512, True),
    (2, 4, 64, 256, True),
    (1, 1, 128, 1024, True),
])
def test_reference_python_test_configs(batch, n_heads, head_dim, seq_len, comp):
    """The reference's tests/test_python.py:63-167 replayed draw for draw:
    torch.manual_seed(42 + seq_len + head_dim), fp16 randn * 0.5 on the device
    for K then V of every step, then one query per checkpoint t in
    {S/4, S/2, S} (a fresh cache of max_seq = t + 4 each), then one more query
    for the binary-vs-compensated comparison.  Checks: parity (2e-3, cosine 0.9999) with
    the oracle at every checkpoint; cosine against exact fp32 attention above
    the reference's 0.85 (:136) wherever the reference algorithm itself (the
    oracle, same inputs) reaches it, else no lower than the oracle's cosine;
    cos_comp >= cos_bin - 0.01 (:158)."""
    from bitcache_amd import _C
    say(f"case reference test_python B={batch} H={n_heads} d={head_dim} S={seq_len} comp={comp}")
    B, H, d, S = batch, n_heads, head_dim, seq_len
    torch.manual_seed(42 + S + d)
    ks, vs = [], []
    for _ in range(S):
        ks.append(torch.randn(B, H, d, device="cuda", dtype=torch.float16) * 0.5)
        vs.append(torch.randn(B, H, d, device="cuda", dtype=torch.float16) * 0.5)
    K = torch.stack(ks, dim=2).float().cpu()
    V = torch.stack(vs, dim=2).float().cpu()
    hk = [to_np(k) for k in ks]
    hv = [to_np(v) for v in vs]

    def exact(q, t):
        p = torch.softmax((K[:, :, :t] @ q.float().cpu().unsqueeze(-1)).squeeze(-1) / math.sqrt(d), -1)
        return (p.unsqueeze(-1) * V[:, :, :t]).sum(2)

    def cos(a, b):
        a, b = a.double().flatten(), b.double().flatten()
        return float(a @ b / (a.norm() * b.norm() + 1e-12))

    for t in sorted({S // 4, S // 2, S}):
        q = torch.randn(B, H, d, device="cuda", dtype=torch.float16) * 0.5
        c = ReferenceCaller(_C, B, H, d, t + 4, comp)
        for s in range(t):
            c.append(ks[s].contiguous(), vs[s].contiguous())
        out = c.attend(q.contiguous())
        ref = ring_oracle_attend(to_np(q), hk[:t], hv[:t], t + 4, B, H, H, d, comp)
        close(to_np(out).astype(np.float32), ref, what=f"t={t}")
        e = exact(q, t)
        cs, cs_ref = cos(e, out.float().cpu()), cos(e, torch.from_numpy(ref))
        say(f"  t={t}: cosine vs exact attention {cs:.4f} (reference algorithm {cs_ref:.4f})")
        assert cs > min(0.85, cs_ref - 1e-4)
    if comp:
        q = torch.randn(B, H, d, device="cuda", dtype=torch.float16) * 0.5
        binc = ReferenceCaller(_C, B, H, d, S + 4, False)
        full = ReferenceCaller(_C, B, H, d, S + 8, True)
        for s in range(S):
            full.append(ks[s], vs[s])
            binc.append(ks[s], vs[s])
        e = exact(q, S)
        c_comp, c_bin = cos(e, full.attend(q).float().cpu()), cos(e, binc.attend(q).float().cpu())
        say(f"  binary {c_bin:.4f} compensated {c_comp:.4f}")
        assert c_comp >= c_bin - 0.01
