"""GPU parity of the BitCache ring buffer (bitcache/__init__.py:29-207) against
the oracle's state machine and encode/attention restatement: stride-correct
reads, wrap-around, GQA, binary mode, prefill == appends, reset."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.gpu_util import close, say, to_np

pytestmark = pytest.mark.gpu


def oracle_attend(q, hist_k, hist_v, ring: O.RingState, B, Hq, Hkv, d, compensated=True):
    """Attention over the tokens currently in the ring (slot order does not
    matter for softmax attention)."""
    n = ring.filled
    slots = {}
    for t, (k, v) in enumerate(zip(hist_k, hist_v)):
        slots[t % ring.max_seq] = (k, v)
    ks = np.stack([slots[s][0] for s in range(n)], axis=2)  # [B, Hkv, n, d]
    vs = np.stack([slots[s][1] for s in range(n)], axis=2)
    Kb, Kr = O.online_encode(ks.reshape(-1, d))
    Vb, Vr = O.online_encode(vs.reshape(-1, d))
    if compensated:
        return O.compensated_attention(q, Kb, Kr, Vb, Vr, B, Hq, n, n_kv_heads=Hkv, return_f32=True)[1]
    return O.binary_attention(q, Kb, Vb, B, Hq, n, n_kv_heads=Hkv, return_f32=True)[1]


@pytest.mark.parametrize("B,Hq,Hkv,d,max_seq,steps,comp", [
    (1, 4, 4, 128, 64, 40, True),     # partially filled, B*H > 1 (reference defect B1 case)
    (2, 4, 4, 64, 16, 37, True),      # wraps twice
    (2, 8, 2, 128, 50, 60, True),     # GQA + wrap
    (1, 2, 2, 128, 32, 20, False),    # binary mode (reference defect B2 case)
])
def test_bitcache_append_attend(B, Hq, Hkv, d, max_seq, steps, comp):
    from bitcache_amd import BitCache
    say(f"case bitcache B={B} Hq={Hq} Hkv={Hkv} d={d} max_seq={max_seq} steps={steps} comp={comp}")
    rng = np.random.default_rng(steps)
    cache = BitCache(B, Hq, d, max_seq, device="cuda", compensated=comp, n_kv_heads=Hkv)
    ring = O.RingState(max_seq)
    hk, hv = [], []
    for t in range(steps):
        k = (rng.standard_normal((B, Hkv, d)) * 0.3).astype(np.float16)
        v = (rng.standard_normal((B, Hkv, d)) * 0.3).astype(np.float16)
        cache.append(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
        ring.append()
        hk.append(k)
        hv.append(v)
        if t in (0, steps // 2, steps - 1):
            q = (rng.standard_normal((B, Hq, d)) * 0.3).astype(np.float16)
            out = cache.attend(torch.from_numpy(q).cuda())
            ref = oracle_attend(q, hk, hv, ring, B, Hq, Hkv, d, comp)
            close(to_np(out).astype(np.float32), ref, what=f"step {t}")
    assert cache.seq_len == ring.filled
    if not comp:
        assert cache._k_res is None
    cache.reset()
    assert cache.seq_len == 0 and torch.count_nonzero(cache._k_bin) == 0


def test_bitcache_prefill_equals_appends():
    from bitcache_amd import BitCache
    say("case bitcache prefill")
    B, Hq, Hkv, d, S, max_seq = 2, 8, 2, 128, 300, 512
    rng = np.random.default_rng(1)
    k = (rng.standard_normal((B, Hkv, S, d)) * 0.2).astype(np.float16)
    v = (rng.standard_normal((B, Hkv, S, d)) * 0.2).astype(np.float16)
    a = BitCache(B, Hq, d, max_seq, n_kv_heads=Hkv)
    b = BitCache(B, Hq, d, max_seq, n_kv_heads=Hkv)
    a.prefill(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
    for s in range(S):
        b.append(torch.from_numpy(np.ascontiguousarray(k[:, :, s])).cuda(),
                 torch.from_numpy(np.ascontiguousarray(v[:, :, s])).cuda())
    for x, y in ((a._k_bin, b._k_bin), (a._v_bin, b._v_bin), (a._k_res, b._k_res), (a._v_res, b._v_res)):
        assert torch.equal(x, y)
    q = torch.from_numpy((rng.standard_normal((B, Hq, d)) * 0.3).astype(np.float16)).cuda()
    assert torch.equal(a.attend(q), b.attend(q))
    assert a.seq_len == b.seq_len == S
    assert abs(a.compression_ratio - (d * 2) / (36 + 130)) < 1e-9


def test_bitcache_rejects_bad_inputs():
    from bitcache_amd import BitCache
    say("case bitcache validation")
    c = BitCache(1, 2, 128, 8)
    with pytest.raises(AssertionError):
        c.attend(torch.zeros((1, 2, 128), dtype=torch.float16, device="cuda"))
    with pytest.raises(AssertionError):
        c.append(torch.zeros((1, 2, 64), dtype=torch.float16, device="cuda"),
                 torch.zeros((1, 2, 64), dtype=torch.float16, device="cuda"))
    with pytest.raises(AssertionError):
        c.append(torch.zeros((1, 2, 128), dtype=torch.float32, device="cuda"),
                 torch.zeros((1, 2, 128), dtype=torch.float32, device="cuda"))
