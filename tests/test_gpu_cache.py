"""GPU parity of the BitCache ring buffer (bitcache/__init__.py:29-207) against
the oracle's state machine and encode/attention restatement: stride-correct
reads, wrap-around, GQA, binary mode, prefill == appends, reset."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.gpu_util import close, ring_oracle_attend, say, slice_enc, to_np

pytestmark = pytest.mark.gpu


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
            ref = ring_oracle_attend(q, hk, hv, max_seq, B, Hq, Hkv, d, comp)
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


def test_config_c4_full_size():
    """Config c4 at full size (B4, GQA 32/8, 16384-token prefill + 256 decode
    steps of append + attend).  Size-independent checks: the one-launch step
    (append_attend, as bench.py runs it) gives the same output at every step
    and the same cache bytes as append() + attend(); the cache after the loop
    is bit-identical to a one-shot prefill of all 16640 tokens (appends ==
    prefill); the outputs of the first, middle and last steps for two head
    groups match the oracle (online encode of the group's tokens, then
    compensated attention over them)."""
    from bitcache_amd import BitCache
    from bitcache_amd import workloads as W
    say("case c4 full size")
    cfg = W.CONFIGS["c4"]
    B, Hq, Hkv, S, d = cfg.batch, cfg.n_heads, cfg.n_kv_heads, cfg.seq_len, cfg.head_dim
    G, T = Hq // Hkv, W.C4_DECODE_STEPS
    _, k, v = W.make_qkv(cfg)
    g = torch.Generator(device="cuda")
    g.manual_seed(cfg.seed + 100)
    qs = (torch.randn((T, B, Hq, d), generator=g, device="cuda") * W.SIGMA).half()
    ks = (torch.randn((T, B, Hkv, d), generator=g, device="cuda") * W.SIGMA).half()
    vs = (torch.randn((T, B, Hkv, d), generator=g, device="cuda") * W.SIGMA).half()
    cache = BitCache(B, Hq, d, S + T, n_kv_heads=Hkv)
    fused = BitCache(B, Hq, d, S + T, n_kv_heads=Hkv)    # the same loop with append_attend
    cache.prefill(k, v)
    fused.prefill(k, v)
    outs = {}
    for t in range(T):
        cache.append(ks[t], vs[t])
        o = cache.attend(qs[t])
        assert torch.equal(fused.append_attend(ks[t], vs[t], qs[t]), o), f"append_attend differs at step {t}"
        if t in (0, T // 2, T - 1):
            outs[t] = o.clone()
    assert cache.seq_len == fused.seq_len == S + T
    for x, y in ((cache._k_bin, fused._k_bin), (cache._v_bin, fused._v_bin),
                 (cache._k_res, fused._k_res), (cache._v_res, fused._v_res)):
        assert torch.equal(x, y)
    kall = torch.cat([k, ks.permute(1, 2, 0, 3)], dim=2).contiguous()
    vall = torch.cat([v, vs.permute(1, 2, 0, 3)], dim=2).contiguous()
    once = BitCache(B, Hq, d, S + T, n_kv_heads=Hkv)
    once.prefill(kall, vall)
    for x, y in ((cache._k_bin, once._k_bin), (cache._v_bin, once._v_bin),
                 (cache._k_res, once._k_res), (cache._v_res, once._v_res)):
        assert torch.equal(x, y)
    for b, kvh in [(0, 0), (3, 7)]:
        Kb, Kr = O.online_encode(to_np(kall[b, kvh]))
        Vb, Vr = O.online_encode(to_np(vall[b, kvh]))
        for t, o in outs.items():
            n = S + t + 1
            enc = [slice_enc(e, 0, n) for e in (Kb, Kr, Vb, Vr)]
            qg = to_np(qs[t, b, kvh * G:(kvh + 1) * G])[None]
            ref = O.compensated_attention(qg, *enc, 1, G, n, n_kv_heads=1, return_f32=True)[1]
            close(to_np(o[b, kvh * G:(kvh + 1) * G]).astype(np.float32), ref[0],
                  what=f"c4 step {t} group {(b, kvh)}")


@pytest.mark.parametrize("B,Hq,Hkv,d,max_seq,prefill,steps,comp", [
    (2, 8, 8, 128, 700, 500, 40, True),      # MHA, fused
    (2, 8, 2, 128, 300, 250, 90, True),      # GQA 4 (the c4 group), fused, wraps at step 50
    (1, 16, 1, 128, 200, 150, 60, True),     # group 16: two query-head groups, two-launch path
    (2, 4, 2, 64, 130, 64, 80, False),       # binary caches, d = 64, wraps
    (1, 4, 4, 256, 96, 0, 120, True),        # d = 256, from empty, wraps
    (1, 4, 2, 96, 64, 30, 50, True),         # d = 96: VALU kernels, two-launch path, wraps
])
def test_append_attend_equals_append_then_attend(B, Hq, Hkv, d, max_seq, prefill, steps, comp):
    """BitCache.append_attend (one launch: the workgroup holding the ring slot
    encodes the token before attending) leaves the same cache bytes and returns
    the same output, bit for bit, as append() followed by attend(), at every
    step, before and after the ring wraps."""
    from bitcache_amd import BitCache
    say(f"case append_attend B={B} Hq={Hq} Hkv={Hkv} d={d} max_seq={max_seq} prefill={prefill} "
        f"steps={steps} comp={comp}")
    g = torch.Generator(device="cuda")
    g.manual_seed(B * 1000 + steps)
    rnd = lambda *s: (torch.randn(s, generator=g, device="cuda") * 0.2).half()
    a = BitCache(B, Hq, d, max_seq, compensated=comp, n_kv_heads=Hkv)
    b = BitCache(B, Hq, d, max_seq, compensated=comp, n_kv_heads=Hkv)
    if prefill:
        k0, v0 = rnd(B, Hkv, prefill, d), rnd(B, Hkv, prefill, d)
        a.prefill(k0, v0)
        b.prefill(k0, v0)
    for t in range(steps):
        k, v, q = rnd(B, Hkv, d), rnd(B, Hkv, d), rnd(B, Hq, d)
        a.append(k, v)
        want = a.attend(q)
        got = b.append_attend(k, v, q)
        assert torch.equal(got, want), f"output differs at step {t}"
        assert a.seq_len == b.seq_len
    pairs = [(a._k_bin, b._k_bin), (a._v_bin, b._v_bin)]
    if comp:
        pairs += [(a._k_res, b._k_res), (a._v_res, b._v_res)]
    for x, y in pairs:
        assert torch.equal(x, y)


def test_append_attend_in_a_hip_graph():
    """A decode loop of append_attend steps captured in one HIP graph: three
    replays, each from the same prefilled cache with eager work and a
    synchronisation in between, give the eager outputs and cache bytes bit for
    bit (the ops allocate only from torch's graph pool and record no memset)."""
    from bitcache_amd import BitCache
    say("case append_attend graph")
    B, Hq, Hkv, d, S, T = 2, 8, 2, 128, 600, 24
    g = torch.Generator(device="cuda")
    g.manual_seed(21)
    rnd = lambda *s: (torch.randn(s, generator=g, device="cuda") * 0.2).half()
    k0, v0 = rnd(B, Hkv, S, d), rnd(B, Hkv, S, d)
    ks, vs, qs = rnd(T, B, Hkv, d), rnd(T, B, Hkv, d), rnd(T, B, Hq, d)
    cache = BitCache(B, Hq, d, S + T, n_kv_heads=Hkv)

    def start():
        cache.reset()
        cache.prefill(k0, v0)
        torch.cuda.synchronize()

    start()
    want = [cache.append_attend(ks[t], vs[t], qs[t]).clone() for t in range(T)]
    want_k = cache._k_res.clone()
    start()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        got = [cache.append_attend(ks[t], vs[t], qs[t]) for t in range(T)]
    for rep in range(3):
        start()
        graph.replay()
        torch.cuda.synchronize()
        for t in range(T):
            assert torch.equal(got[t], want[t]), f"replay {rep}, step {t}"
        assert torch.equal(cache._k_res, want_k), f"replay {rep}: cache bytes"


def test_bitcache_binary_ring_one_head_per_cu():
    """A binary-mode BitCache with one head per CU (the one-workgroup-per-head
    plan) on a partly filled ring (2001 of 3000 tokens): the attention reads
    each head's row at the ring's stride and stops at its last token; eight
    heads against the oracle's binary attention over those tokens (online
    encode)."""
    from bitcache_amd import BitCache
    cu = torch.cuda.get_device_properties(0).multi_processor_count
    if cu % 32:
        pytest.skip(f"{cu} CUs: no batch of 32-head sequences gives one head per CU")
    B, H, d, max_seq, S = cu // 32, 32, 128, 3000, 2001
    say(f"case bitcache binary ring B={B} H={H} S={S} max_seq={max_seq}")
    rng = np.random.default_rng(2001)
    k = (rng.standard_normal((B, H, S, d)) * 0.2).astype(np.float16)
    v = (rng.standard_normal((B, H, S, d)) * 0.2).astype(np.float16)
    q = (rng.standard_normal((B, H, d)) * 0.3).astype(np.float16)
    cache = BitCache(B, H, d, max_seq, compensated=False)
    cache.prefill(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
    out = to_np(cache.attend(torch.from_numpy(q).cuda())).astype(np.float32)
    for (b, h) in [(0, 0), (0, 31), (1, 7), (2, 15), (3, 3), (B - 1, 0), (B - 1, 16), (B // 2, 30)]:
        Kb, _ = O.online_encode(k[b, h])
        Vb, _ = O.online_encode(v[b, h])
        _, ref = O.binary_attention(q[b, h][None, None], Kb, Vb, 1, 1, S, return_f32=True)
        close(out[b, h][None], ref[0], what=f"binary ring head {(b, h)}")


@pytest.mark.parametrize("max_seq,S", [(3000, 2000), (3001, 2000), (3000, 1999)])
def test_bitcache_attend_adaptive_partly_filled(max_seq, S):
    """BitCache.attend_adaptive on a partly filled GQA ring (S of max_seq
    tokens): the selection passes and the attention read rows at the ring's
    stride; max_seq 3000 takes the eight-key scale loads (with S = 1999 the
    last eight-key run of each row ends past the row's tokens), 3001 (stride
    not a multiple of 8) the per-key ones.  Sets bit-exact, outputs against
    the oracle (online encode of each group's tokens)."""
    from bitcache_amd import BitCache
    say(f"case bitcache adaptive partly filled max_seq={max_seq} S={S}")
    B, Hq, Hkv, d, top_k = 2, 8, 2, 128, 200
    G = Hq // Hkv
    rng = np.random.default_rng(max_seq + S)
    k = (rng.standard_normal((B, Hkv, S, d)) * 0.2).astype(np.float16)
    v = (rng.standard_normal((B, Hkv, S, d)) * 0.2).astype(np.float16)
    q = (rng.standard_normal((B, Hq, d)) * 0.3).astype(np.float16)
    cache = BitCache(B, Hq, d, max_seq, n_kv_heads=Hkv)
    cache.prefill(torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
    out, sel = cache.attend_adaptive(torch.from_numpy(q).cuda(), top_k=top_k, return_selected=True)
    out, sel = to_np(out).astype(np.float32), to_np(sel)
    assert sel.shape == (B, Hq, S)
    for b in range(B):
        for kvh in range(Hkv):
            Kb, Kr = O.online_encode(k[b, kvh])
            Vb, Vr = O.online_encode(v[b, kvh])
            qg = q[b, kvh * G:(kvh + 1) * G][None]
            _, ref, sets = O.adaptive_attention(qg, Kb, Kr, Vb, Vr, 1, G, S, top_k, n_kv_heads=1,
                                                return_f32=True, return_sets=True)
            for (_, h), want in sets.items():
                got = np.nonzero(sel[b, kvh * G + h])[0]
                assert np.array_equal(got, want), f"set differs at (b={b}, h={kvh * G + h})"
            close(out[b, kvh * G:(kvh + 1) * G], ref[0], what=f"adaptive ring group {(b, kvh)}")
