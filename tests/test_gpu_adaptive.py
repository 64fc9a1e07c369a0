"""GPU parity of adaptive top-k residual selection: selected index sets are
bit-exact with the oracle (stable sort on the exact key, lowest index first on
ties), outputs within tolerance, and the k = 0 / k = S limits reduce to binary
and compensated attention."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.gpu_util import bin_from_blob, blob_head_tensors, close, res_from_blob, say, to_np

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def F():
    import bitcache_amd.functional as F
    return F


def make(B, Hq, Hkv, S, d, seed, ties=False):
    rng = np.random.default_rng(seed)
    q = (rng.standard_normal((B, Hq, d)) * 0.1).astype(np.float16)
    k = rng.standard_normal((B, Hkv, S, d)) * 0.1
    v = rng.standard_normal((B, Hkv, S, d)) * 0.1
    if ties:
        # few distinct magnitudes and sign patterns -> many equal keys
        k = np.sign(k) * 0.125
        k[..., :100, :] = k[..., 100:200, :] if S >= 200 else k[..., :100, :]
    return q, k.astype(np.float16), v.astype(np.float16)


CASES = [
    # (B, Hq, Hkv, S, d, top_k, ties)
    (1, 4, 4, 1000, 128, 100, False),
    (2, 8, 2, 3000, 128, 300, False),
    (1, 4, 1, 4097, 64, 410, False),
    (1, 2, 2, 2000, 128, 200, True),
    (1, 2, 2, 2000, 128, 1, True),
    (1, 2, 2, 130, 256, 13, False),
    (1, 8, 2, 900, 256, 90, False),     # GQA 4 at d = 256
    (1, 4, 2, 1500, 128, 150, True),    # GQA 2 with ties
    (1, 16, 2, 640, 128, 64, False),    # GQA 8
    # c5 shape at 8K keys: 512 query heads over 128 KV groups, selection
    # passes over key chunks of 1024 (several per head), without and with ties
    (16, 32, 8, 8192, 128, 820, False),
    (16, 32, 8, 8192, 128, 820, True),
    # head dims without the matrix-core kernel (the VALU split kernel's
    # adaptive mode), MHA and GQA
    (1, 2, 2, 300, 32, 30, False),
    (1, 8, 2, 520, 32, 52, True),
    (1, 4, 4, 900, 96, 90, False),
    (1, 8, 2, 700, 96, 70, False),
    (1, 4, 4, 600, 160, 60, True),
    (1, 8, 2, 500, 160, 50, False),
    (1, 4, 2, 400, 192, 40, False),
    (1, 2, 2, 350, 224, 35, False),
    (1, 8, 4, 333, 224, 34, True),
    # contexts beyond the 8192-key sample: the selection ranks a window found
    # from a sample of the keys (ties can overflow it: whole-head select)
    (1, 4, 2, 20000, 128, 2000, True),
    (1, 8, 2, 40000, 128, 4000, False),
    (2, 4, 4, 12000, 64, 1, False),
    (1, 2, 2, 9000, 256, 8999, False),
    # groups of 8 heads at long context (the selection's 8-head instances over
    # many key chunks), with and without ties
    (2, 16, 2, 40000, 128, 4000, False),
    (1, 16, 2, 20000, 64, 2000, True),
]


@pytest.mark.parametrize("case", CASES, ids=[str(c) for c in CASES])
def test_adaptive_sets_and_output(F, case):
    B, Hq, Hkv, S, d, k, ties = case
    say(f"case adaptive {case}")
    q, kx, vx = make(B, Hq, Hkv, S, d, seed=S + k, ties=ties)
    kb, kr = F.encode_fused(torch.from_numpy(kx.reshape(-1, d)).cuda())
    vb, vr = F.encode_fused(torch.from_numpy(vx.reshape(-1, d)).cuda())
    out, sel = F.adaptive_attention(torch.from_numpy(q).cuda(), kb, kr, vb, vr, B, Hq, S, d,
                                    n_kv_heads=Hkv, top_k=k, return_selected=True)
    n = B * Hkv * S
    Kb, Kr = bin_from_blob(kb, n, d), res_from_blob(kr, n, d)
    Vb, Vr = bin_from_blob(vb, n, d), res_from_blob(vr, n, d)
    _, ref, sets = O.adaptive_attention(q, Kb, Kr, Vb, Vr, B, Hq, S, k, n_kv_heads=Hkv,
                                        return_f32=True, return_sets=True)
    sel = to_np(sel)
    for (b, h), idx in sets.items():
        got = np.nonzero(sel[b, h])[0]
        assert np.array_equal(got, idx), f"selected set differs at (b={b}, h={h})"
    close(to_np(out).astype(np.float32), ref, what=f"adaptive {case}")


def test_adaptive_limits(F):
    say("case adaptive limits")
    B, Hq, Hkv, S, d = 1, 4, 2, 700, 128
    q, kx, vx = make(B, Hq, Hkv, S, d, seed=5)
    kb, kr = F.encode_fused(torch.from_numpy(kx.reshape(-1, d)).cuda())
    vb, vr = F.encode_fused(torch.from_numpy(vx.reshape(-1, d)).cuda())
    qt = torch.from_numpy(q).cuda()
    a0, s0 = F.adaptive_attention(qt, kb, kr, vb, vr, B, Hq, S, d, n_kv_heads=Hkv, top_k=0,
                                  return_selected=True)
    aS, sS = F.adaptive_attention(qt, kb, kr, vb, vr, B, Hq, S, d, n_kv_heads=Hkv, top_k=S,
                                  return_selected=True)
    assert int(s0.sum()) == 0 and int(sS.sum()) == B * Hq * S
    b = F.binary_attention(qt, kb, vb, B, Hq, S, d, n_kv_heads=Hkv)
    c = F.compensated_attention(qt, kb, kr, vb, vr, B, Hq, S, d, n_kv_heads=Hkv)
    close(to_np(a0).astype(np.float32), to_np(b).astype(np.float32), rel=1e-3, what="k=0")
    close(to_np(aS).astype(np.float32), to_np(c).astype(np.float32), rel=1e-3, what="k=S")


@pytest.mark.parametrize("S,k", [(10000, 1000), (3000, 300)])
def test_adaptive_all_keys_tied(F, S, k):
    """Every key of a head equal: one score, so the k keys of lowest index are
    taken.  The whole head is one bucket (more keys than the final select
    holds in LDS at S = 10000, so it re-reads the bucket lists each round) and
    more than 512 keys tie, so the cutoff comes from a radix select on the
    index."""
    say(f"case adaptive all tied S={S}")
    B, Hq, Hkv, d = 1, 4, 2, 128
    q, kx, vx = make(B, Hq, Hkv, S, d, seed=21)
    kx[:] = kx[:, :, :1, :]
    kb, kr = F.encode_fused(torch.from_numpy(kx.reshape(-1, d)).cuda())
    vb, vr = F.encode_fused(torch.from_numpy(vx.reshape(-1, d)).cuda())
    _, sel = F.adaptive_attention(torch.from_numpy(q).cuda(), kb, kr, vb, vr, B, Hq, S, d,
                                  n_kv_heads=Hkv, top_k=k, return_selected=True)
    sel = to_np(sel)
    want = np.zeros(S, bool)
    want[:k] = True
    for h in range(Hq):
        assert np.array_equal(sel[0, h].astype(bool), want), f"head {h}"


def test_adaptive_large_bucket_few_ties(F):
    """One sign pattern for every key and per-key magnitudes within 3%: the
    scores of a head fall into one or two first-digit buckets (more keys than
    the final select holds in LDS) with a few hundred keys on each fp16 scale
    value, so the threshold's ties (fewer than 512) are ranked by comparison
    while the bucket is re-read from the lists.  The scenario is asserted on
    the oracle's keys, then the selected sets must be bit-exact."""
    say("case adaptive large bucket, few ties")
    B, Hq, Hkv, S, d, k = 1, 4, 1, 16000, 128, 5000
    rng = np.random.default_rng(1)
    sign = np.where(rng.standard_normal(d) >= 0, 1.0, -1.0)
    g = np.abs(rng.standard_normal(d)) + 0.5
    a = 1.0 + 0.03 * rng.random(S)
    kx = (a[:, None] * (sign * g)[None, :] * 0.05).astype(np.float16).reshape(B, Hkv, S, d)
    q = (rng.standard_normal((B, Hq, d)) * 0.1).astype(np.float16)
    vx = (rng.standard_normal((B, Hkv, S, d)) * 0.1).astype(np.float16)
    Kb, Kr = O.encode_fused(kx.reshape(-1, d))
    Vb, Vr = O.encode_fused(vx.reshape(-1, d))
    # the scenario, on the oracle's ranking keys of head 0
    pc = ((kx[0, 0] >= 0) == (q[0, 0] >= 0)).sum(1)
    key = O.topk_key(Kb.scale, pc, d)
    T = np.sort(key)[::-1][k - 1]
    u = T.astype(np.float32).view(np.uint32)
    ok = np.where(key.view(np.uint32) & 0x80000000, ~key.view(np.uint32), key.view(np.uint32) | 0x80000000)
    ot = (~u) if (u & 0x80000000) else (u | 0x80000000)
    in_bucket = int(((ok >> 19) == (ot >> 19)).sum())
    ties = int((key == T).sum())
    assert in_bucket > 6144 and 1 < ties <= 512, (in_bucket, ties)
    kb, kr = F.encode_fused(torch.from_numpy(kx.reshape(-1, d)).cuda())
    vb, vr = F.encode_fused(torch.from_numpy(vx.reshape(-1, d)).cuda())
    out, sel = F.adaptive_attention(torch.from_numpy(q).cuda(), kb, kr, vb, vr, B, Hq, S, d,
                                    n_kv_heads=Hkv, top_k=k, return_selected=True)
    _, ref, sets = O.adaptive_attention(q, Kb, Kr, Vb, Vr, B, Hq, S, k, n_kv_heads=Hkv,
                                        return_f32=True, return_sets=True)
    sel = to_np(sel)
    for (b, h), idx in sets.items():
        assert np.array_equal(np.nonzero(sel[b, h])[0], idx), f"set differs at {(b, h)}"
    close(to_np(out).astype(np.float32), ref, what="large bucket")


def test_config_c5_sample(F):
    """Config c5 shape on a shortened context (S = 16384, same generator and
    outlier channels): every selected set of two batches is bit-exact and the
    output matches the oracle."""
    from bitcache_amd import workloads as W
    say("case c5 sample")
    cfg = W.CONFIGS["c5"]
    S, d, Hq, Hkv = 16384, cfg.head_dim, cfg.n_heads, cfg.n_kv_heads
    q, k, v = W.make_qkv(cfg, seq_len=S)
    q, k, v = q[:2].contiguous(), k[:2].contiguous(), v[:2].contiguous()
    B = 2
    kb, kr = F.encode_fused(k.view(-1, d))
    vb, vr = F.encode_fused(v.view(-1, d))
    top_k = O.default_top_k(S)
    out, sel = F.adaptive_attention(q, kb, kr, vb, vr, B, Hq, S, d, n_kv_heads=Hkv, top_k=top_k,
                                    return_selected=True)
    n = B * Hkv * S
    Kb, Kr = bin_from_blob(kb, n, d), res_from_blob(kr, n, d)
    Vb, Vr = bin_from_blob(vb, n, d), res_from_blob(vr, n, d)
    _, ref, sets = O.adaptive_attention(to_np(q), Kb, Kr, Vb, Vr, B, Hq, S, top_k, n_kv_heads=Hkv,
                                        return_f32=True, return_sets=True)
    sel = to_np(sel)
    for (b, h), idx in sets.items():
        assert np.array_equal(np.nonzero(sel[b, h])[0], idx), f"set differs at {(b, h)}"
    close(to_np(out).astype(np.float32), ref, what="c5 sample")


def test_config_c5_full_size(F):
    """Config c5 at full size (B16, GQA 32/8, S = 131072, top 10%).  Every one of
    the 512 selected sets is checked against the definition of the top-k, a
    property that does not depend on S: exactly k keys; no unselected key ranks
    above a selected one; keys equal to the threshold are taken lowest index
    first.  The ranking key scale_k * (2pc - d) comes from the GPU independently
    of the kernels under test: 2pc - d = sign(k) . sign(q) is an exact +-1
    matmul in fp32 and the product with the fp16 scale is exact.  All 512
    heads' sets and outputs are compared with the torch-CPU restatement of the
    adaptive attention, and one head group with the numpy oracle from the fp16
    inputs."""
    from bitcache_amd import workloads as W
    say("case c5 full size")
    cfg = W.CONFIGS["c5"]
    B, Hq, Hkv, S, d = cfg.batch, cfg.n_heads, cfg.n_kv_heads, cfg.seq_len, cfg.head_dim
    G = Hq // Hkv
    q, k, v = W.make_qkv(cfg)
    kb, kr = F.encode_fused(k.view(-1, d))
    vb, vr = F.encode_fused(v.view(-1, d))
    top_k = O.default_top_k(S)
    out, sel = F.adaptive_attention(q, kb, kr, vb, vr, B, Hq, S, d, n_kv_heads=Hkv, top_k=top_k,
                                    return_selected=True)
    torch.cuda.synchronize()
    n = B * Hkv * S
    kscale = kb[n * d // 8:n * d // 8 + 2 * n].view(torch.float16).view(B, Hkv, S).float()
    idx = torch.arange(S, device=q.device)
    for b in range(B):
        sk = torch.where(k[b] >= 0, 1.0, -1.0)                                  # [Hkv, S, d]
        sq = torch.where(q[b] >= 0, 1.0, -1.0).view(Hkv, G, d).transpose(1, 2).contiguous()
        dots = torch.bmm(sk, sq)                                                # [Hkv, S, G]
        key = (kscale[b][..., None] * dots).permute(0, 2, 1).reshape(Hq, S)     # exact in fp32
        s = sel[b].bool()
        assert torch.equal(s.sum(-1), torch.full((Hq,), top_k, device=q.device)), f"set sizes, b={b}"
        lo_sel = torch.where(s, key, torch.inf).amin(-1)
        hi_uns = torch.where(~s, key, -torch.inf).amax(-1)
        assert bool((lo_sel >= hi_uns).all()), f"an unselected key ranks above a selected one, b={b}"
        tie = lo_sel == hi_uns
        last_sel = torch.where(s & (key == lo_sel[:, None]), idx, -1).amax(-1)
        first_uns = torch.where(~s & (key == lo_sel[:, None]), idx, S).amin(-1)
        assert bool((last_sel < first_uns)[tie].all()), f"ties not taken lowest index first, b={b}"
    # one head group against the numpy oracle from the fp16 inputs (its own
    # encode, selection and attention)
    b, kvh = 15, 7
    Kb, Kr = O.encode_fused(to_np(k[b, kvh]))
    Vb, Vr = O.encode_fused(to_np(v[b, kvh]))
    qg = to_np(q[b, kvh * G:(kvh + 1) * G])[None]
    _, ref, sets = O.adaptive_attention(qg, Kb, Kr, Vb, Vr, 1, G, S, top_k, n_kv_heads=1,
                                        return_f32=True, return_sets=True)
    for (_, h), want in sets.items():
        got = np.nonzero(to_np(sel[b, kvh * G + h]))[0]
        assert np.array_equal(got, want), f"set differs at (b={b}, h={kvh * G + h})"
    close(to_np(out[b, kvh * G:(kvh + 1) * G]).astype(np.float32), ref[0],
          what=f"c5 full size group {(b, kvh)}")
    del k, v
    # every one of the 512 heads against the torch-CPU restatement of the
    # adaptive attention on the same device blobs: the selected set bit for
    # bit, the output within 2e-3 max-abs relative error, cosine >= 0.9999
    torch.set_num_threads(min(16, len(__import__("os").sched_getaffinity(0))))
    kbc, krc, vbc, vrc, qc = kb.cpu(), kr.cpu(), vb.cpu(), vr.cpu(), q.cpu()
    selc = sel.cpu().bool()
    got = to_np(out).astype(np.float32)
    ref = np.empty((B, Hq, d), np.float32)
    for b in range(B):
        for kvh in range(Hkv):
            args = blob_head_tensors(kbc, krc, vbc, vrc, n, d, (b * Hkv + kvh) * S, S)
            o, s = O.adaptive_attention_torch_cpu(qc[b, kvh * G:(kvh + 1) * G], *args, top_k)
            assert torch.equal(s, selc[b, kvh * G:(kvh + 1) * G]), f"set differs in group {(b, kvh)}"
            ref[b, kvh * G:(kvh + 1) * G] = o.float().numpy()
        say(f"  c5 batch {b}: sets and outputs checked")
    close(got, ref, what="c5 all heads")
    cosh = (got * ref).sum(-1) / (np.linalg.norm(got, axis=-1) * np.linalg.norm(ref, axis=-1))
    say(f"c5 all 512 heads vs torch-CPU restatement: min cosine {cosh.min():.7f}")
    assert cosh.min() >= 0.9999
    del q, kb, kr, vb, vr, out, sel
    torch.cuda.empty_cache()


def test_adaptive_special_scales(F):
    """Selected sets with planted K scales: +-inf, NaN, +-0, negative, the
    fp16 maximum and a subnormal.  Waves holding a non-finite scale rank by the
    exact key, the others by exact float scores; both must give the oracle's
    order (NaN below every key, -0 as +0, ties lowest index first).  Only the
    sets are compared: non-finite scales make the outputs non-finite."""
    say("case adaptive special scales")
    B, Hq, Hkv, S, d, k = 1, 8, 2, 2048, 128, 300
    q, kx, vx = make(B, Hq, Hkv, S, d, seed=11)
    kb, kr = F.encode_fused(torch.from_numpy(kx.reshape(-1, d)).cuda())
    vb, vr = F.encode_fused(torch.from_numpy(vx.reshape(-1, d)).cuda())
    n = B * Hkv * S
    scales = kb[n * d // 8:n * d // 8 + 2 * n].view(torch.float16)
    rng = np.random.default_rng(12)
    special = [np.inf, -np.inf, np.nan, 0.0, -0.0, -0.05, 65504.0, 6e-8, 0.5, 0.5]
    pos = rng.choice(n, size=60, replace=False)
    vals = torch.tensor([special[i % len(special)] for i in range(len(pos))], dtype=torch.float16)
    scales[torch.from_numpy(pos).cuda()] = vals.cuda()
    torch.cuda.synchronize()
    out, sel = F.adaptive_attention(torch.from_numpy(q).cuda(), kb, kr, vb, vr, B, Hq, S, d,
                                    n_kv_heads=Hkv, top_k=k, return_selected=True)
    Kb, Kr = bin_from_blob(kb, n, d), res_from_blob(kr, n, d)
    Vb, Vr = bin_from_blob(vb, n, d), res_from_blob(vr, n, d)
    with np.errstate(all="ignore"):
        _, _, sets = O.adaptive_attention(q, Kb, Kr, Vb, Vr, B, Hq, S, k, n_kv_heads=Hkv,
                                          return_f32=True, return_sets=True)
    sel = to_np(sel)
    for (b, h), idx in sets.items():
        assert np.array_equal(np.nonzero(sel[b, h])[0], idx), f"set differs at {(b, h)}"
