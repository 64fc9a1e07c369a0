"""GPU parity of the attention path against the oracle: exact popcounts and
binary scores, compensated / binary attention within 2e-3 max-abs relative
error and cosine >= 0.9999, GQA, ring strides, edge sizes, entropy and the
fp16 reference kernel; plus full-size checks at configs c1, c2 and c3."""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.gpu_util import (assert_same_bin, assert_same_res, bin_from_blob, bin_head_tensors,
                            blob_head_tensors, close, res_from_blob, say, slice_enc, to_np)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def F():
    import bitcache_amd.functional as F
    return F


def make(B, Hq, Hkv, S, d, seed, scale=0.09, lognorm=0.0):
    rng = np.random.default_rng(seed)
    q = (rng.standard_normal((B, Hq, d)) * scale).astype(np.float16)
    k = rng.standard_normal((B, Hkv, S, d)) * scale
    v = rng.standard_normal((B, Hkv, S, d)) * scale
    if lognorm:
        k = k * np.exp(rng.standard_normal((B, Hkv, S, 1)) * lognorm)
        v = v * np.exp(rng.standard_normal((B, Hkv, S, 1)) * lognorm)
    return q, k.astype(np.float16), v.astype(np.float16)


def encode_gpu(F, x):
    xt = torch.from_numpy(np.ascontiguousarray(x.reshape(-1, x.shape[-1]))).cuda()
    return F.encode_fused(xt)


SHAPES = [
    # (B, Hq, Hkv, S, d)
    (1, 32, 32, 4096, 128),   # config c1 shape
    (2, 4, 4, 1, 128),
    (1, 2, 2, 63, 64),
    (1, 2, 2, 65, 32),
    (2, 8, 2, 1000, 128),     # GQA 4
    (1, 8, 1, 513, 128),      # GQA 8
    (1, 6, 2, 300, 128),      # GQA 3 (query heads processed one by one)
    (1, 4, 2, 700, 128),      # GQA 2 (int8-MFMA residual dots)
    (2, 4, 2, 333, 64),       # GQA 2 at d = 64 (binary: int8 value path, two heads)
    (1, 4, 2, 301, 256),      # GQA 2 at d = 256
    (2, 8, 2, 333, 64),       # GQA 4 at d = 64 (lane-piece residual dots)
    (1, 8, 2, 500, 256),      # GQA 4 at d = 256 (two code pieces per lane)
    (1, 16, 2, 300, 256),     # GQA 8 at d = 256
    (1, 4, 4, 777, 256),
    (1, 2, 2, 300, 96),
    (1, 3, 3, 2000, 160),
    (1, 2, 2, 129, 192),
    (1, 2, 2, 200, 224),
]


@pytest.mark.parametrize("shape", SHAPES, ids=[str(s) for s in SHAPES])
def test_compensated_and_binary_vs_oracle(F, shape):
    B, Hq, Hkv, S, d = shape
    say(f"case attention {shape}")
    q, k, v = make(B, Hq, Hkv, S, d, seed=S + d, lognorm=0.25)
    kb, kr = encode_gpu(F, k)
    vb, vr = encode_gpu(F, v)
    qt = torch.from_numpy(q).cuda()
    kw = dict(n_kv_heads=Hkv) if Hkv != Hq else {}
    out = F.compensated_attention(qt, kb, kr, vb, vr, B, Hq, S, d, **kw)
    outb = F.binary_attention(qt, kb, vb, B, Hq, S, d, **kw)
    n = B * Hkv * S
    Kb, Kr = bin_from_blob(kb, n, d), res_from_blob(kr, n, d)
    Vb, Vr = bin_from_blob(vb, n, d), res_from_blob(vr, n, d)
    _, ref = O.compensated_attention(q, Kb, Kr, Vb, Vr, B, Hq, S, n_kv_heads=Hkv, return_f32=True)
    _, refb = O.binary_attention(q, Kb, Vb, B, Hq, S, n_kv_heads=Hkv, return_f32=True)
    close(to_np(out).astype(np.float32), ref, what=f"compensated {shape}")
    close(to_np(outb).astype(np.float32), refb, what=f"binary {shape}")


# launches with more (b, head group) workgroups than a round of resident
# workgroups holds (one split each, several rounds), and the split-phase API
LAUNCH_SHAPES = [
    (48, 32, 32, 300, 128),    # 1536 MHA groups
    (64, 32, 8, 520, 128),     # 512 GQA-4 groups, 520 keys
    (24, 64, 8, 200, 64),      # GQA 8 at d = 64, ragged last tile
]


@pytest.mark.parametrize("shape", LAUNCH_SHAPES, ids=[str(s) for s in LAUNCH_SHAPES])
def test_many_groups_and_split_phase_api(F, shape):
    """Full attention calls and the split-phase pair (partials, then combine;
    a fixed split plan for either mode) against the oracle."""
    from bitcache_amd import _C
    B, Hq, Hkv, S, d = shape
    say(f"case launch {shape}")
    q, k, v = make(B, Hq, Hkv, S, d, seed=S + B, lognorm=0.25)
    kb, kr = encode_gpu(F, k)
    vb, vr = encode_gpu(F, v)
    qt = torch.from_numpy(q).cuda()
    n = B * Hkv * S
    Kb, Kr = bin_from_blob(kb, n, d), res_from_blob(kr, n, d)
    Vb, Vr = bin_from_blob(vb, n, d), res_from_blob(vr, n, d)
    _, ref = O.compensated_attention(q, Kb, Kr, Vb, Vr, B, Hq, S, n_kv_heads=Hkv, return_f32=True)
    _, refb = O.binary_attention(q, Kb, Vb, B, Hq, S, n_kv_heads=Hkv, return_f32=True)
    out = F.compensated_attention(qt, kb, kr, vb, vr, B, Hq, S, d, n_kv_heads=Hkv)
    outb = F.binary_attention(qt, kb, vb, B, Hq, S, d, n_kv_heads=Hkv)
    close(to_np(out).astype(np.float32), ref, what=f"compensated {shape}")
    close(to_np(outb).astype(np.float32), refb, what=f"binary {shape}")
    ws = _C.attention_partial(qt, kb, kr, vb, vr, B, Hq, Hkv, S, S, d)
    outp = _C.attention_combine(ws, B, Hq, Hkv, S, d)
    wsb = _C.attention_partial(qt, kb, None, vb, None, B, Hq, Hkv, S, S, d)
    outpb = _C.attention_combine(wsb, B, Hq, Hkv, S, d)
    close(to_np(outp).astype(np.float32), ref, what=f"split-phase compensated {shape}")
    close(to_np(outpb).astype(np.float32), refb, what=f"split-phase binary {shape}")
    if shape == LAUNCH_SHAPES[0]:
        # 1536 MHA groups fill a round with one split each, in both plans: the
        # full call writes the output from the split kernel (no merge launch),
        # bit for bit what the merge of the single partial gives.  (Binary
        # attention with exactly one head per CU runs one 8-wave workgroup per
        # head instead; test_config_c2_full_size_scores covers it.)
        assert torch.equal(out, outp) and torch.equal(outb, outpb)


def make_rising(B, Hq, Hkv, S, d, seed):
    """Keys and values that move a wave's running softmax reference and its
    weight plan mid-stream while the keys before each move still carry a
    visible share of the output.  Every key sits at score level 0 except,
    in the second half, one key in 32 at level 1 (about 5.7 above, in log2
    units) and, in the last quarter, one in 2048 at level 2.  V magnitudes
    cycle x1, x2, x4, x8 over consecutive 256-key runs, so the tiles that one
    wave takes (256 keys apart) raise the largest value scale at a power of
    two up to three times."""
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, Hq, d)).astype(np.float16)
    s = np.arange(S)
    level = np.zeros(S, np.int64)
    level[(s >= S // 2) & (s % 32 == 0)] = 1
    level[(s >= 3 * S // 4) & (s % 2048 == 7)] = 2
    kmag = np.array([0.1, 0.9, 1.7])[level]
    # keys agree in sign with their group's first query head on ~75% of dims
    qh = q.reshape(B, Hkv, Hq // Hkv, d)[:, :, 0].astype(np.float32)
    agree = rng.random((B, Hkv, S, d)) < 0.75
    sgn = np.where(agree, np.sign(qh + 1e-30)[:, :, None, :], rng.choice([-1.0, 1.0], size=(B, Hkv, S, d)))
    k = np.abs(rng.standard_normal((B, Hkv, S, d))) * sgn * kmag[None, None, :, None]
    vmag = 0.09 * 2.0 ** ((s // 256) % 4)
    v = rng.standard_normal((B, Hkv, S, d)) * vmag[None, None, :, None]
    return q, k.astype(np.float16), v.astype(np.float16)


@pytest.mark.parametrize("shape", [(2, 16, 16, 8192, 128), (2, 16, 4, 8192, 64), (1, 16, 4, 8192, 256)],
                         ids=lambda s: str(s))
def test_rising_scores_and_value_scales(F, shape):
    """Binary, compensated and adaptive (top 10%) attention against the
    oracle on make_rising data: the rescales of a wave's partial sums (a score past the running
    reference plus its headroom, a value scale past the weight plan) happen
    mid-stream, between tiles whose keys all contribute."""
    B, Hq, Hkv, S, d = shape
    say(f"case rising {shape}")
    q, k, v = make_rising(B, Hq, Hkv, S, d, seed=11 + d)
    kb, kr = encode_gpu(F, k)
    vb, vr = encode_gpu(F, v)
    qt = torch.from_numpy(q).cuda()
    kw = dict(n_kv_heads=Hkv) if Hkv != Hq else {}
    outb = F.binary_attention(qt, kb, vb, B, Hq, S, d, **kw)
    out = F.compensated_attention(qt, kb, kr, vb, vr, B, Hq, S, d, **kw)
    n = B * Hkv * S
    Kb, Kr = bin_from_blob(kb, n, d), res_from_blob(kr, n, d)
    Vb, Vr = bin_from_blob(vb, n, d), res_from_blob(vr, n, d)
    _, refb = O.binary_attention(q, Kb, Vb, B, Hq, S, n_kv_heads=Hkv, return_f32=True)
    _, ref = O.compensated_attention(q, Kb, Kr, Vb, Vr, B, Hq, S, n_kv_heads=Hkv, return_f32=True)
    close(to_np(outb).astype(np.float32), refb, what=f"binary {shape}")
    close(to_np(out).astype(np.float32), ref, what=f"compensated {shape}")
    top_k = S // 10
    outa, sel = F.adaptive_attention(qt, kb, kr, vb, vr, B, Hq, S, d, n_kv_heads=Hkv, top_k=top_k,
                                     return_selected=True)
    _, refa, sets = O.adaptive_attention(q, Kb, Kr, Vb, Vr, B, Hq, S, top_k, n_kv_heads=Hkv,
                                         return_f32=True, return_sets=True)
    sel = to_np(sel)
    for (b, h), idx in sets.items():
        assert np.array_equal(np.nonzero(sel[b, h])[0], idx), f"selected set differs at (b={b}, h={h})"
    close(to_np(outa).astype(np.float32), refa, what=f"adaptive {shape}")


@pytest.mark.parametrize("H,Hkv,d", [(4, 4, 128), (8, 2, 128), (8, 2, 256)])
def test_kv_stride_and_zero_length(F, H, Hkv, d):
    say(f"case kv_stride H={H} Hkv={Hkv} d={d}")
    B, S, stride = 2, 100, 160
    q, k, v = make(B, H, Hkv, stride, d, seed=3)
    kb, kr = encode_gpu(F, k)
    vb, vr = encode_gpu(F, v)
    qt = torch.from_numpy(q).cuda()
    out = F.compensated_attention(qt, kb, kr, vb, vr, B, H, S, d, kv_stride=stride, n_kv_heads=Hkv)
    # oracle on the first S positions of every (b, kv head)
    ks, vs = k[:, :, :S], v[:, :, :S]
    Kb, Kr = O.encode_fused(ks.reshape(-1, d))
    Vb, Vr = O.encode_fused(vs.reshape(-1, d))
    _, ref = O.compensated_attention(q, Kb, Kr, Vb, Vr, B, H, S, n_kv_heads=Hkv, return_f32=True)
    close(to_np(out).astype(np.float32), ref, what="stride")
    z = F.compensated_attention(qt, kb, kr, vb, vr, B, H, 0, d, kv_stride=stride, n_kv_heads=Hkv)
    assert torch.count_nonzero(z) == 0


@pytest.mark.parametrize("S", [(1 << 20) - 37, 1 << 21])
def test_long_context_heads(F, S):
    """One- and two-million-key heads (the split plan at its 2048-split cap, the
    merge kernel's largest weight table, 32-bit buffer offsets per split, a
    ragged last tile): compensated and binary attention against the torch-CPU
    restatements at the fp bar."""
    say(f"case long context S={S}")
    B, H, d = 1, 2, 128
    g = torch.Generator(device="cuda")
    g.manual_seed(S % 9973)
    q = (torch.randn((B, H, d), generator=g, device="cuda") * 0.2).half()
    k = (torch.randn((B * H * S, d), generator=g, device="cuda") * 0.2).half()
    kb, kr = F.encode_fused(k)
    del k
    v = (torch.randn((B * H * S, d), generator=g, device="cuda") * 0.2).half()
    vb, vr = F.encode_fused(v)
    del v
    comp = to_np(F.compensated_attention(q, kb, kr, vb, vr, B, H, S, d)).astype(np.float32)
    binr = to_np(F.binary_attention(q, kb, vb, B, H, S, d)).astype(np.float32)
    torch.set_num_threads(min(16, len(__import__("os").sched_getaffinity(0))))
    n = B * H * S
    kbc, krc, vbc, vrc, qc = kb.cpu(), kr.cpu(), vb.cpu(), vr.cpu(), q.cpu()
    del kb, kr, vb, vr
    rc = np.empty((B, H, d), np.float32)
    rb = np.empty((B, H, d), np.float32)
    for h in range(H):
        args = blob_head_tensors(kbc, krc, vbc, vrc, n, d, h * S, S)
        rc[0, h] = O.compensated_attention_torch_cpu(qc[0, h], *args).float().numpy()
        rb[0, h] = O.binary_attention_torch_cpu(qc[0, h][None], args[0], args[1], args[4],
                                                args[5])[0].float().numpy()
    close(comp, rc, what=f"compensated S={S}")
    close(binr, rb, what=f"binary S={S}")
    torch.cuda.empty_cache()


# (B, Hq, Hkv, S): MHA, GQA, and a group of 32 heads (two head batches per workgroup row)
@pytest.mark.parametrize("shape", [(2, 8, 8, 1500), (2, 8, 2, 1500), (1, 32, 1, 700)])
def test_binary_scores_exact(F, shape):
    say(f"case binary_scores {shape}")
    B, Hq, Hkv, S = shape
    d = 128
    q, k, _ = make(B, Hq, Hkv, S, d, seed=11)
    kb = F.encode(torch.from_numpy(k.reshape(-1, d)).cuda())
    sc, pc = F.binary_scores(torch.from_numpy(q).cuda(), kb, B, Hq, S, d, n_kv_heads=Hkv)
    Kb = bin_from_blob(kb, B * Hkv * S, d)
    esc = O.binary_scores(q, Kb, B, Hq, S, n_kv_heads=Hkv)
    epc = O.binary_popcounts(q, Kb, B, Hq, S, n_kv_heads=Hkv)
    assert np.array_equal(to_np(pc), epc)
    assert np.array_equal(to_np(sc).view(np.uint32), esc.view(np.uint32))


def test_entropy_vs_oracle(F):
    say("case entropy")
    B, H, S, d = 2, 4, 3000, 128
    q, k, _ = make(B, H, H, S, d, seed=13, scale=0.3)
    kb = F.encode(torch.from_numpy(k.reshape(-1, d)).cuda())
    ent = to_np(F.compute_head_entropy(torch.from_numpy(q).cuda(), kb, B, H, S, d))
    Kb = bin_from_blob(kb, B * H * S, d)
    ref = O.head_entropy(q, Kb, B, H, S)
    np.testing.assert_allclose(ent, ref, rtol=2e-4, atol=2e-4)
    modes = to_np(F.adaptive_select(torch.from_numpy(ent).cuda(), float(np.median(ent))))
    assert np.array_equal(modes, (ent < np.median(ent)).astype(np.uint8))


@pytest.mark.parametrize("B,Hq,Hkv,S,stride,d", [(1, 4, 4, 40000, 40000, 128), (2, 8, 2, 30001, 30001, 64),
                                                 (1, 2, 2, 17000, 17000, 256), (1, 4, 1, 9000, 9000, 96),
                                                 (2, 4, 2, 20000, 23456, 128)])
def test_entropy_key_split_vs_oracle_and_single_block(F, B, Hq, Hkv, S, stride, d):
    """The key-split entropy pass (several blocks per head, partials merged by a
    second launch; what the operator module runs when a head's keys span more
    than one chunk) against the oracle, and against the single-block kernel of
    the reference-signature C entry point to fp32 rounding; GQA groups and a
    ring stride past the filled keys included."""
    import ctypes
    import os
    say(f"case entropy split B={B} Hq={Hq} Hkv={Hkv} S={S} stride={stride} d={d}")
    q, k, _ = make(B, Hq, Hkv, stride, d, seed=S % 1000, scale=0.3)
    kb = F.encode(torch.from_numpy(k.reshape(-1, d)).cuda())
    qt = torch.from_numpy(q).cuda()
    k = np.ascontiguousarray(k[:, :, :S])
    L = ctypes.CDLL(os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                                 "bitcache_amd", "libbitcache_hip.so"))
    n = ctypes.c_size_t(0)
    L.bc_entropy_workspace_size.argtypes = [ctypes.c_int] * 3 + [ctypes.POINTER(ctypes.c_size_t)]
    assert L.bc_entropy_workspace_size(B, Hq, S, ctypes.byref(n)) == 0
    assert n.value > 0, "this shape should take the key-split pass"
    ent = to_np(F.compute_head_entropy(qt, kb, B, Hq, S, d, n_kv_heads=Hkv, kv_stride=stride))
    Kb = O.binary_encode(k.reshape(-1, d))
    ref = O.head_entropy(q, Kb, B, Hq, S, n_kv_heads=Hkv)
    np.testing.assert_allclose(ent, ref, rtol=2e-4, atol=2e-4)
    one = torch.empty((B, Hq), dtype=torch.float32, device="cuda")
    P = ctypes.c_void_p
    L.bc_compute_head_entropy_gqa.argtypes = [P, P, P] + [ctypes.c_int] * 6 + [P]
    assert L.bc_compute_head_entropy_gqa(P(qt.data_ptr()), P(kb.data_ptr()), P(one.data_ptr()), B, Hq,
                                         Hkv, S, stride, d, P(torch.cuda.current_stream().cuda_stream)) == 0
    torch.cuda.synchronize()
    np.testing.assert_allclose(ent, to_np(one), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("shape", [(1, 4, 4, 1000, 128), (2, 8, 2, 777, 64), (1, 2, 2, 64, 256),
                                   # head dims whose rows do not fill a power-of-two lane slot
                                   (1, 4, 2, 500, 32), (1, 4, 4, 333, 96), (1, 2, 2, 300, 160),
                                   (1, 4, 2, 257, 192), (1, 8, 2, 200, 224)])
def test_reference_attention_vs_oracle(F, shape):
    B, Hq, Hkv, S, d = shape
    say(f"case reference_attention {shape}")
    q, k, v = make(B, Hq, Hkv, S, d, seed=17, scale=0.3)
    out = F.reference_attention(torch.from_numpy(q).cuda(), torch.from_numpy(k).cuda(),
                                torch.from_numpy(v).cuda(), B, Hq, S, d, n_kv_heads=Hkv)
    _, ref = O.reference_attention(q, k, v, B, Hq, S, n_kv_heads=Hkv, return_f32=True)
    close(to_np(out).astype(np.float32), ref, what="reference")


def test_config_c2_full_size_scores(F):
    """Config c2 at full size: all 8.4M popcounts equal 2*pc-d == sign(q).sign(k)
    (exact +-1 matmul on the GPU); two heads bit-exact against the oracle, and
    Kendall tau of binary vs exact scores reported."""
    from bitcache_amd import workloads as W
    cfg = W.CONFIGS["c2"]
    say("case c2 full size")
    B, H, S, d = cfg.batch, cfg.n_heads, cfg.seq_len, cfg.head_dim
    q, k, mask = W.make_c2(cfg)
    kb = F.encode(k.view(-1, d))
    sc, pc = F.binary_scores(q, kb, B, H, S, d)
    sq = torch.where(q.float() >= 0, 1.0, -1.0)
    sk = torch.where(k.float() >= 0, 1.0, -1.0)
    dots = (sk @ sq[..., None]).squeeze(-1)
    assert torch.equal((2 * pc - d).float(), dots)
    Kb = bin_from_blob(kb, B * H * S, d)
    for (b, h) in [(0, 0), (7, 31)]:
        Kh = slice_enc(Kb, (b * H + h) * S, (b * H + h + 1) * S)
        qh = to_np(q[b, h])[None, None]
        esc = O.binary_scores(qh, Kh, 1, 1, S)
        assert np.array_equal(to_np(sc[b, h]).view(np.uint32), esc[0, 0].view(np.uint32))
    # Kendall tau-a (the reference's statistic, tests/test_correctness.cu:58-71)
    # and tau-b of the binary scores against exact q.k over all 256 heads
    # (reported; the README's "> 0.95" is not a gate)
    exact = torch.matmul(k.float(), q.float().unsqueeze(-1)).squeeze(-1).cpu().numpy()
    scn = to_np(sc)
    taus = np.array([W.kendall_tau_ab(scn[b, h], exact[b, h]) for b in range(B) for h in range(H)])
    say(f"c2 Kendall tau over {len(taus)} heads: tau-a mean {taus[:, 0].mean():.4f} "
        f"min {taus[:, 0].min():.4f}; tau-b mean {taus[:, 1].mean():.4f} min {taus[:, 1].min():.4f}")
    assert taus[:, 1].min() > 0.2 and np.all(taus[:, 0] <= taus[:, 1] + 1e-12)
    del sq, sk, dots, exact
    # binary attention on c2's inputs (the correlated-key softmax regime), all
    # 256 heads against the torch-CPU restatement of the reference's binary
    # attention (src/binary_attention.cu:8-82) on the same device blobs
    v = W.make_c2_values(cfg)
    vb = F.encode(v.view(-1, d))
    out = F.binary_attention(q, kb, vb, B, H, S, d)
    torch.cuda.synchronize()
    torch.set_num_threads(min(16, len(__import__("os").sched_getaffinity(0))))
    n = B * H * S
    kbc, vbc, qc = kb.cpu(), vb.cpu(), q.cpu()
    ref = np.empty((B, H, d), np.float32)
    for b in range(B):
        for h in range(H):
            kw, ks = bin_head_tensors(kbc, n, d, (b * H + h) * S, S)
            vw, vs = bin_head_tensors(vbc, n, d, (b * H + h) * S, S)
            ref[b, h] = O.binary_attention_torch_cpu(qc[b, h][None], kw, ks, vw, vs)[0].float().numpy()
    got = to_np(out).astype(np.float32)
    close(got, ref, what="c2 binary attention, all heads")
    cosh = (got * ref).sum(-1) / (np.linalg.norm(got, axis=-1) * np.linalg.norm(ref, axis=-1))
    say(f"c2 binary attention, all 256 heads vs torch-CPU restatement: min cosine {cosh.min():.7f}")
    assert cosh.min() >= 0.9999


@pytest.mark.parametrize("d", [64, 128, 256])
def test_wide_binary_longest_context(F, d):
    """Binary MHA attention with one head per CU runs one 8-wave workgroup per
    head (no split partials, no merge launch) at every matrix-core head dim;
    at the longest context that plan takes (131072 keys: 16384 keys, 256
    tiles, per wave) 16 heads spread over the batch agree with the torch-CPU
    restatement of the reference's binary attention
    (src/binary_attention.cu:8-82).  Keys equal to 2q sit at 200 positions of
    the last quarter, so each wave's running softmax reference moves after
    thousands of keys and those keys carry most of the weight."""
    import ctypes
    import os
    cu = torch.cuda.get_device_properties(0).multi_processor_count
    if cu % 32:
        pytest.skip(f"{cu} CUs: no batch of 32-head sequences gives one head per CU")
    B, H, S = cu // 32, 32, 131072
    lib = ctypes.CDLL(os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                                   "bitcache_amd", "libbitcache_hip.so"))
    ns, pb, wb = ctypes.c_int(0), ctypes.c_size_t(0), ctypes.c_size_t(0)
    assert lib.bc_attention_split_plan(0, B, H, H, S, d, 0, ctypes.byref(ns), ctypes.byref(pb),
                                       ctypes.byref(wb)) == 0
    assert ns.value == 1, "binary MHA with one head per CU plans one wide workgroup per head"
    say(f"case wide binary B={B} H={H} S={S} d={d}")
    g = torch.Generator(device="cuda")
    g.manual_seed(131)
    q = (torch.randn((B, H, d), generator=g, device="cuda") * 0.1).half()
    k = (torch.randn((B, H, S, d), generator=g, device="cuda") * 0.1).half()
    late = torch.arange(200, device="cuda") * 97 + 3 * S // 4
    k[:, :, late, :] = (2.0 * q.float()).half()[:, :, None, :]
    kb = F.encode(k.view(-1, d))
    del k
    v = (torch.randn((B * H * S, d), generator=g, device="cuda") * 0.1).half()
    vb = F.encode(v)
    del v
    out = F.binary_attention(q, kb, vb, B, H, S, d)
    torch.cuda.synchronize()
    torch.set_num_threads(min(16, len(os.sched_getaffinity(0))))
    n = B * H * S
    heads = [(b, h) for b in range(B) for h in (0, 31)]
    got = np.stack([to_np(out[b, h]).astype(np.float32) for (b, h) in heads])
    ref = np.empty_like(got)
    qc = q.cpu()
    for i, (b, h) in enumerate(heads):
        kw, ks = bin_head_tensors(kb, n, d, (b * H + h) * S, S)
        vw, vs = bin_head_tensors(vb, n, d, (b * H + h) * S, S)
        ref[i] = O.binary_attention_torch_cpu(qc[b, h][None], kw, ks, vw, vs)[0].float().numpy()
    close(got, ref, what=f"wide binary attention, 131072 keys, d = {d}")


def test_fp32_order_kats(F):
    """Hand-derived known answers on the GPU (derivations in
    tests/test_oracle.py): the encode scale's 128-lane tree order (d = 128:
    fp16 0x2001; d = 64: 0x2401; a sequential sum gives 0x2000 / 0x2400), the
    sequential scale_q (score = inv_sqrt(128) exactly = 0x3DB504F3; the tree
    order or a reversed sum move it), and the association
    (scale_q*scale_k)*(2pc-d) of the binary score (0x3F07E5AA; the other
    association gives 0x3F07E5AB)."""
    say("case fp32 order KATs")
    for d, want in ((128, 0x2001), (64, 0x2401)):
        x = np.array([[1.0, 2.0 ** -11] + [2.0 ** -24] * (d - 2)] * 3, np.float16)
        x[1] *= -1
        kb = F.encode(torch.from_numpy(x).cuda())
        got = bin_from_blob(kb, 3, d).scale.view(np.uint16)
        assert list(got) == [want] * 3, (d, [hex(g) for g in got])
    c = 1 + 2.0 ** -10
    q = np.array([[[1.0] + [2.0 ** -24] * 127], [[127.0, 1.0, 3 * 2.0 ** -16] + [0.0] * 125]],
                 np.float16)                                    # [B=2, H=1, 128]
    k = np.array([[1.0] * 128, [c] * 67 + [-c] * 61], np.float16)   # one key per batch
    kb = F.encode(torch.from_numpy(k).cuda())
    sc, pc = F.binary_scores(torch.from_numpy(q).cuda(), kb, 2, 1, 1, 128)
    assert list(to_np(pc).reshape(-1)) == [128, 67]
    assert [hex(v) for v in to_np(sc).reshape(-1).view(np.uint32)] == ["0x3db504f3", "0x3f07e5aa"]


def test_config_c3_full_size(F):
    """Config c3 at full size (B8 H32 S65536): every one of the 256 (b, h)
    heads against the torch-CPU restatement of the reference algorithm on the
    same device blobs, within the parity bar (max-abs error relative to
    max |ref| <= 2e-3 over the step, cosine >= 0.9999 per head); the encoded
    bytes of two heads against the oracle's encoders; and every head against
    the exact fp16 attention as a quality report."""
    from bitcache_amd import workloads as W
    cfg = W.CONFIGS["c3"]
    say("case c3 full size")
    B, H, S, d = cfg.batch, cfg.n_heads, cfg.seq_len, cfg.head_dim
    q, k, v = W.make_qkv(cfg)
    kb, kr = F.encode_fused(k.view(-1, d))
    vb, vr = F.encode_fused(v.view(-1, d))
    out = F.compensated_attention(q, kb, kr, vb, vr, B, H, S, d)
    torch.cuda.synchronize()
    n = B * H * S
    for (b, h) in [(0, 0), (5, 17)]:
        lo = (b * H + h) * S
        Kb, Kr = O.encode_fused(to_np(k[b, h]))
        assert_same_bin(slice_enc(bin_from_blob(kb, n, d), lo, lo + S), Kb, f"c3 head {(b, h)}")
        assert_same_res(slice_enc(res_from_blob(kr, n, d), lo, lo + S), Kr, f"c3 head {(b, h)}")
    torch.set_num_threads(min(16, len(__import__("os").sched_getaffinity(0))))
    ref = np.empty((B, H, d), np.float32)
    got = to_np(out).astype(np.float32)
    qc = q.cpu()
    for b in range(B):
        for h in range(H):
            args = blob_head_tensors(kb, kr, vb, vr, n, d, (b * H + h) * S, S)
            ref[b, h] = O.compensated_attention_torch_cpu(qc[b, h], *args).float().numpy()
        say(f"  c3 batch {b}: heads checked")
    close(got, ref, what="c3 all heads")
    cosh = (got * ref).sum(-1) / (np.linalg.norm(got, axis=-1) * np.linalg.norm(ref, axis=-1))
    say(f"c3 all 256 heads vs torch-CPU restatement: min cosine {cosh.min():.7f}")
    assert cosh.min() >= 0.9999
    exact = F.reference_attention(q, k, v, B, H, S, d).float()
    cos = torch.nn.functional.cosine_similarity(out.float().view(-1, d), exact.view(-1, d), dim=1)
    say(f"c3 compensated vs exact fp16 attention: mean cos {cos.mean().item():.5f} "
        f"min {cos.min().item():.5f}")
    assert cos.mean().item() > 0.9


def test_config_c1(F):
    """Config c1 on its own inputs (W.make_qkv: B1 H32 S4096, N(0, 1/128),
    seed 0) through the reference's two-step path (encode, compute_residual,
    compensated_attention): bytes against the oracle's encoders, output
    against the oracle within 2e-3 / cosine 0.9999, and against fp16
    reference attention (the reference checks cosine and max-abs error
    there; reported, cosine gated at > 0.9)."""
    from bitcache_amd import workloads as W
    cfg = W.CONFIGS["c1"]
    say("case c1")
    B, H, S, d = cfg.batch, cfg.n_heads, cfg.seq_len, cfg.head_dim
    q, k, v = W.make_qkv(cfg)
    kf, vf = k.view(-1, d), v.view(-1, d)
    kb = F.encode(kf)
    kr = F.compute_residual(kf, kb)
    vb = F.encode(vf)
    vr = F.compute_residual(vf, vb)
    out = F.compensated_attention(q, kb, kr, vb, vr, B, H, S, d)
    n = B * H * S
    Kb, Kr = O.binary_encode(to_np(kf)), None
    Kr = O.residual_encode(to_np(kf), Kb)
    Vb = O.binary_encode(to_np(vf))
    Vr = O.residual_encode(to_np(vf), Vb)
    assert_same_bin(bin_from_blob(kb, n, d), Kb, "c1 K")
    assert_same_res(res_from_blob(kr, n, d), Kr, "c1 K")
    assert_same_bin(bin_from_blob(vb, n, d), Vb, "c1 V")
    assert_same_res(res_from_blob(vr, n, d), Vr, "c1 V")
    _, ref = O.compensated_attention(to_np(q), Kb, Kr, Vb, Vr, B, H, S, return_f32=True)
    got = to_np(out).astype(np.float32)
    err, c = close(got, ref, what="c1 vs oracle")
    exact = F.reference_attention(q, k, v, B, H, S, d).float()
    _, eref = O.reference_attention(to_np(q), to_np(k), to_np(v), B, H, S, return_f32=True)
    close(to_np(exact), eref, what="c1 fp16 reference attention vs oracle")
    g, e = torch.from_numpy(got).view(-1, d), exact.cpu().view(-1, d)
    cos = torch.nn.functional.cosine_similarity(g, e, dim=1)
    mae = (g - e).abs().max().item()
    say(f"c1: vs oracle rel err {err:.2e} cos {c:.7f}; vs fp16 attention mean cos "
        f"{cos.mean().item():.5f} min {cos.min().item():.5f} max-abs err {mae:.3e}")
    assert cos.mean().item() > 0.9


@pytest.mark.parametrize("group,d", [(2, 128), (4, 128), (8, 128), (4, 64), (4, 256)])
def test_gqa_equals_mha_on_repeated_kv(F, group, d):
    """GQA head mapping pinned by its closed form: attention with n_kv_heads =
    Hq / group equals MHA attention over K/V whose heads are repeated group
    times (each repeated vector encodes to the same bits).  The two run
    different kernels (int8-MFMA residual dots over a head group against
    per-head v_dot8 dots) and split plans; their outputs agree to the output
    tolerance."""
    B, Hq, S = 2, 16, 1500
    Hkv = Hq // group
    say(f"case gqa==mha group={group} d={d}")
    q, k, v = make(B, Hq, Hkv, S, d, seed=group * 1000 + d, lognorm=0.25)
    kr_ = np.repeat(k, group, axis=1)
    vr_ = np.repeat(v, group, axis=1)
    kb, kr = encode_gpu(F, k)
    vb, vr = encode_gpu(F, v)
    kbm, krm = encode_gpu(F, kr_)
    vbm, vrm = encode_gpu(F, vr_)
    qt = torch.from_numpy(q).cuda()
    for comp in (True, False):
        if comp:
            g = F.compensated_attention(qt, kb, kr, vb, vr, B, Hq, S, d, n_kv_heads=Hkv)
            m = F.compensated_attention(qt, kbm, krm, vbm, vrm, B, Hq, S, d)
        else:
            g = F.binary_attention(qt, kb, vb, B, Hq, S, d, n_kv_heads=Hkv)
            m = F.binary_attention(qt, kbm, vbm, B, Hq, S, d)
        close(to_np(g).astype(np.float32), to_np(m).astype(np.float32),
              what=f"gqa vs mha group={group} d={d} comp={comp}")


@pytest.mark.parametrize("B,Hq,Hkv,S,d", [(2, 8, 8, 1500, 128), (2, 16, 4, 2000, 128),
                                          (1, 8, 2, 900, 64), (1, 4, 4, 700, 256),
                                          # more query-head groups than one block of the
                                          # group compaction takes at a time (1024)
                                          (40, 32, 32, 130, 64), (48, 32, 8, 200, 128),
                                          # the VALU kernel's per-head modes
                                          (1, 4, 4, 500, 32), (1, 8, 2, 600, 96),
                                          (1, 4, 2, 300, 160), (1, 8, 4, 250, 224)])
def test_head_mode_attention(F, B, Hq, Hkv, S, d):
    """Per-head dispatch in one launch: heads with mode 0 match the oracle's
    binary attention, heads with mode 1 its compensated attention (modes mixed
    inside GQA groups); all-compensated modes agree with compensated attention
    to rounding (the same arithmetic, which the compiler may contract into
    FMAs differently in the two kernels)."""
    say(f"case head modes B={B} Hq={Hq} Hkv={Hkv} S={S} d={d}")
    q, k, v = make(B, Hq, Hkv, S, d, seed=S + d, lognorm=0.25)
    kb, kr = encode_gpu(F, k)
    vb, vr = encode_gpu(F, v)
    qt = torch.from_numpy(q).cuda()
    rng = np.random.default_rng(S)
    modes = rng.integers(0, 2, size=(B, Hq)).astype(np.uint8)
    # a query-head group of binary heads only (its workgroups read no
    # residual bytes) and one of compensated heads only
    G = Hq // Hkv
    modes[0, :G], modes[-1, -G:] = 0, 1
    out = to_np(F.head_mode_attention(qt, kb, kr, vb, vr, torch.from_numpy(modes).cuda(), B, Hq, S, d,
                                      n_kv_heads=Hkv)).astype(np.float32)
    n = B * Hkv * S
    Kb, Kr = bin_from_blob(kb, n, d), res_from_blob(kr, n, d)
    Vb, Vr = bin_from_blob(vb, n, d), res_from_blob(vr, n, d)
    _, rb = O.binary_attention(q, Kb, Vb, B, Hq, S, n_kv_heads=Hkv, return_f32=True)
    _, rc = O.compensated_attention(q, Kb, Kr, Vb, Vr, B, Hq, S, n_kv_heads=Hkv, return_f32=True)
    for b in range(B):
        for h in range(Hq):
            ref = rc[b, h] if modes[b, h] else rb[b, h]
            close(out[b, h], ref, what=f"head ({b}, {h}) mode {modes[b, h]}")
    ones = torch.ones((B, Hq), dtype=torch.uint8, device="cuda")
    allc = F.head_mode_attention(qt, kb, kr, vb, vr, ones, B, Hq, S, d, n_kv_heads=Hkv)
    comp = F.compensated_attention(qt, kb, kr, vb, vr, B, Hq, S, d, n_kv_heads=Hkv)
    close(to_np(allc).astype(np.float32), to_np(comp).astype(np.float32), rel=1e-3, cos=0.999999,
          what="all heads compensated")
    # every head binary: no workgroup reads a residual byte; the binary
    # kernel's output to rounding
    allb = F.head_mode_attention(qt, kb, kr, vb, vr, torch.zeros_like(ones), B, Hq, S, d, n_kv_heads=Hkv)
    binr = F.binary_attention(qt, kb, vb, B, Hq, S, d, n_kv_heads=Hkv)
    close(to_np(allb).astype(np.float32), to_np(binr).astype(np.float32), rel=1e-3, cos=0.999999,
          what="all heads binary")


def test_entropy_dispatch_attention(F):
    """The reference's adaptive precision end to end (MHA): entropy per head,
    mode = binary where entropy >= threshold, one launch; modes and outputs
    against the oracle."""
    say("case entropy dispatch")
    B, H, S, d = 2, 8, 2500, 128
    q, k, v = make(B, H, H, S, d, seed=31, scale=0.3)
    kb, kr = encode_gpu(F, k)
    vb, vr = encode_gpu(F, v)
    qt = torch.from_numpy(q).cuda()
    n = B * H * S
    Kb, Kr = bin_from_blob(kb, n, d), res_from_blob(kr, n, d)
    Vb, Vr = bin_from_blob(vb, n, d), res_from_blob(vr, n, d)
    ent = O.head_entropy(q, Kb, B, H, S)
    thr = float(np.median(ent))
    out, modes = F.entropy_dispatch_attention(qt, kb, kr, vb, vr, B, H, S, d, thr)
    modes = to_np(modes)
    want = (ent < thr).astype(np.uint8).reshape(B, H)
    # heads within float rounding of the threshold may land either side
    near = np.abs(ent.reshape(B, H) - thr) <= 2e-4 * max(1.0, abs(thr))
    assert np.array_equal(modes[~near], want[~near])
    _, rb = O.binary_attention(q, Kb, Vb, B, H, S, return_f32=True)
    _, rc = O.compensated_attention(q, Kb, Kr, Vb, Vr, B, H, S, return_f32=True)
    out = to_np(out).astype(np.float32)
    for b in range(B):
        for h in range(H):
            close(out[b, h], rc[b, h] if modes[b, h] else rb[b, h], what=f"head ({b}, {h})")
