"""GPU parity: encode kernels are bit-exact with the oracle (sign words, fp16
scales, INT4 codes and residual scales), for every supported head_dim."""
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.gpu_util import (assert_same_bin, assert_same_res, bin_from_blob, res_from_blob, say,
                            to_np)

pytestmark = pytest.mark.gpu

GOLDEN = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden.npz"))
ALL_DIMS = (32, 64, 96, 128, 160, 192, 224, 256)


@pytest.fixture(scope="module")
def F():
    import bitcache_amd.functional as F
    return F


def rand_x(n, d, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((n, d)) * rng.lognormal(0, 1.5, (n, 1))).astype(np.float16)
    if n >= 3:
        x[0] = 0.5
        x[1, ::2] = np.float16(-0.0)
        x[2, :3] = [np.inf, -np.inf, np.nan]
    if n >= 200:
        # fp16 subnormals only (7 / absmax may overflow), the largest finite
        # magnitudes, zeros of both signs, and small integers (exact ties of
        # r * 7 / absmax at .5), each far from the NaN row so that whole waves
        # of such vectors take the fast quantisation path
        x[64] = (rng.integers(-1023, 1024, d) * 2.0 ** -24).astype(np.float16)
        x[65] = rng.choice([-65504.0, 65504.0, -32768.0, 1.0], d).astype(np.float16)
        x[66] = np.where(rng.random(d) < 0.5, np.float16(-0.0), np.float16(0.0))
        x[67] = np.float16(2.0 ** -24)
        x[100:200] = rng.integers(-8, 9, (100, d)).astype(np.float16)
    return x


@pytest.mark.parametrize("d", (32, 64, 128, 256))
def test_encode_golden(F, d):
    say(f"case encode_golden d={d}")
    x = GOLDEN[f"enc_d{d}_x"]
    n = x.shape[0]
    xt = torch.from_numpy(x).cuda()
    b = F.encode(xt)
    r = F.compute_residual(xt, b)
    got_b = bin_from_blob(b, n, d)
    assert np.array_equal(got_b.words, GOLDEN[f"enc_d{d}_words"])
    assert np.array_equal(got_b.scale.view(np.uint16), GOLDEN[f"enc_d{d}_scale"])
    got_r = res_from_blob(r, n, d)
    assert np.array_equal(got_r.codes, GOLDEN[f"enc_d{d}_codes"])
    assert np.array_equal(got_r.scale.view(np.uint16), GOLDEN[f"enc_d{d}_rscale"])
    b1, r1 = F.encode_fused(xt, fp32_scale=True)
    got_r1 = res_from_blob(r1, n, d)
    assert np.array_equal(got_r1.codes, GOLDEN[f"enc_d{d}_codes_online"])
    assert np.array_equal(got_r1.scale.view(np.uint16), GOLDEN[f"enc_d{d}_rscale_online"])
    pb = n * (d // 8 + 2)    # payload bytes; the rest of each blob is unused capacity
    assert torch.equal(b1[:pb], b[:pb])


@pytest.mark.parametrize("d", ALL_DIMS)
def test_encode_random_all_dims(F, d):
    say(f"case encode_random d={d}")
    n = 3001
    x = rand_x(n, d, d)
    xt = torch.from_numpy(x).cuda()
    b = F.encode(xt)
    r = F.compute_residual(xt, b)
    eb = O.binary_encode(x)
    er = O.residual_encode(x, eb)
    assert_same_bin(bin_from_blob(b, n, d), eb, f"d={d}")
    assert_same_res(res_from_blob(r, n, d), er, f"d={d}")
    # fused prefill encode produces identical bytes (the tail of each blob beyond
    # the payload is untouched scratch and not compared)
    fb, fr = F.encode_fused(xt, fp32_scale=False)
    pb, pr = n * (d // 8 + 2), n * (d // 2 + 2)
    assert torch.equal(fb[:pb], b[:pb]) and torch.equal(fr[:pr], r[:pr])
    _, on = O.online_encode(x)
    _, fr1 = F.encode_fused(xt, fp32_scale=True)
    assert_same_res(res_from_blob(fr1, n, d), on, f"online d={d}")


def test_encode_empty_and_single(F):
    say("case encode_empty_single")
    e = F.encode(torch.zeros((0, 128), dtype=torch.float16, device="cuda"))
    assert e.numel() == 0
    x = rand_x(1, 64, 5)[:1]
    b = F.encode(torch.from_numpy(x).cuda())
    assert_same_bin(bin_from_blob(b, 1, 64), O.binary_encode(x))


def test_online_encode_ring_slots():
    """online_encode_token writes slot current_len % max_seq of each (b,h) and
    nothing else (src/online_encode.cu:31-34,139)."""
    import bitcache_amd as bc
    say("case online_encode_ring")
    B, H, d, max_seq = 2, 3, 128, 5
    n = B * H * max_seq
    kb = torch.zeros(n * 36, dtype=torch.uint8, device="cuda")
    kr = torch.zeros(n * 130, dtype=torch.uint8, device="cuda")
    rng = np.random.default_rng(7)
    toks = []
    for step in range(7):
        x = (rng.standard_normal((B, H, d)) * 0.3).astype(np.float16)
        toks.append(x)
        bc._C.online_encode_token(torch.from_numpy(x).cuda(), kb, kr, B, H, d, step, max_seq)
    got_b = bin_from_blob(kb, n, d)
    got_r = res_from_blob(kr, n, d)
    # slot s holds the last token written there
    for slot in range(max_seq):
        last = max(t for t in range(7) if t % max_seq == slot)
        x = toks[last].reshape(B * H, d)
        eb, er = O.online_encode(x)
        idx = np.arange(B * H) * max_seq + slot
        assert np.array_equal(got_b.words[idx], eb.words)
        assert np.array_equal(got_b.scale[idx].view(np.uint16), eb.scale.view(np.uint16))
        assert np.array_equal(got_r.codes[idx], er.codes)
        assert np.array_equal(got_r.scale[idx].view(np.uint16), er.scale.view(np.uint16))
    # binary-only cache: residual pointer None writes nothing else
    kb2 = torch.zeros(n * 36, dtype=torch.uint8, device="cuda")
    bc._C.online_encode_token(torch.from_numpy(toks[0]).cuda(), kb2, None, B, H, d, 0, max_seq)
    torch.cuda.synchronize()
    eb, _ = O.online_encode(toks[0].reshape(B * H, d))
    got = bin_from_blob(kb2, n, d)
    assert np.array_equal(got.words[np.arange(B * H) * max_seq], eb.words)


def test_encode_into_cache_equals_appends():
    import bitcache_amd as bc
    say("case encode_into_cache")
    B, H, S, d, max_seq, start = 2, 2, 37, 64, 50, 3
    rows = B * H
    n = rows * max_seq
    rng = np.random.default_rng(9)
    x = (rng.standard_normal((rows, S, d)) * 0.2).astype(np.float16)
    kb = torch.zeros(n * 36, dtype=torch.uint8, device="cuda")
    kr = torch.zeros(n * 130, dtype=torch.uint8, device="cuda")
    bc._C.encode_into_cache(torch.from_numpy(x).cuda(), kb, kr, rows, S, d, start, max_seq, True)
    kb2 = torch.zeros_like(kb)
    kr2 = torch.zeros_like(kr)
    for s in range(S):
        tok = torch.from_numpy(np.ascontiguousarray(x[:, s])).cuda()
        bc._C.online_encode_token(tok, kb2, kr2, B, H, d, start + s, max_seq)
    assert torch.equal(kb, kb2) and torch.equal(kr, kr2)


@pytest.mark.parametrize("B,S,H,d,max_seq,start,res", [
    (2, 300, 4, 128, 320, 7, True),
    (3, 77, 8, 64, 77, 0, True),
    (1, 513, 2, 256, 600, 40, True),
    (2, 50, 3, 96, 64, 5, True),      # head dim of the one-vector-per-wave encoder
    (2, 33, 5, 128, 40, 1, False),    # binary-only cache, odd head count
])
def test_encode_into_cache_bshd(B, S, H, d, max_seq, start, res):
    """[batch, seq, heads, d] prefill source: the same cache bytes as the
    [batch, heads, seq, d] prefill of its transpose (online-encode math and
    two-step math), and as appending its tokens one by one."""
    import bitcache_amd as bc
    say(f"case encode_into_cache_bshd B={B} S={S} H={H} d={d} start={start} res={res}")
    rows, n = B * H, B * H * max_seq
    rng = np.random.default_rng(S + d)
    x = (rng.standard_normal((B, S, H, d)) * 0.2).astype(np.float16)
    xt = torch.from_numpy(x).cuda()
    xh = xt.permute(0, 2, 1, 3).contiguous()
    for fp32 in (True, False):
        blobs = []
        for layout in ("bshd", "bhsd"):
            kb = torch.zeros(n * 36, dtype=torch.uint8, device="cuda")
            kr = torch.zeros(n * 130, dtype=torch.uint8, device="cuda") if res else None
            if layout == "bshd":
                bc._C.encode_into_cache_bshd(xt, kb, kr, B, S, H, d, start, max_seq, fp32)
            else:
                bc._C.encode_into_cache(xh, kb, kr, rows, S, d, start, max_seq, fp32)
            blobs.append((kb, kr))
        assert torch.equal(blobs[0][0], blobs[1][0])
        if res:
            assert torch.equal(blobs[0][1], blobs[1][1])
    # == token-by-token appends (online-encode math)
    kb2 = torch.zeros(n * 36, dtype=torch.uint8, device="cuda")
    kr2 = torch.zeros(n * 130, dtype=torch.uint8, device="cuda") if res else None
    for s in range(S):
        bc._C.online_encode_token(xt[:, s].contiguous(), kb2, kr2, B, H, d, start + s, max_seq)
    kb, kr = torch.zeros_like(kb2), (torch.zeros_like(kr2) if res else None)
    bc._C.encode_into_cache_bshd(xt, kb, kr, B, S, H, d, start, max_seq, True)
    assert torch.equal(kb, kb2) and (not res or torch.equal(kr, kr2))


def test_bitcache_prefill_bshd():
    from bitcache_amd import BitCache
    say("case bitcache prefill bshd")
    B, Hq, Hkv, S, d = 2, 8, 2, 200, 128
    rng = np.random.default_rng(4)
    k = torch.from_numpy((rng.standard_normal((B, S, Hkv, d)) * 0.2).astype(np.float16)).cuda()
    v = torch.from_numpy((rng.standard_normal((B, S, Hkv, d)) * 0.2).astype(np.float16)).cuda()
    a = BitCache(B, Hq, d, 256, n_kv_heads=Hkv)
    b = BitCache(B, Hq, d, 256, n_kv_heads=Hkv)
    a.prefill(k, v, layout="bshd")
    b.prefill(k.permute(0, 2, 1, 3).contiguous(), v.permute(0, 2, 1, 3).contiguous())
    for x, y in ((a._k_bin, b._k_bin), (a._v_bin, b._v_bin), (a._k_res, b._k_res), (a._v_res, b._v_res)):
        assert torch.equal(x, y)
    assert a.seq_len == b.seq_len == S


def test_reference_layout_conversion(F):
    from bitcache_amd import layout
    say("case layout_conversion")
    for d in (64, 128, 256):
        n = 257
        x = rand_x(n, d, 100 + d)
        xt = torch.from_numpy(x).cuda()
        b = F.encode(xt)
        r = F.compute_residual(xt, b)
        ref_b = to_np(layout.to_reference(b, d, False)).reshape(n, 36)
        ref_r = to_np(layout.to_reference(r, d, True)).reshape(n, 130)
        eb = O.binary_encode(x)
        er = O.residual_encode(x, eb)
        # reference struct: u32 words[8] (unused words zero) + fp16 scale at byte 32
        words = np.zeros((n, 8), np.uint32)
        words[:, : d // 32] = eb.words
        assert np.array_equal(ref_b[:, :32].copy().view("<u4"), words)
        assert np.array_equal(ref_b[:, 32:34].copy().view(np.float16)[:, 0].view(np.uint16),
                              eb.scale.view(np.uint16))
        nib = np.zeros((n, 128), np.uint8)
        nib[:, : d // 2] = O.pack_nibbles(er.codes)
        assert np.array_equal(ref_r[:, :128], nib)
        assert np.array_equal(ref_r[:, 128:130].copy().view(np.float16)[:, 0].view(np.uint16),
                              er.scale.view(np.uint16))
        pb, pr = n * (d // 8 + 2), n * (d // 2 + 2)
        assert torch.equal(layout.from_reference(layout.to_reference(b, d, False), d, False)[:pb], b[:pb])
        assert torch.equal(layout.from_reference(layout.to_reference(r, d, True), d, True)[:pr], r[:pr])


def test_layout_planes_of_a_bitcache_prefix_view(F):
    """layout.binary_planes / residual_planes / to_reference on the prefix
    views the reference's BitCache.attend slices (bitcache/__init__.py:134-139)
    read the planes of the whole ring blob the view belongs to: the same
    tensors as on the whole blob, and the slots written so far hold the
    oracle's online-encode bytes of the appended vectors."""
    from bitcache_amd import BitCache, layout
    say("case layout prefix view")
    B, H, d, max_seq, steps = 2, 2, 128, 40, 13
    c = BitCache(B, H, d, max_seq)
    rng = np.random.default_rng(41)
    ks = []
    for _ in range(steps):
        k = (rng.standard_normal((B, H, d)) * 0.3).astype(np.float16)
        c.append(torch.from_numpy(k).cuda(), torch.from_numpy(k).cuda())
        ks.append(k)
    n = B * H * max_seq
    vb = c._k_bin[:B * H * steps * 36]
    vr = c._k_res[:B * H * steps * 130]
    assert vb.numel() < c._k_bin.numel()
    for got, want in zip(layout.binary_planes(vb, d), layout.binary_planes(c._k_bin, d)):
        assert got.shape[0] == n and torch.equal(got, want)
    for got, want in zip(layout.residual_planes(vr, d), layout.residual_planes(c._k_res, d)):
        assert got.shape[0] == n and torch.equal(got, want)
    assert torch.equal(layout.to_reference(vb, d, False), layout.to_reference(c._k_bin, d, False))
    signs, scale = layout.binary_planes(vb, d)
    codes, rscale = layout.residual_planes(vr, d)
    x = np.stack(ks, axis=2).reshape(B * H * steps, d)          # row (b, h), slot s
    eb, er = O.online_encode(x)
    rows = (np.arange(B * H)[:, None] * max_seq + np.arange(steps)[None]).reshape(-1)
    assert np.array_equal(to_np(signs)[rows].view(np.uint32), eb.words)
    assert np.array_equal(to_np(scale)[rows].view(np.uint16), eb.scale.view(np.uint16))
    assert np.array_equal(O.unpack_nibbles(to_np(codes)[rows]), er.codes)
    assert np.array_equal(to_np(rscale)[rows].view(np.uint16), er.scale.view(np.uint16))


def test_encode_prefill_scale_property(F):
    """c3-sized prefill slice: fused fp16-scale encode == two-step encode bytes
    on 2M vectors, and a random sample of vectors matches the oracle."""
    say("case encode_prefill_2M")
    n, d = 2 * 1024 * 1024, 128
    g = torch.Generator(device="cuda")
    g.manual_seed(2)
    x = (torch.randn((n, d), generator=g, device="cuda") / np.sqrt(128.0)
         * torch.exp(0.25 * torch.randn((n, 1), generator=g, device="cuda"))).half()
    b = F.encode(x)
    r = F.compute_residual(x, b)
    fb, fr = F.encode_fused(x)
    pb, pr = n * (d // 8 + 2), n * (d // 2 + 2)
    assert torch.equal(fb[:pb], b[:pb]) and torch.equal(fr[:pr], r[:pr])
    idx = np.random.default_rng(0).choice(n, 4096, replace=False)
    xs = to_np(x[torch.from_numpy(idx).cuda()])
    eb = O.binary_encode(xs)
    er = O.residual_encode(xs, eb)
    gb = bin_from_blob(b, n, d)
    gr = res_from_blob(r, n, d)
    assert np.array_equal(gb.words[idx], eb.words)
    assert np.array_equal(gb.scale[idx].view(np.uint16), eb.scale.view(np.uint16))
    assert np.array_equal(gr.codes[idx], er.codes)


@pytest.mark.parametrize("n_bytes", [16, 4096 * 16 + 48, 3 << 20])
def test_read_probe_reads_every_word_once(n_bytes):
    """The read-ceiling probe's per-wave XOR words combine to the XOR of every
    32-bit word of the source: each 16-byte piece is read (an odd number of
    times, i.e. once), the ragged tail and a source smaller than the grid
    included."""
    from bitcache_amd import _C
    say(f"case read probe {n_bytes}")
    g = torch.Generator(device="cuda")
    g.manual_seed(n_bytes)
    src = torch.randint(-2 ** 31, 2 ** 31 - 1, (n_bytes // 4,), dtype=torch.int32, device="cuda", generator=g)
    out = _C.read_probe(src)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    wgs = min(cus * 4, 4096, n_bytes // 16)
    got = np.bitwise_xor.reduce(out[: 4 * wgs].cpu().numpy())
    want = np.bitwise_xor.reduce(src.cpu().numpy())
    assert got == want


@pytest.mark.parametrize("n_write,nt", [(4096, False), (4096 * 1021, True), (4096 * 9000, False)])
def test_mix_probe_writes_each_word_once(n_write, nt):
    """The mixed read/write probe: output word j (16 bytes) is the XOR of the
    three input words 768 * (j // 256) + 256 r + j % 256, r = 0..2, so every
    input is read once and every output written once; a guard region past
    dst stays untouched."""
    from bitcache_amd import _C
    say(f"case mix probe {n_write} nt={nt}")
    g = torch.Generator(device="cuda")
    g.manual_seed(n_write)
    src = torch.randint(-2 ** 31, 2 ** 31 - 1, (3 * n_write // 4,), dtype=torch.int32, device="cuda",
                        generator=g)
    buf = torch.full((n_write // 4 + 1024,), 0x5A5A5A5A, dtype=torch.int32, device="cuda")
    dst = buf[: n_write // 4]
    _C.mix_probe(src, dst, nt)
    torch.cuda.synchronize()
    w = src.cpu().numpy().reshape(-1, 3, 256, 4)             # [block, r, word, 4 x u32]
    want = (w[:, 0] ^ w[:, 1] ^ w[:, 2]).reshape(-1)
    assert np.array_equal(dst.cpu().numpy(), want)
    assert bool((buf[n_write // 4:] == 0x5A5A5A5A).all())


@pytest.mark.parametrize("d,n", [(64, 5000), (128, 3001), (256, 777)])
def test_traffic_probe_stays_in_its_blobs(d, n):
    """The encoder's traffic probe (same loads and stores, no arithmetic)
    writes only inside the two blobs it is given: guard bytes after each blob
    keep their value, and the source is not modified."""
    from bitcache_amd import _C
    say(f"case traffic_probe d={d} n={n}")
    x = torch.from_numpy(rand_x(n, d, 7)).cuda()
    x0 = x.clone()
    guard = 4096
    bfull = torch.full((n * 36 + guard,), 0xA5, dtype=torch.uint8, device="cuda")
    rfull = torch.full((n * 130 + guard,), 0x5A, dtype=torch.uint8, device="cuda")
    _C.encode_traffic_probe(x, bfull[:n * 36], rfull[:n * 130])
    torch.cuda.synchronize()
    assert torch.all(bfull[n * 36:] == 0xA5) and torch.all(rfull[n * 130:] == 0x5A)
    assert torch.equal(x.view(torch.int16), x0.view(torch.int16))   # bitwise (x holds a NaN)
