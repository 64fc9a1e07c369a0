"""The C ABI on its own: libbitcache_hip.so called through ctypes with raw
device pointers, the workspace a caller allocates and the caller's stream, as
a non-PyTorch binding would (include/bitcache.h).  Outputs and cache bytes
must equal, bit for bit, those of the operator module built on the same
library."""
import ctypes
import os

import numpy as np
import pytest
import torch

from tests.gpu_util import say

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "bitcache_amd", "libbitcache_hip.so")
P, I32, I64, SZ = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_size_t


@pytest.fixture(scope="module")
def lib():
    L = ctypes.CDLL(LIB)
    L.bc_status_string.restype = ctypes.c_char_p
    L.bc_last_error.restype = ctypes.c_char_p
    L.bc_encode_fused.argtypes = [P, P, P, I64, I32, I32, P]
    L.bc_attention_workspace_size.argtypes = [I32] * 5 + [ctypes.POINTER(SZ)]
    L.bc_compensated_attention.argtypes = [P] * 6 + [I32] * 4 + [P, SZ, P]
    L.bc_attention_gqa.argtypes = [P] * 6 + [I32] * 6 + [P, SZ, P]
    L.bc_append_attention.argtypes = [P] * 8 + [I32] * 4 + [I64, I32, P, SZ, P]
    return L


def ok(lib, st):
    assert st == 0, f"{lib.bc_status_string(st).decode()}: {lib.bc_last_error().decode()}"


def ptr(t):
    return P(t.data_ptr())


def stream():
    return P(torch.cuda.current_stream().cuda_stream)


def workspace(lib, B, Hq, Hkv, S, d):
    n = SZ(0)
    ok(lib, lib.bc_attention_workspace_size(B, Hq, Hkv, S, d, ctypes.byref(n)))
    return torch.empty(max(n.value, 1), dtype=torch.uint8, device="cuda"), n.value


def test_cabi_encode_and_attention_match_the_operators(lib):
    """bc_encode_fused + bc_compensated_attention (MHA) and bc_attention_gqa
    through ctypes against bitcache_amd._C on the same inputs."""
    from bitcache_amd import _C
    say("case cabi encode + attention")
    B, Hq, Hkv, S, d = 2, 8, 2, 1500, 128
    g = torch.Generator(device="cuda")
    g.manual_seed(7)
    q = (torch.randn((B, Hq, d), generator=g, device="cuda") * 0.2).half()
    k = (torch.randn((B, Hkv, S, d), generator=g, device="cuda") * 0.2).half()
    v = (torch.randn((B, Hkv, S, d), generator=g, device="cuda") * 0.2).half()
    n = B * Hkv * S
    blobs = []
    for x in (k, v):
        b = torch.zeros(n * 36, dtype=torch.uint8, device="cuda")
        r = torch.zeros(n * 130, dtype=torch.uint8, device="cuda")
        ok(lib, lib.bc_encode_fused(ptr(x), ptr(b), ptr(r), n, d, 0, stream()))
        blobs += [b, r]
    kb, kr, vb, vr = blobs
    kb2, kr2 = _C.encode_fused(k.view(-1, d), False)
    vb2, vr2 = _C.encode_fused(v.view(-1, d), False)
    # the planes (signs + scales, codes + scales); the rest of a
    # reference-sized blob is unused and left as allocated
    nb, nr = n * (d // 8 + 2), n * (d // 2 + 2)
    for x, y, m in ((kb, kb2, nb), (kr, kr2, nr), (vb, vb2, nb), (vr, vr2, nr)):
        assert torch.equal(x[:m], y[:m])
    # GQA through bc_attention_gqa
    ws, nws = workspace(lib, B, Hq, Hkv, S, d)
    out = torch.empty((B, Hq, d), dtype=torch.float16, device="cuda")
    ok(lib, lib.bc_attention_gqa(ptr(q), ptr(kb), ptr(kr), ptr(vb), ptr(vr), ptr(out), B, Hq, Hkv, S, S,
                                 d, ptr(ws), nws, stream()))
    want = _C.attention(q, kb, kr, vb, vr, B, Hq, Hkv, S, S, d)
    assert torch.equal(out, want)
    # the reference's MHA signature: one head per kv head
    qm = q[:, :Hkv].contiguous()
    ws, nws = workspace(lib, B, Hkv, Hkv, S, d)
    outm = torch.empty((B, Hkv, d), dtype=torch.float16, device="cuda")
    ok(lib, lib.bc_compensated_attention(ptr(qm), ptr(kb), ptr(kr), ptr(vb), ptr(vr), ptr(outm), B, Hkv,
                                         S, d, ptr(ws), nws, stream()))
    assert torch.equal(outm, _C.compensated_attention(qm, kb, kr, vb, vr, B, Hkv, S, d))


def test_cabi_append_attention_matches_bitcache(lib):
    """bc_append_attention through ctypes, step by step on a ring that wraps,
    against BitCache.append + attend on a second cache."""
    from bitcache_amd import BitCache
    say("case cabi append_attention")
    B, Hq, Hkv, d, max_seq, steps = 2, 8, 2, 128, 40, 70
    ref = BitCache(B, Hq, d, max_seq, n_kv_heads=Hkv)
    cap = B * Hkv * max_seq
    kb = torch.zeros(cap * 36, dtype=torch.uint8, device="cuda")
    vb = torch.zeros(cap * 36, dtype=torch.uint8, device="cuda")
    kr = torch.zeros(cap * 130, dtype=torch.uint8, device="cuda")
    vr = torch.zeros(cap * 130, dtype=torch.uint8, device="cuda")
    ws, nws = workspace(lib, B, Hq, Hkv, max_seq, d)   # the largest step's workspace
    g = torch.Generator(device="cuda")
    g.manual_seed(8)
    for t in range(steps):
        k = (torch.randn((B, Hkv, d), generator=g, device="cuda") * 0.2).half()
        v = (torch.randn((B, Hkv, d), generator=g, device="cuda") * 0.2).half()
        q = (torch.randn((B, Hq, d), generator=g, device="cuda") * 0.2).half()
        out = torch.empty((B, Hq, d), dtype=torch.float16, device="cuda")
        ok(lib, lib.bc_append_attention(ptr(q), ptr(k), ptr(v), ptr(kb), ptr(kr), ptr(vb), ptr(vr),
                                        ptr(out), B, Hq, Hkv, d, t, max_seq, ptr(ws), nws, stream()))
        ref.append(k, v)
        assert torch.equal(out, ref.attend(q)), f"step {t}"
    for x, y in ((kb, ref._k_bin), (vb, ref._v_bin), (kr, ref._k_res), (vr, ref._v_res)):
        assert torch.equal(x, y)
    assert np.isfinite(out.float().cpu().numpy()).all()


def test_split_partials_stay_inside_the_reported_workspace(lib):
    """Regression: every attention mode's split plan writes its partials inside
    the workspace bc_attention_workspace_size reports.  Binary GQA plans the
    most workgroups per CU; at these shapes its plan holds more splits than a
    workspace sized over fewer policies.  The workspace is the reported size
    followed by a guard region of known bytes that must come back untouched,
    and each output equals the operator module's."""
    from bitcache_amd import _C
    L = lib
    L.bc_attention_split_plan.argtypes = [I32] * 7 + [ctypes.POINTER(I32), ctypes.POINTER(SZ),
                                                      ctypes.POINTER(SZ)]
    L.bc_head_mode_attention.argtypes = [P] * 7 + [I32] * 6 + [P, SZ, P]
    guard = 1 << 20
    g = torch.Generator(device="cuda")
    g.manual_seed(11)
    for (B, Hq, Hkv, S, d) in [(4, 32, 8, 16384, 128), (2, 32, 8, 32768, 128),
                               (1, 32, 8, 65536, 128)]:
        say(f"case workspace guard B={B} Hq={Hq} Hkv={Hkv} S={S} d={d}")
        n = B * Hkv * S
        q = (torch.randn((B, Hq, d), generator=g, device="cuda") * 0.2).half()
        kb, kr = _C.encode_fused((torch.randn((n, d), generator=g, device="cuda") * 0.2).half(), False)
        vb, vr = _C.encode_fused((torch.randn((n, d), generator=g, device="cuda") * 0.2).half(), False)
        modes = (torch.arange(B * Hq, device="cuda") % 3 == 0).to(torch.uint8)
        nws = SZ(0)
        ok(L, L.bc_attention_workspace_size(B, Hq, Hkv, S, d, ctypes.byref(nws)))
        for mode in (0, 1, 3):
            ns, part, total = I32(0), SZ(0), SZ(0)
            ok(L, L.bc_attention_split_plan(mode, B, Hq, Hkv, S, d, 0, ctypes.byref(ns),
                                            ctypes.byref(part), ctypes.byref(total)))
            assert total.value == nws.value and part.value <= nws.value, (mode, ns.value)
            ws = torch.full((nws.value + guard,), 0xA5, dtype=torch.uint8, device="cuda")
            out = torch.empty((B, Hq, d), dtype=torch.float16, device="cuda")
            if mode == 3:
                ok(L, L.bc_head_mode_attention(ptr(q), ptr(kb), ptr(kr), ptr(vb), ptr(vr),
                                               ptr(modes), ptr(out), B, Hq, Hkv, S, S, d, ptr(ws),
                                               nws.value, stream()))
                want = _C.head_mode_attention(q, kb, kr, vb, vr, modes, B, Hq, Hkv, S, S, d)
            else:
                kr_, vr_ = (kr, vr) if mode == 1 else (None, None)
                ok(L, L.bc_attention_gqa(ptr(q), ptr(kb), P(kr_.data_ptr()) if mode else None,
                                         ptr(vb), P(vr_.data_ptr()) if mode else None, ptr(out), B,
                                         Hq, Hkv, S, S, d, ptr(ws), nws.value, stream()))
                want = _C.attention(q, kb, kr_, vb, vr_, B, Hq, Hkv, S, S, d)
            torch.cuda.synchronize()
            tail = ws[nws.value:]
            assert bool((tail == 0xA5).all()), f"mode {mode}: partials written past the workspace"
            assert torch.equal(out, want), f"mode {mode}"
