"""bc_attention_gqa_noalloc (the entry point for callers that cannot allocate:
split partials in a library-owned device array) through the C ABI against
bc_attention_gqa with a caller workspace: the same outputs, bit for bit, on
two calls in a row, the second smaller, in compensated and binary modes.
(The rejection of a shape whose partials exceed the array is a CPU test:
tests/test_abi.py::test_attention_argument_errors.)"""
import ctypes
import os

import pytest
import torch

from tests.gpu_util import say

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "bitcache_amd", "libbitcache_hip.so")
P, I32, SZ = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t


def test_noalloc_attention_matches_workspace_entry_point():
    from bitcache_amd import _C
    L = ctypes.CDLL(LIB)
    L.bc_status_string.restype = ctypes.c_char_p
    L.bc_last_error.restype = ctypes.c_char_p
    L.bc_attention_workspace_size.argtypes = [I32] * 5 + [ctypes.POINTER(SZ)]
    L.bc_attention_gqa.argtypes = [P] * 6 + [I32] * 6 + [P, SZ, P]
    L.bc_attention_gqa_noalloc.argtypes = [P] * 6 + [I32] * 6 + [P]

    def ok(st):
        assert st == 0, f"{L.bc_status_string(st).decode()}: {L.bc_last_error().decode()}"

    ptr = lambda t: P(t.data_ptr()) if t is not None else None
    st = P(torch.cuda.current_stream().cuda_stream)
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    # two calls in a row, the second with a smaller input (fewer heads, a
    # shorter context, another head dim): the array keeps the first call's
    # partials, which the second must not see
    for (B, Hq, Hkv, S, stride, d) in [(4, 32, 8, 5000, 5100, 128), (1, 8, 8, 700, 700, 64)]:
        say(f"case noalloc B={B} Hq={Hq} Hkv={Hkv} S={S} stride={stride} d={d}")
        q = (torch.randn((B, Hq, d), generator=g, device="cuda") * 0.1).half()
        k = (torch.randn((B * Hkv * stride, d), generator=g, device="cuda") * 0.1).half()
        v = (torch.randn((B * Hkv * stride, d), generator=g, device="cuda") * 0.1).half()
        kb, kr = _C.encode_fused(k, False)
        vb, vr = _C.encode_fused(v, False)
        n = SZ(0)
        ok(L.bc_attention_workspace_size(B, Hq, Hkv, S, d, ctypes.byref(n)))
        ws = torch.empty(max(n.value, 1), dtype=torch.uint8, device="cuda")
        for res in (True, False):
            a = torch.empty((B, Hq, d), dtype=torch.float16, device="cuda")
            b = torch.full((B, Hq, d), float("nan"), dtype=torch.float16, device="cuda")
            kr_, vr_ = (kr, vr) if res else (None, None)
            ok(L.bc_attention_gqa(ptr(q), ptr(kb), ptr(kr_), ptr(vb), ptr(vr_), ptr(a), B, Hq, Hkv,
                                  S, stride, d, ptr(ws), n.value, st))
            ok(L.bc_attention_gqa_noalloc(ptr(q), ptr(kb), ptr(kr_), ptr(vb), ptr(vr_), ptr(b), B,
                                          Hq, Hkv, S, stride, d, st))
            torch.cuda.synchronize()
            assert torch.equal(a, b), f"outputs differ (residual={res})"
