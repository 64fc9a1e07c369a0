"""CPU checks of the C ABI and the extension boundary (no GPU work is issued):
the library loads, exports every function include/bitcache.h declares, reports
the reference's struct sizes, and rejects invalid arguments with the right
status before touching the device."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "bitcache.h")
LIB = os.path.join(ROOT, "bitcache_amd", "libbitcache_hip.so")

BC_OK, BC_ERR_INVALID_ARGUMENT, BC_ERR_UNSUPPORTED, BC_ERR_WORKSPACE, BC_ERR_HIP = range(5)


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(bc_[a-z0-9_]+)\s*\(", text)))


def _gpu_visible() -> bool:
    try:
        import torch
        return torch.cuda.device_count() > 0
    except Exception:
        return False


@pytest.fixture()
def no_gpu():
    """The argument-error cases pass a fake device address and rely on the
    entry point rejecting the call before any launch; they run only where no
    GPU could receive a launch if a validation ever regressed."""
    if _gpu_visible():
        pytest.skip("fake-pointer argument checks run only without a GPU")


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.skip("libbitcache_hip.so not built (run python -m bitcache_amd.build)")
    L = ctypes.CDLL(LIB)
    L.bc_status_string.restype = ctypes.c_char_p
    L.bc_last_error.restype = ctypes.c_char_p
    L.bc_sizeof_binary_vec.restype = ctypes.c_int64
    L.bc_sizeof_residual_vec.restype = ctypes.c_int64
    return L


def test_exports_every_declared_symbol(lib):
    names = declared_functions()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"


def test_sizes_and_strings(lib):
    assert lib.bc_sizeof_binary_vec() == 36
    assert lib.bc_sizeof_residual_vec() == 130
    assert lib.bc_abi_version() == 1
    assert lib.bc_status_string(BC_OK) == b"ok"
    assert lib.bc_status_string(BC_ERR_WORKSPACE) == b"workspace too small"


def test_encode_argument_errors(lib, no_gpu):
    P = ctypes.c_void_p
    fake = P(0x1000)
    f = lib.bc_binary_encode
    f.argtypes = [P, P, ctypes.c_int64, ctypes.c_int, P]
    assert f(fake, fake, 10, 48, None) == BC_ERR_UNSUPPORTED
    assert b"multiple of 32" in lib.bc_last_error()
    assert f(fake, fake, 10, 288, None) == BC_ERR_UNSUPPORTED
    assert f(fake, fake, -1, 128, None) == BC_ERR_INVALID_ARGUMENT
    assert f(None, fake, 10, 128, None) == BC_ERR_INVALID_ARGUMENT
    assert f(None, None, 0, 128, None) == BC_OK          # empty input: nothing to do
    g = lib.bc_encode_fused
    g.argtypes = [P, P, P, ctypes.c_int64, ctypes.c_int, ctypes.c_int, P]
    assert g(fake, fake, fake, 10, 128, 7, None) == BC_ERR_INVALID_ARGUMENT
    h = lib.bc_online_encode_token
    h.argtypes = [P, P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int64, ctypes.c_int, P]
    assert h(fake, fake, fake, 1, 1, 128, 0, 0, None) == BC_ERR_INVALID_ARGUMENT   # max_seq 0
    assert h(fake, fake, fake, 1, 1, 128, -1, 4, None) == BC_ERR_INVALID_ARGUMENT  # current_len < 0
    e = lib.bc_encode_into_cache
    e.argtypes = [P, P, P, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                  ctypes.c_int, P]
    assert e(fake, fake, fake, 2, 10, 128, 8, 16, 1, None) == BC_ERR_INVALID_ARGUMENT  # overflows ring
    t = lib.bc_encode_traffic_probe
    t.argtypes = [P, P, P, ctypes.c_int64, ctypes.c_int, P]
    assert t(fake, fake, fake, 10, 96, None) == BC_ERR_UNSUPPORTED        # row encoder dims only
    assert t(fake, fake, fake, -1, 128, None) == BC_ERR_INVALID_ARGUMENT
    assert t(fake, None, fake, 10, 128, None) == BC_ERR_INVALID_ARGUMENT
    assert t(None, None, None, 0, 128, None) == BC_OK
    m = lib.bc_mix_probe
    m.argtypes = [P, P, ctypes.c_int64, ctypes.c_int, P]
    assert m(fake, fake, 4096 + 16, 0, None) == BC_ERR_INVALID_ARGUMENT   # not whole 4 KiB blocks
    assert m(fake, fake, 24, 0, None) == BC_ERR_INVALID_ARGUMENT
    assert m(fake, P(0x1008), 4096, 0, None) == BC_ERR_INVALID_ARGUMENT  # unaligned
    assert m(None, fake, 4096, 0, None) == BC_ERR_INVALID_ARGUMENT
    assert m(None, None, 0, 0, None) == BC_OK
    r = lib.bc_read_probe
    r.argtypes = [P, ctypes.c_int64, P, P]
    assert r(fake, 24, fake, None) == BC_ERR_INVALID_ARGUMENT        # not a multiple of 16
    assert r(fake, -16, fake, None) == BC_ERR_INVALID_ARGUMENT
    assert r(None, 64, fake, None) == BC_ERR_INVALID_ARGUMENT
    assert r(P(0x1008), 64, fake, None) == BC_ERR_INVALID_ARGUMENT   # unaligned
    assert r(None, 0, None, None) == BC_OK


def test_attention_argument_errors(lib, no_gpu):
    P = ctypes.c_void_p
    fake = P(0x1000)
    size_t = ctypes.c_size_t
    ws = lib.bc_attention_workspace_size
    ws.argtypes = [ctypes.c_int] * 5 + [ctypes.POINTER(size_t)]
    n = size_t(0)
    assert ws(8, 32, 32, 65536, 128, ctypes.byref(n)) == BC_OK and n.value > 0
    assert ws(1, 6, 4, 10, 128, ctypes.byref(n)) == BC_ERR_INVALID_ARGUMENT   # 6 % 4 != 0
    assert ws(1, 4, 4, 10, 100, ctypes.byref(n)) == BC_ERR_UNSUPPORTED
    aws = lib.bc_adaptive_attention_workspace_size
    aws.argtypes = [ctypes.c_int] * 5 + [ctypes.POINTER(size_t)]
    # the selection lists index keys within chunks of 2^16, at most 2^10 chunks
    assert aws(1, 4, 4, (1 << 26) + 1, 128, ctypes.byref(n)) == BC_ERR_UNSUPPORTED
    g = lib.bc_attention_gqa
    g.argtypes = [P] * 6 + [ctypes.c_int] * 6 + [P, size_t, P]
    # workspace too small is rejected before any launch
    assert g(fake, fake, fake, fake, fake, fake, 1, 4, 4, 100, 100, 128, fake, 1, None) == BC_ERR_WORKSPACE
    assert g(fake, fake, fake, fake, fake, fake, 1, 4, 4, 100, 50, 128, fake, 1 << 30, None) == BC_ERR_INVALID_ARGUMENT
    assert g(fake, fake, fake, fake, None, fake, 1, 4, 4, 100, 100, 128, fake, 1 << 30, None) == BC_ERR_INVALID_ARGUMENT
    a = lib.bc_adaptive_attention
    a.argtypes = [P] * 7 + [ctypes.c_int] * 7 + [P, size_t, P]
    assert a(fake, fake, fake, fake, fake, fake, None, 1, 4, 4, 100, 100, 128, -1, fake, 1 << 30, None) == BC_ERR_INVALID_ARGUMENT
    f = lib.bc_append_attention
    f.argtypes = [P] * 8 + [ctypes.c_int] * 4 + [ctypes.c_int64, ctypes.c_int, P, size_t, P]
    assert f(*[fake] * 4, fake, fake, None, fake, 1, 4, 4, 128, 0, 16, fake, 1 << 30, None) == BC_ERR_INVALID_ARGUMENT
    assert f(*[fake] * 8, 1, 4, 4, 128, 0, 0, fake, 1 << 30, None) == BC_ERR_INVALID_ARGUMENT    # max_seq 0
    assert f(*[fake] * 8, 1, 4, 4, 128, -1, 16, fake, 1 << 30, None) == BC_ERR_INVALID_ARGUMENT  # current_len < 0
    assert f(*[fake] * 8, 1, 6, 4, 128, 0, 16, fake, 1 << 30, None) == BC_ERR_INVALID_ARGUMENT   # 6 % 4 != 0
    assert f(*[fake] * 8, 1, 4, 4, 100, 0, 16, fake, 1 << 30, None) == BC_ERR_UNSUPPORTED
    assert f(*[fake] * 8, 1, 4, 4, 128, 5, 16, fake, 1, None) == BC_ERR_WORKSPACE   # before the token is written
    r = lib.bc_reference_attention
    r.argtypes = [P] * 4 + [ctypes.c_int] * 5 + [P, size_t, P]
    assert r(fake, fake, fake, fake, 1, 4, 4, 100, 100, fake, 1 << 30, None) == BC_ERR_UNSUPPORTED
    h = lib.bc_head_mode_attention
    h.argtypes = [P] * 7 + [ctypes.c_int] * 6 + [P, size_t, P]
    modes = P(0x2000)
    assert h(*[fake] * 5, modes, fake, 1, 4, 4, 100, 100, 100, fake, 1 << 30, None) == BC_ERR_UNSUPPORTED
    assert h(*[fake] * 5, None, fake, 1, 4, 4, 100, 100, 128, fake, 1 << 30, None) == BC_ERR_INVALID_ARGUMENT
    assert h(fake, fake, None, fake, fake, modes, fake, 1, 4, 4, 100, 100, 128, fake, 1 << 30, None) == BC_ERR_INVALID_ARGUMENT
    assert h(*[fake] * 5, modes, fake, 1, 4, 4, 100, 100, 128, fake, 1, None) == BC_ERR_WORKSPACE
    # the allocation-free entry point rejects a shape whose partials exceed
    # its array before it looks the array up or launches anything
    na = lib.bc_attention_gqa_noalloc
    na.argtypes = [P] * 6 + [ctypes.c_int] * 6 + [P]
    assert na(*[fake] * 6, 4096, 64, 8, 1 << 20, 1 << 20, 128, None) == BC_ERR_WORKSPACE
    assert b"allocation-free" in lib.bc_last_error()
    ew = lib.bc_entropy_workspace_size
    ew.argtypes = [ctypes.c_int] * 3 + [ctypes.POINTER(size_t)]
    assert ew(1, 4, 100, ctypes.byref(n)) == BC_OK and n.value == 0        # one block per head
    assert ew(8, 32, 65536, ctypes.byref(n)) == BC_OK and n.value > 0      # key chunks
    assert ew(-1, 4, 100, ctypes.byref(n)) == BC_ERR_INVALID_ARGUMENT
    es = lib.bc_compute_head_entropy_ws
    es.argtypes = [P, P, P] + [ctypes.c_int] * 6 + [P, size_t, P]
    assert es(fake, fake, fake, 8, 32, 32, 65536, 65536, 128, fake, 1, None) == BC_ERR_WORKSPACE
    assert es(fake, fake, fake, 1, 6, 4, 100, 100, 128, None, 0, None) == BC_ERR_INVALID_ARGUMENT
    e = lib.bc_compute_head_entropy_gqa
    e.argtypes = [P, P, P] + [ctypes.c_int] * 6 + [P]
    assert e(fake, fake, fake, 1, 6, 4, 100, 100, 128, None) == BC_ERR_INVALID_ARGUMENT  # 6 % 4
    assert e(fake, fake, fake, 1, 4, 2, 100, 50, 128, None) == BC_ERR_INVALID_ARGUMENT   # stride < S
    assert e(fake, fake, None, 1, 4, 2, 100, 100, 128, None) == BC_ERR_INVALID_ARGUMENT  # null output
    assert e(fake, fake, fake, 1, 4, 2, 100, 100, 80, None) == BC_ERR_UNSUPPORTED


def test_workspace_covers_every_split_plan(lib):
    """The workspace bc_attention_workspace_size reports holds the split
    partials of the plan every attention mode launches, on devices of several
    CU counts (the plan depends on the CU count), over shapes where the
    policies' split counts differ: MHA and GQA groups 1-8, short and long
    contexts, the c1-c5 config shapes among them.  No launch: the plan is host
    arithmetic.  (On a host without a GPU each mode plans at its largest
    workgroups-per-CU policy, the case with the most splits.)"""
    size_t = ctypes.c_size_t
    f = lib.bc_attention_split_plan
    f.argtypes = [ctypes.c_int] * 7 + [ctypes.POINTER(ctypes.c_int), ctypes.POINTER(size_t),
                                       ctypes.POINTER(size_t)]
    ws = lib.bc_attention_workspace_size
    ws.argtypes = [ctypes.c_int] * 5 + [ctypes.POINTER(size_t)]
    shapes = [(8, 32, 32, 32768, 128), (8, 32, 32, 65536, 128), (4, 32, 8, 16384, 128),
              (4, 32, 8, 16640, 128), (2, 32, 8, 32768, 128), (1, 32, 8, 65536, 128),
              (16, 32, 8, 131072, 128), (1, 8, 1, 100000, 64), (3, 16, 2, 9000, 256),
              (1, 4, 4, 700, 96), (2, 64, 8, 50000, 128), (1, 32, 16, 4096, 128),
              (1, 1, 1, 1, 128), (1, 32, 8, 1 << 20, 128)]
    n, part, total, ref = ctypes.c_int(0), size_t(0), size_t(0), size_t(0)
    checked = 0
    for (B, Hq, Hkv, S, d) in shapes:
        for cu in (0, 80, 256, 304):
            for mode in range(4):
                assert f(mode, B, Hq, Hkv, S, d, cu, ctypes.byref(n), ctypes.byref(part),
                         ctypes.byref(total)) == BC_OK, lib.bc_last_error()
                assert 1 <= n.value <= 2048
                assert part.value == B * Hq * n.value * (d + 2) * 4
                assert part.value <= total.value, (
                    f"mode {mode} shape {(B, Hq, Hkv, S, d)} cu {cu}: plan writes "
                    f"{part.value} B, workspace {total.value} B")
                checked += 1
            if cu == 0:
                assert ws(B, Hq, Hkv, S, d, ctypes.byref(ref)) == BC_OK
                assert ref.value == total.value
    assert checked == len(shapes) * 16
    assert f(4, 1, 4, 4, 100, 128, 0, ctypes.byref(n), ctypes.byref(part),
             ctypes.byref(total)) == BC_ERR_INVALID_ARGUMENT


def test_wide_binary_plan(lib):
    """Binary MHA attention at d = 64, 128, 256 with one head per CU (and a
    context of at most 131072 keys) plans one split per head: one wide
    workgroup takes all of a head's keys and writes the output.  Other modes,
    GQA groups, the head dims without the matrix-core kernel, longer contexts
    and other head counts keep the split plans."""
    size_t = ctypes.c_size_t
    f = lib.bc_attention_split_plan
    f.argtypes = [ctypes.c_int] * 7 + [ctypes.POINTER(ctypes.c_int), ctypes.POINTER(size_t),
                                       ctypes.POINTER(size_t)]
    n, part, total = ctypes.c_int(0), size_t(0), size_t(0)

    def splits(mode, B, Hq, Hkv, S, d, cu):
        assert f(mode, B, Hq, Hkv, S, d, cu, ctypes.byref(n), ctypes.byref(part),
                 ctypes.byref(total)) == BC_OK, lib.bc_last_error()
        assert part.value == B * Hq * n.value * (d + 2) * 4 <= total.value
        return n.value

    assert splits(0, 8, 32, 32, 32768, 128, 256) == 1        # c2: 256 heads on 256 CUs
    assert splits(0, 4, 32, 32, 131072, 128, 128) == 1       # the longest wide context
    assert splits(0, 8, 32, 32, 32768, 128, 80) > 1          # 256 heads on 80 CUs
    assert splits(0, 8, 32, 32, 32768, 128, 512) > 1         # half a round
    assert splits(0, 4, 32, 32, 131136, 128, 128) > 1        # past the wide context
    assert splits(0, 8, 32, 32, 32768, 64, 256) == 1         # d = 64
    assert splits(0, 8, 32, 32, 32768, 256, 256) == 1        # d = 256
    assert splits(0, 8, 32, 32, 32768, 96, 256) > 1          # a VALU-kernel head dim
    assert splits(0, 8, 32, 8, 32768, 128, 64) > 1           # GQA groups
    assert splits(1, 8, 32, 32, 32768, 128, 256) > 1         # compensated
    assert splits(3, 8, 32, 32, 32768, 128, 256) > 1         # per-head modes


def test_extension_rejects_cpu_tensors():
    torch = pytest.importorskip("torch")
    import bitcache_amd
    if not bitcache_amd._HAS_EXTENSION:
        pytest.skip("extension not built")
    import bitcache_amd.functional as F
    x = torch.zeros((4, 128), dtype=torch.float16)
    with pytest.raises(AssertionError):
        F.encode(x)
    with pytest.raises(RuntimeError, match="ROCm"):
        bitcache_amd._C.binary_encode(x)
    with pytest.raises(RuntimeError):
        bitcache_amd.BitCache(1, 2, 128, 8, device="cpu")
    assert F.sizeof_binary_vec() == 36 and F.sizeof_residual_vec() == 130


def test_product_never_imports_oracle():
    """The product package must not import, call or read the oracle."""
    pkg = os.path.join(ROOT, "bitcache_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".cpp", ".hip", ".h")):
                text = open(os.path.join(dirpath, f)).read()
                assert "oracle" not in text.replace("oracles", ""), f"{f} mentions the oracle"
