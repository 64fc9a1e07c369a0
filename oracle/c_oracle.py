"""ctypes wrapper over the scalar C oracle (oracle/bitcache_oracle.c).

TEST INFRASTRUCTURE ONLY (imported by tests/ and tests/golden/make_golden.py).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        src = os.path.join(_HERE, "bitcache_oracle.c")
        if (not os.path.exists(_LIB_PATH)) or os.path.getmtime(_LIB_PATH) < os.path.getmtime(src):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        I = ctypes.c_int
        _lib.orc_half_to_float.restype = ctypes.c_float
        _lib.orc_half_to_float.argtypes = [ctypes.c_uint16]
        _lib.orc_float_to_half.restype = ctypes.c_uint16
        _lib.orc_float_to_half.argtypes = [ctypes.c_float]
        _lib.orc_binary_encode.argtypes = [P, I, I, P, P, P]
        _lib.orc_residual_encode.argtypes = [P, P, P, I, I, P, P]
        _lib.orc_query_prep.argtypes = [P, I, I, P, P]
        _lib.orc_query_prep_tree.argtypes = [P, I, I, P, P]
        _lib.orc_xnor_scores.argtypes = [P, ctypes.c_float, P, P, I, I, P, P]
        _lib.orc_entropy.restype = ctypes.c_float
        _lib.orc_entropy.argtypes = [P, I]
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def half_to_float(h: int) -> float:
    return lib().orc_half_to_float(h)


def float_to_half_bits(f: float) -> int:
    return lib().orc_float_to_half(f)


def binary_encode(x16: np.ndarray):
    x = np.ascontiguousarray(x16, dtype=np.float16)
    n, d = x.shape
    words = np.zeros((n, d // 32), np.uint32)
    scale = np.zeros(n, np.uint16)
    mean = np.zeros(n, np.float32)
    lib().orc_binary_encode(_p(x.view(np.uint16)), n, d, _p(words), _p(scale), _p(mean))
    return words, scale.view(np.float16), mean


def residual_encode(x16: np.ndarray, words: np.ndarray, s32: np.ndarray):
    x = np.ascontiguousarray(x16, dtype=np.float16)
    n, d = x.shape
    words = np.ascontiguousarray(words, np.uint32)
    s32 = np.ascontiguousarray(s32, np.float32)
    codes = np.zeros((n, d), np.int8)
    rs = np.zeros(n, np.uint16)
    lib().orc_residual_encode(_p(x.view(np.uint16)), _p(words), _p(s32), n, d, _p(codes), _p(rs))
    return codes, rs.view(np.float16)


def query_prep(q16: np.ndarray, tree: bool = False):
    q = np.ascontiguousarray(q16, dtype=np.float16)
    nq, d = q.shape
    qw = np.zeros((nq, d // 32), np.uint32)
    sq = np.zeros(nq, np.float32)
    fn = lib().orc_query_prep_tree if tree else lib().orc_query_prep
    fn(_p(q.view(np.uint16)), nq, d, _p(qw), _p(sq))
    return qw, sq


def xnor_scores(qw: np.ndarray, sq: float, kw: np.ndarray, ks16: np.ndarray, d: int):
    kw = np.ascontiguousarray(kw, np.uint32)
    ks = np.ascontiguousarray(ks16, np.float16).view(np.uint16)
    qw = np.ascontiguousarray(qw, np.uint32)
    S = kw.shape[0]
    pc = np.zeros(S, np.int32)
    xd = np.zeros(S, np.float32)
    lib().orc_xnor_scores(_p(qw), float(sq), _p(kw), _p(ks), S, d, _p(pc), _p(xd))
    return pc, xd


def entropy(scores: np.ndarray) -> float:
    s = np.ascontiguousarray(scores, np.float32)
    return float(lib().orc_entropy(_p(s), s.shape[0]))
