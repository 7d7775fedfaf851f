"""ctypes loader for oracle/liboracle_c.so — TEST INFRASTRUCTURE ONLY.

Wraps the C restatement (oracle_c.c) with numpy arrays.  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg use it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_c.so")
_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        LL = ctypes.c_longlong
        I = ctypes.c_int
        L.oracle_decode_attention.argtypes = [P, P, P, P, P, P, LL, LL, I, P, I]
        L.oracle_decode_attention.restype = I
        L.oracle_prefill_attention.argtypes = [P, P, P, P, P, P, LL, LL, I, I, P, I]
        L.oracle_prefill_attention.restype = I
        L.oracle_gemm_i8_i32.argtypes = [P, P, P, LL, LL, LL, I]
        L.oracle_gemm_i8_i32.restype = I
        L.oracle_max_threads.argtypes = []
        L.oracle_max_threads.restype = I
        _lib = L
    return _lib


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def max_threads() -> int:
    return lib().oracle_max_threads()


def decode_attention(Qi, Ki, Vi, sQ, sK, sV, threads: int = 0):
    Qi = _c(Qi, np.int8)
    BH, D = Qi.shape
    Ki, Vi = _c(Ki, np.int8), _c(Vi, np.int8)
    S = Ki.shape[1]
    sQ, sK, sV = _c(sQ, np.float32), _c(sK, np.float32), _c(sV, np.float32)
    out = np.empty((BH, D), np.float64)
    rc = lib().oracle_decode_attention(_p(Qi), _p(Ki), _p(Vi), _p(sQ), _p(sK), _p(sV), BH, S, D,
                                       _p(out), threads)
    if rc:
        raise RuntimeError("oracle_decode_attention failed")
    return out


def prefill_attention(Qi, Ki, Vi, sQ, sK, sV, causal=False, threads: int = 0):
    Qi = _c(Qi, np.int8)
    BH, S, D = Qi.shape
    Ki, Vi = _c(Ki, np.int8), _c(Vi, np.int8)
    sQ, sK, sV = _c(sQ, np.float32), _c(sK, np.float32), _c(sV, np.float32)
    out = np.empty((BH, S, D), np.float64)
    rc = lib().oracle_prefill_attention(_p(Qi), _p(Ki), _p(Vi), _p(sQ), _p(sK), _p(sV), BH, S,
                                        D, int(bool(causal)), _p(out), threads)
    if rc:
        raise RuntimeError("oracle_prefill_attention failed")
    return out


def gemm_i8_i32(A, B, threads: int = 0):
    A, B = _c(A, np.int8), _c(B, np.int8)
    M, K = A.shape
    K2, N = B.shape
    assert K == K2
    C = np.empty((M, N), np.int32)
    if lib().oracle_gemm_i8_i32(_p(A), _p(B), _p(C), M, N, K, threads):
        raise OverflowError("int32 accumulator overflow")
    return C
