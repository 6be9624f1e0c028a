"""GEMM oracles. Test infrastructure only (see oracle/__init__.py).

gemm_f64      -- exact-product float64 reference, the accuracy oracle of
                 reference tests/test_invariance.py:114-146 (a64 @ b64).
gemm_fixed32  -- the fixed-order fp32 restatement of reference
                 _gemm.py:62-129 (oracle/csrc/oracle.c: oracle_gemm), rounded
                 once to the element type.
"""

import ctypes
import os

import numpy as np

from . import bits as _bits

_LIB = None


def clib():
    global _LIB
    if _LIB is None:
        path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "liboracle.so")
        if not os.path.exists(path):
            from . import build
            build.build(verbose=False)
        L = ctypes.CDLL(path)
        f32p = ctypes.POINTER(ctypes.c_float)
        i64 = ctypes.c_int64
        L.oracle_gemm.argtypes = [f32p, f32p, f32p, f32p, i64, i64, i64, ctypes.c_int,
                                  ctypes.c_float, ctypes.c_float]
        L.oracle_gemm.restype = None
        L.oracle_gemm_bt.argtypes = [f32p, f32p, f32p, i64, i64, i64]
        L.oracle_gemm_bt.restype = None
        L.oracle_sdpa.argtypes = [f32p, f32p, f32p, f32p, i64, i64, i64, f32p, f32p,
                                  i64, i64, i64, i64, i64, i64, i64, ctypes.c_float,
                                  ctypes.c_int, i64]
        L.oracle_sdpa.restype = None
        _LIB = L
    return _LIB


def fptr(x):
    if x is None:
        return None
    return x.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def gemm_f64(a, b, bias=None, alpha=1.0, beta=1.0, trans_b=False):
    """float64 a @ B (B = b.T if trans_b) with the reference epilogue
    alpha * acc + beta * bias (reference _gemm.py:125-127). Products of fp32
    values are exact in float64 when both have at most 26 significant bits,
    which covers bf16 and f16 inputs exactly."""
    a64 = np.asarray(a, dtype=np.float64)
    b64 = np.asarray(b, dtype=np.float64)
    if trans_b:
        b64 = b64.T
    acc = a64 @ b64
    if bias is not None:
        acc = alpha * acc + beta * np.asarray(bias, dtype=np.float64)
    return acc


def abs_products(a, b, trans_b=False):
    """sum_k |a[m, k] * B[k, n]| in float64 (the scale of the cancellation floor)."""
    a64 = np.abs(np.asarray(a, dtype=np.float64))
    b64 = np.abs(np.asarray(b, dtype=np.float64))
    return a64 @ (b64.T if trans_b else b64)


def gemm_fixed32(a, b, bias=None, alpha=1.0, beta=1.0, trans_b=False, out_dtype="float32"):
    """Reference-order fp32 accumulation (C), then one RNE rounding to out_dtype.
    a, b, bias are float32 arrays holding the (already rounded) input values."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    M, K = a.shape
    N = b.shape[0] if trans_b else b.shape[1]
    out = np.empty((M, N), dtype=np.float32)
    bias_c = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    clib().oracle_gemm(fptr(a), fptr(b), fptr(bias_c), fptr(out), M, N, K, int(trans_b),
                       float(alpha), float(beta))
    return _bits.round_f32_to(out, out_dtype)
