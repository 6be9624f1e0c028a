"""Affine-quantized weight oracle. Test infrastructure only (see oracle/__init__.py).

unpack      -- restates reference _gemm.py:163-169 (the dequantizing B load of
               bi_qgemm): weight element k of row n is
               (word[n][k // (32 / bits)] >> (bits * (k % (32 / bits)))) & mask.
dequantize  -- reference _gemm.py:170-173: v = float(scale) * float(q) +
               float(bias) in fp32. The product is exact (at most 11 + 8
               significant bits), so v has one rounding. The reference keeps v
               in fp32: it is stored to a float B tile (_gemm.py:46, :80) and
               enters the product unrounded.
qgemm_f64   -- the exact value the reference's quantized GEMM approximates
               with fp32 arithmetic: float64 x @ v.T (x has at most 11
               significant bits and v 24, so every product is exact in
               float64).

Pinned in tests/test_oracle.py by hand-worked words (known answers), a planted
big-endian packing mistake, and closed-form weights whose fp32 values are not
representable in the element type (a planted element-type rounding of v fails).
"""

import numpy as np

from . import bits as _bits


def unpack(words, bits, K):
    """(N, K * bits / 32) uint32 words -> (N, K) integer codes."""
    per = 32 // bits
    w = np.asarray(words).astype(np.int64) & 0xFFFFFFFF
    N = w.shape[0]
    q = np.empty((N, K), dtype=np.int64)
    for k in range(K):
        q[:, k] = (w[:, k // per] >> (bits * (k % per))) & ((1 << bits) - 1)
    return q


def dequantize(words, scales, biases, group_size, bits):
    """(N, K) float64 array holding the fp32 dequantized weights."""
    s = np.asarray(scales, dtype=np.float64)
    b = np.asarray(biases, dtype=np.float64)
    K = np.asarray(words).shape[1] * (32 // bits)
    q = unpack(words, bits, K).astype(np.float64)
    g = np.arange(K) // group_size
    return (s[:, g] * q + b[:, g]).astype(np.float32).astype(np.float64)


def dequantize_to(words, scales, biases, group_size, bits, dtype_name):
    """The fp32 weights rounded once (RNE) to an element type: what a
    dequantize-then-dense path would multiply by."""
    v32 = dequantize(words, scales, biases, group_size, bits).astype(np.float32)
    return _bits.round_f32_to(v32, dtype_name).astype(np.float64)


def qgemm_f64(x, words, scales, biases, group_size, bits):
    """float64 x @ v.T with v the fp32 dequantized weights."""
    v = dequantize(words, scales, biases, group_size, bits)
    return np.asarray(x, dtype=np.float64) @ v.T
