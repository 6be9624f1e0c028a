"""Affine-quantized weight oracle. Test infrastructure only (see oracle/__init__.py).

unpack      -- restates reference _gemm.py:163-173 (the dequantizing B load of
               bi_qgemm): weight element k of row n is
               (word[n][k // (32 / bits)] >> (bits * (k % (32 / bits)))) & mask.
dequantize  -- scale * q + bias in fp32 (reference :172-173; the product is
               exact, so the fp32 result has one rounding), then one rounding
               to the element type (MLX dequantize returns the scales' dtype).

Pinned in tests/test_oracle.py by hand-worked words (known answers) and a
planted big-endian packing mistake.
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


def dequantize(words, scales, biases, group_size, bits, dtype_name):
    """(N, K) float64 values of the weight as the element type holds them."""
    s = np.asarray(scales, dtype=np.float64)
    b = np.asarray(biases, dtype=np.float64)
    K = np.asarray(words).shape[1] * (32 // bits)
    q = unpack(words, bits, K).astype(np.float64)
    g = np.arange(K) // group_size
    v32 = (s[:, g] * q + b[:, g]).astype(np.float32)  # exact product, one rounding
    return _bits.round_f32_to(v32, dtype_name).astype(np.float64)
