"""Shared helpers for the test suite (mirrors reference tests/test_invariance.py:14-33)."""

import numpy as np
import torch

from oracle.bits import bits  # noqa: F401  (re-exported for the tests)

BATCHES = [1, 2, 3, 5, 8, 16, 31, 32, 33, 64, 128, 256]
DTYPES = [("float32", torch.float32), ("float16", torch.float16), ("bfloat16", torch.bfloat16)]


def rn(shape, dtype, seed, std=1.0, device="cpu"):
    """Seeded N(0, std^2) values rounded to dtype (CPU generator, then moved)."""
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g, dtype=torch.float32) * std).to(dtype).to(device)


def batch_with(ref, pool, B, idx):
    """Batch of size B holding `ref` at position `idx` and pool rows elsewhere
    (reference tests/test_invariance.py:28-33)."""
    if B == 1:
        return ref
    parts = ([pool[:idx]] if idx > 0 else []) + [ref] + ([pool[idx + 1:B]] if idx + 1 < B else [])
    return torch.cat(parts).contiguous()


def f64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def ndiff(a, b):
    return int((bits(a) != bits(b)).sum())


def pack_codes(q, bits):
    """(N, K) integer codes -> (N, K * bits / 32) int32 words, little-endian
    within each word (the packing the quantized kernels read)."""
    q = np.asarray(q, dtype=np.int64)
    per = 32 // bits
    N, K = q.shape
    shifts = np.arange(per, dtype=np.int64) * bits
    words = (q.reshape(N, K // per, per) << shifts).sum(-1)
    return torch.from_numpy((words & 0xFFFFFFFF).astype(np.uint32).view(np.int32))


def closed_form_quant(M, N, K, group_size, bits, dtype, seed):
    """Quantized weights whose fp32 values need more significant bits than the
    element type holds, and small-integer activations, so that the exact
    x @ v.T is reached by any fp32 accumulation order (every partial sum is a
    multiple of 2^-11 below 2^13). Returns torch CPU tensors (x, words,
    scales, biases) and the exact float64 product."""
    g = np.random.default_rng(seed)
    G = K // group_size
    assert 9 * K < 2 ** 13
    scales = 2.0 ** g.integers(-11, -8, size=(N, G))            # 2^-11 .. 2^-9
    biases = g.choice([1.0, -1.0, 1.5, -1.25], size=(N, G))
    q = g.integers(0, 1 << bits, size=(N, K))
    x = g.integers(-3, 4, size=(M, K)).astype(np.float64)
    v = scales.repeat(group_size, axis=1) * q + biases.repeat(group_size, axis=1)
    exact = x @ v.T
    to = lambda a: torch.from_numpy(a.astype(np.float32)).to(dtype)
    return to(x), pack_codes(q, bits), to(scales), to(biases), exact
