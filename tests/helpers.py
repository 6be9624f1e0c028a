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
