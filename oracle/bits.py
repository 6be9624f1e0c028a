"""Bit-level helpers: raw views, ULP distance, RNE rounding, ULP size.

Test infrastructure only (see oracle/__init__.py).
"""

import numpy as np

# Precision p (significand bits incl. the implicit one) of each format.
PRECISION = {"float32": 24, "float16": 11, "bfloat16": 8}


def bits(t):
    """Raw bit patterns of a torch tensor as a flat numpy uint array.

    Reference tests/test_invariance.py:20-21 (`bits`): invariance is compared on
    bit patterns, never with allclose.
    """
    import torch

    u = {torch.float32: torch.int32, torch.float16: torch.int16, torch.bfloat16: torch.int16}
    x = t.detach().contiguous().reshape(-1).view(u[t.dtype]).cpu().numpy()
    return x.view(np.uint32 if x.dtype == np.int32 else np.uint16)


def ulp_distance(x, y, nbits):
    """IEEE754 ULP distance between two uint bit-pattern arrays of width nbits.

    Reference probe/probe.py:39-45: map sign-magnitude patterns onto a line of
    integers (negative values mirrored below zero) and subtract.
    """
    top = 1 << (nbits - 1)
    xi, yi = x.astype(np.int64), y.astype(np.int64)
    xo = np.where(xi >= top, top - xi, xi)
    yo = np.where(yi >= top, top - yi, yi)
    return np.abs(xo - yo)


def round_f32_to(x, name):
    """Round float32 values to `name` with round-to-nearest-even; returns float64
    values of the rounded numbers. NaN stays NaN, overflow goes to +-inf."""
    x = np.asarray(x, dtype=np.float32)
    if name == "float32":
        return x.astype(np.float64)
    if name == "float16":
        with np.errstate(over="ignore"):  # overflow rounds to +-inf, as intended
            return x.astype(np.float16).astype(np.float64)
    if name == "bfloat16":
        u = x.view(np.uint32).astype(np.uint64)
        lsb = (u >> 16) & 1
        r = ((u + 0x7FFF + lsb) >> 16) & 0xFFFF
        nan = np.isnan(x)
        r = np.where(nan, 0x7FC0, r).astype(np.uint32)
        return (r << 16).view(np.float32).astype(np.float64)
    raise ValueError(name)


def ulp_of(x, name):
    """Size of one unit in the last place of |x| in format `name` (float64).
    Subnormal spacing at the bottom of the range."""
    p = PRECISION[name]
    emin = {"float32": -126, "float16": -14, "bfloat16": -126}[name]
    ax = np.abs(np.asarray(x, dtype=np.float64))
    _, e = np.frexp(np.where(ax > 0, ax, 1.0))  # ax = m * 2**e, m in [0.5, 1)
    e = np.where(ax > 0, np.maximum(e - 1, emin), emin)
    return np.ldexp(1.0, (e - (p - 1)).astype(np.int64))
