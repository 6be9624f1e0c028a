"""Attention oracles. Test infrastructure only (see oracle/__init__.py).

sdpa_f64      -- float64 softmax attention with GQA head mapping, masks, sinks
                 and the reference's conventions (fully masked row -> 0,
                 mask values <= -3e38 drop the key, causal aligned by
                 causal_offset). Accuracy oracle of reference
                 tests/test_invariance.py:408-432.
sdpa_fixed32  -- the fixed-order fp32 restatement of reference
                 _attention.py:68-148 (oracle/csrc/oracle.c: oracle_sdpa).
"""

import math

import numpy as np

from . import bits as _bits
from .gemm import clib, fptr


def _mask_value(mask, b, h, s):
    """Row of an (already broadcast-shaped, 4-D) additive mask."""
    Bm, Hm, Lm, _ = mask.shape
    return mask[0 if Bm == 1 else b, 0 if Hm == 1 else h, 0 if Lm == 1 else s]


def sdpa_f64(q, k, v, scale=None, mask=None, sinks=None, causal_offset=None):
    """q (B,H,qL,D), k (B,Hkv,N,D), v (B,Hkv,N,V) float arrays; mask: None, or a
    4-D additive float array broadcastable to (B,H,qL,N); causal_offset: if not
    None, key i is visible to row s iff i <= s + causal_offset. Returns float64
    (B,H,qL,V)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    B, H, qL, D = q.shape
    Hkv, N = k.shape[1], k.shape[2]
    V = v.shape[3]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    g = H // Hkv
    out = np.zeros((B, H, qL, V))
    for b in range(B):
        for h in range(H):
            kk, vv = k[b, h // g], v[b, h // g]
            for s in range(qL):
                sc = (kk @ q[b, h, s]) * scale
                use = np.ones(N, dtype=bool)
                if causal_offset is not None:
                    use &= np.arange(N) <= s + causal_offset
                if mask is not None:
                    mv = np.asarray(_mask_value(mask, b, h, s), dtype=np.float64)
                    use &= mv > -3.0e38
                    sc = sc + np.where(use, mv, 0.0)
                logits = list(sc[use])
                if sinks is not None:
                    logits.append(float(sinks[h]))
                if not use.any():
                    continue  # fully masked row -> 0 (reference _attention.py:139)
                mx = max(logits)
                w = np.exp(sc[use] - mx)
                den = w.sum() + (math.exp(float(sinks[h]) - mx) if sinks is not None else 0.0)
                out[b, h, s] = (w @ vv[use]) / den
    return out


def sdpa_fixed32(q, k, v, scale=None, mask=None, sinks=None, causal_offset=None,
                 out_dtype="float32"):
    """Reference-order fp32 restatement (C), then one RNE rounding to out_dtype.
    Arguments as sdpa_f64, holding the (already rounded) input values."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    B, H, qL, D = q.shape
    Hkv, N = k.shape[1], k.shape[2]
    V = v.shape[3]
    if D > 1024 or V > 1024:
        raise ValueError("oracle_sdpa handles head dims up to 1024")
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    mode, ms, m = 0, (0, 0, 0), None
    if causal_offset is not None:
        mode = 1
    if mask is not None:
        if mode == 1:
            raise ValueError("causal and an array mask together are not a reference mode")
        mode = 2
        m = np.ascontiguousarray(mask, dtype=np.float32)
        Bm, Hm, Lm, _ = m.shape
        ms = (0 if Bm == 1 else Hm * Lm * N, 0 if Hm == 1 else Lm * N, 0 if Lm == 1 else N)
    sk = None if sinks is None else np.ascontiguousarray(sinks, dtype=np.float32)
    out = np.empty((B, H, qL, V), dtype=np.float32)
    clib().oracle_sdpa(fptr(q), fptr(k), fptr(v), fptr(m), ms[0], ms[1], ms[2], fptr(sk),
                       fptr(out), B, H, Hkv, qL, N, D, V, float(scale), mode,
                       int(causal_offset or 0))
    return _bits.round_f32_to(out, out_dtype)
