"""Batch-invariant single-pass scaled dot product attention.

Mirrors reference mlx_batch_invariant/_attention.py:173-250 (mask
normalisation, validation, sinks, launch) on top of the HIP kernels in
csrc/ (bi_sdpa.hip: fp32 on the vector ALUs; bi_sdpa_mfma_kernel.h: bf16 and
f16 on matrix cores), reached through the C ABI ``bi_sdpa`` (include/bi.h).

One workgroup owns the entire reduction over the keys for each of its query
rows. fp32 splits it into 32 partial online softmaxes by key index (key i
belongs to partial i mod 32); bf16/f16 into 4 chains of 32-key blocks (block b
belongs to chain b mod 4); the partials are combined in a fixed order. Nothing
in that order depends on the number of query rows, the batch, or how far the
key sequence extends past the keys a row can see.
"""

import ctypes
import math

import torch

from . import _lib

PARTIALS = 32     # partial softmaxes per row = stride over the key sequence
GROUP_LANES = 8   # lanes that share one key's dot product
# Built (D, V) head-dim pairs: D for queries and keys, V for values
# (csrc/bi_sdpa_args.h BI_SDPA_DIM_PAIRS).
HEAD_DIMS = tuple((d, d) for d in range(32, 513, 32)) + (
    (192, 128), (128, 64), (64, 128), (256, 128), (128, 256), (576, 512))
HEAD_DIM_MULTIPLE = 32      # the reference's own requirement (_attention.py:224-227)

_SUPPORTED = (torch.float32, torch.float16, torch.bfloat16)


def supported_head_dims(D, V):
    return (D, V) in HEAD_DIMS


def _mask_args(mask, B, H, qL, N, dtype):
    """Returns (mask tensor or None, (b, h, q) element strides, mode).

    Reference _attention.py:173-202: None -> no mask, "causal" -> causal,
    otherwise an additive or boolean array broadcastable to (B, H, qL, N).
    A boolean mask keeps the keys where it is True.
    """
    if mask is None:
        return None, (0, 0, 0), _lib.MASK_NONE
    if isinstance(mask, str):
        if mask != "causal":
            raise ValueError("string mask must be 'causal', got %r" % (mask,))
        return None, (0, 0, 0), _lib.MASK_CAUSAL

    m = mask
    if m.dtype == torch.bool:
        m = torch.where(m, torch.zeros((), dtype=dtype, device=m.device),
                        torch.full((), float("-inf"), dtype=dtype, device=m.device))
    m = m.to(dtype)
    if m.ndim > 4:
        raise ValueError("mask must have at most 4 dimensions, got %d" % mask.ndim)
    while m.ndim < 4:
        m = m.unsqueeze(0)
    Bm, Hm, Lm, Nm = m.shape
    if Nm != N or Lm not in (1, qL) or Hm not in (1, H) or Bm not in (1, B):
        raise ValueError("mask shape %s is not broadcastable to (%d, %d, %d, %d)"
                         % (tuple(m.shape), B, H, qL, N))
    m = m.contiguous()
    strides = (0 if Bm == 1 else Hm * Lm * N, 0 if Hm == 1 else Lm * N, 0 if Lm == 1 else N)
    return m, strides, _lib.MASK_ARRAY


def _kernel_view(t):
    """t itself if the kernel can read it in place (last dim contiguous, 16-byte
    aligned rows and base), else a contiguous copy."""
    if t.data_ptr() % 16 == 0:
        if t.is_contiguous() and (t.shape[-1] * t.element_size()) % 16 == 0:
            return t
        ce = 16 // t.element_size()
        st = t.stride()
        if st[-1] == 1 and all(s % ce == 0 for s in st[:-1]):
            return t
    return t.contiguous()


_NO_MASK_STRIDES = _lib.i64_array((0, 0, 0))
_I64x9 = ctypes.c_int64 * 9


def _sdpa(q, k, v, scale, mask_mode, mask, mstrides, causal_offset, sinks):
    """Launch after validation: q (B,H,qL,D), k (B,Hkv,N,D), v (B,Hkv,N,V).
    While torch.compile traces, the launch is recorded as the opaque op
    mlx_bi::sdpa."""
    if torch.compiler.is_compiling():
        from . import _ops  # noqa: F401  (registers the ops)

        return torch.ops.mlx_bi.sdpa(q, k, v, float(scale), int(mask_mode), mask,
                                     [int(x) if isinstance(x, int) else x for x in mstrides],
                                     int(causal_offset), sinks)
    return _sdpa_eager(q, k, v, scale, mask_mode, mask, mstrides, causal_offset, sinks)


def _sdpa_eager(q, k, v, scale, mask_mode, mask, mstrides, causal_offset, sinks, shape=None):
    """The launch; `shape` forces a launch shape (bi_sdpa_with_shape,
    include/bi_testing.h) instead of the one bi_sdpa picks."""
    B, H, qL, D = q.shape
    _, Hkv, N, _ = k.shape
    V = v.shape[-1]
    out = torch.empty((B, H, qL, V), dtype=q.dtype, device=q.device)
    if out.numel() == 0:
        return out
    q, k, v = _kernel_view(q), _kernel_view(k), _kernel_view(v)
    qs, ks, vs = q.stride(), k.stride(), v.stride()
    strides = _I64x9(qs[0], qs[1], qs[2], ks[0], ks[1], ks[2], vs[0], vs[1], vs[2])
    L = _lib.lib()
    ms = _NO_MASK_STRIDES if mask is None else _lib.i64_array(mstrides)
    args = (q.data_ptr(), k.data_ptr(), v.data_ptr(),
            mask.data_ptr() if mask is not None else None, ms,
            sinks.data_ptr() if sinks is not None else None, out.data_ptr(),
            B, H, Hkv, qL, N, D, V, strides, float(scale), int(mask_mode),
            int(causal_offset), _lib.DTYPE_CODES[q.dtype])
    stream, switch = _lib.launch_stream(q.device)
    if shape is None:
        fn, tail = L.bi_sdpa, (stream,)
    else:
        fn, tail = L.bi_sdpa_with_shape, (int(shape), stream)
    if switch:
        with torch.cuda.device(q.device):
            rc = fn(*args, *tail)
    else:
        rc = fn(*args, *tail)
    if rc:
        _lib.check(rc, "bi_sdpa")
    return out


def launch_shape(q, k, v, mask_mode=_lib.MASK_NONE):
    """The launch shape bi_sdpa picks for these operands and mask mode
    (include/bi_testing.h): _lib.SDPA_ROWS ... for bf16/f16, log2(query heads
    per workgroup) for fp32."""
    B, H, qL, D = q.shape
    L = _lib.lib()
    rc = L.bi_sdpa_pick_shape(B, H, k.shape[1], qL, D, v.shape[-1], _lib.DTYPE_CODES[q.dtype],
                              int(mask_mode), 0)
    if rc < 0:
        _lib.check(rc, "bi_sdpa_pick_shape")
    return rc


def scaled_dot_product_attention(q, k, v, *, scale=None, mask=None, sinks=None):
    """Bitwise-invariant SDPA. ``q`` is (B, H, L, D), ``k``/``v`` are (B, Hkv, N, ...).

    ``mask`` may be ``None``, ``"causal"`` (aligned to the end of the key
    sequence: query row s sees keys i <= N - L + s), or an additive/boolean
    array broadcastable over the batch, head and query dimensions. ``sinks`` is
    an optional per-query-head logit of shape ``(H,)``. A row whose keys are all
    masked is 0. Reference _attention.py:205-250.
    """
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("q, k and v must be 4-dimensional (B, H, L, D)")
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError("q, k and v must share a dtype")
    if q.dtype not in _SUPPORTED:
        raise ValueError("unsupported dtype %s" % q.dtype)

    B, H, qL, D = q.shape
    Bk, Hkv, N, Dk = k.shape
    Bv, Hv, Nv, V = v.shape
    if (Bk, Hv, Nv, Dk) != (B, Hkv, N, D) or Bv != B:
        raise ValueError("inconsistent q/k/v shapes: %s %s %s"
                         % (tuple(q.shape), tuple(k.shape), tuple(v.shape)))
    if H % Hkv:
        raise ValueError("head count %d is not a multiple of kv head count %d" % (H, Hkv))
    if D % HEAD_DIM_MULTIPLE or V % HEAD_DIM_MULTIPLE:
        raise ValueError("head dimensions must be multiples of %d, got D=%d V=%d"
                         % (HEAD_DIM_MULTIPLE, D, V))
    if not supported_head_dims(D, V):
        raise NotImplementedError("head dimensions D=%d V=%d are not built (built (D, V): %s)"
                                  % (D, V, HEAD_DIMS))

    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    m, mstrides, mode = _mask_args(mask, B, H, qL, N, q.dtype)
    if sinks is not None:
        if tuple(sinks.shape) != (H,):
            raise ValueError("sinks must have shape (%d,), got %s" % (H, tuple(sinks.shape)))
        sinks = sinks.to(q.dtype).contiguous()
    dev = q.device
    devs = (q, k, v) if m is None and sinks is None else \
        [q, k, v] + ([m] if m is not None else []) + ([sinks] if sinks is not None else [])
    if not q.is_cuda or any(t.device != dev for t in devs[1:]):
        raise ValueError("batch-invariant kernels run on the GPU; all operands must be "
                         "on one cuda device")
    return _sdpa(q, k, v, scale, mode, m, mstrides, N - qL, sinks)
