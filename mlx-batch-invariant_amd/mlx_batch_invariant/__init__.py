"""Batch-invariant GEMM and attention for PyTorch on AMD Instinct MI355X.

Every function here returns bitwise identical results for a given row of input
regardless of what else was in the batch, how many query tokens were submitted
together, how long the key sequence has grown, or whether the call was captured
in a HIP graph.

    import mlx_batch_invariant as bi

    with bi.batch_invariant_mode():
        logits = model(tokens)

Drop-in for the reference package's API (reference mlx_batch_invariant/
__init__.py): the same functions and context manager, re-targeted from MLX to
torch. The kernels are hand-written CDNA4 HIP (csrc/), reached through the C
ABI in include/bi.h.
"""

import contextlib
import math

import torch
import torch.nn.functional as F

from ._attention import HEAD_DIMS, scaled_dot_product_attention, supported_head_dims
from ._attention import _mask_args, _sdpa
from ._gemm import TILE, addmm, geometries, linear, matmul
from ._quant import (QUANT_BITS, QuantizedLinear, dequantize, quantize, quantized_linear,
                     quantized_matmul)

__all__ = [
    "matmul",
    "addmm",
    "linear",
    "scaled_dot_product_attention",
    "quantized_linear",
    "quantized_matmul",
    "quantize",
    "dequantize",
    "QuantizedLinear",
    "QUANT_BITS",
    "batch_invariant_mode",
    "is_enabled",
    "TILE",
    "HEAD_DIMS",
    "__version__",
]

__version__ = "0.2.0"

_depth = 0
_strict_flag = True
_FLOATS = (torch.float32, torch.float16, torch.bfloat16)


def is_enabled():
    """True inside a :func:`batch_invariant_mode` block (reference __init__.py:41-43)."""
    return _depth > 0


def _strict():
    """strict= of the outermost active batch_invariant_mode."""
    return _strict_flag


def _unsupported(what, strict, fallback, *args, **kwargs):
    """Reference __init__.py:46-53: raise under strict, else call stock torch."""
    if strict:
        raise NotImplementedError(
            "%s is not batch-invariant in this build. Pass strict=False to "
            "batch_invariant_mode() to fall back to stock PyTorch for this call, "
            "accepting that its result is not invariant." % what
        )
    return fallback(*args, **kwargs)


def _kernel_ready(*tensors):
    """The operands can go to the invariant kernels: one cuda device, a built
    float dtype, and no autograd graph to record (the kernels have no backward)."""
    ts = [t for t in tensors if t is not None]
    if not all(isinstance(t, torch.Tensor) for t in ts):
        return False
    dev, dt = ts[0].device, ts[0].dtype
    if dev.type != "cuda" or dt not in _FLOATS:
        return False
    if any(t.device != dev or t.dtype != dt for t in ts):
        return False
    if torch.is_grad_enabled() and any(t.requires_grad for t in ts):
        return False
    return True


class _Patches:
    """Attribute patches that restore exactly what was there before."""

    def __init__(self):
        self._saved = []

    def set(self, owner, name, value):
        had_own = name in vars(owner)
        self._saved.append((owner, name, had_own, vars(owner).get(name)))
        setattr(owner, name, value)

    def restore(self):
        for owner, name, had_own, old in reversed(self._saved):
            if had_own:
                setattr(owner, name, old)
            else:
                delattr(owner, name)
        self._saved = []


@contextlib.contextmanager
def batch_invariant_mode(strict=True):
    """Route torch.matmul, torch.mm, torch.addmm, ``@``, nn.Linear / F.linear
    and F.scaled_dot_product_attention through the invariant kernels
    (torch.bmm and torch.einsum are not routed: they stay stock and
    batch-variant).

    Calls the kernels cannot make invariant raise ``NotImplementedError``. With
    ``strict=False`` they fall back to stock PyTorch instead, which means the
    result is no longer guaranteed bitwise reproducible -- use it to find out
    what a model needs, not to ship. Reference __init__.py:56-147.

    Process-global and not thread-safe, like the reference: it patches module
    attributes. Nesting is counted; only the outermost exit restores.
    """
    global _depth, _strict_flag

    if _depth:  # already patched; nesting must not stack another set of shims
        _depth += 1
        try:
            yield
        finally:
            _depth -= 1
        return

    saved = {
        "matmul": torch.matmul,
        "addmm": torch.addmm,
        "tensor_matmul_op": torch.Tensor.__matmul__,
        "tensor_matmul": torch.Tensor.matmul,
        "mm": torch.mm,
        "tensor_mm": torch.Tensor.mm,
        "linear_forward": torch.nn.Linear.forward,
        "F_linear": F.linear,
        "sdpa": F.scaled_dot_product_attention,
    }

    def bi_matmul(a, b, *args, **kwargs):
        if (args or kwargs or not _kernel_ready(a, b) or a.ndim < 2 or b.ndim != 2):
            return _unsupported(
                "matmul with shapes %s @ %s" % (_shape(a), _shape(b)),
                strict, saved["matmul"], a, b, *args, **kwargs)
        return matmul(a, b)

    def bi_mm(a, b, *args, **kwargs):
        # torch.mm takes two 2-D matrices; the same kernel as matmul.
        if (args or kwargs or not _kernel_ready(a, b) or a.ndim != 2 or b.ndim != 2):
            return _unsupported(
                "mm with shapes %s @ %s" % (_shape(a), _shape(b)),
                strict, saved["mm"], a, b, *args, **kwargs)
        return matmul(a, b)

    def bi_addmm(c, a, b, *args, beta=1, alpha=1, **kwargs):
        if (args or kwargs or not _kernel_ready(c, a, b) or a.ndim < 2 or b.ndim != 2
                or c.ndim != 1 or c.shape[0] != b.shape[-1] or beta == 0):
            return _unsupported(
                "addmm with shapes %s, %s @ %s" % (_shape(c), _shape(a), _shape(b)),
                strict, saved["addmm"], c, a, b, *args, beta=beta, alpha=alpha, **kwargs)
        return addmm(c, a, b, alpha, beta)

    def bi_linear(x, w, bias=None):
        # The reference routes x.ndim >= 2 and lets 1-D input through stock
        # (reference __init__.py:125-129); here a 1-D input is routed as a
        # one-row batch so it gets the same bits as that row in any batch.
        if not isinstance(w, torch.Tensor) or w.ndim != 2 or not isinstance(x, torch.Tensor) \
                or x.ndim < 1:
            return saved["F_linear"](x, w, bias)
        if not _kernel_ready(x, w, bias):
            return _unsupported("linear with shapes %s, %s" % (_shape(x), _shape(w)),
                                strict, saved["F_linear"], x, w, bias)
        if x.ndim == 1:
            return linear(x.unsqueeze(0), w, bias).squeeze(0)
        return linear(x, w, bias)

    def bi_linear_forward(self, x):
        return bi_linear(x, self.weight, self.bias)

    def bi_sdpa(query, key, value, attn_mask=None, dropout_p=0.0, is_causal=False,
                scale=None, enable_gqa=False, **kwargs):
        args = (query, key, value)
        kw = dict(attn_mask=attn_mask, dropout_p=dropout_p, is_causal=is_causal, scale=scale,
                  enable_gqa=enable_gqa, **kwargs)
        ok = (not kwargs and _kernel_ready(query, key, value) and query.ndim == 4
              and key.ndim == 4 and value.ndim == 4 and dropout_p == 0.0
              and supported_head_dims(query.shape[-1], value.shape[-1])
              and key.shape[-1] == query.shape[-1]
              and query.shape[0] == key.shape[0] == value.shape[0]
              and key.shape[1:3] == value.shape[1:3]
              and (query.shape[1] == key.shape[1]
                   or (enable_gqa and query.shape[1] % key.shape[1] == 0))
              and not (is_causal and attn_mask is not None)
              and (attn_mask is None or (isinstance(attn_mask, torch.Tensor)
                                         and attn_mask.device == query.device)))
        if not ok:
            return _unsupported("attention with shapes %s, %s, %s"
                                % (_shape(query), _shape(key), _shape(value)),
                                strict, saved["sdpa"], *args, **kw)
        B, H, qL, D = query.shape
        N = key.shape[2]
        sc = 1.0 / math.sqrt(D) if scale is None else float(scale)
        if is_causal:
            # torch's is_causal is aligned to the start: row s sees keys i <= s.
            return _sdpa(query, key, value, sc, 1, None, (0, 0, 0), 0, None)
        try:
            m, mstrides, mode = _mask_args(attn_mask, B, H, qL, N, query.dtype)
        except ValueError:
            return _unsupported("attention mask of shape %s" % (_shape(attn_mask),),
                                strict, saved["sdpa"], *args, **kw)
        return _sdpa(query, key, value, sc, mode, m, mstrides, 0, None)

    patches = _Patches()
    patches.set(torch, "matmul", bi_matmul)
    patches.set(torch, "addmm", bi_addmm)
    patches.set(torch.Tensor, "__matmul__", lambda a, b: bi_matmul(a, b))
    patches.set(torch.Tensor, "matmul", lambda a, b: bi_matmul(a, b))
    patches.set(torch, "mm", bi_mm)
    patches.set(torch.Tensor, "mm", lambda a, b: bi_mm(a, b))
    patches.set(torch.nn.Linear, "forward", bi_linear_forward)
    patches.set(F, "linear", bi_linear)
    patches.set(F, "scaled_dot_product_attention", bi_sdpa)
    _depth = 1
    _strict_flag = bool(strict)
    try:
        yield
    finally:
        _depth = 0
        _strict_flag = True
        patches.restore()


def _shape(t):
    return tuple(t.shape) if isinstance(t, torch.Tensor) else type(t).__name__
