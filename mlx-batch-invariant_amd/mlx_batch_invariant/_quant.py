"""Batch-invariant GEMM on affine-quantized weights.

Mirrors reference mlx_batch_invariant/_gemm.py:159-177 and 243-285
(``quantized_linear``: ``x @ dequantize(w).T`` without materialising the
dequantized weight) and the shim's ``quantized_matmul`` route
(reference __init__.py:109-123), on top of the HIP kernel behind ``bi_qgemm``
(include/bi.h).

Weight format (MLX's affine layout): ``w`` is (N, K * bits / 32) 32-bit words;
weight element k of row n sits in bits ``bits * (k % (32 / bits))`` onward of
word ``k // (32 / bits)`` of row n (little-endian packing). ``scales`` and
``biases`` are (N, K / group_size) in the activation dtype. Torch has no
uint32 arithmetic, so packed words are held in int32 tensors (same bits);
uint32 is accepted too.

Arithmetic: the reference's kernel (_gemm.py:170-173, into a float B tile)
multiplies by the fp32 value ``v = scale * q + bias`` and accumulates in
fp32. The kernel here forms the same sum per group, ``scale * sum(x * q) +
bias * sum(x)``, with exact products in its MFMAs and fp32 roundings only, in
a fixed order per element, so invariance holds exactly as for the dense GEMM
and the result is within fp32 accumulation error of the reference's. Note
that :func:`dequantize` returns v rounded to the element type (what
``mx.dequantize`` returns); ``linear(x, dequantize(w))`` therefore differs from
``quantized_linear`` by that rounding of the weights.
"""

import torch
import torch.nn.functional as F

from . import _lib

QUANT_BITS = (2, 4, 8)
GROUP_SIZES = (32, 64, 128)
_ACT_DTYPES = (torch.float16, torch.bfloat16)


def _unpack(w, bits, K):
    """(N, K * bits / 32) words -> (N, K) integer codes (int64)."""
    per = 32 // bits
    words = w.to(torch.int64) & 0xFFFFFFFF
    shifts = torch.arange(per, device=w.device, dtype=torch.int64) * bits
    q = (words.unsqueeze(-1) >> shifts) & ((1 << bits) - 1)
    return q.reshape(w.shape[0], K)


def _pack(q, bits):
    """(N, K) integer codes -> (N, K * bits / 32) int32 words."""
    per = 32 // bits
    N, K = q.shape
    shifts = torch.arange(per, device=q.device, dtype=torch.int64) * bits
    words = (q.to(torch.int64).reshape(N, K // per, per) << shifts).sum(-1)
    words = torch.where(words >= 2 ** 31, words - 2 ** 32, words)
    return words.to(torch.int32)


def quantize(w, group_size=64, bits=4):
    """Affine-quantize a (N, K) weight into the layout above.

    Per group: bias = min, scale = (max - min) / (2**bits - 1) (1 for a
    constant group), both rounded to w's dtype; codes are round((w - bias) /
    scale) clipped to [0, 2**bits - 1]. Returns (packed int32, scales, biases).
    """
    if bits not in QUANT_BITS:
        raise ValueError("bits must be one of %s, got %r" % (QUANT_BITS, bits))
    if group_size not in GROUP_SIZES:
        raise ValueError("group_size must be one of %s, got %r" % (GROUP_SIZES, group_size))
    if w.ndim != 2 or w.shape[1] % group_size:
        raise ValueError("expected a 2-d weight whose columns are a multiple of %d, got %s"
                         % (group_size, tuple(w.shape)))
    N, K = w.shape
    n = (1 << bits) - 1
    g = w.float().reshape(N, K // group_size, group_size)
    lo, hi = g.amin(-1), g.amax(-1)
    scale = torch.where(hi > lo, (hi - lo) / n, torch.ones_like(lo)).to(w.dtype)
    bias = lo.to(w.dtype)
    q = torch.round((g - bias.float().unsqueeze(-1)) / scale.float().unsqueeze(-1)).clamp(0, n)
    return _pack(q.reshape(N, K), bits), scale, bias


def dequantize(w, scales, biases, group_size=64, bits=4):
    """The (N, K) weight in the dtype of ``scales``: T(fp32(scale * q + bias)),
    one rounding of the fp32 value the quantized GEMM multiplies by."""
    if bits not in QUANT_BITS:
        raise ValueError("bits must be one of %s, got %r" % (QUANT_BITS, bits))
    K = w.shape[1] * (32 // bits)
    q = _unpack(w, bits, K).to(torch.float32)
    s = scales.float().repeat_interleave(group_size, dim=1)
    b = biases.float().repeat_interleave(group_size, dim=1)
    return (s * q + b).to(scales.dtype)


def quantized_linear(x, w, scales, biases, group_size, bits):
    """``x @ dequantize(w).T`` for an affine-quantized w, batch-invariant
    (reference _gemm.py:243-285). While torch.compile traces, the launch is
    recorded as the opaque op mlx_bi::qgemm."""
    if torch.compiler.is_compiling():
        from . import _ops  # noqa: F401  (registers the ops)

        return torch.ops.mlx_bi.qgemm(x, w, scales, biases, int(group_size), int(bits))
    return _quantized_linear_eager(x, w, scales, biases, group_size, bits)


def _quantized_linear_eager(x, w, scales, biases, group_size, bits):
    if bits not in QUANT_BITS:
        raise ValueError("bits must be one of %s, got %r" % (QUANT_BITS, bits))
    if x.ndim < 2 or w.ndim != 2 or scales.ndim != 2 or biases.ndim != 2:
        raise ValueError("expected x.ndim >= 2 and 2-d w, scales and biases")
    lead, K = tuple(x.shape[:-1]), x.shape[-1]
    M = 1
    for d in lead:
        M *= d
    N = w.shape[0]
    if w.shape[1] * (32 // bits) != K:
        raise ValueError("packed weight %s does not describe %d columns at %d bits"
                         % (tuple(w.shape), K, bits))
    if group_size not in GROUP_SIZES:
        raise ValueError("group_size must be one of %s, got %r" % (GROUP_SIZES, group_size))
    if K % group_size:
        raise ValueError("group size %d does not divide K=%d" % (group_size, K))
    if tuple(scales.shape) != (N, K // group_size) or biases.shape != scales.shape:
        raise ValueError("scales/biases must have shape (%d, %d), got %s and %s"
                         % (N, K // group_size, tuple(scales.shape), tuple(biases.shape)))
    if w.dtype not in (torch.int32, torch.uint32):
        raise ValueError("packed weight must be int32 or uint32, got %s" % w.dtype)
    if scales.dtype != x.dtype or biases.dtype != x.dtype:
        raise ValueError("scales and biases must share the dtype of x (%s), got %s and %s"
                         % (x.dtype, scales.dtype, biases.dtype))
    dev = x.device
    if dev.type != "cuda" or any(t.device != dev for t in (w, scales, biases)):
        raise ValueError("batch-invariant kernels run on one GPU; got %s"
                         % sorted({str(t.device) for t in (x, w, scales, biases)}))
    if x.dtype not in _ACT_DTYPES:
        raise NotImplementedError("quantized weights are built for float16/bfloat16 "
                                  "activations, got %s" % x.dtype)

    x2 = x.reshape(M, K)
    if not x2.is_contiguous() or x2.data_ptr() % 16:
        x2 = x2.contiguous() if not x2.is_contiguous() else x2.clone()
    w_c = w if w.is_contiguous() and w.data_ptr() % 16 == 0 else w.clone(
        memory_format=torch.contiguous_format)
    s_c, b_c = scales.contiguous(), biases.contiguous()
    out = torch.empty((M, N), dtype=x.dtype, device=dev)
    if M and N:
        L = _lib.lib()
        args = (x2.data_ptr(), w_c.data_ptr(), s_c.data_ptr(), b_c.data_ptr(), out.data_ptr(),
                M, N, K, int(group_size), int(bits), _lib.DTYPE_CODES[x.dtype])
        stream, switch = _lib.launch_stream(dev)
        if switch:
            with torch.cuda.device(dev):
                rc = L.bi_qgemm(*args, stream)
        else:
            rc = L.bi_qgemm(*args, stream)
        if rc:
            _lib.check(rc, "bi_qgemm")
    return out.reshape(*lead, N)


def quantized_matmul(x, w, scales, biases=None, transpose=True, group_size=None, bits=None,
                     mode="affine"):
    """MLX's ``quantized_matmul`` signature. Outside batch_invariant_mode this
    is stock torch (dequantize, then F.linear); inside it routes to the
    invariant kernel when it can (reference __init__.py:109-123) and otherwise
    raises (strict) or falls back to stock."""
    from . import _strict, _unsupported, is_enabled

    if transpose and x.ndim >= 2 and w.ndim == 2 and scales.ndim == 2:
        K = x.shape[-1]
        bits = 32 * w.shape[1] // K if bits is None else bits
        group_size = K // scales.shape[1] if group_size is None else group_size

    def stock(x, w, scales, biases, transpose, group_size, bits, mode):
        if mode != "affine" or biases is None:
            raise ValueError("only the affine mode with biases is supported")
        wd = dequantize(w, scales, biases, group_size, bits)
        return F.linear(x, wd) if transpose else x @ wd

    if not is_enabled():
        return stock(x, w, scales, biases, transpose, group_size, bits, mode)
    if (not transpose or x.ndim < 2 or mode != "affine" or biases is None
            or bits not in QUANT_BITS or x.dtype not in _ACT_DTYPES or x.device.type != "cuda"
            or (torch.is_grad_enabled() and x.requires_grad)):
        return _unsupported("quantized_matmul with transpose=%s x.ndim=%d mode=%s bits=%s dtype=%s"
                            % (transpose, x.ndim, mode, bits, x.dtype),
                            _strict(), stock, x, w, scales, biases, transpose, group_size,
                            bits, mode)
    return quantized_linear(x, w, scales, biases, group_size, bits)


class QuantizedLinear(torch.nn.Module):
    """A linear layer with an affine-quantized weight (MLX nn.QuantizedLinear's
    role): ``quantized_matmul(x, w, ...) + bias``; batch-invariant inside
    batch_invariant_mode."""

    def __init__(self, weight, scales, biases, bias=None, group_size=64, bits=4):
        super().__init__()
        self.group_size, self.bits = group_size, bits
        self.register_buffer("weight", weight)
        self.register_buffer("scales", scales)
        self.register_buffer("biases", biases)
        self.bias = None if bias is None else torch.nn.Parameter(bias, requires_grad=False)

    @classmethod
    def from_linear(cls, lin, group_size=64, bits=4):
        w, s, b = quantize(lin.weight.detach(), group_size, bits)
        bias = None if lin.bias is None else lin.bias.detach().clone()
        return cls(w, s, b, bias, group_size, bits)

    def forward(self, x):
        y = quantized_matmul(x, self.weight, self.scales, self.biases, True, self.group_size,
                             self.bits)
        return y if self.bias is None else y + self.bias
