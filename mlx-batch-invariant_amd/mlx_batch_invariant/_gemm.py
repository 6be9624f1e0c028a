"""Batch-invariant GEMM: ``matmul``, ``addmm``, ``linear``.

Mirrors reference mlx_batch_invariant/_gemm.py:185-240 (validation, leading-dim
flattening, bias/epilogue, public entry points) on top of the HIP kernel in
csrc/bi_gemm.hip, reached through the C ABI ``bi_gemm`` (include/bi.h).

Every output row is computed by the same fixed sequence of MFMA instructions
over K, whatever else is in the batch: the workgroup that owns a tile owns its
whole K reduction, and the K loop depends on K alone.
"""

import ctypes

import torch

from . import _lib

# Fixed per-element arithmetic of the kernel. The reference exports its single
# tile (BM, BN, BK, SG_M, SG_N) as TILE (reference _gemm.py:25-27) and a test
# pins it (reference tests/test_invariance.py:468-470). This build keeps those
# keys for the unit of fixed arithmetic -- one wave's 16 x 16 MFMA output tile
# (BM x BN), fed BK = 32 elements of K per chunk-step for bf16/f16 (fp32: 16,
# K_CHUNK_FP32), by one wave (SG_M x SG_N = 1 x 1) -- and pins the rest of what
# decides an element's bits: the MFMA instructions, the fp32 chain rule and the
# epilogue. Workgroup footprints (how many such units a workgroup holds, and
# the K bytes each footprint stages per pipeline step) are listed separately by
# geometries(); they do not enter any element's arithmetic.
TILE = dict(
    BM=16,                               # rows of the fixed unit (one MFMA tile)
    BN=16,                               # columns of the fixed unit
    BK=32,                               # K per chunk-step, bf16 / f16
    SG_M=1,                              # waves per unit, along M
    SG_N=1,                              # waves per unit, along N
    MFMA_16BIT="v_mfma_f32_16x16x32",   # bf16 / f16 inputs, fp32 accumulate
    MFMA_FP32="v_mfma_f32_16x16x4_f32",
    K_CHUNK_16BIT=32,                    # K per MFMA for 16-bit inputs
    K_CHUNK_FP32=16,                     # K per chunk-step (4 MFMAs) for fp32
    FP32_CHAINS=2,                       # fp32: chunk-step j feeds chain j; acc = c0 + c1
    EPILOGUE="fma(alpha, acc, beta * bias) then one RNE rounding",
)

_SUPPORTED = (torch.float32, torch.float16, torch.bfloat16)


def geometries():
    """[(block_m, block_n, waves)] of the workgroup footprints built into libbi.so."""
    L = _lib.lib()
    out = []
    for g in range(L.bi_gemm_num_geometries()):
        bm, bn, w = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        _lib.check(L.bi_gemm_geometry_info(g, ctypes.byref(bm), ctypes.byref(bn),
                                           ctypes.byref(w)), "bi_gemm_geometry_info")
        out.append((bm.value, bn.value, w.value))
    return out


def _check_device(*tensors):
    dev = tensors[0].device
    if dev.type != "cuda":
        raise ValueError("batch-invariant kernels run on the GPU; got a %s tensor" % dev.type)
    for t in tensors[1:]:
        if t.device != dev:
            raise ValueError("all operands must be on %s, got %s" % (dev, t.device))


def _gemm(a, b, bias, transpose_b, alpha=1.0, beta=1.0, geometry=None):
    """Validation and launch; reference _gemm.py:185-222. While torch.compile
    traces, the launch is recorded as the opaque op mlx_bi::gemm."""
    if geometry is None and torch.compiler.is_compiling():
        from . import _ops  # noqa: F401  (registers the ops)

        return torch.ops.mlx_bi.gemm(a, b, bias, bool(transpose_b), float(alpha), float(beta))
    return _gemm_eager(a, b, bias, transpose_b, alpha, beta, geometry)


def _gemm_eager(a, b, bias, transpose_b, alpha=1.0, beta=1.0, geometry=None, events=None):
    if a.dtype != b.dtype:
        raise ValueError("a and b must share a dtype, got %s and %s" % (a.dtype, b.dtype))
    if a.ndim < 2 or b.ndim != 2:
        raise ValueError("expected a.ndim >= 2 and b.ndim == 2")
    if a.dtype not in _SUPPORTED:
        raise ValueError("unsupported dtype %s (float32, float16 and bfloat16 are built)"
                         % a.dtype)

    lead, K = tuple(a.shape[:-1]), a.shape[-1]
    M = 1
    for d in lead:
        M *= d
    kb, N = (b.shape[1], b.shape[0]) if transpose_b else (b.shape[0], b.shape[1])
    if kb != K:
        raise ValueError("inner dimensions do not match: %d vs %d" % (K, kb))
    if bias is not None:
        if tuple(bias.shape) != (N,):
            raise ValueError("bias must have shape (%d,), got %s" % (N, tuple(bias.shape)))
        if bias.dtype != a.dtype:
            raise ValueError("bias must share the dtype of a, got %s and %s"
                             % (bias.dtype, a.dtype))
        _check_device(a, b, bias)
    else:
        _check_device(a, b)

    a2 = a if len(lead) == 1 else a.reshape(M, K)
    if not a2.is_contiguous():
        a2 = a2.contiguous()
    # A (K, N) operand that is the transpose of a contiguous (N, K) tensor is
    # read in place through the (N, K) kernel: both layouts feed each MFMA the
    # same K elements in the same lane slots, so the bits are the same.
    if not transpose_b and not b.is_contiguous() and b.t().is_contiguous():
        b, transpose_b = b.t(), True
    elif not b.is_contiguous():
        b = b.contiguous()
    bias_c = None if bias is None else bias.contiguous()

    out = torch.empty((M, N), dtype=a.dtype, device=a.device)
    if M and N:
        L = _lib.lib()
        args = (a2.data_ptr(), b.data_ptr(), bias_c.data_ptr() if bias_c is not None else None,
                out.data_ptr(), M, N, K, _lib.DTYPE_CODES[a.dtype], int(transpose_b),
                float(alpha), float(beta))
        stream, switch = _lib.launch_stream(a.device)
        if switch:
            with torch.cuda.device(a.device):
                rc = _launch(L, args, geometry, stream, events)
        else:
            rc = _launch(L, args, geometry, stream, events)
        if rc:
            _lib.check(rc, "bi_gemm")
    return out if len(lead) == 1 else out.reshape(*lead, N)


def _launch(L, args, geometry, stream, events=None):
    if events is not None:
        return L.bi_gemm_timed(*args, events[0].cuda_event, events[1].cuda_event, stream)
    if geometry is None:
        return L.bi_gemm(*args, stream)
    return L.bi_gemm_with_geometry(*args, int(geometry), stream)


def matmul_timed(a, b, start, stop):
    """matmul(a, b) whose kernel records its own start and end timestamps into
    the torch.cuda.Events `start` and `stop` (bi_gemm_timed): times one launch
    without event markers between kernels. Both events must have been recorded
    once before (torch creates the underlying event on its first record)."""
    return _gemm_eager(a, b, None, False, events=(start, stop))


def linear_timed(x, w, start, stop):
    """linear(x, w) timed like matmul_timed (the kernel's own timestamps)."""
    return _gemm_eager(x, w, None, True, events=(start, stop))


def matmul(a, b):
    """a @ b with b laid out (K, N). Bitwise independent of a's leading dimensions."""
    return _gemm(a, b, None, transpose_b=False)


def addmm(c, a, b, alpha=1.0, beta=1.0):
    """alpha * (a @ b) + beta * c, with b laid out (K, N) and c of shape (N,)."""
    return _gemm(a, b, c, transpose_b=False, alpha=alpha, beta=beta)


def linear(x, w, bias=None):
    """x @ w.T (+ bias) with w laid out (N, K), the nn.Linear convention.

    Takes the weight in its stored layout so no transposed copy is made.
    """
    return _gemm(x, w, bias, transpose_b=True)
