"""Batch-invariant GEMM on affine-quantized weights (reference
_gemm.py:159-177 and 243-285; tests/test_invariance.py's quantized cases).

The kernel's result is defined as bi.linear(x, bi.dequantize(w, ...)), bit for
bit: it dequantizes every weight to the element type exactly as the oracle
does (pinned in tests/test_oracle.py) and then runs the dense kernel's
arithmetic, whose parity with the GEMM oracle is pinned in test_gpu_gemm.py.
"""

import numpy as np
import pytest
import torch

import mlx_batch_invariant as bi
from mlx_batch_invariant import _lib

from helpers import batch_with, bits, rn

pytestmark = pytest.mark.gpu

QDTYPES = [("float16", torch.float16), ("bfloat16", torch.bfloat16)]


def _qweight(N, K, dtype, seed, gs, nbits, device):
    w = rn((N, K), dtype, seed, std=K ** -0.5)
    q, s, b = bi.quantize(w, gs, nbits)
    return q.to(device), s.to(device), b.to(device)


def _dense(x, q, s, b, gs, nbits):
    return bi.linear(x, bi.dequantize(q, s, b, gs, nbits))


@pytest.mark.parametrize("dname,dtype", QDTYPES)
@pytest.mark.parametrize("nbits", [2, 4, 8])
def test_qgemm_equals_dense_on_dequantized_weight(cuda, dname, dtype, nbits):
    for gs in (32, 64, 128):
        for M, N, K in [(1, 256, 512), (7, 200, 384), (64, 512, 1024), (300, 384, 640)]:
            q, s, b = _qweight(N, K, dtype, 101 + nbits + gs, gs, nbits, cuda)
            x = rn((M, K), dtype, 102 + M, device=cuda)
            got = bi.quantized_linear(x, q, s, b, gs, nbits)
            want = _dense(x, q, s, b, gs, nbits)
            assert got.dtype == dtype and got.shape == (M, N)
            assert np.array_equal(bits(got), bits(want)), (dname, nbits, gs, M, N, K)


def test_qgemm_every_geometry_gives_the_same_bits(cuda):
    """The footprint never enters an element's arithmetic, as for the dense kernel."""
    L = _lib.lib()
    ng = L.bi_gemm_num_geometries()
    M, N, K, gs = 96, 272, 768, 64
    for dname, dtype in QDTYPES:
        for nbits in (2, 4, 8):
            q, s, b = _qweight(N, K, dtype, 103 + nbits, gs, nbits, cuda)
            x = rn((M, K), dtype, 104, device=cuda)
            want = bits(_dense(x, q, s, b, gs, nbits))
            for g in range(ng):
                out = torch.empty((M, N), dtype=dtype, device=cuda)
                stream, _ = _lib.launch_stream(x.device)
                rc = L.bi_qgemm_with_geometry(x.data_ptr(), q.data_ptr(), s.data_ptr(),
                                              b.data_ptr(), out.data_ptr(), M, N, K, gs, nbits,
                                              _lib.DTYPE_CODES[dtype], g, stream)
                _lib.check(rc, "bi_qgemm_with_geometry")
                assert np.array_equal(bits(out), want), (dname, nbits, g)


@pytest.mark.parametrize("dname,dtype", QDTYPES)
def test_quantized_linear_is_batch_invariant(cuda, dname, dtype):
    """Row i of a batch equals the batch-1 result, whatever the other rows
    (reference tests/test_invariance.py, quantized linear invariance)."""
    N, K, gs, nbits = 4096, 4096, 64, 4
    q, s, b = _qweight(N, K, dtype, 105, gs, nbits, cuda)
    ref = rn((1, K), dtype, 106, device=cuda)
    pool = rn((256, K), dtype, 107, device=cuda)
    base = bits(bi.quantized_linear(ref, q, s, b, gs, nbits)[0])
    for B in (2, 3, 8, 16, 33, 64, 128, 256):
        idx = B // 2
        got = bits(bi.quantized_linear(batch_with(ref, pool, B, idx), q, s, b, gs, nbits)[idx])
        assert int((got != base).sum()) == 0, "quantized %s B=%d" % (dname, B)


def test_quantized_module_under_mode(cuda):
    """QuantizedLinear (with bias, 3-d input) is invariant inside the mode and
    equals the dense invariant linear on the dequantized weight plus bias."""
    torch.manual_seed(108)
    lin = torch.nn.Linear(512, 384).to(torch.bfloat16)
    mod = bi.QuantizedLinear.from_linear(lin, group_size=32, bits=8).to(cuda)
    x_ref = rn((1, 1, 512), torch.bfloat16, 109, device=cuda)
    pool = rn((32, 1, 512), torch.bfloat16, 110, device=cuda)
    with bi.batch_invariant_mode(strict=True), torch.no_grad():
        base = bits(mod(x_ref)[0])
        for B in (2, 5, 32):
            got = bits(mod(batch_with(x_ref, pool, B, B - 1))[B - 1])
            assert np.array_equal(got, base), B
        wd = bi.dequantize(mod.weight, mod.scales, mod.biases, 32, 8)
        want = bits((bi.linear(x_ref, wd) + mod.bias)[0])
    assert np.array_equal(base, want)


def test_quantized_accuracy_against_float64(cuda):
    """The product is the float64 product of x and the dequantized weight to
    within the fp32-accumulation and output-rounding error."""
    M, N, K, gs = 16, 256, 2048, 64
    for dname, dtype in QDTYPES:
        q, s, b = _qweight(N, K, dtype, 111, gs, 4, cuda)
        x = rn((M, K), dtype, 112, device=cuda)
        got = bi.quantized_linear(x, q, s, b, gs, 4).double().cpu()
        wd = bi.dequantize(q, s, b, gs, 4).double().cpu()
        want = x.double().cpu() @ wd.T
        tol = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11
        err = ((got - want).abs() / (want.abs() + 1e-2)).max().item()
        assert err < 4 * tol, (dname, err)


def test_quantized_edges(cuda):
    dtype = torch.float16
    # K = one group, N not a multiple of 16, M = 1
    q, s, b = _qweight(37, 32, dtype, 113, 32, 2, cuda)
    x = rn((1, 32), dtype, 114, device=cuda)
    assert np.array_equal(bits(bi.quantized_linear(x, q, s, b, 32, 2)),
                          bits(_dense(x, q, s, b, 32, 2)))
    # empty batch
    out = bi.quantized_linear(x[:0], q, s, b, 32, 2)
    assert out.shape == (0, 37)
    # a non-contiguous (strided) activation is copied, not misread
    xs = rn((4, 64), dtype, 115, device=cuda)[:, :32]
    assert np.array_equal(bits(bi.quantized_linear(xs, q, s, b, 32, 2)),
                          bits(_dense(xs.contiguous(), q, s, b, 32, 2)))
    # float32 activations are not built
    with pytest.raises(NotImplementedError):
        bi.quantized_linear(x.float(), q, s.float(), b.float(), 32, 2)
    # the C ABI refuses float32 with BI_EUNSUPPORTED and a message
    L = _lib.lib()
    rc = L.bi_qgemm(None, None, None, None, None, 1, 1, 32, 32, 2, _lib.DTYPE_CODES[torch.float32],
                    None)
    assert rc != 0 and b"float16/bfloat16" in L.bi_last_error()


def test_quantized_matmul_routes_inside_the_mode(cuda):
    q, s, b = _qweight(128, 256, torch.bfloat16, 116, 64, 4, cuda)
    x = rn((3, 256), torch.bfloat16, 117, device=cuda)
    with bi.batch_invariant_mode(strict=True):
        got = bi.quantized_matmul(x, q, s, b, transpose=True, group_size=64, bits=4)
        with pytest.raises(NotImplementedError):
            bi.quantized_matmul(x, q, s, b, transpose=False, group_size=64, bits=4)
    assert np.array_equal(bits(got), bits(bi.quantized_linear(x, q, s, b, 64, 4)))
