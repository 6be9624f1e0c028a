"""Batch-invariant GEMM on affine-quantized weights (reference
_gemm.py:159-177 and 243-285; tests/test_invariance.py:477-592).

Parity: the reference dequantizes each weight to an fp32 value v and
multiplies in fp32 (its B tile is float). The kernel forms the same sum per
group as scale * sum(x q) + bias * sum(x), with exact products and fp32
roundings only, so on inputs whose partial sums are exact in fp32 its result
is the exact product rounded once, bit for bit, and on random inputs it is
within 1 ULP of the exact product with the fp32 weights (the dense GEMM's
bound). The oracle is oracle/quant.py, pinned in tests/test_oracle.py.
"""

import numpy as np
import pytest
import torch

import mlx_batch_invariant as bi
from mlx_batch_invariant import _lib
from oracle import bits as obits
from oracle import gemm as ogemm
from oracle import quant as oquant

from helpers import batch_with, bits, closed_form_quant, f64, rn

pytestmark = pytest.mark.gpu

QDTYPES = [("float16", torch.float16), ("bfloat16", torch.bfloat16)]


def _qweight(N, K, dtype, seed, gs, nbits, device):
    w = rn((N, K), dtype, seed, std=K ** -0.5)
    q, s, b = bi.quantize(w, gs, nbits)
    return q.to(device), s.to(device), b.to(device)


def _exact(x, q, s, b, gs, nbits):
    return oquant.qgemm_f64(f64(x), q.cpu().numpy(), f64(s), f64(b), gs, nbits)


def _launch(L, x, q, s, b, gs, nbits, g):
    M, K = x.shape
    N = q.shape[0]
    out = torch.empty((M, N), dtype=x.dtype, device=x.device)
    stream, _ = _lib.launch_stream(x.device)
    rc = L.bi_qgemm_with_geometry(x.data_ptr(), q.data_ptr(), s.data_ptr(), b.data_ptr(),
                                  out.data_ptr(), M, N, K, gs, nbits, _lib.DTYPE_CODES[x.dtype],
                                  g, stream)
    _lib.check(rc, "bi_qgemm_with_geometry")
    return out


@pytest.mark.parametrize("dname,dtype", QDTYPES)
@pytest.mark.parametrize("nbits", [2, 4, 8])
def test_closed_form_products_are_exact(cuda, dname, dtype, nbits):
    """Weights whose fp32 values are not representable in the element type and
    small-integer activations (every partial sum a multiple of 2^-11 below
    2^13): the result is the exact product rounded once, bitwise. A kernel
    that rounded the weights to the element type first fails this
    (tests/test_oracle.py shows the planted rounding changes >20% of these
    outputs)."""
    for gs in (32, 64, 128):
        for M, N, K in [(1, 48, 256), (19, 64, 512), (70, 130, 384)]:
            x, q, s, b, exact = closed_form_quant(M, N, K, gs, nbits, dtype, 100 + nbits + gs + M)
            want = obits.round_f32_to(exact.astype(np.float32), dname)
            got = f64(bi.quantized_linear(x.to(cuda), q.to(cuda), s.to(cuda), b.to(cuda), gs,
                                          nbits))
            bad = int((got != want).sum())
            assert bad == 0, "%s bits=%d gs=%d M=%d N=%d K=%d: %d differ" % (
                dname, nbits, gs, M, N, K, bad)


@pytest.mark.parametrize("dname,dtype", QDTYPES)
def test_within_one_ulp_of_exact(cuda, dname, dtype):
    """Random weights and activations: every element within 1 ULP of the exact
    product with the fp32 weights, the ULP taken at max(|exact|, 2^-p * sum_k
    |x_k v_k|) as for the dense GEMM."""
    p = obits.PRECISION[dname]
    for nbits in (2, 4, 8):
        for gs in (32, 64, 128):
            for M, N, K in [(1, 256, 2048), (33, 200, 640), (130, 384, 1024)]:
                q, s, b = _qweight(N, K, dtype, 101 + nbits + gs, gs, nbits, cuda)
                x = rn((M, K), dtype, 102 + M, device=cuda)
                exact = _exact(x, q, s, b, gs, nbits)
                v = oquant.dequantize(q.cpu().numpy(), f64(s), f64(b), gs, nbits)
                floor = ogemm.abs_products(f64(x), v, trans_b=True) * 2.0 ** -p
                ulp = obits.ulp_of(np.maximum(np.abs(exact), floor), dname)
                got = f64(bi.quantized_linear(x, q, s, b, gs, nbits))
                worst = (np.abs(got - exact) / ulp).max()
                assert worst <= 1.0, "%s bits=%d gs=%d M=%d: %.3f ULP" % (dname, nbits, gs, M,
                                                                           worst)


def test_reference_accuracy_bounds(cuda):
    """Reference tests:564-592: against x @ dequantize(w) (weights rounded to
    the element type, as mx.dequantize returns them) the max-normalised error
    is below 5e-3, and no larger than twice that of the stock path."""
    for nbits in bi.QUANT_BITS:
        for gs in (32, 64, 128):
            w = rn((256, 512), torch.float16, 50)
            q, s, b = (t.to(cuda) for t in bi.quantize(w, gs, nbits))
            x = rn((5, 512), torch.float16, 49, device=cuda)
            wd = bi.dequantize(q, s, b, gs, nbits)
            exact = f64(x) @ f64(wd).T
            got = f64(bi.quantized_linear(x, q, s, b, gs, nbits))
            err = np.abs(got - exact).max() / np.abs(exact).max()
            assert err < 5e-3, (nbits, gs, err)
            stock = f64(torch.nn.functional.linear(x, wd))
            assert np.abs(got - exact).max() <= 2 * np.abs(stock - exact).max() + 1e-6


def test_every_geometry_gives_the_same_bits(cuda):
    """The footprint never enters an element's arithmetic."""
    L = _lib.lib()
    ng = L.bi_qgemm_num_geometries()
    M, N, K, gs = 96, 272, 768, 64
    for dname, dtype in QDTYPES:
        for nbits in (2, 4, 8):
            q, s, b = _qweight(N, K, dtype, 103 + nbits, gs, nbits, cuda)
            x = rn((M, K), dtype, 104, device=cuda)
            want = bits(bi.quantized_linear(x, q, s, b, gs, nbits))
            built = 0
            for g in range(ng):
                try:
                    out = _launch(L, x, q, s, b, gs, nbits, g)
                except NotImplementedError:
                    continue
                built += 1
                assert np.array_equal(bits(out), want), (dname, nbits, g)
            assert built >= 4


@pytest.mark.parametrize("dname,dtype", QDTYPES)
def test_decode_footprint_gives_the_same_bits(cuda, dname, dtype):
    """The decode footprint (2-, 4- and 8-bit weights, at most 8 rows: the waves of
    a workgroup split K by groups, the codes reach the matrix cores through a
    transpose across lane groups) gives the 16x16 footprint's bits: one
    group, blocks cut short by K, K over several rounds, N not a multiple
    of 16, one to eight rows. More rows are refused."""
    L = _lib.lib()
    dec = L.bi_gemm_num_geometries()
    assert L.bi_qgemm_num_geometries() == dec + 1
    for nbits in (2, 4, 8):
        for gs in (32, 64, 128):
            for M, N, K in [(1, 37, gs), (2, 48, 3 * gs), (1, 272, 768), (4, 130, 4096),
                            (3, 64, 8192 + 3 * gs), (1, 200, 4096 + gs), (5, 40, 256),
                            (8, 96, 4096 + 5 * gs), (7, 33, 2 * gs)]:
                q, s, b = _qweight(N, K, dtype, 120 + gs + M + nbits, gs, nbits, cuda)
                x = rn((M, K), dtype, 121 + K, device=cuda)
                want = bits(_launch(L, x, q, s, b, gs, nbits, 0))
                got = bits(_launch(L, x, q, s, b, gs, nbits, dec))
                bad = int((got != want).sum())
                assert bad == 0, "%s bits=%d gs=%d M=%d N=%d K=%d: %d differ" % (
                    dname, nbits, gs, M, N, K, bad)
    q, s, b = _qweight(64, 256, dtype, 122, 64, 4, cuda)
    with pytest.raises(NotImplementedError):
        _launch(L, rn((9, 256), dtype, 123, device=cuda), q, s, b, 64, 4, dec)


@pytest.mark.parametrize("dname,dtype", QDTYPES)
def test_quantized_linear_is_batch_invariant(cuda, dname, dtype):
    """Row i of a batch equals the batch-1 result, whatever the other rows
    (reference tests:513-535)."""
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
    """QuantizedLinear (with bias, 3-d input: the prefill-vs-decode case of
    reference tests:537-552) is invariant inside the mode and equals
    quantized_linear plus the bias."""
    torch.manual_seed(108)
    lin = torch.nn.Linear(512, 384).to(torch.bfloat16)
    mod = bi.QuantizedLinear.from_linear(lin, group_size=32, bits=8).to(cuda)
    x_ref = rn((1, 5, 512), torch.bfloat16, 109, device=cuda)
    pool = rn((32, 5, 512), torch.bfloat16, 110, device=cuda)
    with bi.batch_invariant_mode(strict=True), torch.no_grad():
        base = bits(mod(x_ref)[0])
        for B in (2, 5, 32):
            got = bits(mod(batch_with(x_ref, pool, B, B - 1))[B - 1])
            assert np.array_equal(got, base), B
        want = bits((bi.quantized_linear(x_ref, mod.weight, mod.scales, mod.biases, 32, 8)
                     + mod.bias)[0])
    assert np.array_equal(base, want)


def test_quantized_edges(cuda):
    dtype = torch.float16
    # K = one group, N not a multiple of 16, M = 1
    x, q, s, b, exact = closed_form_quant(1, 37, 32, 32, 2, dtype, 113)
    want = obits.round_f32_to(exact.astype(np.float32), "float16")
    q, s, b = q.to(cuda), s.to(cuda), b.to(cuda)
    assert (f64(bi.quantized_linear(x.to(cuda), q, s, b, 32, 2)) == want).all()
    # empty batch
    out = bi.quantized_linear(x.to(cuda)[:0], q, s, b, 32, 2)
    assert out.shape == (0, 37)
    # a non-contiguous (strided) activation is copied, not misread
    xs = rn((4, 64), dtype, 115, device=cuda)[:, :32]
    assert np.array_equal(bits(bi.quantized_linear(xs, q, s, b, 32, 2)),
                          bits(bi.quantized_linear(xs.contiguous(), q, s, b, 32, 2)))
    # float32 activations are not built
    with pytest.raises(NotImplementedError):
        bi.quantized_linear(xs.float(), q, s.float(), b.float(), 32, 2)
    # the C ABI refuses float32 with BI_EUNSUPPORTED and a message
    L = _lib.lib()
    rc = L.bi_qgemm(None, None, None, None, None, 1, 1, 32, 32, 2,
                    _lib.DTYPE_CODES[torch.float32], None)
    assert rc != 0 and b"float16/bfloat16" in L.bi_last_error()


def test_quantized_matmul_routes_inside_the_mode(cuda):
    q, s, b = _qweight(128, 256, torch.bfloat16, 116, 64, 4, cuda)
    x = rn((3, 256), torch.bfloat16, 117, device=cuda)
    with bi.batch_invariant_mode(strict=True):
        got = bi.quantized_matmul(x, q, s, b, transpose=True, group_size=64, bits=4)
        with pytest.raises(NotImplementedError):
            bi.quantized_matmul(x, q, s, b, transpose=False, group_size=64, bits=4)
    assert np.array_equal(bits(got), bits(bi.quantized_linear(x, q, s, b, 64, 4)))
