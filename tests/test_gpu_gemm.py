"""GPU parity tests of the invariant GEMM (bi.matmul / bi.addmm / bi.linear).

Invariance is self-referential (bits of a row alone vs the same row in any
batch); accuracy is checked against the float64 oracle (oracle/gemm.py) with
the bounds the north star and reference tests state; closed forms pin exact
bits. Mirrors reference tests/test_invariance.py:36-158.
"""

import numpy as np
import pytest
import torch

import mlx_batch_invariant as bi
from mlx_batch_invariant import _gemm
from oracle import bits as obits
from oracle import gemm as ogemm

from helpers import BATCHES, DTYPES, batch_with, bits, f64, ndiff, rn

pytestmark = pytest.mark.gpu

SHAPES = [(512, 512), (1024, 1024), (4096, 4096), (11008, 4096), (4096, 11008), (333, 200)]


def test_linear_config1_row0_bitwise(cuda):
    """x (M,4096) @ W(4096,4096)^T + bias, bf16, seed 0."""
    g = torch.Generator().manual_seed(0)
    x = torch.randn(8, 4096, generator=g).to(torch.bfloat16).to(cuda)
    w = (torch.randn(4096, 4096, generator=g) / 64.0).to(torch.bfloat16).to(cuda)
    b = torch.randn(4096, generator=g).to(torch.bfloat16).to(cuda)
    base = bits(bi.linear(x[:1].contiguous(), w, b)[0])
    assert (base != 0).any()
    for M in (2, 3, 8):
        y = bi.linear(x[:M].contiguous(), w, b)
        for r in range(M):
            one = bits(bi.linear(x[r:r + 1].contiguous(), w, b)[0])
            assert (bits(y[r]) == one).all(), "M=%d row %d differs from its M=1 result" % (M, r)
        assert (bits(y[0]) == base).all()


@pytest.mark.parametrize("op", ["matmul", "addmm", "linear"])
def test_batch_invariance_sweep(cuda, op):
    """Row at positions 0, B//2, B-1 is bitwise equal to its B=1 result for every
    batch size 1..256 (reference TestBitwiseInvariance)."""
    for dname, dtype in DTYPES:
        for K, N in SHAPES:
            wshape = (N, K) if op == "linear" else (K, N)
            W = rn(wshape, dtype, 1, std=K ** -0.5, device=cuda)
            c = rn((N,), dtype, 4, device=cuda)
            ref = rn((1, K), dtype, 3, device=cuda)
            pool = rn((max(BATCHES), K), dtype, 2, device=cuda)
            if op == "matmul":
                fn = lambda x: bi.matmul(x, W)
            elif op == "addmm":
                fn = lambda x: bi.addmm(c, x, W, 0.75, -1.25)
            else:
                fn = lambda x: bi.linear(x, W, c)
            base = fn(ref)
            assert bool((base != 0).any()), "degenerate all-zero output"
            base = bits(base[0])
            for B in BATCHES[1:]:
                for idx in sorted({0, B // 2, B - 1}):
                    y = fn(batch_with(ref, pool, B, idx))
                    d = int((bits(y[idx]) != base).sum())
                    assert d == 0, "%s %s K=%d N=%d B=%d idx=%d: %d elements differ" % (
                        op, dname, K, N, B, idx, d)


def test_config2_widest_shape_sweep(cuda):
    """BASELINE configs[1] at its widest (K, N) = (4096, 32000), (M,K)x(K,N),
    N(0,1/K) weights, M in {1, 2, 4, ..., 256}, all three dtypes: the row at
    positions 0, M//2 and M-1 has its M=1 bits. M = 256 takes the bench's
    dominant 256 x 128 footprint; smaller M cross every other footprint."""
    K, N = 4096, 32000
    for dname, dtype in DTYPES:
        W = rn((K, N), dtype, 1, std=K ** -0.5, device=cuda)
        ref = rn((1, K), dtype, 3, device=cuda)
        pool = rn((256, K), dtype, 2, device=cuda)
        base = bi.matmul(ref, W)
        assert bool((base != 0).any())
        base = bits(base[0])
        for M in (2, 4, 8, 16, 32, 64, 128, 256):
            for idx in sorted({0, M // 2, M - 1}):
                y = bi.matmul(batch_with(ref, pool, M, idx), W)
                d = int((bits(y[idx]) != base).sum())
                assert d == 0, "%s M=%d idx=%d: %d differ" % (dname, M, idx, d)
        del W, pool
        torch.cuda.empty_cache()


def test_every_row_slot(cuda):
    """A row gives the same bits in every slot of every tile: a batch made of
    copies of one row must return copies of that row's B=1 result."""
    for dname, dtype in DTYPES:
        for K, N in [(1024, 768), (4096, 4096)]:
            W = rn((N, K), dtype, 7, std=K ** -0.5, device=cuda)
            ref = rn((1, K), dtype, 8, device=cuda)
            one = bits(bi.linear(ref, W)[0])
            for M in (17, 64, 256, 300):
                y = bi.linear(ref.expand(M, K).contiguous(), W)
                yb = bits(y).reshape(M, N)
                bad = np.nonzero((yb != one[None, :]).any(axis=1))[0]
                assert bad.size == 0, "%s K=%d N=%d M=%d: rows %s differ" % (
                    dname, K, N, M, bad[:10].tolist())


@pytest.mark.parametrize("trans_b", [False, True])
def test_all_geometries_agree(cuda, trans_b):
    """Every workgroup footprint computes bitwise the same output: the direct
    proof that the footprint the launcher picks cannot change a result."""
    geos = _gemm.geometries()
    assert len(geos) >= 2
    ran = set()
    for dname, dtype in DTYPES:
        for M, K, N in [(300, 1000, 300), (1, 4096, 512), (77, 520, 130), (260, 4096, 520)]:
            a = rn((M, K), dtype, 11, device=cuda)
            b = rn((N, K) if trans_b else (K, N), dtype, 12, std=K ** -0.5, device=cuda)
            c = rn((N,), dtype, 13, device=cuda)
            for bias in (None, c):
                outs = {}
                for gi in range(len(geos)):
                    try:
                        y = _gemm._gemm(a, b, bias, trans_b, 1.5, 0.5, geometry=gi)
                    except NotImplementedError:
                        continue  # geometry built for 16-bit, aligned operands only
                    outs[gi] = bits(y)
                    ran.add((gi, dname))
                assert 0 in outs
                for gi, o in outs.items():
                    d = int((o != outs[0]).sum())
                    assert d == 0, "%s M=%d K=%d N=%d bias=%s geometry %s vs %s: %d differ" % (
                        dname, M, K, N, bias is not None, geos[gi], geos[0], d)
    # every geometry ran on some 16-bit case
    assert {gi for gi, dn in ran if dn != "float32"} == set(range(len(geos)))


@pytest.mark.parametrize("trans_b", [False, True])
def test_large_footprints_agree(cuda, trans_b):
    """The large-M footprints (128 x 128, 256 x 128 with loading waves, 256 x
    256 ping-pong, 256 x 256 with four waves) over several rounds of
    workgroups, with ragged M, N and K tails and a partial group of row
    blocks, give the same bits; at M = 4096 bi_gemm picks a 256 x 256
    footprint and a row keeps its M = 1 bits there."""
    geos = _gemm.geometries()
    big = [geos.index(f) for f in ((128, 128, 8), (256, 128, 12), (256, 256, 16), (256, 256, 4))]
    for dname, dtype in DTYPES[1:]:
        M, K, N = 4360, 1032, 4104
        a = rn((M, K), dtype, 41, device=cuda)
        b = rn((N, K) if trans_b else (K, N), dtype, 42, std=K ** -0.5, device=cuda)
        c = rn((N,), dtype, 43, device=cuda)
        outs = [bits(_gemm._gemm(a, b, c, trans_b, 0.75, -1.5, geometry=g)) for g in big]
        for g, o in zip(big[1:], outs[1:]):
            d = int((o != outs[0]).sum())
            assert d == 0, "%s trans_b=%s geometry %s: %d differ" % (dname, trans_b, geos[g], d)
        M, N = 4096, 4096
        a = rn((M, K), dtype, 44, device=cuda)
        b = rn((N, K) if trans_b else (K, N), dtype, 45, std=K ** -0.5, device=cuda)
        from mlx_batch_invariant import _lib
        assert geos[_lib.lib().bi_gemm_pick_geometry(M, N, K, _lib.DTYPE_CODES[dtype],
                                                     int(trans_b))] == (
            (256, 256, 4) if trans_b else (256, 256, 16))
        y = bits(_gemm._gemm(a, b, None, trans_b)).reshape(M, N)
        for r in (0, 1, 2047, 4095):
            one = bits(_gemm._gemm(a[r:r + 1].contiguous(), b, None, trans_b))
            assert (y[r] == one).all(), "%s trans_b=%s row %d" % (dname, trans_b, r)


def test_unaligned_operands_leave_the_aligned_only_footprint(cuda):
    """The 256x128 footprint (its loading waves issue every load) takes
    16-byte aligned operands only: forcing it on others raises, and bi_gemm
    launches the 128x128 footprint instead. Misaligned bases and a K that is
    not a multiple of 8 give the bits of the same values in aligned storage
    and of every footprint that takes them."""
    from mlx_batch_invariant import _lib
    geos = _gemm.geometries()
    g_pl = geos.index((256, 128, 12))
    L = _lib.lib()
    for dname, dtype in DTYPES[1:]:
        for K in (1024, 1001):
            M, N = 256, 25600
            assert L.bi_gemm_pick_geometry(M, N, K, _lib.DTYPE_CODES[dtype], 0) == g_pl
            a = rn((M, K), dtype, 31, device=cuda)
            b = rn((K, N), dtype, 32, std=K ** -0.5, device=cuda)
            ref = bits(bi.matmul(a, b))
            buf = torch.empty(M * K + 1, dtype=dtype, device=cuda)
            au = buf[1:].view(M, K)
            au.copy_(a)
            assert au.data_ptr() % 16 != 0
            assert (bits(bi.matmul(au, b)) == ref).all(), "%s K=%d: misaligned A" % (dname, K)
            with pytest.raises(NotImplementedError):
                _gemm._gemm(au, b, None, False, geometry=g_pl)
            if K % 8:
                with pytest.raises(NotImplementedError):
                    _gemm._gemm(a, b, None, False, geometry=g_pl)
            else:
                assert (bits(_gemm._gemm(a, b, None, False, geometry=g_pl)) == ref).all()
            for gi in (2, 3):
                assert (bits(_gemm._gemm(au, b, None, False, geometry=gi)) == ref).all(), (
                    "%s K=%d geometry %s" % (dname, K, geos[gi]))


def test_kn_and_nk_layouts_agree(cuda):
    """matmul on a (K, N) weight and linear on the same weight stored (N, K)
    feed the MFMAs identically, so they give the same bits; a transposed view
    is read in place with the same result."""
    for dname, dtype in DTYPES:
        for M, K, N in [(5, 1024, 1024), (256, 4096, 4096), (33, 520, 136)]:
            x = rn((M, K), dtype, 21, device=cuda)
            w = rn((N, K), dtype, 22, std=K ** -0.5, device=cuda)
            y_nk = bi.linear(x, w)
            y_kn = bi.matmul(x, w.t().contiguous())
            y_view = bi.matmul(x, w.t())
            assert ndiff(y_nk, y_kn) == 0, "%s M=%d K=%d N=%d" % (dname, M, K, N)
            assert ndiff(y_nk, y_view) == 0


def test_leading_dims_collapse_invariantly(cuda):
    """(B, S, K) and (B*S, K) give the same bits (reference tests:93-103)."""
    for dname, dtype in DTYPES:
        K, N = 1024, 512
        W = rn((K, N), dtype, 1, std=K ** -0.5, device=cuda)
        x = rn((24, K), dtype, 5, device=cuda)
        flat = bi.matmul(x, W)
        shaped = bi.matmul(x.reshape(4, 6, K), W).reshape(24, N)
        assert ndiff(flat, shaped) == 0


ACC_CASES = [(17, 1024, 512), (128, 2048, 256), (1, 4096, 512), (8, 11008, 4096),
             (128, 11008, 4096), (256, 4096, 4096),
             (256, 4096, 32000), (1, 4096, 32000)]   # configs[1]'s widest shape


def test_fp32_accuracy(cuda):
    """fp32: max-abs-err / max|exact| <= 4.5e-6 against float64 (north star; the
    reference's own test bound is 2e-5, tests:127) and no worse than 8x the
    error of stock torch.matmul (tests:128-129)."""
    for M, K, N in ACC_CASES:
        a = rn((M, K), torch.float32, 11, device=cuda)
        b = rn((K, N), torch.float32, 12, device=cuda)
        exact = ogemm.gemm_f64(f64(a), f64(b))
        scale = np.abs(exact).max()
        ours = np.abs(f64(bi.matmul(a, b)) - exact).max() / scale
        stock = np.abs(f64(torch.matmul(a, b)) - exact).max() / scale
        assert ours < 4.5e-6, "M=%d K=%d N=%d rel err %g (stock %g)" % (M, K, N, ours, stock)
        assert ours < 8 * stock + 1e-9, "M=%d K=%d N=%d ours %g stock %g" % (M, K, N, ours, stock)


def test_low_precision_within_one_ulp(cuda):
    """bf16/f16: every element within 1 ULP of the exact result, the ULP taken
    at max(|exact|, 2^-p * sum_k |a_k b_k|) so cancellation outputs are judged
    against the accumulation they came from (p = 8 bf16, 11 f16). Also the
    reference's max-normalised bounds (f16 < 5e-3, bf16 < 4e-2, tests:131-146)."""
    for dname, dtype, bound in (("float16", torch.float16, 5e-3), ("bfloat16", torch.bfloat16, 4e-2)):
        p = obits.PRECISION[dname]
        for M, K, N in ACC_CASES:
            a = rn((M, K), dtype, 11, device=cuda)
            b = rn((K, N), dtype, 12, device=cuda)
            a64, b64 = f64(a), f64(b)
            exact = ogemm.gemm_f64(a64, b64)
            floor = ogemm.abs_products(a64, b64) * 2.0 ** -p
            ulp = obits.ulp_of(np.maximum(np.abs(exact), floor), dname)
            got = f64(bi.matmul(a, b))
            worst = (np.abs(got - exact) / ulp).max()
            assert worst <= 1.0, "%s M=%d K=%d N=%d: %.3f ULP" % (dname, M, K, N, worst)
            rel = np.abs(got - exact).max() / np.abs(exact).max()
            assert rel < bound


def test_addmm_epilogue_single_rounding_bitwise(cuda):
    """Bias is applied to the fp32 accumulator as fma(alpha, acc, beta * c) and
    rounded once. Small-integer inputs make acc exact in any order, so the
    expected bits follow in numpy float32 arithmetic (tightens tests:148-158)."""
    for dname, dtype in DTYPES[1:] + DTYPES[:1]:
        g = torch.Generator().manual_seed(31)
        M, K, N = 40, 96, 72
        a = torch.randint(-4, 5, (M, K), generator=g).to(dtype)
        b = torch.randint(-4, 5, (K, N), generator=g).to(dtype)
        c = (torch.randn(N, generator=g) * 3).to(dtype)
        for alpha, beta in ((1.0, 1.0), (0.1, 0.3), (-2.5, 0.7)):
            acc = f64(a) @ f64(b)  # exact integers, |acc| < 2^11
            cb = (np.float32(beta) * f64(c).astype(np.float32)).astype(np.float64)
            # fma(alpha, acc, cb): alpha * acc + cb is exact in float64 at these
            # magnitudes (< 53 significant bits), so one rounding to fp32 follows.
            want = (np.float64(np.float32(alpha)) * acc + cb).astype(np.float32)
            want = obits.round_f32_to(want, dname)
            got = f64(bi.addmm(c.to(cuda), a.to(cuda), b.to(cuda), alpha, beta))
            assert (got == want).all(), "%s alpha=%g beta=%g: %d differ" % (
                dname, alpha, beta, int((got != want).sum()))


def test_closed_forms(cuda):
    for dname, dtype in DTYPES:
        # K = 1: out = RNE(a * b) exactly.
        a = rn((9, 1), dtype, 41, device=cuda)
        b = rn((1, 33), dtype, 42, device=cuda)
        want = obits.round_f32_to((f64(a) * f64(b)).astype(np.float32), dname)
        assert (f64(bi.matmul(a, b)) == want).all()
        # Identity weight: out = x bitwise.
        x = rn((70, 96), dtype, 43, device=cuda)
        eye = torch.eye(96, dtype=dtype, device=cuda)
        assert ndiff(bi.linear(x, eye), x) == 0
        assert ndiff(bi.matmul(x, eye), x) == 0
        # Integer-valued inputs: exact sums, order-independent.
        g = torch.Generator().manual_seed(44)
        ai = torch.randint(-3, 4, (50, 2000), generator=g).to(dtype)
        bi_ = torch.randint(-3, 4, (2000, 40), generator=g).to(dtype)
        exact = f64(ai) @ f64(bi_)  # partial sums stay below 2^24: exact in fp32
        want = obits.round_f32_to(exact.astype(np.float32), dname)
        assert (f64(bi.matmul(ai.to(cuda), bi_.to(cuda))) == want).all()
        # Zero K-padding does not change results: K=513 vs the same zero-padded to 528.
        a = rn((20, 513), dtype, 45, device=cuda)
        w = rn((64, 513), dtype, 46, std=0.05, device=cuda)
        ap = torch.nn.functional.pad(a, (0, 15))
        wp = torch.nn.functional.pad(w, (0, 15))
        assert ndiff(bi.linear(a, w), bi.linear(ap, wp)) == 0


def test_k_zero_and_empty(cuda):
    for dname, dtype in DTYPES:
        a = torch.empty((5, 0), dtype=dtype, device=cuda)
        b = torch.empty((0, 7), dtype=dtype, device=cuda)
        assert (bi.matmul(a, b) == 0).all()
        c = rn((7,), dtype, 1, device=cuda)
        assert ndiff(bi.addmm(c, a, b), c.expand(5, 7)) == 0
        assert bi.matmul(torch.empty((0, 8), dtype=dtype, device=cuda),
                         rn((8, 3), dtype, 2, device=cuda)).shape == (0, 3)


def test_graph_capture_replays_bitwise(cuda):
    """Captured in a HIP graph and replayed several times, with eager work in
    between, the result is bitwise the eager result every time."""
    for dname, dtype in DTYPES:
        x = rn((48, 1024), dtype, 51, device=cuda)
        w = rn((512, 1024), dtype, 52, std=1 / 32, device=cuda)
        b = rn((512,), dtype, 53, device=cuda)
        eager = bi.linear(x, w, b).clone()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            bi.linear(x, w, b)  # warm up on the capture stream
        torch.cuda.current_stream().wait_stream(s)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            y = bi.linear(x, w, b)
        for rep in range(4):
            graph.replay()
            torch.cuda.synchronize()
            assert ndiff(y, eager) == 0, "%s replay %d" % (dname, rep)
            _ = bi.linear(x[:3].contiguous(), w, b)  # eager work between replays
            torch.cuda.synchronize()


def test_stock_matmul_is_batch_variant(cuda):
    """Negative control (reference TestStockMLXIsStillBroken, tests:161-180): if
    stock torch.matmul were batch-invariant everywhere, the invariance tests
    would prove nothing."""
    found = []
    for dname, dtype in DTYPES:
        for K, N in [(2048, 1024), (4096, 4096), (11008, 4096)]:
            W = rn((K, N), dtype, 1, std=K ** -0.5, device=cuda)
            ref, pool = rn((1, K), dtype, 3, device=cuda), rn((256, K), dtype, 2, device=cuda)
            base = bits(torch.matmul(ref, W)[0])
            for B in (2, 33, 128, 256):
                y = torch.matmul(batch_with(ref, pool, B, 0), W)
                if int((bits(y[0]) != base).sum()):
                    found.append("%s K=%d N=%d B=%d" % (dname, K, N, B))
    assert found, "stock torch.matmul looks batch-invariant everywhere"


def test_wavefront_is_64(cuda):
    """The fixed reduction shapes assume 64-lane wavefronts (the analogue of the
    reference's SIMD-width guard, tests:459-466)."""
    import ctypes

    from mlx_batch_invariant import _lib

    w = ctypes.c_int()
    _lib.check(_lib.lib().bi_device_wavefront_size(ctypes.byref(w)), "wavefront")
    assert w.value == 64


def test_timed_launch_matches_and_records_the_kernel(cuda):
    """bi_gemm_timed runs the same kernel as bi_gemm (same bits) and writes the
    launch's own start/end timestamps into the two events."""
    g = torch.Generator().manual_seed(3)
    a = torch.randn(256, 4096, generator=g).to(torch.bfloat16).to(cuda)
    b = (torch.randn(4096, 4096, generator=g) / 64).to(torch.bfloat16).to(cuda)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    e1.record()
    y = _gemm.matmul_timed(a, b, e0, e1)
    torch.cuda.synchronize()
    assert (bits(y) == bits(bi.matmul(a, b))).all()
    assert 0.0 < e0.elapsed_time(e1) < 100.0  # milliseconds


def test_padding_steps_change_no_bit(cuda):
    """The pipelined loop finishes its last round of stages with chunk-steps
    that see only zeros. Those add exact zeros to an accumulator that starts at
    +0.0, so every footprint gives the same bits for ragged K, exact-zero sums
    (which must stay +0.0), negative zeros in the inputs and infinities."""
    geos = _gemm.geometries()
    for dname, dtype in DTYPES:
        for K in (520, 1000, 4104):
            a = rn((70, K), dtype, 21, device=cuda)
            b = rn((K, 96), dtype, 22, std=K ** -0.5, device=cuda)
            a[0] = 0.0                     # all products zero
            a[1] = -0.0
            a[2, 0::2], a[2, 1::2] = 1.0, -1.0  # with b[:, 0] = 1: an exact-zero sum
            b[:, 0] = 1.0
            b[:, 1] = -0.0
            a[3, 5] = float("inf")
            for trans_b, bb in ((False, b), (True, b.t().contiguous())):
                outs = {}
                for gi in range(len(geos)):
                    try:
                        outs[gi] = bits(_gemm._gemm(a, bb, None, trans_b, geometry=gi))
                    except NotImplementedError:
                        continue
                ref = outs[0]
                for gi, o in outs.items():
                    assert (o == ref).all(), "%s K=%d trans_b=%s geometry %s differs" % (
                        dname, K, trans_b, geos[gi])
            y = _gemm._gemm(a, b, None, False)
            z = torch.zeros((), dtype=dtype, device=cuda)
            for r, c in [(0, 0), (0, 7), (1, 3), (2, 0), (0, 1)]:
                assert bits(y[r, c:c + 1])[0] == bits(z.reshape(1))[0], \
                    "%s K=%d: element (%d, %d) is not +0.0" % (dname, K, r, c)
