"""torch.compile around the invariant kernels (reference
tests/test_invariance.py:595-640, TestCompiled). The compiler may reorder and
fuse the graph around them, never inside: traced calls become the opaque ops
mlx_bi::gemm / mlx_bi::qgemm / mlx_bi::sdpa, with no graph break. backend="aot_eager" traces
through Dynamo and AOTAutograd and runs the graph's kernels as they are, so
no code is generated for the surrounding ops."""

import numpy as np
import pytest
import torch

import mlx_batch_invariant as bi

from helpers import DTYPES, batch_with, bits, rn

pytestmark = pytest.mark.gpu


def _compile(fn, **kw):
    torch._dynamo.reset()
    return torch.compile(fn, backend="aot_eager", **kw)


def test_attention_is_invariant_under_compile(cuda):
    H, Hkv, N, D = 16, 8, 2048, 128
    qls = [1, 2, 4, 8, 9, 16]
    for dname, dtype in DTYPES:
        k, v = rn((1, Hkv, N, D), dtype, 51, device=cuda), rn((1, Hkv, N, D), dtype, 52, device=cuda)
        qf = rn((1, H, max(qls), D), dtype, 53, device=cuda)
        fn = _compile(lambda q: bi.scaled_dot_product_attention(q, k, v), fullgraph=True)
        base = None
        for qL in qls:
            q = qf[:, :, max(qls) - qL:, :].contiguous()
            got = bits(fn(q)[:, :, -1, :])
            eager = bits(bi.scaled_dot_product_attention(q, k, v)[:, :, -1, :])
            assert np.array_equal(got, eager), "compiled != eager %s qL=%d" % (dname, qL)
            if base is None:
                base = got
            else:
                assert int((got != base).sum()) == 0, "compiled sdpa %s qL=%d" % (dname, qL)


def test_mode_holds_for_function_compiled_inside(cuda):
    """A module first traced inside the mode captures the invariant kernels and
    stays invariant for every later call inside it."""
    torch.manual_seed(54)
    net = torch.nn.Sequential(torch.nn.Linear(256, 512), torch.nn.GELU(),
                              torch.nn.Linear(512, 128)).to(cuda, torch.float16)
    net.requires_grad_(False)
    ref = rn((1, 256), torch.float16, 55, device=cuda)
    pool = rn((16, 256), torch.float16, 56, device=cuda)
    with bi.batch_invariant_mode(strict=True):
        fn = _compile(net)
        base = None
        for B in (1, 2, 3, 8, 16):
            idx = B // 2
            got = bits(fn(batch_with(ref, pool, B, idx))[idx])
            if base is None:
                base = got
            else:
                assert int((got != base).sum()) == 0, "compiled-inside mode B=%d" % B
        eager = bits(net(ref)[0])
    assert np.array_equal(base, eager)


def test_compiled_gemm_is_one_graph_and_matches_eager(cuda):
    w = rn((384, 512), torch.bfloat16, 57, std=512 ** -0.5, device=cuda)
    c = rn((384,), torch.bfloat16, 58, device=cuda)
    x = rn((5, 7, 512), torch.bfloat16, 59, device=cuda)
    fn = _compile(lambda t: torch.relu(bi.linear(t, w, c)) + 1, fullgraph=True)
    assert np.array_equal(bits(fn(x)), bits(torch.relu(bi.linear(x, w, c)) + 1))


def test_ops_pass_opcheck(cuda):
    a = rn((33, 256), torch.bfloat16, 60, device=cuda)
    w = rn((64, 256), torch.bfloat16, 61, device=cuda)
    from mlx_batch_invariant import _ops

    torch.library.opcheck(_ops.gemm, (a, w, None, True, 1.0, 1.0))
    q = rn((1, 4, 3, 64), torch.bfloat16, 62, device=cuda)
    k = rn((1, 2, 40, 64), torch.bfloat16, 63, device=cuda)
    torch.library.opcheck(_ops.sdpa, (q, k, k, 0.125, 1, None, [0, 0, 0], 37, None))
    wq, s, b = bi.quantize(rn((64, 256), torch.bfloat16, 64), 64, 4)
    torch.library.opcheck(_ops.qgemm, (a, wq.to(cuda), s.to(cuda), b.to(cuda), 64, 4))


def test_compiled_quantized_linear_matches_eager(cuda):
    wq, s, b = (t.to(cuda) for t in bi.quantize(rn((256, 512), torch.float16, 65), 32, 8))
    x = rn((3, 5, 512), torch.float16, 66, device=cuda)
    fn = _compile(lambda t: bi.quantized_linear(t, wq, s, b, 32, 8) * 2, fullgraph=True)
    assert np.array_equal(bits(fn(x)), bits(bi.quantized_linear(x, wq, s, b, 32, 8) * 2))
