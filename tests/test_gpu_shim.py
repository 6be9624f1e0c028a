"""batch_invariant_mode on the GPU: routed torch calls run the invariant
kernels (same bits as the direct bi.* calls), a small model's rows are
invariant across batch sizes, and unsupported calls follow strict / non-strict
(reference tests/test_invariance.py:622-684)."""

import math

import pytest
import torch
import torch.nn.functional as F

import mlx_batch_invariant as bi

from helpers import batch_with, bits, ndiff, rn

pytestmark = pytest.mark.gpu


def test_routed_calls_match_direct_kernels(cuda):
    dtype = torch.bfloat16
    a = rn((37, 1024), dtype, 1, device=cuda)
    w = rn((1024, 768), dtype, 2, std=1 / 32, device=cuda)
    c = rn((768,), dtype, 3, device=cuda)
    lin = torch.nn.Linear(1024, 768, dtype=dtype, device=cuda)
    q = rn((2, 16, 5, 128), dtype, 4, device=cuda)
    k = rn((2, 4, 300, 128), dtype, 5, device=cuda)
    v = rn((2, 4, 300, 128), dtype, 6, device=cuda)
    with torch.no_grad():
        direct = dict(mm=bi.matmul(a, w), addmm=bi.addmm(c, a, w, 0.5, 2.0),
                      lin=bi.linear(a, lin.weight, lin.bias),
                      sdpa=bi.scaled_dot_product_attention(q, k, v, scale=0.3))
        with bi.batch_invariant_mode():
            routed = dict(mm=torch.matmul(a, w), addmm=torch.addmm(c, a, w, beta=2.0, alpha=0.5),
                          lin=lin(a),
                          sdpa=F.scaled_dot_product_attention(q, k, v, scale=0.3, enable_gqa=True))
            op = a @ w
            mm_fn, mm_method = torch.mm(a, w), a.mm(w)
    for key in direct:
        assert ndiff(direct[key], routed[key]) == 0, key
    assert ndiff(op, direct["mm"]) == 0
    assert ndiff(mm_fn, direct["mm"]) == 0 and ndiff(mm_method, direct["mm"]) == 0


def test_is_causal_is_aligned_to_the_start(cuda):
    """torch's is_causal masks key i > query row s (top-left); the reference's
    "causal" string aligns to the end (row s sees i <= N - L + s)."""
    dtype = torch.float32
    q = rn((1, 4, 6, 64), dtype, 7, device=cuda)
    k = rn((1, 4, 10, 64), dtype, 8, device=cuda)
    v = rn((1, 4, 10, 64), dtype, 9, device=cuda)
    stock = F.scaled_dot_product_attention(q, k, v, is_causal=True)
    with torch.no_grad(), bi.batch_invariant_mode():
        routed = F.scaled_dot_product_attention(q, k, v, is_causal=True)
    assert (routed - stock).abs().max().item() < 1e-5
    tl = torch.arange(10, device=cuda)[None, :] <= torch.arange(6, device=cuda)[:, None]
    assert ndiff(routed, bi.scaled_dot_product_attention(q, k, v, mask=tl)) == 0


def test_model_rows_invariant_under_mode(cuda):
    """A small decoder-style stack (linear, attention, MLP) under the mode: a
    sequence's logits have the same bits alone and in any batch (reference
    tests:622-640, bench/bench.py:217-246)."""
    torch.manual_seed(0)
    D, H, Hkv, hd, V = 512, 8, 2, 64, 1000
    dtype = torch.bfloat16

    class Block(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.q = torch.nn.Linear(D, H * hd, bias=False)
            self.kv = torch.nn.Linear(D, 2 * Hkv * hd, bias=False)
            self.o = torch.nn.Linear(H * hd, D, bias=False)
            self.up = torch.nn.Linear(D, 4 * D)
            self.down = torch.nn.Linear(4 * D, D)

        def forward(self, x):
            B, L, _ = x.shape
            q = self.q(x).view(B, L, H, hd).transpose(1, 2)
            k, v = self.kv(x).view(B, L, 2, Hkv, hd).permute(2, 0, 3, 1, 4)
            a = F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True)
            x = x + self.o(a.transpose(1, 2).reshape(B, L, H * hd))
            return x + self.down(F.silu(self.up(x)))

    model = torch.nn.Sequential(Block(), Block(), torch.nn.Linear(D, V)).to(cuda, dtype)
    ref = rn((1, 24, D), dtype, 11, device=cuda)
    pool = rn((8, 24, D), dtype, 12, device=cuda)
    with torch.no_grad(), bi.batch_invariant_mode():
        base = bits(model(ref)[0, -1])
        for B in (2, 3, 8):
            y = model(batch_with(ref, pool, B, B // 2))
            assert (bits(y[B // 2, -1]) == base).all(), "B=%d" % B


def test_strict_mode_on_gpu(cuda):
    q = rn((1, 4, 1, 48), torch.float16, 61, device=cuda)
    k = rn((1, 4, 128, 48), torch.float16, 62, device=cuda)
    with bi.batch_invariant_mode(strict=True):
        with pytest.raises(NotImplementedError):
            F.scaled_dot_product_attention(q, k, k, scale=0.1)
    with bi.batch_invariant_mode(strict=False):
        y = F.scaled_dot_product_attention(q, k, k, scale=0.1)
    assert y.shape == (1, 4, 1, 48)
