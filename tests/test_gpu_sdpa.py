"""GPU parity tests of the invariant attention (bi.scaled_dot_product_attention).

Mirrors reference tests/test_invariance.py:242-364, 408-455 and 595-620:
query-length, batch, mask and sink invariance on raw bits; accuracy against
the float64 oracle (oracle/sdpa.py); plus the north star's context-growth and
graph-capture axes and closed forms.
"""

import math

import numpy as np
import pytest
import torch

import mlx_batch_invariant as bi
from oracle import bits as obits
from oracle import sdpa as osdpa

from helpers import DTYPES, batch_with, bits, f64, ndiff, rn

pytestmark = pytest.mark.gpu

QLS = [1, 2, 3, 4, 7, 8, 9, 16, 17]
CASES = [
    (32, 8, 512, 128),    # GQA 4, short context
    (16, 8, 4096, 128),   # GQA 2 at 4096
    (8, 8, 4096, 128),    # MHA
    (32, 8, 8192, 128),   # GQA long context
    (4, 4, 333, 64),      # ragged N, small head dim
    (8, 2, 700, 256),     # large head dim
]


def _last_row(y):
    return bits(y[:, :, -1, :])


def test_query_length_invariance(cuda):
    for dname, dtype in DTYPES:
        for H, Hkv, N, D in CASES:
            k = rn((1, Hkv, N, D), dtype, 11, device=cuda)
            v = rn((1, Hkv, N, D), dtype, 12, device=cuda)
            qf = rn((1, H, max(QLS), D), dtype, 13, device=cuda)
            base = None
            for qL in QLS:
                q = qf[:, :, max(QLS) - qL:, :].contiguous()
                y = bi.scaled_dot_product_attention(q, k, v)
                got = _last_row(y)
                if base is None:
                    base = got
                    assert bool((y != 0).any()), "degenerate output"
                else:
                    d = int((got != base).sum())
                    assert d == 0, "sdpa %s H=%d/%d N=%d qL=%d: %d differ" % (dname, H, Hkv, N, qL, d)


def test_batch_invariance(cuda):
    H, Hkv, N, D = 16, 8, 2048, 128
    for dname, dtype in DTYPES:
        k1, v1 = rn((1, Hkv, N, D), dtype, 21, device=cuda), rn((1, Hkv, N, D), dtype, 22, device=cuda)
        q1 = rn((1, H, 1, D), dtype, 23, device=cuda)
        kp, vp = rn((16, Hkv, N, D), dtype, 24, device=cuda), rn((16, Hkv, N, D), dtype, 25, device=cuda)
        qp = rn((16, H, 1, D), dtype, 26, device=cuda)
        base = None
        for B in (1, 2, 3, 8, 16):
            for idx in sorted({0, B // 2, B - 1}):
                y = bi.scaled_dot_product_attention(batch_with(q1, qp, B, idx),
                                                    batch_with(k1, kp, B, idx),
                                                    batch_with(v1, vp, B, idx))
                got = bits(y[idx])
                if base is None:
                    base = got
                else:
                    assert int((got != base).sum()) == 0, "sdpa %s B=%d idx=%d" % (dname, B, idx)


@pytest.mark.parametrize("H,Hkv,D,batches", [(32, 8, 128, (1, 32, 64)),
                                              (32, 4, 64, (1, 32, 64, 128)),
                                              (64, 1, 128, (1, 3, 300)),    # MQA: 64 columns per kv head
                                              (16, 16, 256, (1, 8, 20))])
def test_head_grouping_does_not_change_bits(cuda, H, Hkv, D, batches):
    """The launch shape follows the grid: bf16/f16 decode grids that fill the
    GPU run one workgroup per kv head, smaller ones split the output dims over
    2, 4 or 8 workgroups, and more than 16 query columns per kv head (MQA)
    take the prefill shape; the fp32 kernel groups query heads per workgroup
    by grid size. The batch sizes here cross those choices: a row's bits must
    not move."""
    N = 256
    for dname, dtype in DTYPES:
        q1 = rn((1, H, 1, D), dtype, 31, device=cuda)
        k1, v1 = rn((1, Hkv, N, D), dtype, 32, device=cuda), rn((1, Hkv, N, D), dtype, 33, device=cuda)
        B = max(batches)
        qp = rn((B, H, 1, D), dtype, 34, device=cuda)
        kp, vp = rn((B, Hkv, N, D), dtype, 35, device=cuda), rn((B, Hkv, N, D), dtype, 36, device=cuda)
        base = bits(bi.scaled_dot_product_attention(q1, k1, v1, mask="causal")[0])
        for B in batches[1:]:
            idx = B - 1
            y = bi.scaled_dot_product_attention(batch_with(q1, qp, B, idx), batch_with(k1, kp, B, idx),
                                                batch_with(v1, vp, B, idx), mask="causal")
            assert int((bits(y[idx]) != base).sum()) == 0, "%s H=%d Hkv=%d D=%d B=%d" % (
                dname, H, Hkv, D, B)


def test_causal_and_masks_are_invariant(cuda):
    H, Hkv, N, D = 8, 4, 1024, 128
    for dname, dtype in DTYPES:
        k, v = rn((1, Hkv, N, D), dtype, 31, device=cuda), rn((1, Hkv, N, D), dtype, 32, device=cuda)
        qf = rn((1, H, 16, D), dtype, 33, device=cuda)
        add = rn((1, 1, 1, N), dtype, 34, device=cuda)
        keep = torch.rand(1, 1, 1, N, generator=torch.Generator().manual_seed(35)) > 0.3
        keep = keep.to(cuda)
        for label, mk in (("causal", lambda qL: "causal"), ("additive", lambda qL: add),
                          ("bool", lambda qL: keep)):
            base = None
            for qL in (1, 4, 8, 9, 16):
                q = qf[:, :, 16 - qL:, :].contiguous()
                got = _last_row(bi.scaled_dot_product_attention(q, k, v, mask=mk(qL)))
                if base is None:
                    base = got
                else:
                    assert int((got != base).sum()) == 0, "sdpa %s %s qL=%d" % (label, dname, qL)


def test_masked_decode_is_batch_invariant(cuda):
    """An additive and a boolean mask per batch entry: a sequence's row has the
    same bits alone and at batch sizes whose grids take every launch shape
    (bf16/f16: dims split over 8, 4, 2 workgroups and unsplit; fp32: one, two
    and four query heads per workgroup, whose mask rows sit at offsets of the
    head stride)."""
    H, Hkv, N, D = 32, 8, 1000, 128
    g = torch.Generator().manual_seed(36)
    for dname, dtype in DTYPES:
        q1, k1, v1 = (rn((1, H, 1, D), dtype, 37, device=cuda), rn((1, Hkv, N, D), dtype, 38, device=cuda),
                      rn((1, Hkv, N, D), dtype, 39, device=cuda))
        qp, kp, vp = (rn((64, H, 1, D), dtype, 40, device=cuda), rn((64, Hkv, N, D), dtype, 41, device=cuda),
                      rn((64, Hkv, N, D), dtype, 42, device=cuda))
        add = rn((64, 1, 1, N), dtype, 43, device=cuda)
        add[:, :, :, ::5] = -float("inf")
        keep = (torch.rand(64, 1, 1, N, generator=g) > 0.2).to(cuda)
        for label, mpool in (("additive", add), ("bool", keep)):
            m1 = mpool[7:8]
            base = bits(bi.scaled_dot_product_attention(q1, k1, v1, mask=m1)[0])
            for B in (2, 5, 17, 40, 64):
                idx = B // 2
                mb = torch.cat([mpool[:idx], m1, mpool[idx + 1:B]]) if B > 1 else m1
                y = bi.scaled_dot_product_attention(batch_with(q1, qp, B, idx), batch_with(k1, kp, B, idx),
                                                    batch_with(v1, vp, B, idx), mask=mb)
                assert int((bits(y[idx]) != base).sum()) == 0, "%s %s B=%d" % (label, dname, B)


def test_values_behind_a_mask_are_never_read(cuda):
    """The reference skips masked keys (_attention.py:94-96), so whatever their
    value rows hold (here NaN, as in an unwritten cache slot behind a padding
    mask) cannot reach the output: bitwise equal to the same call with those
    rows zeroed, for decode and prefill shapes."""
    H, Hkv, N, D = 8, 2, 300, 128
    for dname, dtype in DTYPES:
        for B, qL in ((3, 1), (1, 40)):
            q = rn((B, H, qL, D), dtype, 44, device=cuda)
            k = rn((B, Hkv, N, D), dtype, 45, device=cuda)
            v = rn((B, Hkv, N, D), dtype, 46, device=cuda)
            keep = torch.ones(B, 1, 1, N, dtype=torch.bool)
            keep[..., 250:] = False   # padding past each sequence's end
            keep[..., 7::11] = False  # and scattered holes
            keep = keep.to(cuda)
            vnan = v.clone()
            vnan[:, :, ~keep[0, 0, 0]] = float("nan")
            vzero = v.clone()
            vzero[:, :, ~keep[0, 0, 0]] = 0
            got = bi.scaled_dot_product_attention(q, k, vnan, mask=keep)
            want = bi.scaled_dot_product_attention(q, k, vzero, mask=keep)
            assert torch.isfinite(got).all(), "%s B=%d qL=%d" % (dname, B, qL)
            assert np.array_equal(bits(got), bits(want)), "%s B=%d qL=%d" % (dname, B, qL)


def test_context_growth_chunked_prefill(cuda):
    """32/8 heads, D=128, bf16; KV grown 4000 -> 4200 with the
    new keys masked. A query row's result computed over the first N' keys must
    not change when the cache holds more keys that the row cannot see, nor with
    the number of query rows submitted together (1..16)."""
    H, Hkv, D, NMAX = 32, 8, 128, 4200
    for dname, dtype in DTYPES:
        k = rn((1, Hkv, NMAX, D), dtype, 41, device=cuda)
        v = rn((1, Hkv, NMAX, D), dtype, 42, device=cuda)
        qf = rn((1, H, 16, D), dtype, 43, device=cuda)
        for n_vis in (4000, 4096, 4097, 4133):
            base = None
            for n_phys in (n_vis, n_vis + 1, n_vis + 31, n_vis + 64, NMAX):
                keep = (torch.arange(n_phys, device=cuda) < n_vis).reshape(1, 1, 1, n_phys)
                for qL in (1, 5, 16):
                    q = qf[:, :, 16 - qL:, :].contiguous()
                    kk, vv = k[:, :, :n_phys], v[:, :, :n_phys]
                    mask = keep if n_phys > n_vis else None
                    got = _last_row(bi.scaled_dot_product_attention(q, kk, vv, mask=mask))
                    if base is None:
                        base = got
                    else:
                        d = int((got != base).sum())
                        assert d == 0, "%s visible=%d cache=%d qL=%d: %d differ" % (
                            dname, n_vis, n_phys, qL, d)


def test_causal_rows_match_masked_prefix(cuda):
    """Causal row s (aligned to the end) equals an explicit boolean prefix mask
    and equals the same row computed alone over its visible keys."""
    H, Hkv, N, D = 32, 8, 4200, 128
    dtype = torch.bfloat16
    k, v = rn((1, Hkv, N, D), dtype, 51, device=cuda), rn((1, Hkv, N, D), dtype, 52, device=cuda)
    q = rn((1, H, 16, D), dtype, 53, device=cuda)
    yc = bi.scaled_dot_product_attention(q, k, v, mask="causal")
    tri = torch.arange(N, device=cuda)[None, :] <= (N - 16 + torch.arange(16, device=cuda))[:, None]
    ym = bi.scaled_dot_product_attention(q, k, v, mask=tri.reshape(1, 1, 16, N))
    assert ndiff(yc, ym) == 0
    for s in (0, 7, 15):
        n_vis = N - 16 + s + 1
        alone = bi.scaled_dot_product_attention(q[:, :, s:s + 1].contiguous(),
                                                k[:, :, :n_vis], v[:, :, :n_vis])
        assert ndiff(alone[:, :, 0], yc[:, :, s]) == 0, "row %d" % s


def test_sinks_are_query_length_invariant(cuda):
    H, Hkv, N, D = 32, 8, 1024, 128
    for dname, dtype in DTYPES:
        k, v = rn((1, Hkv, N, D), dtype, 71, device=cuda), rn((1, Hkv, N, D), dtype, 72, device=cuda)
        qf = rn((1, H, 17, D), dtype, 73, device=cuda)
        sinks = rn((H,), dtype, 74, device=cuda)
        base = None
        for qL in (1, 2, 3, 7, 8, 9, 16, 17):
            q = qf[:, :, 17 - qL:, :].contiguous()
            got = _last_row(bi.scaled_dot_product_attention(q, k, v, sinks=sinks))
            if base is None:
                base = got
            else:
                assert int((got != base).sum()) == 0, "sinks %s qL=%d" % (dname, qL)


def test_sinks_change_the_answer(cuda):
    H, Hkv, N, D = 8, 8, 256, 64
    q, k = rn((1, H, 1, D), torch.float32, 75, device=cuda), rn((1, Hkv, N, D), torch.float32, 76, device=cuda)
    v = rn((1, Hkv, N, D), torch.float32, 77, device=cuda)
    sinks = torch.full((H,), 10.0, dtype=torch.float32, device=cuda)
    without = bi.scaled_dot_product_attention(q, k, v)
    with_ = bi.scaled_dot_product_attention(q, k, v, sinks=sinks)
    assert ndiff(without, with_) > 0


@pytest.mark.parametrize("dname,dtype,tol", [("float32", torch.float32, 2e-6),
                                             ("float16", torch.float16, 5e-3),
                                             ("bfloat16", torch.bfloat16, 3e-2)])
def test_accuracy_against_float64(cuda, dname, dtype, tol):
    """Reference tests:408-432: fp32 < 2e-6, bf16 < 3e-2 (max-normalised)."""
    for H, Hkv, qL, N, D, mask in ((8, 4, 4, 2048, 128, None), (32, 8, 16, 4200, 128, "causal"),
                                   (4, 2, 3, 777, 64, "add"), (8, 8, 2, 300, 256, None)):
        q, k, v = (rn((1, H, qL, D), dtype, 51, device=cuda), rn((1, Hkv, N, D), dtype, 52, device=cuda),
                   rn((1, Hkv, N, D), dtype, 53, device=cuda))
        add = rn((1, 1, qL, N), dtype, 54, device=cuda) if mask == "add" else None
        m = add if mask == "add" else mask
        ours = f64(bi.scaled_dot_product_attention(q, k, v, mask=m))
        want = osdpa.sdpa_f64(f64(q), f64(k), f64(v), mask=None if add is None else f64(add),
                              causal_offset=(N - qL) if mask == "causal" else None)
        err = np.abs(ours - want).max() / np.abs(want).max()
        assert err < tol, "%s H=%d/%d qL=%d N=%d D=%d mask=%s: %.3e" % (dname, H, Hkv, qL, N, D, mask, err)
        # No worse than the reference-order fp32 restatement (4x, tests:430-431).
        fixed = osdpa.sdpa_fixed32(f64(q), f64(k), f64(v), mask=None if add is None else f64(add),
                                   causal_offset=(N - qL) if mask == "causal" else None,
                                   out_dtype=dname)
        err_fixed = np.abs(fixed - want).max() / np.abs(want).max()
        assert err < 4 * err_fixed + 1e-7, "%s: ours %.3e vs restatement %.3e" % (dname, err, err_fixed)


def test_decode_config3_accuracy_and_batch(cuda):
    """BASELINE config 3 shapes: 32/8 heads, D=128, q_len 1, bf16, no mask."""
    H, Hkv, D = 32, 8, 128
    for B, N in ((1, 128), (4, 1000), (2, 8192), (64, 256)):
        q = rn((B, H, 1, D), torch.bfloat16, 61, device=cuda)
        k = rn((B, Hkv, N, D), torch.bfloat16, 62, device=cuda)
        v = rn((B, Hkv, N, D), torch.bfloat16, 63, device=cuda)
        y = bi.scaled_dot_product_attention(q, k, v, scale=1 / math.sqrt(128))
        want = osdpa.sdpa_f64(f64(q), f64(k), f64(v))
        err = np.abs(f64(y) - want).max() / np.abs(want).max()
        assert err < 3e-2
        for b in (0, B - 1):
            one = bi.scaled_dot_product_attention(q[b:b + 1], k[b:b + 1], v[b:b + 1],
                                                  scale=1 / math.sqrt(128))
            assert ndiff(one[0], y[b]) == 0, "B=%d N=%d b=%d" % (B, N, b)


def test_closed_forms(cuda):
    for dname, dtype in DTYPES:
        # One key: out = v_0 exactly.
        q, k, v = (rn((2, 4, 3, 64), dtype, 81, device=cuda), rn((2, 2, 1, 64), dtype, 82, device=cuda),
                   rn((2, 2, 1, 64), dtype, 83, device=cuda))
        y = bi.scaled_dot_product_attention(q, k, v)
        assert ndiff(y, v.repeat_interleave(2, dim=1).expand(2, 4, 3, 64)) == 0
        # All keys equal: out = mean of v; v in multiples of 1/4 over 64 keys is exact.
        N = 64
        kk = rn((1, 2, 1, 128), dtype, 84, device=cuda).expand(1, 2, N, 128).contiguous()
        g = torch.Generator().manual_seed(85)
        vv = (torch.randint(-8, 9, (1, 2, N, 128), generator=g) / 4.0).to(dtype).to(cuda)
        qq = rn((1, 4, 2, 128), dtype, 86, device=cuda)
        y = f64(bi.scaled_dot_product_attention(qq, kk, vv))
        mean = f64(vv).mean(axis=2, keepdims=True).repeat(2, axis=1)  # exact in fp32
        mean = obits.round_f32_to(mean.astype(np.float32), dname)
        assert (y == np.broadcast_to(mean, y.shape)).all()
        # Fully masked rows are 0 (reference _attention.py:139).
        none = torch.zeros(1, 1, 1, N, dtype=torch.bool, device=cuda)
        y = bi.scaled_dot_product_attention(qq, kk, vv, mask=none)
        assert (y == 0).all()
        # Causal with more query rows than keys: the leading rows see nothing -> 0.
        y = bi.scaled_dot_product_attention(rn((1, 4, 8, 128), dtype, 87, device=cuda),
                                            kk[:, :, :5], vv[:, :, :5], mask="causal")
        assert (y[:, :, :3] == 0).all() and bool((y[:, :, 3:] != 0).any())
        # No keys at all (an empty cache): every row is 0, with or without a sink.
        e = torch.empty(1, 2, 0, 128, dtype=dtype, device=cuda)
        assert (bi.scaled_dot_product_attention(qq, e, e) == 0).all()
        assert (bi.scaled_dot_product_attention(qq, e, e, sinks=torch.ones(4, dtype=dtype,
                                                                           device=cuda)) == 0).all()
        # A dominant sink drives the output to ~0.
        sinks = torch.full((4,), 60.0, dtype=dtype, device=cuda)
        y = f64(bi.scaled_dot_product_attention(qq, kk, vv, sinks=sinks))
        assert np.abs(y).max() < 1e-6


def test_strided_kv_cache_view(cuda):
    """A KV-cache slice k[:, :, :N] is read in place and matches a compact copy."""
    dtype = torch.bfloat16
    cache_k = rn((2, 8, 5000, 128), dtype, 91, device=cuda)
    cache_v = rn((2, 8, 5000, 128), dtype, 92, device=cuda)
    q = rn((2, 32, 3, 128), dtype, 93, device=cuda)
    a = bi.scaled_dot_product_attention(q, cache_k[:, :, :4100], cache_v[:, :, :4100])
    b = bi.scaled_dot_product_attention(q, cache_k[:, :, :4100].contiguous(),
                                        cache_v[:, :, :4100].contiguous())
    assert ndiff(a, b) == 0


def test_graph_capture_replays_bitwise(cuda):
    for dname, dtype in DTYPES:
        q = rn((2, 16, 4, 128), dtype, 95, device=cuda)
        k = rn((2, 8, 1500, 128), dtype, 96, device=cuda)
        v = rn((2, 8, 1500, 128), dtype, 97, device=cuda)
        eager = bi.scaled_dot_product_attention(q, k, v, mask="causal").clone()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            bi.scaled_dot_product_attention(q, k, v, mask="causal")
        torch.cuda.current_stream().wait_stream(s)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            y = bi.scaled_dot_product_attention(q, k, v, mask="causal")
        for rep in range(4):
            graph.replay()
            torch.cuda.synchronize()
            assert ndiff(y, eager) == 0, "%s replay %d" % (dname, rep)
            _ = bi.scaled_dot_product_attention(q[:1], k[:1], v[:1])
            torch.cuda.synchronize()


def test_stock_sdpa_is_query_length_variant(cuda):
    """Negative control (reference TestStockAttentionIsQueryVariant): stock
    torch SDPA must change a fixed query row's bits somewhere when the number of
    query rows submitted with it changes, else the attention half proves
    nothing. Sweeps several shapes and dtypes and needs one variant case."""
    import torch.nn.functional as F

    found = []
    for dname, dtype in DTYPES:
        for H, Hkv, N, D in ((32, 8, 512, 128), (8, 8, 4096, 128), (16, 16, 1000, 64)):
            k = rn((1, Hkv, N, D), dtype, 61, device=cuda).repeat_interleave(H // Hkv, dim=1)
            v = rn((1, Hkv, N, D), dtype, 62, device=cuda).repeat_interleave(H // Hkv, dim=1)
            qf = rn((1, H, 64, D), dtype, 63, device=cuda)
            base = None
            for qL in (1, 2, 8, 9, 16, 17, 64):
                q = qf[:, :, 64 - qL:, :].contiguous()
                got = _last_row(F.scaled_dot_product_attention(q, k, v))
                if base is None:
                    base = got
                elif int((got != base).sum()):
                    found.append("%s H=%d N=%d qL=%d" % (dname, H, N, qL))
    assert found, "stock torch SDPA looks query-length invariant everywhere"
