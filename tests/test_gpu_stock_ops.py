"""Stock torch-ROCm ops a decoder uses around the invariant GEMM and attention
must themselves give a row the same bits in any batch (reference
tests/test_invariance.py:183-212, which guards the same property of stock
MLX). batch_invariant_mode does not wrap these; if a torch upgrade changes
their reduction strategy with the row count, this is where it shows.

Not every stock reduction qualifies: a generic fp32 ``x.sum(-1)`` /
``x.mean(-1)`` changes its reduction split with the number of rows on this
stack, so a hand-written RMSNorm built on ``pow(2).mean(-1)`` in fp32 is
batch-variant; ``F.rms_norm`` / ``nn.RMSNorm`` is not.
"""

import pytest
import torch
import torch.nn.functional as F

from helpers import DTYPES, batch_with, bits, rn

pytestmark = pytest.mark.gpu

BATCHES = (1, 2, 3, 8, 16, 64, 128)


def _assert_invariant(label, fn, ref, pool):
    base = None
    for B in BATCHES:
        idx = B // 2
        got = bits(fn(batch_with(ref, pool, B, idx))[idx])
        if base is None:
            base = got
        else:
            assert int((got != base).sum()) == 0, "%s B=%d" % (label, B)


@pytest.mark.parametrize("D", [1024, 4096, 8192])
def test_norms_and_softmax(cuda, D):
    for dname, dtype in DTYPES:
        w, b = rn((D,), dtype, 1, device=cuda), rn((D,), dtype, 4, device=cuda)
        ref, pool = rn((1, D), dtype, 3, device=cuda), rn((128, D), dtype, 2, device=cuda)
        for label, fn in (
            ("rms_norm", lambda x: F.rms_norm(x, (D,), w, 1e-5)),
            ("layer_norm", lambda x: F.layer_norm(x, (D,), w, b, 1e-5)),
            ("softmax", lambda x: torch.softmax(x, dim=-1)),
            ("silu_mul", lambda x: F.silu(x) * x),
            ("residual", lambda x: x + w),
        ):
            _assert_invariant("%s %s D=%d" % (label, dname, D), fn, ref, pool)


def test_embedding_rows(cuda):
    for dname, dtype in DTYPES:
        table = rn((1000, 512), dtype, 5, device=cuda)
        g = torch.Generator().manual_seed(6)
        ref = torch.randint(0, 1000, (1, 64), generator=g).to(cuda)
        pool = torch.randint(0, 1000, (128, 64), generator=g).to(cuda)
        _assert_invariant("embedding %s" % dname, lambda ids: F.embedding(ids, table), ref, pool)
