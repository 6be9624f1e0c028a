"""GPU kernels against the exact known-answer vectors (tests/golden/kats.json),
every element type, both weight layouts, every GEMM geometry."""

import json
import os

import numpy as np
import pytest
import torch

import mlx_batch_invariant as bi
from mlx_batch_invariant import _gemm
from oracle import bits as obits

from helpers import DTYPES, f64

pytestmark = pytest.mark.gpu

KATS = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "kats.json")))


@pytest.mark.parametrize("i", range(len(KATS["gemm"])))
def test_gemm_kats(cuda, i):
    case = KATS["gemm"][i]
    want = np.array(case["out"])
    for dname, dtype in DTYPES:
        a = torch.tensor(case["a"], dtype=dtype, device=cuda)
        b = torch.tensor(case["b"], dtype=dtype, device=cuda)
        c = None if case["bias"] is None else torch.tensor(case["bias"], dtype=dtype, device=cuda)
        for g in range(len(_gemm.geometries())):
            try:
                y = _gemm._gemm(a, b, c, case["trans_b"], case["alpha"], case["beta"], geometry=g)
            except NotImplementedError:
                continue  # geometry built for 16-bit, aligned operands only
            assert (f64(y) == want).all(), (dname, g)


@pytest.mark.parametrize("i", range(len(KATS["sdpa"])))
def test_sdpa_kats(cuda, i):
    case = KATS["sdpa"][i]
    want = np.array(case["out"], dtype=np.float32)
    for dname, dtype in DTYPES:
        q = torch.tensor(case["q"], dtype=dtype, device=cuda)
        k = torch.tensor(case["k"], dtype=dtype, device=cuda)
        v = torch.tensor(case["v"], dtype=dtype, device=cuda)
        mask = None
        if case["mask"] is not None:
            mask = torch.tensor(case["mask"], dtype=torch.bool, device=cuda)
        if case["causal"]:
            mask = "causal"
        got = f64(bi.scaled_dot_product_attention(q, k, v, mask=mask))
        assert (got == obits.round_f32_to(want, dname)).all(), (case["name"], dname)
