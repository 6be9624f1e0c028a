"""Pins the CPU oracle (oracle/) before it is trusted as the checker.

The reference ships no golden vectors and its MLX/Metal kernels cannot run on
Linux, so each oracle function is checked against something other than itself:
exact rational known answers (tests/golden/kats.json), torch's own float64
CPU attention, brute force on tiny inputs, and cases chosen so that a
plausible mistake fails (a transposed operand, a dropped bias, a wrong head
mapping, a reordered K sum, a wrong causal alignment). The "planted mistake"
tests at the end run those checks against deliberately broken copies of the
oracle and require them to fail.
"""

import json
import math
import os

import numpy as np
import pytest
import torch

from oracle import bits as obits
from oracle import gemm as ogemm
from oracle import sdpa as osdpa

KATS = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "kats.json")))


# ------------------------------------------------------------------ bit tools

def test_comparator_self_test():
    """A 1-ULP perturbation reads as exactly 1 ULP; +0 and -0 are 0 ULP apart;
    -1 ULP and +1 ULP around zero are 2 apart (reference probe/probe.py:390-408)."""
    for dt, n in ((torch.float32, 32), (torch.float16, 16), (torch.bfloat16, 16)):
        a = obits.bits(torch.tensor([1.0, -3.5], dtype=dt))
        b = a + 1
        u = obits.ulp_distance(a, b, n)
        assert (u == 1).all()
        z = obits.bits(torch.tensor([0.0, -0.0], dtype=dt))
        assert obits.ulp_distance(z[:1], z[1:], n)[0] == 0
        tiny = torch.tensor([1e-40 if dt == torch.float32 else 1e-7], dtype=dt)
        pm = obits.bits(torch.cat([tiny, -tiny]))
        assert obits.ulp_distance(pm[:1], pm[1:], n)[0] == 2 * int(pm[0])


def test_rne_rounding_matches_torch():
    """round_f32_to agrees bitwise with torch's (round-to-nearest-even)
    conversions, including ties, subnormals, overflow and NaN."""
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 10,
                        np.array([0.0, -0.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 65520.0, 3.4e38,
                                  1e-40, -1e-42, np.inf, -np.inf], dtype=np.float32)])
    # exact ties for bf16: low 16 bits == 0x8000
    ties = (rng.integers(0, 2 ** 31, 2000, dtype=np.uint32) & 0xFFFF0000) | 0x8000
    x = np.concatenate([x, ties.astype(np.uint32).view(np.float32)])
    x = x[np.isfinite(x) | np.isinf(x)]
    for name, dt in (("bfloat16", torch.bfloat16), ("float16", torch.float16)):
        want = torch.from_numpy(x).to(dt).to(torch.float64).numpy()
        got = obits.round_f32_to(x, name)
        same = (got == want) | (np.isnan(got) & np.isnan(want))
        assert same.all(), (name, x[~same][:5], got[~same][:5], want[~same][:5])
    nan = obits.round_f32_to(np.array([np.nan], dtype=np.float32), "bfloat16")
    assert np.isnan(nan).all()


def test_ulp_of_known_values():
    assert obits.ulp_of(1.0, "bfloat16") == 2 ** -7
    assert obits.ulp_of(1.0, "float16") == 2 ** -10
    assert obits.ulp_of(1.0, "float32") == 2 ** -23
    assert obits.ulp_of(1.9, "bfloat16") == 2 ** -7
    assert obits.ulp_of(2.0, "bfloat16") == 2 ** -6
    assert obits.ulp_of(-6.0, "float16") == 2 ** -8
    assert obits.ulp_of(1e-30, "float16") == 2 ** -24  # subnormal spacing
    assert obits.ulp_of(0.0, "float32") == 2 ** -149


# ----------------------------------------------------------------------- GEMM

def _kat_gemm(case):
    a = np.array(case["a"], dtype=np.float32)
    b = np.array(case["b"], dtype=np.float32)
    c = None if case["bias"] is None else np.array(case["bias"], dtype=np.float32)
    return a, b, c


@pytest.mark.parametrize("i", range(len(KATS["gemm"])))
def test_gemm_oracles_match_known_answers(i):
    case = KATS["gemm"][i]
    a, b, c = _kat_gemm(case)
    want = np.array(case["out"])
    f64 = ogemm.gemm_f64(a, b, c, case["alpha"], case["beta"], trans_b=case["trans_b"])
    assert (f64 == want).all()
    for name in ("float32", "float16", "bfloat16"):
        f32 = ogemm.gemm_fixed32(a, b, c, case["alpha"], case["beta"], trans_b=case["trans_b"],
                                 out_dtype=name)
        assert (f32 == want).all(), name


def test_gemm_f64_against_brute_force():
    rng = np.random.default_rng(1)
    a = rng.standard_normal((3, 5))
    b = rng.standard_normal((5, 4))
    c = rng.standard_normal(4)
    want = [[2.5 * sum(a[m, k] * b[k, n] for k in range(5)) - 0.5 * c[n] for n in range(4)]
            for m in range(3)]
    assert np.allclose(ogemm.gemm_f64(a, b, c, 2.5, -0.5), want, rtol=1e-14, atol=0)
    assert np.allclose(ogemm.gemm_f64(a, b.T, c, 2.5, -0.5, trans_b=True), want, rtol=1e-14,
                       atol=0)


def test_abs_products_against_brute_force():
    """The cancellation floor's scale is sum_k |a[m, k] * b[k, n]| -- not
    |sum_k a b| (which cancellation drives to 0) -- in both layouts."""
    rng = np.random.default_rng(3)
    a = rng.standard_normal((3, 6))
    b = rng.standard_normal((6, 5))
    want = [[sum(abs(a[m, k] * b[k, n]) for k in range(6)) for n in range(5)] for m in range(3)]
    assert np.allclose(ogemm.abs_products(a, b), want, rtol=1e-14, atol=0)
    assert np.allclose(ogemm.abs_products(a, b.T, trans_b=True), want, rtol=1e-14, atol=0)
    # A cancelling row: the floor stays at the size of the terms.
    assert ogemm.abs_products(np.array([[1.0, -1.0]]), np.array([[3.0], [3.0]]))[0, 0] == 6.0


def test_gemm_fixed32_is_sequential_k_ascending():
    """In fp32, 1 - 1e8 rounds to -1e8. Terms (1e8, -1e8, 1) summed in
    ascending k give (1e8 - 1e8) + 1 = 1; summed from the other end they give
    (1 - 1e8) + 1e8 = 0. Both arrangements pin the direction."""
    b = np.ones((3, 1), dtype=np.float32)
    assert ogemm.gemm_fixed32(np.array([[1e8, -1e8, 1.0]], dtype=np.float32), b)[0, 0] == 1.0
    assert ogemm.gemm_fixed32(np.array([[1.0, -1e8, 1e8]], dtype=np.float32), b)[0, 0] == 0.0


def test_gemm_fixed32_epilogue_is_one_fma():
    """out = fma(alpha, acc, beta * bias) in fp32: with acc = 1 + 2^-23 and
    alpha = 1 - 2^-24, the fused product-sum differs from rounding alpha*acc
    first (the separately rounded product is exactly 1)."""
    acc = np.float32(1 + 2 ** -23)
    alpha = float(np.float32(1 - 2 ** -24))
    a = np.array([[acc]], dtype=np.float32)
    b = np.ones((1, 1), dtype=np.float32)
    bias = np.array([-1.0], dtype=np.float32)
    got = ogemm.gemm_fixed32(a, b, bias, alpha, 1.0)[0, 0]
    exact = float(alpha) * float(acc) - 1.0          # fma: one rounding of the exact value
    assert got == float(np.float32(exact))
    assert got != float(np.float32(np.float32(alpha * np.float64(acc)) - 1))


def test_gemm_fixed32_within_fp32_bound_of_f64():
    rng = np.random.default_rng(2)
    for M, K, N in ((7, 1000, 33), (2, 4096, 64)):
        a = rng.standard_normal((M, K)).astype(np.float32)
        b = (rng.standard_normal((K, N)) / math.sqrt(K)).astype(np.float32)
        exact = ogemm.gemm_f64(a, b)
        bound = K * 2.0 ** -24 * ogemm.abs_products(a, b) * 1.01
        assert (np.abs(ogemm.gemm_fixed32(a, b) - exact) <= bound).all()
        assert (ogemm.gemm_fixed32(a, b) == ogemm.gemm_fixed32(a, b.T.copy(), trans_b=True)).all()


# ----------------------------------------------------------------------- SDPA

def _kat_sdpa(case):
    q = np.array(case["q"], dtype=np.float32)
    k = np.array(case["k"], dtype=np.float32)
    v = np.array(case["v"], dtype=np.float32)
    mask = None
    if case["mask"] is not None:
        m = np.array(case["mask"], dtype=bool)
        mask = np.where(m, 0.0, -np.inf).astype(np.float32)
    off = case["N"] - case["qL"] if case["causal"] else None
    return q, k, v, mask, off


@pytest.mark.parametrize("i", range(len(KATS["sdpa"])))
def test_sdpa_oracles_match_known_answers(i):
    case = KATS["sdpa"][i]
    q, k, v, mask, off = _kat_sdpa(case)
    want = np.array(case["out"])
    assert np.allclose(osdpa.sdpa_f64(q, k, v, mask=mask, causal_offset=off), want,
                       rtol=0, atol=1e-12), case["name"]
    for name in ("float32", "bfloat16"):
        got = osdpa.sdpa_fixed32(q, k, v, mask=mask, causal_offset=off, out_dtype=name)
        expect = obits.round_f32_to(want.astype(np.float32), name)
        assert (got == expect).all(), (case["name"], name)


def _torch_sdpa64(q, k, v, mask=None, causal_offset=None, scale=None):
    """torch's float64 CPU attention as an independent implementation."""
    tq, tk, tv = (torch.from_numpy(np.asarray(x, dtype=np.float64)) for x in (q, k, v))
    g = tq.shape[1] // tk.shape[1]
    tk, tv = tk.repeat_interleave(g, dim=1), tv.repeat_interleave(g, dim=1)
    qL, N = tq.shape[2], tk.shape[2]
    bias = torch.zeros(1, 1, qL, N, dtype=torch.float64)
    if causal_offset is not None:
        keep = torch.arange(N)[None, :] <= (torch.arange(qL)[:, None] + causal_offset)
        bias = bias.masked_fill(~keep, float("-inf"))
    if mask is not None:
        bias = bias + torch.from_numpy(np.asarray(mask, dtype=np.float64))
    return torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, attn_mask=bias,
                                                            scale=scale).numpy()


def test_sdpa_f64_matches_torch_float64():
    rng = np.random.default_rng(3)
    for B, H, Hkv, qL, N, D, causal, with_mask in ((2, 8, 2, 5, 37, 64, False, False),
                                                    (1, 4, 4, 6, 20, 32, True, False),
                                                    (1, 6, 3, 3, 50, 64, False, True)):
        q = rng.standard_normal((B, H, qL, D))
        k = rng.standard_normal((B, Hkv, N, D))
        v = rng.standard_normal((B, Hkv, N, D))
        mask = rng.standard_normal((1, 1, qL, N)) if with_mask else None
        off = N - qL if causal else None
        got = osdpa.sdpa_f64(q, k, v, mask=mask, causal_offset=off)
        want = _torch_sdpa64(q, k, v, mask=mask, causal_offset=off)
        assert np.allclose(got, want, rtol=1e-12, atol=1e-13)


def test_sdpa_sink_closed_form():
    """One key with score s and a sink logit z: out = v * e^s / (e^s + e^z)."""
    q = np.ones((1, 1, 1, 32))
    k = np.full((1, 1, 1, 32), 0.25)
    v = np.full((1, 1, 1, 32), 3.0)
    s = 32 * 0.25 / math.sqrt(32)
    z = 1.5
    want = 3.0 * math.exp(s) / (math.exp(s) + math.exp(z))
    assert abs(osdpa.sdpa_f64(q, k, v, sinks=[z])[0, 0, 0, 0] - want) < 1e-14
    got = osdpa.sdpa_fixed32(q, k, v, sinks=np.array([z], dtype=np.float32))[0, 0, 0, 0]
    assert abs(got - want) < 1e-6


def test_sdpa_fixed32_close_to_f64():
    rng = np.random.default_rng(4)
    for B, H, Hkv, qL, N, D, causal in ((1, 8, 2, 4, 300, 128, False), (2, 4, 4, 7, 70, 64, True)):
        q = rng.standard_normal((B, H, qL, D)).astype(np.float32)
        k = rng.standard_normal((B, Hkv, N, D)).astype(np.float32)
        v = rng.standard_normal((B, Hkv, N, D)).astype(np.float32)
        off = N - qL if causal else None
        want = osdpa.sdpa_f64(q, k, v, causal_offset=off)
        got = osdpa.sdpa_fixed32(q, k, v, causal_offset=off)
        assert np.abs(got - want).max() / np.abs(want).max() < 2e-6


def test_sdpa_masked_keys_do_not_change_bits():
    """Appending masked keys leaves the fixed-order restatement's bits unchanged
    (key i stays in partial i mod 32; masked keys are skipped)."""
    rng = np.random.default_rng(5)
    q = rng.standard_normal((1, 4, 2, 64)).astype(np.float32)
    k = rng.standard_normal((1, 2, 150, 64)).astype(np.float32)
    v = rng.standard_normal((1, 2, 150, 64)).astype(np.float32)
    base = osdpa.sdpa_fixed32(q, k[:, :, :100], v[:, :, :100])
    mask = np.where(np.arange(150) < 100, 0.0, -np.inf).astype(np.float32).reshape(1, 1, 1, 150)
    grown = osdpa.sdpa_fixed32(q, k, v, mask=mask)
    assert (base == grown).all()


# ------------------------------------------------------------- planted mistakes

def _gemm_checks_pass(gemm_fn):
    """The GEMM known-answer checks, parameterised by the function under test."""
    for case in KATS["gemm"]:
        a, b, c = _kat_gemm(case)
        try:
            got = gemm_fn(a, b, c, case["alpha"], case["beta"], trans_b=case["trans_b"])
        except ValueError:
            return False
        if got.shape != np.array(case["out"]).shape or not (got == np.array(case["out"])).all():
            return False
    return True


def _sdpa_checks_pass(sdpa_fn):
    rng = np.random.default_rng(6)
    q = rng.standard_normal((1, 8, 3, 32))
    k = rng.standard_normal((1, 2, 9, 32))
    v = rng.standard_normal((1, 2, 9, 32))
    for off in (None, 9 - 3):
        if not np.allclose(sdpa_fn(q, k, v, causal_offset=off), _torch_sdpa64(q, k, v, causal_offset=off),
                           rtol=1e-10, atol=1e-12):
            return False
    return True


def test_planted_gemm_mistakes_are_caught():
    assert _gemm_checks_pass(ogemm.gemm_f64)

    def transposed_b(a, b, c, al, be, trans_b):
        # the same memory indexed with the other layout's formula
        return ogemm.gemm_f64(a, b.reshape(b.shape[::-1]), c, al, be, trans_b=not trans_b)

    def dropped_bias(a, b, c, al, be, trans_b):
        return ogemm.gemm_f64(a, b, None, al, be, trans_b=trans_b)

    def swapped_coef(a, b, c, al, be, trans_b):
        return ogemm.gemm_f64(a, b, c, be, al, trans_b=trans_b)

    for bad in (transposed_b, dropped_bias, swapped_coef):
        assert not _gemm_checks_pass(bad), bad.__name__


def test_planted_sdpa_mistakes_are_caught():
    assert _sdpa_checks_pass(osdpa.sdpa_f64)

    def wrong_gqa(q, k, v, causal_offset=None):
        # head h reads kv head h % Hkv instead of h // (H / Hkv)
        H, Hkv = q.shape[1], k.shape[1]
        idx = [h % Hkv for h in range(H)]
        kk = np.stack([k[:, i] for i in idx], 1)
        vv = np.stack([v[:, i] for i in idx], 1)
        return osdpa.sdpa_f64(q, kk, vv, causal_offset=causal_offset)

    def top_left_causal(q, k, v, causal_offset=None):
        return osdpa.sdpa_f64(q, k, v, causal_offset=None if causal_offset is None else 0)

    def unscaled(q, k, v, causal_offset=None):
        return osdpa.sdpa_f64(q, k, v, scale=1.0, causal_offset=causal_offset)

    for bad in (wrong_gqa, top_left_causal, unscaled):
        assert not _sdpa_checks_pass(bad), bad.__name__


# ---------------------------------------------------------------- quantized weights

def _big_endian_unpack(words, bits, K):
    """A planted mistake: codes taken from the high end of each word."""
    per = 32 // bits
    w = np.asarray(words).astype(np.int64) & 0xFFFFFFFF
    q = np.empty((w.shape[0], K), dtype=np.int64)
    for k in range(K):
        q[:, k] = (w[:, k // per] >> (bits * (per - 1 - k % per))) & ((1 << bits) - 1)
    return q


QUANT_KATS = [
    # (bits, words of one row, codes of that row): worked by hand
    (4, [0x76543210, 0xFEDCBA98], list(range(16))),
    (8, [0x04030201, 0x000000FF], [1, 2, 3, 4, 255, 0, 0, 0]),
    (2, [0x1BE4], [0, 1, 2, 3, 3, 2, 1, 0] + [0] * 8),
]


@pytest.mark.parametrize("i", range(len(QUANT_KATS)))
def test_quant_unpack_known_words(i):
    from oracle import quant as oquant

    bits, words, codes = QUANT_KATS[i]
    got = oquant.unpack(np.array([words], dtype=np.int64), bits, len(codes))
    assert got.tolist() == [codes]
    # the planted big-endian reading disagrees with the hand-worked codes
    assert _big_endian_unpack(np.array([words]), bits, len(codes)).tolist() != [codes]


def test_quant_dequantize_closed_form_and_rounding():
    from oracle import quant as oquant

    # scale 0.5, bias -1: every value -1 + q/2 is exact
    words = np.array([[0x76543210, 0xFEDCBA98]], dtype=np.int64)
    got = oquant.dequantize(words, [[0.5]], [[-1.0]], 16, 4)
    assert got.tolist() == [[-1.0 + q / 2 for q in range(16)]]
    # 1 + 3 * 2**-9 is an fp32 value and not a bfloat16: the reference keeps it
    # in fp32; dequantize_to rounds it once to the element type
    words = np.array([[0x3]], dtype=np.int64)
    s, b = 2.0 ** -9, 1.0
    assert oquant.dequantize(words, [[s]], [[b]], 16, 2)[0, 0] == 1 + 3 * s
    got = oquant.dequantize_to(words, [[s]], [[b]], 16, 2, "bfloat16")[0, 0]
    want = float(torch.tensor(1 + 3 * s, dtype=torch.float32).to(torch.bfloat16).float())
    assert got == want and got != 1 + 3 * s
    # fp32 rounding of v: bias 2^10 and scale 2^-20 need more than 24 bits
    words = np.array([[0x1]], dtype=np.int64)
    v = oquant.dequantize(words, [[2.0 ** -20]], [[1024.0]], 16, 2)[0, 0]
    assert v == 1024.0  # 1024 + 2^-20 rounds to 1024 in fp32


@pytest.mark.parametrize("dname", ["bfloat16", "float16"])
def test_quant_closed_form_discriminates_weight_rounding(dname):
    """The closed-form quantized inputs the GPU tests use: the oracle's exact
    product equals x @ v.T for the fp32 weights, and a planted mistake --
    weights rounded to the element type before the product -- changes many
    outputs, so a kernel that rounds them cannot pass the bitwise test."""
    from oracle import quant as oquant

    from helpers import closed_form_quant

    dt = {"bfloat16": torch.bfloat16, "float16": torch.float16}[dname]
    for bits in (2, 4, 8):
        x, w, s, b, exact = closed_form_quant(8, 64, 256, 32, bits, dt, 3 + bits)
        xs, ss, bs = (t.float().numpy().astype(np.float64) for t in (x, s, b))
        got = oquant.qgemm_f64(xs, w.numpy(), ss, bs, 32, bits)
        assert (got == exact).all()
        want = obits.round_f32_to(exact.astype(np.float32), dname)
        assert (obits.round_f32_to(got.astype(np.float32), dname) == want).all()
        vt = oquant.dequantize_to(w.numpy(), ss, bs, 32, bits, dname)
        planted = obits.round_f32_to((xs @ vt.T).astype(np.float32), dname)
        assert (planted != want).mean() > 0.2, bits
