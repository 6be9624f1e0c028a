"""GPU parity tests of the attention launch shapes and head dims.

bi_sdpa picks a launch shape from the grid (include/bi_testing.h): for
bf16/f16 the prefill "rows" shape (several 16-column tiles per workgroup), the
prefill "shared" shape (one column tile per wave, every key block loaded once
for all waves), one tile, or one tile with the output dims split over 2/4/8
workgroups; for fp32 how many query heads share a workgroup's loads. The reference has a single
launch shape (_attention.py:241-250) and rejects any route switch on query
length (reference ROADMAP.md:91-94), so every shape must give the same bits:

  * every shape, forced through bi_sdpa_with_shape, gives identical bits on the
    same input, for every built (D, V) pair, element type and mask mode;
  * the prefill rows and shared shapes, selected by bi_sdpa itself at the
    shapes they are built for, give each row the bits of that row computed
    alone at query length 1 over its visible keys (a one-tile shape), are
    accurate against the float64 oracle (reference
    tests/test_invariance.py:408-432), and give each other's bits;
  * keys no query row can see (an unwritten cache tail) never reach the
    output, whatever they hold (reference _attention.py:92-98).
"""

import ctypes
import math

import numpy as np
import pytest
import torch

from mlx_batch_invariant import _attention, _lib
from oracle import sdpa as osdpa

from helpers import bits, f64, rn

pytestmark = pytest.mark.gpu

LOW = [("float16", torch.float16), ("bfloat16", torch.bfloat16)]
TOL = {"float32": 2e-6, "float16": 5e-3, "bfloat16": 3e-2}
PAIRS = list(_attention.HEAD_DIMS)


def _mask_mode(spec, q, k):
    """(mode, mask, strides, causal_offset) for a mask spec: None, "end"
    (bi mask="causal": row s sees keys i <= N - qL + s), "start" (torch
    is_causal: i <= s) or an additive / boolean tensor."""
    B, H, qL, _ = q.shape
    N = k.shape[2]
    if spec is None:
        return _lib.MASK_NONE, None, (0, 0, 0), 0
    if isinstance(spec, str):
        return _lib.MASK_CAUSAL, None, (0, 0, 0), (N - qL if spec == "end" else 0)
    m, ms, mode = _attention._mask_args(spec, B, H, qL, N, q.dtype)
    return mode, m, ms, 0


def run(q, k, v, spec=None, shape=None, sinks=None):
    mode, m, ms, off = _mask_mode(spec, q, k)
    return _attention._sdpa_eager(q, k, v, 1.0 / math.sqrt(q.shape[-1]), mode, m, ms, off, sinks,
                                  shape)


def shapes_for(dtype, D, V, G):
    """Launch shapes built for the head dims (fp32: those dividing G heads)."""
    L = _lib.lib()
    code = _lib.DTYPE_CODES[dtype]
    out = []
    for s in range(_lib.SDPA_NUM_SHAPES):
        c, w = ctypes.c_int(), ctypes.c_int()
        if L.bi_sdpa_shape_info(D, V, code, s, c, w) != _lib.OK:
            continue
        if dtype == torch.float32 and G % c.value:
            continue
        out.append(s)
    return out


def _masks(B, qL, N, dtype, device, seed):
    g = torch.Generator().manual_seed(seed)
    add = (torch.randn(B, 1, qL, N, generator=g)).to(dtype)
    add[torch.rand(B, 1, qL, N, generator=g) < 0.1] = -float("inf")
    keep = torch.rand(1, 1, qL, N, generator=g) > 0.2
    keep[..., N - max(1, N // 10):] = False  # a padding tail
    return add.to(device), keep.to(device)


@pytest.mark.parametrize("D,V", PAIRS)
def test_every_shape_gives_the_same_bits(cuda, D, V):
    """One input through every launch shape, for each element type and mask
    mode: the bits must not move (the attention analogue of the GEMM's
    test_all_geometries_agree)."""
    B, H, Hkv, qL, N = 2, 16, 2, 40, 300
    for dname, dtype in LOW + [("float32", torch.float32)]:
        q = rn((B, H, qL, D), dtype, 101, device=cuda)
        k = rn((B, Hkv, N, D), dtype, 102, device=cuda)
        v = rn((B, Hkv, N, V), dtype, 103, device=cuda)
        sinks = rn((H,), dtype, 104, device=cuda)
        add, keep = _masks(B, qL, N, dtype, cuda, 105)
        shapes = shapes_for(dtype, D, V, H // Hkv)
        assert len(shapes) >= (2 if dtype == torch.float32 else 3), shapes
        for label, spec, sk in (("none", None, None), ("end", "end", None),
                                ("start", "start", None), ("additive", add, None),
                                ("bool", keep, None), ("sinks", None, sinks)):
            ref = None
            for s in shapes:
                if s == _lib.SDPA_SHARED and label in ("additive", "bool"):
                    # Built without array masks: bi_sdpa never picks it for one.
                    continue
                y = run(q, k, v, spec, shape=s, sinks=sk)
                got = bits(y)
                if ref is None:
                    ref = got
                    assert torch.isfinite(y).all() and bool((y != 0).any())
                else:
                    d = int((got != ref).sum())
                    assert d == 0, "%s D=%d V=%d %s shape %d: %d differ" % (
                        dname, D, V, label, s, d)


def test_short_contexts_through_the_loader_wave_shapes(cuda):
    """Decode at D = V = 128 without an array mask takes the dim-split shapes
    with loader waves, whose chains can hold no block at all (N < 97) or
    different block counts. Contexts of 1 to 129 keys, causal and not, with
    and without sinks: the picked shape gives the bits of the rows and
    one-tile shapes, and a single key returns its value row exactly."""
    H, Hkv, D = 32, 8, 128
    for dname, dtype in LOW:
        for B in (1, 8):
            for N in (1, 5, 32, 33, 97, 100, 129):
                q = rn((B, H, 1, D), dtype, 301 + N, device=cuda)
                k = rn((B, Hkv, N, D), dtype, 302 + N, device=cuda)
                v = rn((B, Hkv, N, D), dtype, 303 + N, device=cuda)
                sinks = rn((H,), dtype, 304, device=cuda)
                shape = _attention.launch_shape(q, k, v)
                assert shape in (_lib.SDPA_SPLIT2, _lib.SDPA_SPLIT4, _lib.SDPA_SPLIT8), (B, N, shape)
                for spec, sk in ((None, None), ("end", None), (None, sinks)):
                    y = run(q, k, v, spec, sinks=sk)
                    case = "%s B=%d N=%d %s sinks=%s shape %d" % (dname, B, N, spec, sk is not None, shape)
                    for forced in (_lib.SDPA_TILE, _lib.SDPA_ROWS):
                        d = int((bits(run(q, k, v, spec, shape=forced, sinks=sk)) != bits(y)).sum())
                        assert d == 0, "%s: forced %d: %d differ" % (case, forced, d)
                    if N == 1 and sk is None:
                        want = v.repeat_interleave(H // Hkv, dim=1)
                        assert np.array_equal(bits(y), bits(want.contiguous())), case


def test_long_contexts_through_the_loader_wave_shapes(cuda):
    """The dim-split shapes with loader waves run their chains as a pipeline
    (a step scores block j while it finishes block j - 1, four slots per wave
    at dim split 4 and 8; one block per step at dim split 2). Over 8192 keys
    (65 steps per chain) and 4099 keys (chains of unequal length, a ragged
    last block), each of them forced gives the one-tile shape's bits,
    without a mask, end-aligned causal and with sinks."""
    H, Hkv, D = 32, 8, 128
    for dname, dtype in LOW:
        for N in (8192, 4099):
            q = rn((2, H, 1, D), dtype, 401 + N, device=cuda)
            k = rn((2, Hkv, N, D), dtype, 402 + N, device=cuda)
            v = rn((2, Hkv, N, D), dtype, 403 + N, device=cuda)
            sinks = rn((H,), dtype, 404, device=cuda)
            for spec, sk in ((None, None), ("end", None), (None, sinks)):
                ref = bits(run(q, k, v, spec, shape=_lib.SDPA_TILE, sinks=sk))
                for forced in (_lib.SDPA_SPLIT2, _lib.SDPA_SPLIT4, _lib.SDPA_SPLIT8):
                    d = int((bits(run(q, k, v, spec, shape=forced, sinks=sk)) != ref).sum())
                    assert d == 0, "%s N=%d %s sinks=%s shape %d: %d differ" % (
                        dname, N, spec, sk is not None, forced, d)


def _oracle_rows(q, k, v, spec, rows, b, dname):
    """float64 and reference-order fp32 results for query rows `rows` of batch
    entry b (every head), each row as a one-row problem."""
    B, H, qL, D = q.shape
    N = k.shape[2]
    qh, kh, vh = f64(q[b:b + 1]), f64(k[b:b + 1]), f64(v[b:b + 1])
    want, fixed = [], []
    for s in rows:
        qs = qh[:, :, s:s + 1]
        mask, off = None, None
        if isinstance(spec, str):
            off = s + (N - qL if spec == "end" else 0)
        elif spec is not None:
            m = spec
            if m.dtype == torch.bool:
                m = torch.where(m, 0.0, -float("inf"))
            m = f64(m)
            mask = m[(0 if m.shape[0] == 1 else b):][:1, :, (s if m.shape[2] > 1 else 0):][:, :, :1]
        want.append(osdpa.sdpa_f64(qs, kh, vh, mask=mask, causal_offset=off))
        fixed.append(osdpa.sdpa_fixed32(qs, kh, vh, mask=mask, causal_offset=off,
                                        out_dtype=dname))
    return np.concatenate(want, axis=2), np.concatenate(fixed, axis=2)


def _alone(q, k, v, spec, b, s):
    """Row s of batch entry b computed alone at query length 1 over the keys it
    can see: causal rows as an unmasked call over their visible prefix, masked
    rows with their own mask row."""
    qL, N = q.shape[2], k.shape[2]
    qs = q[b:b + 1, :, s:s + 1].contiguous()
    if isinstance(spec, str):
        nvis = min(N, s + (N - qL if spec == "end" else 0) + 1)
        return run(qs, k[b:b + 1, :, :nvis], v[b:b + 1, :, :nvis])
    m = spec[(0 if spec.shape[0] == 1 else b):][:1, :, (s if spec.shape[2] > 1 else 0):][:, :, :1]
    return run(qs, k[b:b + 1], v[b:b + 1], m)


ROWS_CASES = [(4, 64), (1, 513), (2, 513), (1, 2048), (2, 2048)]


@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("dname,dtype", LOW)
def test_prefill_rows_shape_is_invariant_and_accurate(cuda, dname, dtype, D):
    """The prefill shapes at 32/8 heads: bi_sdpa selects "rows" or (D = 128
    without an array mask, on the larger grids) "shared" for these problems;
    rows 0, middle and last are bitwise equal to the same row computed alone at
    query length 1 (which takes a one-tile shape), and every head of those rows
    is within the reference's float64 bound and no worse than 4x the
    reference-order fp32 restatement (tests:408-432). Where "shared" is built
    (D <= 128, no array mask), it and "rows", forced, give the whole output the
    same bits. Masks: end-aligned causal (mask="causal"), start-aligned causal
    (torch is_causal), additive per row, boolean per row."""
    H, Hkv = 32, 8
    picked = set()
    for B, qL in ROWS_CASES:
        for N in (qL, 4200):
            seed = 1000 * B + qL + N + D
            q = rn((B, H, qL, D), dtype, seed, device=cuda)
            k = rn((B, Hkv, N, D), dtype, seed + 1, device=cuda)
            v = rn((B, Hkv, N, D), dtype, seed + 2, device=cuda)
            add, keep = _masks(B, qL, N, dtype, cuda, seed + 3)
            rows = sorted({0, qL // 2, qL - 1})
            b = B - 1
            for label, spec in (("end", "end"), ("start", "start"), ("additive", add),
                                ("bool", keep)):
                mode = _mask_mode(spec, q, k)[0]
                shape = _attention.launch_shape(q, k, v, mode)
                assert shape in (_lib.SDPA_ROWS, _lib.SDPA_SHARED), (B, qL, D, label, shape)
                picked.add(shape)
                y = run(q, k, v, spec)
                case = "%s D=%d B=%d qL=%d N=%d %s shape %d" % (dname, D, B, qL, N, label, shape)
                assert torch.isfinite(y).all(), case
                if D <= 128 and mode != _lib.MASK_ARRAY:
                    for forced in (_lib.SDPA_ROWS, _lib.SDPA_SHARED):
                        yf = run(q, k, v, spec, shape=forced)
                        d = int((bits(yf) != bits(y)).sum())
                        assert d == 0, "%s: forced shape %d: %d differ" % (case, forced, d)
                for s in rows:
                    alone = _alone(q, k, v, spec, b, s)
                    assert np.array_equal(bits(alone[0, :, 0]), bits(y[b, :, s])), (case, s)
                ours = f64(y[b:b + 1, :, rows])
                want, fixed = _oracle_rows(q, k, v, spec, rows, b, dname)
                scale = max(np.abs(want).max(), 1e-30)
                err = np.abs(ours - want).max() / scale
                err_fixed = np.abs(fixed - want).max() / scale
                assert err < TOL[dname], "%s: %.3e" % (case, err)
                assert err < 4 * err_fixed + 1e-7, "%s: %.3e vs %.3e" % (case, err, err_fixed)
    # bi_sdpa's own choice covers the rows shape everywhere, and the shared
    # shape at D = 128.
    assert _lib.SDPA_ROWS in picked
    assert (_lib.SDPA_SHARED in picked) == (D == 128), picked


@pytest.mark.parametrize("dname,dtype", LOW + [("float32", torch.float32)])
def test_base_moves_in_later_blocks_for_some_columns(cuda, dname, dtype):
    """Scores that rise along the keys for some (row, head) columns and stay
    flat for others: head dim 0 carries k_i[0] = i / 2 and q[0] = a slope of
    0, 0.5, 1 or 1.5 by (row + head) mod 4, so a chain's lazily moved base
    (reference _attention.py:99-114, the online softmax) moves again in later
    blocks for some columns of a wave or workgroup (every block of a chain at
    the steeper slopes, every other block at 0.5) and never after the first
    for the flat ones. A block whose base moves for some columns takes the
    full step for the whole wave, where the others keep m and f = 1. Every
    launch shape gives the same bits, without a mask and end-aligned causal,
    and rows 0, 31 and 63 are no worse than 4x the reference-order fp32
    restatement against float64, and within the float64 bound (bf16, f16;
    fp32 within 2e-5: on these scores the restatement itself exceeds the
    random-input bound of 2e-6)."""
    B, H, Hkv, qL, N, D = 1, 8, 2, 64, 640, 128
    q = rn((B, H, qL, D), torch.float32, 121, std=0.3)
    k = rn((B, Hkv, N, D), torch.float32, 122, std=0.3)
    v = rn((B, Hkv, N, D), dtype, 123, device=cuda)
    slope = ((torch.arange(qL).view(1, 1, qL) + torch.arange(H).view(1, H, 1)) % 4) * 0.5
    q[..., 0] = slope.to(torch.float32)
    k[..., 0] = torch.arange(N, dtype=torch.float32).view(1, 1, N) / 2
    q, k = q.to(dtype).to(cuda), k.to(dtype).to(cuda)
    shapes = shapes_for(dtype, D, D, H // Hkv)
    assert len(shapes) >= (2 if dtype == torch.float32 else 5), shapes
    rows = [0, 31, 63]
    for label, spec in (("none", None), ("end", "end")):
        ref = None
        for sh in shapes:
            y = run(q, k, v, spec, shape=sh)
            case = "%s %s shape %d" % (dname, label, sh)
            assert torch.isfinite(y).all(), case
            if ref is None:
                ref = bits(y)
                ours = f64(y[0:1, :, rows])
                want, fixed = _oracle_rows(q, k, v, spec, rows, 0, dname)
                scale = max(np.abs(want).max(), 1e-30)
                err = np.abs(ours - want).max() / scale
                err_fixed = np.abs(fixed - want).max() / scale
                # fp32: scores in the hundreds, rescaled block after block,
                # take the reference-order restatement past the random-input
                # bound too; the restatement ratio is the check there.
                tol = 2e-5 if dtype == torch.float32 else TOL[dname]
                assert err < tol, "%s: %.3e (restatement %.3e)" % (case, err, err_fixed)
                assert err < 4 * err_fixed + 1e-7, "%s: %.3e vs %.3e" % (case, err, err_fixed)
            else:
                d = int((bits(y) != ref).sum())
                assert d == 0, "%s: %d differ" % (case, d)


def test_key_value_views_spanning_more_than_4_gib(cuda):
    """Key and value views whose rows are 1 MiB apart (the first 128 elements
    of each row of a wider cache), so that from a block's first row to the
    last visible row spans more than 4 GiB: the kernels' per-block buffer
    resources cap their byte count at 2^31 - 1 (a block's own rows lie within
    32 rows). Every bf16 launch shape gives, at decode and at a causal prefill
    chunk, the bits of the same call on compact copies."""
    dtype = torch.bfloat16
    B, H, Hkv, N, D, RS = 1, 8, 1, 4352, 128, 1 << 19
    assert (N - 1) * RS * 2 > 1 << 32
    kc = rn((B, Hkv, N, D), dtype, 131, device=cuda)
    vc = rn((B, Hkv, N, D), dtype, 132, device=cuda)
    kw = torch.zeros(N, RS, dtype=dtype, device=cuda)
    vw = torch.zeros(N, RS, dtype=dtype, device=cuda)
    kw[:, :D] = kc[0, 0]
    vw[:, :D] = vc[0, 0]
    kv, vv = kw[:, :D][None, None], vw[:, :D][None, None]
    assert kv.shape == (B, Hkv, N, D) and kv.stride()[2:] == (RS, 1)
    try:
        for qL, spec in ((1, None), (64, "end")):
            q = rn((B, H, qL, D), dtype, 133 + qL, device=cuda)
            for sh in [None] + shapes_for(dtype, D, D, H // Hkv):
                case = (qL, spec, sh)
                got, want = run(q, kv, vv, spec, shape=sh), run(q, kc, vc, spec, shape=sh)
                assert torch.isfinite(got).all(), case
                assert np.array_equal(bits(got), bits(want)), case
    finally:
        del kw, vw, kv, vv
        torch.cuda.empty_cache()


@pytest.mark.parametrize("dname,dtype", LOW + [("float32", torch.float32)])
def test_unwritten_cache_tail_never_reaches_the_output(cuda, dname, dtype):
    """Keys past every row's causal horizon hold NaN (an unwritten cache tail):
    the output is finite and bitwise equal to the same call with a zero tail,
    for start-aligned causal (torch is_causal over a longer cache) and for a
    cache view k[:, :, :N] whose storage continues with NaN rows (mask="causal",
    aligned to the end of the view), at decode and prefill shapes: the one
    bi_sdpa picks, and the two prefill shapes forced (bf16/f16)."""
    H, Hkv, D, NP = 32, 8, 128, 1200
    for B, qL in ((1, 1), (3, 5), (1, 300), (2, 700)):
        q = rn((B, H, qL, D), dtype, 111, device=cuda)
        k = rn((B, Hkv, NP, D), dtype, 112, device=cuda)
        v = rn((B, Hkv, NP, D), dtype, 113, device=cuda)
        shapes = [None]
        if dtype != torch.float32 and qL > 16:
            shapes += [_lib.SDPA_ROWS, _lib.SDPA_SHARED]
        for shape in shapes:
            case = (dname, B, qL, shape)
            # Start-aligned: row s sees keys 0..s; keys from qL on are never read.
            kn, vn, kz, vz = k.clone(), v.clone(), k.clone(), v.clone()
            kn[:, :, qL:] = float("nan")
            vn[:, :, qL:] = float("nan")
            kz[:, :, qL:] = 0
            vz[:, :, qL:] = 0
            got, want = run(q, kn, vn, "start", shape), run(q, kz, vz, "start", shape)
            assert torch.isfinite(got).all(), case
            assert np.array_equal(bits(got), bits(want)), case
            # End-aligned over a view of the first N rows; storage past N is NaN.
            N = NP - 77
            kn, vn, kz, vz = k.clone(), v.clone(), k.clone(), v.clone()
            kn[:, :, N:] = float("nan")
            vn[:, :, N:] = float("nan")
            kz[:, :, N:] = 0
            vz[:, :, N:] = 0
            got = run(q, kn[:, :, :N], vn[:, :, :N], "end", shape)
            want = run(q, kz[:, :, :N], vz[:, :, :N], "end", shape)
            assert torch.isfinite(got).all(), case
            assert np.array_equal(bits(got), bits(want)), case


@pytest.mark.parametrize("dname,dtype", LOW)
def test_nan_value_hidden_from_some_rows_by_the_causal_mask(cuda, dname, dtype):
    """A NaN value row at key j of a start-aligned causal prefill (qL = N):
    rows s >= j see it and are all NaN in every launch shape; a row s < j
    cannot see it, and is either bitwise its result with a finite value there
    or all NaN, by launch shape and by which rows share its workgroup and
    32-key block (its zero probability multiplies the value: 0 * NaN = NaN).
    So bit parity across shapes holds for finite values of the keys some row
    of the call can see (include/bi.h); the reference skips such a key per
    row (_attention.py:92-98)."""
    B, H, Hkv, D, L, j = 1, 8, 2, 128, 96, 40
    q = rn((B, H, L, D), dtype, 131, device=cuda)
    k = rn((B, Hkv, L, D), dtype, 132, device=cuda)
    v = rn((B, Hkv, L, D), dtype, 133, device=cuda)
    vn = v.clone()
    vn[:, :, j] = float("nan")
    leaked = {}
    for shape in shapes_for(dtype, D, D, H // Hkv):
        want = bits(run(q, k, v, "start", shape)).reshape(B, H, L, D)
        out = run(q, k, vn, "start", shape)
        got = bits(out).reshape(B, H, L, D)
        nan_rows = torch.isnan(out).all(-1).cpu().numpy()
        assert nan_rows[:, :, j:].all(), (dname, shape)
        same = (got == want).all(-1)
        assert (nan_rows | same)[:, :, :j].all(), (dname, shape)
        leaked[shape] = int(nan_rows[:, :, :j].sum())
    # Every matrix-core shape ran (how many rows before j turn NaN is the
    # shape's business; the finite ones are exact).
    assert len(leaked) >= 5, leaked


@pytest.mark.parametrize("D,V", PAIRS)
def test_head_dims_accuracy_and_query_length_invariance(cuda, D, V):
    """Every built (D, V) pair (the reference takes any multiples of 32,
    _attention.py:224-227): accurate against float64 within the reference's
    bounds, and a query row keeps its bits for query lengths 1..17."""
    H, Hkv, N = 8, 2, 777
    for dname, dtype in LOW + [("float32", torch.float32)]:
        k = rn((1, Hkv, N, D), dtype, 121, device=cuda)
        v = rn((1, Hkv, N, V), dtype, 122, device=cuda)
        qf = rn((1, H, 17, D), dtype, 123, device=cuda)
        base = None
        for qL in (1, 2, 9, 16, 17):
            q = qf[:, :, 17 - qL:].contiguous()
            y = run(q, k, v, "end")
            got = bits(y[:, :, -1])
            if base is None:
                base = got
            else:
                assert np.array_equal(got, base), (dname, D, V, qL)
        want = osdpa.sdpa_f64(f64(qf), f64(k), f64(v), causal_offset=N - 17)
        fixed = osdpa.sdpa_fixed32(f64(qf), f64(k), f64(v), causal_offset=N - 17,
                                   out_dtype=dname)
        err = np.abs(f64(y) - want).max() / np.abs(want).max()
        err_fixed = np.abs(fixed - want).max() / np.abs(want).max()
        assert err < TOL[dname], (dname, D, V, err)
        assert err < 4 * err_fixed + 1e-7, (dname, D, V, err, err_fixed)


def test_large_sinks_stay_accurate(cuda):
    """A sink far above every score (up to 12 in natural-log units, where e^-12
    is below f16's smallest normal) must not push the keys' probabilities out
    of the half-precision planes that carry them into the value products: the
    sink enters the fixed-order merge as its own partial, so f16 and bf16 stay
    within the reference's bounds and within 4x the reference-order fp32
    restatement rounded once."""
    H, Hkv, N, D = 8, 2, 500, 128
    for dname, dtype in LOW + [("float32", torch.float32)]:
        q = rn((1, H, 3, D), dtype, 131, std=0.3, device=cuda)
        k = rn((1, Hkv, N, D), dtype, 132, std=0.3, device=cuda)
        v = rn((1, Hkv, N, D), dtype, 133, device=cuda)
        for level in (4.0, 8.0, 12.0):
            sinks = torch.full((H,), level, dtype=dtype, device=cuda)
            y = run(q, k, v, None, sinks=sinks)
            want = osdpa.sdpa_f64(f64(q), f64(k), f64(v), sinks=f64(sinks))
            fixed = osdpa.sdpa_fixed32(f64(q), f64(k), f64(v), sinks=f64(sinks),
                                       out_dtype=dname)
            err = np.abs(f64(y) - want).max() / np.abs(want).max()
            err_fixed = np.abs(fixed - want).max() / np.abs(want).max()
            assert err < TOL[dname], (dname, level, err)
            assert err < 4 * err_fixed + 1e-7, (dname, level, err, err_fixed)


def test_fp32_head_grouping_prefill(cuda):
    """fp32 groups two query heads per workgroup for prefill (more than 16 query
    rows) and four for decode; with causal and additive masks each row keeps
    the bits of the same row computed alone at query length 1."""
    H, Hkv, qL, N, D = 32, 8, 64, 900, 128
    dtype = torch.float32
    q = rn((1, H, qL, D), dtype, 141, device=cuda)
    k = rn((1, Hkv, N, D), dtype, 142, device=cuda)
    v = rn((1, Hkv, N, D), dtype, 143, device=cuda)
    add, keep = _masks(1, qL, N, dtype, cuda, 144)
    assert _attention.launch_shape(q, k, v) == 1  # two heads per workgroup
    for spec in ("end", "start", add, keep):
        y = run(q, k, v, spec)
        for s in (0, 17, qL - 1):
            alone = _alone(q, k, v, spec, 0, s)
            assert np.array_equal(bits(alone[0, :, 0]), bits(y[0, :, s])), s
