"""Host-side logic, no GPU needed: the C ABI library loads and exports what
include/*.h declares, rejects bad arguments before any HIP call, and the
Python layer keeps the reference's validation, error types and routing-shim
contract (reference tests/test_invariance.py:643-708, __init__.py:41-147,
_gemm.py:185-208, _attention.py:173-239).
"""

import ctypes
import os
import re
import subprocess
import sys

import pytest
import torch
import torch.nn.functional as F

import mlx_batch_invariant as bi
from mlx_batch_invariant import _attention, _lib

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_functions():
    names = set()
    for hdr in ("bi.h", "bi_testing.h"):
        text = open(os.path.join(REPO, "include", hdr)).read()
        names |= set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(bi_\w+)\s*\(", text, re.M))
    return names


def test_library_exports_every_declared_symbol():
    names = _declared_functions()
    assert {"bi_gemm", "bi_sdpa", "bi_abi_version", "bi_last_error"} <= names
    lib = ctypes.CDLL(_lib.LIB_PATH)
    for n in sorted(names):
        assert hasattr(lib, n), n
    assert set(_lib.SIGNATURES) == names


def test_abi_version_and_geometry_table():
    L = _lib.lib()
    assert L.bi_abi_version() == _lib.ABI_VERSION == 1
    geos = bi.geometries()
    assert len(geos) == L.bi_gemm_num_geometries() >= 2
    for bm, bn, w in geos:
        assert bm % 16 == 0 and bn % 16 == 0 and 1 <= w <= 16  # a workgroup holds at most 16 waves
    assert L.bi_gemm_geometry_info(len(geos), None, None, None) == _lib.EINVAL
    for M in (1, 16, 17, 64, 65, 256, 4096):
        assert 0 <= L.bi_gemm_pick_geometry(M, 4096, 4096, _lib.BF16, 1) < len(geos)


def test_footprint_policy():
    """The footprint bi_gemm picks for representative shapes (a performance
    policy, measured on MI355X; every footprint gives the same bits, which the
    GPU tests prove). Footprints are identified by (rows, columns, waves)."""
    L = _lib.lib()
    geos = bi.geometries()

    def pick(M, N, dtype=_lib.BF16, trans_b=1):
        return geos[L.bi_gemm_pick_geometry(M, N, 4096, dtype, trans_b)]

    assert pick(1, 4096) == pick(16, 32000) == (16, 16, 4)      # decode
    # A (K, N) weight gives a 16-column tile 32 bytes per row: wide ones
    # take wider tiles at decode sizes too.
    assert pick(1, 32000, trans_b=0) == (128, 128, 8)
    assert pick(1, 11008, trans_b=0) == (64, 64, 8)
    assert pick(1, 4096, trans_b=0) == (16, 16, 4)
    assert pick(32, 4096) == (16, 16, 4)                        # 17..32 rows, narrow weight
    assert pick(48, 4096) == (64, 16, 4)                        # 33..64 rows, narrow weight
    assert pick(48, 8192) == pick(96, 4096) == (64, 32, 8)
    assert pick(32, 11008) == pick(96, 8192) == (64, 64, 8)
    assert pick(64, 32000) == pick(96, 11008) == (128, 128, 8)  # wide weights, 17..128 rows
    assert pick(192, 22016) == (256, 128, 12)
    # Whole rounds of 256 workgroups: 172 tiles of 256 x 128 fit one round
    # (M = 384), 258 need two, where 516 of 128 x 128 need three (M = 768).
    assert pick(384, 11008) == (256, 128, 12)
    assert pick(512, 11008) == (256, 128, 12)
    # 256 x 256 once its tiles fill most CUs: the four-wave footprint on
    # (N, K) weights, the 16-wave ping-pong one on (K, N) weights.
    assert pick(768, 11008) == (256, 256, 4)
    assert pick(768, 11008, trans_b=0) == (256, 256, 16)
    assert pick(2048, 4096) == (256, 128, 12)                   # 128 tiles of 256 x 256
    assert pick(1024, 4096) == (128, 128, 8)
    assert pick(4096, 4096) == pick(4096, 11008) == pick(1024, 32000) == (256, 256, 4)
    assert (pick(4096, 4096, trans_b=0) == pick(4096, 11008, trans_b=0)
            == pick(1024, 32000, trans_b=0) == (256, 256, 16))
    assert pick(256, 512) == (64, 16, 4)                        # small output
    assert pick(256, 4096) == (64, 64, 8)
    assert pick(256, 11008) == (128, 128, 8)
    assert pick(256, 32000) == (256, 128, 12)                   # the bench's dominant shape
    assert pick(256, 32000, _lib.F32) == (128, 128, 8)          # fp32: registers
    assert pick(256, 11008, _lib.F32) == (64, 64, 8)            # fp32: whole tiles per CU
    assert pick(128, 4096, _lib.F32) == (64, 32, 8)


def test_quantized_footprint_policy():
    """The footprint bi_qgemm picks (a performance policy measured on MI355X;
    every footprint gives the same bits, which the GPU tests prove): the
    decode footprint for few rows, by code width and by whether its column
    blocks fit one round over the CUs, the dense table's footprints above."""
    L = _lib.lib()
    geos = bi.geometries()
    decode = L.bi_qgemm_num_geometries() - 1
    assert decode == len(geos)

    def pick(M, N, K=4096, bits=4):
        g = L.bi_qgemm_pick_geometry(M, N, K, bits)
        assert 0 <= g <= decode
        return "decode" if g == decode else geos[g]

    for bits in (2, 4):
        for M in (1, 4):
            assert pick(M, 4096, bits=bits) == pick(M, 32000, 11008, bits) == "decode"
        assert pick(8, 4096, bits=bits) == "decode"              # 256 column blocks: one round
        assert pick(5, 4112, bits=bits) == (16, 16, 4)           # 257 column blocks
        assert pick(9, 4096, bits=bits) == (16, 16, 4)           # at most 8 rows
    assert pick(1, 32000, 11008, bits=8) == "decode"
    assert pick(8, 4096, bits=8) == "decode"
    assert pick(2, 4096, 11008, bits=8) == (16, 16, 4)           # two rounds of K
    assert pick(2, 11008, bits=8) == (16, 16, 4)
    assert pick(32, 4096) == (16, 16, 4)
    assert pick(32, 32000) == pick(256, 11008) == (64, 64, 8)
    assert pick(256, 32000) == (128, 128, 8)
    assert L.bi_qgemm_pick_geometry(1, 4096, 4096, 3) == _lib.EINVAL


def _err():
    return _lib.lib().bi_last_error().decode()


def test_gemm_abi_rejects_bad_arguments_without_a_gpu():
    L = _lib.lib()
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    args = lambda **kw: (kw.get("a", p), kw.get("b", p), None, kw.get("out", p), kw.get("M", 4),
                         kw.get("N", 4), kw.get("K", 4), kw.get("dtype", _lib.BF16),
                         kw.get("tb", 1), 1.0, 1.0, None)
    assert L.bi_gemm(*args(dtype=7)) == _lib.EINVAL and "dtype" in _err()
    assert L.bi_gemm(*args(M=-1)) == _lib.EINVAL and "negative" in _err()
    assert L.bi_gemm(*args(tb=2)) == _lib.EINVAL
    assert L.bi_gemm(*args(a=None)) == _lib.EINVAL and "null" in _err()
    assert L.bi_gemm(*args(out=None)) == _lib.EINVAL
    assert L.bi_gemm(*args(M=1 << 40)) == _lib.EINVAL
    assert L.bi_gemm(*args(M=0)) == _lib.OK  # empty output: nothing to launch
    assert L.bi_gemm(*args(N=0)) == _lib.OK
    assert L.bi_gemm_with_geometry(*args()[:-1], 99, None) == _lib.EINVAL


def test_sdpa_abi_rejects_bad_arguments_without_a_gpu():
    L = _lib.lib()
    p = ctypes.c_void_p(16)

    def call(B=1, H=8, Hkv=2, qL=1, N=16, D=128, V=128, mode=0, mask=None, dtype=_lib.BF16):
        ms = _lib.i64_array([0, 0, 0]) if mask else None
        return L.bi_sdpa(p, p, p, mask, ms, None, p, B, H, Hkv, qL, N, D, V, None, 0.1, mode, 0,
                         dtype, None)

    assert call(H=6, Hkv=4) == _lib.EINVAL and "multiple" in _err()
    assert call(D=48, V=48) == _lib.EUNSUPPORTED and "head dims" in _err()
    assert call(D=128, V=96) == _lib.EUNSUPPORTED
    assert call(D=544, V=544) == _lib.EUNSUPPORTED
    assert call(mode=5) == _lib.EINVAL
    assert call(mode=2) == _lib.EINVAL and "mask" in _err()
    assert call(dtype=9) == _lib.EINVAL
    assert call(Hkv=0) == _lib.EINVAL
    assert call(B=0) == _lib.OK and call(qL=0) == _lib.OK


def test_sdpa_shape_abi_without_a_gpu():
    """Shape introspection and forcing: unknown shapes are rejected before any
    HIP call; the shape table matches the documented geometry."""
    L = _lib.lib()
    p = ctypes.c_void_p(16)

    def forced(shape, dtype=_lib.BF16, D=128, V=128, H=8, Hkv=2):
        return L.bi_sdpa_with_shape(p, p, p, None, None, None, p, 1, H, Hkv, 1, 16, D, V, None,
                                    0.1, 0, 0, dtype, shape, None)

    assert forced(-1) == _lib.EINVAL
    assert forced(_lib.SDPA_NUM_SHAPES) == _lib.EINVAL and "shape" in _err()
    assert forced(3, dtype=_lib.F32) == _lib.EINVAL      # 8 heads per workgroup: D <= 64 only
    assert forced(2, dtype=_lib.F32, H=8, Hkv=4) == _lib.EINVAL  # 4 heads do not divide 2
    assert forced(0, D=96, V=64) == _lib.EUNSUPPORTED
    assert forced(0, D=544, V=544) == _lib.EUNSUPPORTED

    def info(D, V, shape, dtype=_lib.BF16):
        c, w = ctypes.c_int(), ctypes.c_int()
        rc = L.bi_sdpa_shape_info(D, V, dtype, shape, ctypes.byref(c), ctypes.byref(w))
        return (c.value, w.value) if rc == _lib.OK else rc

    assert info(128, 128, _lib.SDPA_ROWS) == (32, 1)
    assert info(128, 128, _lib.SDPA_TILE) == (16, 1)
    assert info(128, 128, _lib.SDPA_SPLIT8) == (16, 8)
    assert info(64, 64, _lib.SDPA_SPLIT8) == (16, 4)     # at least 16 dims per workgroup
    assert info(256, 256, _lib.SDPA_ROWS) == (16, 2)     # wide heads: one tile, dims split
    assert info(192, 128, _lib.SDPA_ROWS) == (16, 1)
    assert info(96, 96, _lib.SDPA_SPLIT8) == (16, 2)     # 96 = 6 x 16 dims: splits in two
    assert info(192, 192, _lib.SDPA_SPLIT8) == (16, 4)
    assert info(32, 32, _lib.SDPA_SPLIT4) == (16, 2)
    assert info(128, 128, _lib.SDPA_SHARED) == (128, 1)  # 8 waves, one column tile each
    assert info(64, 64, _lib.SDPA_SHARED) == (128, 1)
    assert info(32, 32, _lib.SDPA_SHARED) == (64, 1)     # 4 loads per key block: 4 waves
    assert info(96, 96, _lib.SDPA_SHARED) == _lib.EINVAL
    assert info(256, 256, _lib.SDPA_SHARED) == _lib.EINVAL
    assert info(128, 128, _lib.SDPA_NUM_SHAPES) == _lib.EINVAL
    assert info(64, 64, 3, _lib.F32) == (8, 1)
    assert info(128, 128, 3, _lib.F32) == _lib.EINVAL
    assert info(256, 256, 1, _lib.F32) == (2, 1)
    assert info(128, 64, _lib.SDPA_ROWS) == (32, 1) and info(64, 128, _lib.SDPA_SPLIT8) == (16, 8)
    assert info(576, 512, _lib.SDPA_ROWS) == (16, 2)     # latent-attention heads: one tile
    assert info(64, 128, _lib.SDPA_SHARED) == _lib.EINVAL  # shared: D = V only
    assert info(512, 512, _lib.SDPA_SPLIT8) == (16, 8)


def test_sdpa_shape_policy():
    """The launch shape bi_sdpa picks on a 256-CU GPU for representative
    problems (a performance policy; every shape gives the same bits, which the
    GPU tests prove by forcing each one)."""
    L = _lib.lib()

    def pick(B, qL, H=32, Hkv=8, D=128, V=128, dtype=_lib.BF16, mask=_lib.MASK_NONE):
        return L.bi_sdpa_pick_shape(B, H, Hkv, qL, D, V, dtype, mask, 256)

    assert pick(64, 1) == pick(32, 1) == _lib.SDPA_TILE  # configs[2] decode, B >= 32
    assert pick(16, 1) == _lib.SDPA_SPLIT2
    assert pick(8, 1) == _lib.SDPA_SPLIT4
    assert pick(1, 1) == pick(4, 1) == _lib.SDPA_SPLIT8  # dims over 8 workgroups
    # Whole rounds of workgroups (a loader-wave split fills a CU, one tile
    # takes half): B=6 fits 4-way splits in one round, B=12 2-way, B=24 tiles.
    assert pick(6, 1) == _lib.SDPA_SPLIT4
    assert pick(12, 1) == _lib.SDPA_SPLIT2
    assert pick(24, 1) == _lib.SDPA_TILE
    assert pick(1, 16) == _lib.SDPA_SPLIT8      # configs[3] chunk of 16 query rows
    assert pick(1, 64) == _lib.SDPA_SPLIT2      # 8 streams x 16 tiles: too few for rows
    assert pick(4, 64) == pick(1, 256) == _lib.SDPA_ROWS  # prefill: rows fill 256 CUs
    assert pick(2, 513) == _lib.SDPA_ROWS       # 272 shared workgroups: a second round barely used
    # Shared runs one workgroup per CU at a time: it takes over once its grid
    # covers 4/5 of the CUs and fills 3/4 of its rounds.
    assert pick(1, 768) == pick(1, 1280) == _lib.SDPA_ROWS     # 192 / 320 workgroups
    assert pick(1, 896) == pick(1, 1024) == pick(1, 1536) == _lib.SDPA_SHARED  # 224, 256, 384
    assert pick(1, 2048) == pick(4, 1024) == _lib.SDPA_SHARED  # D = V = 128, no array mask
    assert pick(1, 2048, mask=_lib.MASK_CAUSAL) == _lib.SDPA_SHARED
    # Multi-token decode at large batch: shared only from 64 columns per kv
    # head (half of its 128), rows below.
    assert pick(64, 5) == pick(64, 8) == pick(32, 8) == _lib.SDPA_ROWS
    assert pick(64, 17) == pick(32, 17) == _lib.SDPA_SHARED
    assert pick(1, 2048, mask=_lib.MASK_ARRAY) == _lib.SDPA_ROWS
    assert pick(1, 2048, D=64, V=64) == _lib.SDPA_ROWS
    assert pick(1, 2048, D=256, V=256) == _lib.SDPA_ROWS
    assert pick(1, 2048, mask=7) == _lib.EINVAL
    assert pick(64, 1, dtype=_lib.F32) == 2     # fp32: four query heads per workgroup
    assert pick(1, 2048, dtype=_lib.F32) == 1   # fp32 prefill: two
    assert pick(1, 1, dtype=_lib.F32) == 0
    assert pick(1, 1, D=96, V=64) == _lib.EUNSUPPORTED


def test_status_codes_map_to_reference_exceptions():
    L = _lib.lib()
    L.bi_gemm(None, None, None, None, -1, 1, 1, 0, 0, 1.0, 1.0, None)
    with pytest.raises(ValueError):
        _lib.check(_lib.EINVAL, "x")
    with pytest.raises(NotImplementedError):
        _lib.check(_lib.EUNSUPPORTED, "x")
    with pytest.raises(RuntimeError):
        _lib.check(_lib.ELAUNCH, "x")
    _lib.check(_lib.OK, "x")


def test_tile_contract_is_pinned():
    """Guard against anyone changing the per-element arithmetic (the analogue
    of reference tests/test_invariance.py:468-470)."""
    assert bi.TILE == dict(BM=16, BN=16, BK=32, SG_M=1, SG_N=1,
                           MFMA_16BIT="v_mfma_f32_16x16x32", MFMA_FP32="v_mfma_f32_16x16x4_f32",
                           K_CHUNK_16BIT=32, K_CHUNK_FP32=16, FP32_CHAINS=2,
                           EPILOGUE="fma(alpha, acc, beta * bias) then one RNE rounding")
    # The reference's keys are all there, with the unit of fixed arithmetic.
    assert {"BM", "BN", "BK", "SG_M", "SG_N"} <= set(bi.TILE)
    assert bi.TILE["BK"] == bi.TILE["K_CHUNK_16BIT"]
    assert _attention.PARTIALS == 32 and _attention.GROUP_LANES == 8
    assert bi.HEAD_DIMS == tuple((d, d) for d in range(32, 513, 32)) + (
        (192, 128), (128, 64), (64, 128), (256, 128), (128, 256), (576, 512))


# ------------------------------------------------------------ Python validation

def _t(*shape, dtype=torch.bfloat16):
    return torch.zeros(*shape, dtype=dtype)


def test_gemm_validation_matches_reference():
    with pytest.raises(ValueError, match="share a dtype"):
        bi.matmul(_t(2, 4), _t(4, 3, dtype=torch.float16))
    with pytest.raises(ValueError, match="ndim"):
        bi.matmul(_t(4), _t(4, 3))
    with pytest.raises(ValueError, match="ndim"):
        bi.matmul(_t(2, 4), _t(2, 4, 3))
    with pytest.raises(ValueError, match="inner dimensions"):
        bi.matmul(_t(2, 4), _t(5, 3))
    with pytest.raises(ValueError, match="inner dimensions"):
        bi.linear(_t(2, 4), _t(3, 5))
    with pytest.raises(ValueError, match="bias must have shape"):
        bi.addmm(_t(4), _t(2, 4), _t(4, 3))
    with pytest.raises(ValueError, match="unsupported dtype"):
        bi.matmul(_t(2, 4, dtype=torch.float64), _t(4, 3, dtype=torch.float64))
    with pytest.raises(ValueError, match="GPU"):
        bi.matmul(_t(2, 4), _t(4, 3))  # valid shapes, but CPU tensors: no fallback


def test_sdpa_validation_matches_reference():
    q, k, v = _t(1, 8, 2, 64), _t(1, 2, 16, 64), _t(1, 2, 16, 64)
    with pytest.raises(ValueError, match="4-dimensional"):
        bi.scaled_dot_product_attention(q[0], k, v)
    with pytest.raises(ValueError, match="share a dtype"):
        bi.scaled_dot_product_attention(q, k.float(), v)
    with pytest.raises(ValueError, match="inconsistent"):
        bi.scaled_dot_product_attention(q, k, _t(1, 2, 15, 64))
    with pytest.raises(ValueError, match="multiple"):
        bi.scaled_dot_product_attention(_t(1, 6, 2, 64), _t(1, 4, 16, 64), _t(1, 4, 16, 64))
    with pytest.raises(ValueError, match="multiples of 32"):
        bi.scaled_dot_product_attention(_t(1, 4, 1, 48), _t(1, 4, 8, 48), _t(1, 4, 8, 48))
    with pytest.raises(NotImplementedError, match="not built"):  # D != V pairs not compiled
        bi.scaled_dot_product_attention(_t(1, 4, 1, 96), _t(1, 4, 8, 96), _t(1, 4, 8, 64))
    with pytest.raises(NotImplementedError, match="not built"):  # above 512
        bi.scaled_dot_product_attention(_t(1, 4, 1, 544), _t(1, 4, 8, 544), _t(1, 4, 8, 544))
    with pytest.raises(ValueError, match="sinks"):  # reference tests:355-364
        bi.scaled_dot_product_attention(q, k, v, sinks=torch.zeros(4))
    with pytest.raises(ValueError, match="causal"):
        bi.scaled_dot_product_attention(q, k, v, mask="tril")
    with pytest.raises(ValueError, match="broadcastable"):
        bi.scaled_dot_product_attention(q, k, v, mask=torch.zeros(1, 1, 3, 16))
    with pytest.raises(ValueError, match="GPU"):
        bi.scaled_dot_product_attention(q, k, v)


def test_mask_normalisation():
    """Reference _attention.py:173-202: bool -> 0 / -inf in q's dtype, left-pad
    to 4-D, zero strides on broadcast dimensions."""
    m, strides, mode = _attention._mask_args(None, 2, 8, 3, 16, torch.bfloat16)
    assert m is None and mode == _lib.MASK_NONE
    _, _, mode = _attention._mask_args("causal", 2, 8, 3, 16, torch.bfloat16)
    assert mode == _lib.MASK_CAUSAL
    keep = torch.tensor([True, False] * 8)
    m, strides, mode = _attention._mask_args(keep, 2, 8, 3, 16, torch.bfloat16)
    assert mode == _lib.MASK_ARRAY and m.shape == (1, 1, 1, 16) and strides == (0, 0, 0)
    assert m.dtype == torch.bfloat16 and m[0, 0, 0, 0] == 0 and m[0, 0, 0, 1] == float("-inf")
    m, strides, _ = _attention._mask_args(torch.zeros(2, 1, 3, 16), 2, 8, 3, 16, torch.float16)
    assert strides == (3 * 16, 0, 16) and m.dtype == torch.float16
    m, strides, _ = _attention._mask_args(torch.zeros(8, 1, 16), 2, 8, 3, 16, torch.float16)
    assert m.shape == (1, 8, 1, 16) and strides == (0, 16, 0)
    with pytest.raises(ValueError):
        _attention._mask_args(torch.zeros(1, 1, 1, 1, 16), 2, 8, 3, 16, torch.float16)


# ----------------------------------------------------------------- routing shim

class _Recorder:
    def __init__(self):
        self.calls = []

    def __call__(self, name):
        def fn(*args, **kwargs):
            self.calls.append(name)
            t = torch.zeros(1, 1)
            t.routed_to = "bi:" + name
            return t
        return fn


@pytest.fixture
def stubbed(monkeypatch):
    """Kernels replaced by recording stubs and every operand treated as
    kernel-ready, so the shim's routing runs on the CPU (test-only)."""
    rec = _Recorder()
    monkeypatch.setattr(bi, "_kernel_ready", lambda *t: all(
        x is None or (isinstance(x, torch.Tensor)
                      and not (torch.is_grad_enabled() and x.requires_grad)) for x in t))
    monkeypatch.setattr(bi, "matmul", rec("matmul"))
    monkeypatch.setattr(bi, "addmm", rec("addmm"))
    monkeypatch.setattr(bi, "linear", rec("linear"))
    monkeypatch.setattr(bi, "_sdpa", rec("sdpa"))
    return rec


def test_shim_routes_supported_calls(stubbed):
    a, w, c = torch.randn(3, 8), torch.randn(8, 5), torch.randn(5)
    with bi.batch_invariant_mode(), torch.no_grad():
        assert bi.is_enabled()
        assert torch.matmul(a, w).routed_to == "bi:matmul"
        assert (a @ w).routed_to == "bi:matmul"
        assert a.matmul(w).routed_to == "bi:matmul"
        assert torch.mm(a, w).routed_to == "bi:matmul"
        assert a.mm(w).routed_to == "bi:matmul"
        assert torch.addmm(c, a, w).routed_to == "bi:addmm"
        lin = torch.nn.Linear(8, 5)
        assert lin(a).routed_to == "bi:linear"
        assert F.linear(a, w.T).routed_to == "bi:linear"
        n_lin = stubbed.calls.count("linear")
        lin(torch.randn(8))  # 1-D input routed as a one-row batch
        assert stubbed.calls.count("linear") == n_lin + 1
        q, k = torch.randn(1, 8, 2, 64), torch.randn(1, 2, 16, 64)
        assert F.scaled_dot_product_attention(q, k, k, enable_gqa=True).routed_to == "bi:sdpa"
        y = F.scaled_dot_product_attention(q, k, k, is_causal=True, enable_gqa=True)
        assert y.routed_to == "bi:sdpa"
    assert not bi.is_enabled()
    assert stubbed.calls.count("matmul") == 5 and "addmm" in stubbed.calls


def test_strict_raises_and_non_strict_falls_back(stubbed):
    """Reference tests:646-662: head dim 48 raises under strict and falls back
    to stock otherwise."""
    q, k = torch.randn(1, 4, 1, 48), torch.randn(1, 4, 8, 48)
    stock = F.scaled_dot_product_attention(q, k, k, scale=0.1)
    with bi.batch_invariant_mode(strict=True):
        with pytest.raises(NotImplementedError, match="strict=False"):
            F.scaled_dot_product_attention(q, k, k, scale=0.1)
        with pytest.raises(NotImplementedError):
            torch.matmul(torch.randn(4), torch.randn(4, 3))  # 1-D @ 2-D
        with pytest.raises(NotImplementedError):
            torch.addmm(torch.randn(3, 5), torch.randn(3, 8), torch.randn(8, 5))  # 2-D input
        with pytest.raises(NotImplementedError):
            torch.mm(torch.randn(2, 3, 8), torch.randn(8, 5))  # mm takes 2-D operands only
        with pytest.raises(NotImplementedError):
            F.scaled_dot_product_attention(torch.randn(1, 4, 2, 64), torch.randn(1, 4, 8, 64),
                                           torch.randn(1, 4, 8, 64), dropout_p=0.1)
        g = torch.randn(3, 8, requires_grad=True)
        with pytest.raises(NotImplementedError):
            torch.matmul(g, torch.randn(8, 5))  # autograd: the kernels have no backward
    with bi.batch_invariant_mode(strict=False):
        y = F.scaled_dot_product_attention(q, k, k, scale=0.1)
    assert torch.equal(y, stock)


def test_originals_restored_even_on_exception():
    """Reference tests:686-698."""
    before = (torch.matmul, torch.addmm, torch.Tensor.__matmul__, torch.Tensor.matmul,
              torch.mm, torch.Tensor.mm, torch.nn.Linear.forward, F.linear,
              F.scaled_dot_product_attention)
    had = {n: n in vars(torch.Tensor) for n in ("__matmul__", "matmul", "mm")}
    with pytest.raises(RuntimeError):
        with bi.batch_invariant_mode():
            assert bi.is_enabled()
            raise RuntimeError("boom")
    after = (torch.matmul, torch.addmm, torch.Tensor.__matmul__, torch.Tensor.matmul,
             torch.mm, torch.Tensor.mm, torch.nn.Linear.forward, F.linear,
             F.scaled_dot_product_attention)
    assert before == after
    assert {n: n in vars(torch.Tensor) for n in had} == had
    assert not bi.is_enabled()


def test_nesting_restores_only_at_outermost_exit():
    """Reference tests:700-708."""
    stock = torch.matmul
    with bi.batch_invariant_mode():
        patched = torch.matmul
        assert patched is not stock
        with bi.batch_invariant_mode():
            assert torch.matmul is patched
        assert torch.matmul is patched, "inner exit unpatched too early"
    assert torch.matmul is stock


def test_cpu_tensors_raise_under_strict_and_fall_back_otherwise():
    a, w = torch.randn(3, 8), torch.randn(8, 5)
    with bi.batch_invariant_mode(strict=True):
        with pytest.raises(NotImplementedError):
            torch.matmul(a, w)
    with bi.batch_invariant_mode(strict=False):
        assert torch.equal(torch.matmul(a, w), a @ w)


# -------------------------------------------------------------- CLI and bench

def test_cli_usage_exit_code(capsys):
    from mlx_batch_invariant._cli import main

    assert main([]) == 2
    assert "usage: mlx-bi verify" in capsys.readouterr().err


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_decoder_harness_on_cpu():
    """The synthetic decoder builds and runs on the CPU (stock ops only: the
    invariant kernels need the GPU); prompts and weights follow their seeds."""
    from mlx_batch_invariant import decoder

    c = decoder.DecoderConfig(hidden=64, inter=128, heads=4, kv_heads=2, head_dim=16,
                              layers=2, vocab=100)
    m1 = decoder.build(c, device="cpu", dtype=torch.float32, seed=3)
    m2 = decoder.build(c, device="cpu", dtype=torch.float32, seed=3)
    assert all(torch.equal(a, b) for a, b in zip(m1.parameters(), m2.parameters()))
    ids = decoder.prompts(c, 4, 10, seed=1, device="cpu")
    assert ids.shape == (4, 10) and torch.equal(ids, decoder.prompts(c, 4, 10, seed=1, device="cpu"))
    with torch.no_grad():
        y = m1(ids)
    assert y.shape == (4, c.vocab) and torch.isfinite(y).all()
    got = decoder.determinism(m1, length=10, batches=(2, 4), seed=1, invariant=False)
    assert set(got) == {2, 4} and all(v >= 0 for v in got.values())


def test_custom_op_fake_shapes():
    """torch.compile sees bi.* calls as the opaque ops mlx_bi::gemm / mlx_bi::sdpa;
    their fake implementations give the output shapes without a GPU."""
    from torch._subclasses.fake_tensor import FakeTensorMode

    from mlx_batch_invariant import _ops

    with FakeTensorMode():
        a = torch.empty(3, 5, 64, dtype=torch.bfloat16)
        assert _ops.gemm(a, torch.empty(96, 64, dtype=torch.bfloat16), None, True, 1.0,
                         1.0).shape == (3, 5, 96)
        assert _ops.gemm(a, torch.empty(64, 80, dtype=torch.bfloat16), None, False, 1.0,
                         1.0).shape == (3, 5, 80)
        q, k = torch.empty(2, 8, 3, 64), torch.empty(2, 2, 10, 64)
        assert _ops.sdpa(q, k, torch.empty(2, 2, 10, 32), 0.1, 0, None, [0, 0, 0], 0,
                         None).shape == (2, 8, 3, 32)


def test_quant_pack_layout_matches_the_oracle():
    """bi's packing is the reference layout: the oracle's restatement of the
    reference unpack reads back the codes bi packed; bi.dequantize is the
    oracle's fp32 weight rounded once to the element type."""
    from oracle import quant as oquant

    from helpers import pack_codes
    from mlx_batch_invariant import _quant

    g = torch.Generator().manual_seed(7)
    for bits in bi.QUANT_BITS:
        q = torch.randint(0, 1 << bits, (6, 128), generator=g)
        w = _quant._pack(q, bits)
        assert w.dtype == torch.int32 and w.shape == (6, 128 * bits // 32)
        assert torch.equal(w, pack_codes(q.numpy(), bits))
        assert torch.equal(_quant._unpack(w, bits, 128), q)
        assert (oquant.unpack(w.numpy(), bits, 128) == q.numpy()).all()
        for dtype, name in ((torch.bfloat16, "bfloat16"), (torch.float16, "float16")):
            for gs in (32, 64, 128):
                s = (torch.rand(6, 128 // gs, generator=g) * 0.1 + 1e-3).to(dtype)
                b = (torch.randn(6, 128 // gs, generator=g)).to(dtype)
                got = bi.dequantize(w, s, b, gs, bits)
                want = oquant.dequantize_to(w.numpy(), s.float().numpy(), b.float().numpy(),
                                            gs, bits, name)
                assert got.dtype == dtype
                assert (got.double().numpy() == want).all(), (bits, name, gs)


def test_quantize_error_is_within_half_a_step():
    g = torch.Generator().manual_seed(8)
    w = torch.randn(32, 256, generator=g).to(torch.bfloat16)
    for bits in bi.QUANT_BITS:
        for gs in (32, 64, 128):
            q, s, b = bi.quantize(w, gs, bits)
            err = (bi.dequantize(q, s, b, gs, bits).float() - w.float()).abs()
            step = s.float().repeat_interleave(gs, dim=1)
            assert (err <= step * 0.5 + w.float().abs() * 2 ** -7 + 1e-6).all(), (bits, gs)


def test_quantized_linear_validation():
    x = torch.zeros(3, 128, dtype=torch.bfloat16)
    w, s, b = bi.quantize(torch.zeros(64, 128, dtype=torch.bfloat16), 64, 4)
    with pytest.raises(ValueError):
        bi.quantized_linear(x, w, s, b, 64, 3)            # bits
    with pytest.raises(ValueError):
        bi.quantized_linear(x[:, :96], w, s, b, 64, 4)    # K mismatch
    with pytest.raises(ValueError):
        bi.quantized_linear(x, w, s[:, :1], b, 64, 4)     # scales shape
    with pytest.raises(ValueError):
        bi.quantized_linear(x, w, s.float(), b, 64, 4)    # scales dtype
    with pytest.raises(ValueError):
        bi.quantized_linear(x, w, s, b, 64, 4)            # CPU tensors
    # outside the mode quantized_matmul is stock: dequantize, then F.linear
    y = bi.quantized_matmul(x, w, s, b, True, 64, 4)
    assert torch.equal(y, F.linear(x, bi.dequantize(w, s, b, 64, 4)))
