"""ctypes binding of libbi.so, the C ABI declared in include/bi.h.

This is the boundary the reference crosses with ``mx.fast.metal_kernel``
(reference mlx_batch_invariant/_gemm.py:142-149, _attention.py:151-158): the
Python side validates and lays out the arguments, allocates the output, and
hands raw device pointers plus the current HIP stream to one C call. There is
no other compute path: if libbi.so is missing the ops raise.
"""

import ctypes
import os

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libbi.so")

# enum bi_dtype / bi_status / bi_mask_mode (include/bi.h)
F32, F16, BF16 = 0, 1, 2
OK, EINVAL, EUNSUPPORTED, ELAUNCH = 0, -1, -2, -3
MASK_NONE, MASK_CAUSAL, MASK_ARRAY = 0, 1, 2

DTYPE_CODES = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}

_c_i64 = ctypes.c_int64
_c_vp = ctypes.c_void_p
_c_int = ctypes.c_int
_c_float = ctypes.c_float
_c_i64p = ctypes.POINTER(ctypes.c_int64)

# name -> (restype, argtypes); every symbol include/bi.h and include/bi_testing.h declare.
SIGNATURES = {
    "bi_abi_version": (_c_int, []),
    "bi_last_error": (ctypes.c_char_p, []),
    "bi_gemm": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_int, _c_int,
                         _c_float, _c_float, _c_vp]),
    "bi_sdpa": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_i64p, _c_vp, _c_vp,
                         _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                         _c_i64p, _c_float, _c_int, _c_i64, _c_int, _c_vp]),
    "bi_gemm_num_geometries": (_c_int, []),
    "bi_gemm_geometry_info": (_c_int, [_c_int, ctypes.POINTER(_c_int), ctypes.POINTER(_c_int),
                                       ctypes.POINTER(_c_int)]),
    "bi_gemm_pick_geometry": (_c_int, [_c_i64, _c_i64, _c_i64, _c_int, _c_int]),
    "bi_gemm_with_geometry": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64,
                                       _c_int, _c_int, _c_float, _c_float, _c_int, _c_vp]),
    "bi_gemm_timed": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_int,
                               _c_int, _c_float, _c_float, _c_vp, _c_vp, _c_vp]),
    "bi_feed_probe": (_c_int, [_c_vp, _c_i64, _c_int, _c_int, _c_int, _c_vp, _c_vp, _c_vp]),
    "bi_qgemm": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_int,
                          _c_int, _c_int, _c_vp]),
    "bi_qgemm_num_geometries": (_c_int, []),
    "bi_qgemm_pick_geometry": (_c_int, [_c_i64, _c_i64, _c_i64, _c_int]),
    "bi_qgemm_with_geometry": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64,
                                        _c_i64, _c_int, _c_int, _c_int, _c_int, _c_vp]),
    "bi_sdpa_pick_shape": (_c_int, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int,
                                    _c_int, _c_int]),
    "bi_sdpa_shape_info": (_c_int, [_c_i64, _c_i64, _c_int, _c_int, ctypes.POINTER(_c_int),
                                    ctypes.POINTER(_c_int)]),
    "bi_sdpa_with_shape": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_i64p, _c_vp, _c_vp,
                                    _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                    _c_i64p, _c_float, _c_int, _c_i64, _c_int, _c_int, _c_vp]),
    "bi_device_wavefront_size": (_c_int, [ctypes.POINTER(_c_int)]),
}

# Attention launch shapes (include/bi_testing.h): bf16 / f16 on matrix cores.
SDPA_ROWS, SDPA_TILE, SDPA_SPLIT2, SDPA_SPLIT4, SDPA_SPLIT8, SDPA_SHARED = 0, 1, 2, 3, 4, 5
SDPA_NUM_SHAPES = 6

ABI_VERSION = 1

_lib = None


def lib():
    """The loaded libbi.so; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                "libbi.so is not built (%s). Build it with "
                "`python mlx-batch-invariant_amd/csrc/build.py`; there is no "
                "fallback path." % LIB_PATH)
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        if handle.bi_abi_version() != ABI_VERSION:
            raise RuntimeError("libbi.so ABI version %d, expected %d"
                               % (handle.bi_abi_version(), ABI_VERSION))
        _lib = handle
    return _lib


def check(rc, what):
    """Turns a bi_status into the exception the reference raises for it."""
    if rc == OK:
        return
    msg = lib().bi_last_error().decode(errors="replace")
    if rc == EINVAL:
        raise ValueError("%s: %s" % (what, msg))
    if rc == EUNSUPPORTED:
        raise NotImplementedError("%s: %s" % (what, msg))
    raise RuntimeError("%s: %s" % (what, msg))


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def launch_stream(device):
    """(stream handle as int, needs_device_switch) for a launch on `device`.

    The raw handle of torch's current stream, read without building a Stream
    object (the launch path is host-bound for small problems). A launch on a
    device other than the current one runs under torch.cuda.device: the null
    (default) stream always means the current device to HIP.
    """
    idx = device.index
    cur = torch.cuda.current_device()
    if idx is None:
        idx = cur
    if _raw_stream is not None:
        handle = _raw_stream(idx)
    else:
        handle = torch.cuda.current_stream(idx).cuda_stream
    return handle, idx != cur


def i64_array(values):
    return (ctypes.c_int64 * len(values))(*[int(v) for v in values])
