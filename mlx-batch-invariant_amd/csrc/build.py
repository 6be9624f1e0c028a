"""Builds libbi.so (the HIP kernels + C ABI) for gfx950 with hipcc, in-tree.

    python mlx-batch-invariant_amd/csrc/build.py

Objects go to mlx-batch-invariant_amd/_build/, the library to
mlx-batch-invariant_amd/mlx_batch_invariant/libbi.so, where the Python package
loads it from. Always recompiles (the driver uses this as its build check).
"""

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.dirname(HERE)
REPO = os.path.dirname(PKG_ROOT)
INCLUDE = os.path.join(REPO, "include")
BUILD = os.path.join(PKG_ROOT, "_build")
LIB = os.path.join(PKG_ROOT, "mlx_batch_invariant", "libbi.so")

# Attention: one instantiation unit per built head-dim pair (BI_SDPA_DIM_PAIRS).
SDPA_MFMA_UNITS = sorted(f for f in os.listdir(HERE)
                         if f.startswith("bi_sdpa_mfma_d") and f.endswith(".hip"))
SOURCES = ["bi_abi.cpp", "bi_gemm.hip", "bi_gemm_f32.hip", "bi_gemm_f16.hip", "bi_gemm_bf16.hip",
           "bi_qgemm_f16.hip", "bi_qgemm_bf16.hip", "bi_sdpa.hip", *SDPA_MFMA_UNITS]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# -ffp-contract=off: every fused multiply-add in the kernels is written out
# explicitly, so the compiler may not contract anything else -- the per-element
# arithmetic is part of the invariance contract.
# -packed-fp32-ops: keep the compiler from emitting packed fp32 VALU ops.
DEVICE_FLAGS = [
    "--offload-arch=" + ARCH, "-O3", "-std=c++17", "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]

# The quantized GEMM and the MFMA attention work on MFMA results with VALU
# arithmetic (group folds; softmax and rescaling); with the results in
# accumulation registers every such step would copy them out and back. This
# keeps MFMA operands and results in VGPRs.
EXTRA_FLAGS = {
    "bi_qgemm_f16.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "bi_qgemm_bf16.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    **{u: ["-mllvm", "-amdgpu-mfma-vgpr-form"] for u in SDPA_MFMA_UNITS},
}


def _compile(src):
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [HIPCC, *DEVICE_FLAGS, *EXTRA_FLAGS.get(src, []), "-I", INCLUDE, "-I", HERE, "-c",
           os.path.join(HERE, src), "-o", obj]
    if src.endswith(".cpp"):
        cmd[cmd.index("-c"):cmd.index("-c")] = ["-x", "hip"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError("hipcc failed for %s:\n%s" % (src, err))
    return obj


def build(verbose=True):
    os.makedirs(BUILD, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 8)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    # --no-undefined: a kernel whose host stub was not emitted fails here, not
    # at load time on the GPU box.
    cmd = [HIPCC, "--offload-arch=" + ARCH, "-shared", "-fPIC", "-Wl,--no-undefined", *objs,
           "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stderr)
    os.replace(tmp, LIB)
    if verbose:
        print("built", os.path.relpath(LIB, REPO))
    return LIB


if __name__ == "__main__":
    try:
        build()
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)
