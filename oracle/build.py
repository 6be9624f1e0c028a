"""Builds oracle/liboracle.so from oracle/csrc/oracle.c with gcc.

Test infrastructure only. The reference's own kernels are MLX/Metal source
strings (reference _gemm.py:29-130, _attention.py:32-149) with no C/C++ build,
so there is no oracle/_ref build: the reference cannot be compiled or run on
Linux.
"""

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "csrc", "oracle.c")
LIB = os.path.join(HERE, "liboracle.so")


def build(verbose=True):
    tmp = LIB + ".tmp"
    cmd = ["gcc", "-O2", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off", "-std=c11",
           SRC, "-o", tmp, "-lm"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("oracle build failed:\n" + r.stderr)
    os.replace(tmp, LIB)
    if verbose:
        print("built", os.path.relpath(LIB, os.path.dirname(HERE)))
    return LIB


if __name__ == "__main__":
    try:
        build()
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)
