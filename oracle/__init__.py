"""CPU oracle for the batch-invariant GEMM and attention path.

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this package, and only as the checker (or, for the
CPU baseline, as the thing timed on the host). The product path
(mlx-batch-invariant_amd/) never imports it and has no CPU fallback.

Contents:
  bits.py  -- raw bit views, ULP distance and round-to-nearest-even helpers
              (reference probe/probe.py:33-45, tests/test_invariance.py:20-21)
  gemm.py  -- float64 GEMM oracle (reference tests/test_invariance.py:114-146)
              and the fixed-order fp32 restatement of reference
              _gemm.py:62-129 (C, csrc/oracle.c)
  sdpa.py  -- float64 softmax-attention oracle (reference
              tests/test_invariance.py:408-432) and the fixed-order fp32
              restatement of reference _attention.py:68-148 (C)

How each function is pinned (checked against something other than itself) is
listed in tests/test_oracle.py; the reference ships no golden vectors and its
MLX/Metal code cannot run here, so the pins are closed forms, exact integer
arithmetic, brute force on tiny inputs and agreement of the two independent
implementations above. Bitwise parity with the reference's own outputs is
unpinned: those depend on Apple's simdgroup MMA and simd_sum orders.
"""
