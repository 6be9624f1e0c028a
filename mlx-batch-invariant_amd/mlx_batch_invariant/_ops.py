"""torch.library custom ops over the kernel launches, for torch.compile.

The reference's kernels are opaque to ``mx.compile``, which may reorder and
fuse the graph around them but never inside (reference
tests/test_invariance.py:595-640). The same holds here: while torch.compile
traces, ``bi.*`` calls become the ops ``mlx_bi::gemm``, ``mlx_bi::qgemm`` and
``mlx_bi::sdpa``, which the compiler treats as opaque nodes (their fake
implementations give only output shapes) and which run the HIP kernels
unchanged. Eager calls skip
the dispatcher and launch directly.
"""

from typing import List, Optional

import torch


@torch.library.custom_op("mlx_bi::gemm", mutates_args=())
def gemm(a: torch.Tensor, b: torch.Tensor, bias: Optional[torch.Tensor], trans_b: bool,
         alpha: float, beta: float) -> torch.Tensor:
    from . import _gemm

    return _gemm._gemm_eager(a, b, bias, trans_b, alpha, beta, None)


@gemm.register_fake
def _gemm_fake(a, b, bias, trans_b, alpha, beta):
    n = b.shape[0] if trans_b else b.shape[1]
    return a.new_empty((*a.shape[:-1], n))


@torch.library.custom_op("mlx_bi::sdpa", mutates_args=())
def sdpa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float, mask_mode: int,
         mask: Optional[torch.Tensor], mstrides: List[int], causal_offset: int,
         sinks: Optional[torch.Tensor]) -> torch.Tensor:
    from . import _attention

    return _attention._sdpa_eager(q, k, v, scale, mask_mode, mask, mstrides, causal_offset,
                                  sinks)


@sdpa.register_fake
def _sdpa_fake(q, k, v, scale, mask_mode, mask, mstrides, causal_offset, sinks):
    return q.new_empty((q.shape[0], q.shape[1], q.shape[2], v.shape[-1]))


@torch.library.custom_op("mlx_bi::qgemm", mutates_args=())
def qgemm(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
          group_size: int, bits: int) -> torch.Tensor:
    from . import _quant

    return _quant._quantized_linear_eager(x, w, scales, biases, group_size, bits)


@qgemm.register_fake
def _qgemm_fake(x, w, scales, biases, group_size, bits):
    return x.new_empty((*x.shape[:-1], w.shape[0]))
