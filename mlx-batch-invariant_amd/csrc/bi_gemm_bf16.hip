// GEMM kernels for __bf16 operands (one translation unit per element type so the
// instantiations compile in parallel).
#include "bi_gemm_kernel.h"

bi_gemm_dev::KernelFn bi_gemm_kernel_bf16(int g, bool trans_b) {
  return bi_gemm_dev::kernel_for<__bf16>(g, trans_b);
}
