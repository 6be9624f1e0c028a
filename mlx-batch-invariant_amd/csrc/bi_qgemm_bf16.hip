// Quantized-B GEMM kernels for __bf16 activations (own translation unit so the
// instantiations compile in parallel with the dense ones).
#include "bi_gemm_kernel.h"

bi_gemm_dev::KernelFn bi_qgemm_kernel_bf16(int g, int bits, int group) {
  return bi_gemm_dev::qkernel_for<__bf16>(g, bits, group);
}

bi_gemm_dev::KernelFn bi_qdecode_kernel_bf16(int group, int rows, int bits) {
  return bi_gemm_dev::qdecode_kernel_for<__bf16>(group, rows, bits);
}
