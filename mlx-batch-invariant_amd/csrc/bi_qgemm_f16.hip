// Quantized-B GEMM kernels for _Float16 activations (own translation unit so the
// instantiations compile in parallel with the dense ones).
#include "bi_gemm_kernel.h"

bi_gemm_dev::KernelFn bi_qgemm_kernel_f16(int g, int bits, int group) {
  return bi_gemm_dev::qkernel_for<_Float16>(g, bits, group);
}

bi_gemm_dev::KernelFn bi_qdecode_kernel_f16(int group, int rows, int bits) {
  return bi_gemm_dev::qdecode_kernel_for<_Float16>(group, rows, bits);
}
