// bf16 / f16 attention kernels for head dims D = 64, V = 128 (bi_sdpa_mfma_kernel.h);
// one unit per head-dim pair so the library builds in parallel.
#include "bi_sdpa_mfma_kernel.h"

BI_SDPA_MFMA_DEFINE(64, 128)
