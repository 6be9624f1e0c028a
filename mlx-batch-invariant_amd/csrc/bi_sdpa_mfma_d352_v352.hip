// bf16 / f16 attention kernels for head dims D = 352, V = 352 (bi_sdpa_mfma_kernel.h);
// one unit per head-dim pair so the library builds in parallel.
#include "bi_sdpa_mfma_kernel.h"

BI_SDPA_MFMA_DEFINE(352, 352)
