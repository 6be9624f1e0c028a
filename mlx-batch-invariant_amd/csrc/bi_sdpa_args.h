// Launch arguments shared by the attention kernels (bi_sdpa.hip, the VALU
// kernel for fp32; bi_sdpa_mfma.hip, the MFMA kernel for bf16 and f16).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

struct SdpaArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* mask;
  const void* sinks;
  void* out;
  int64_t B, H, Hkv, qL, N;
  int64_t qs[3], ks[3], vs[3], ms[3];  // element strides for (b, h, s|n)
  float scale2;                        // scale * log2(e)
  int mask_mode;
  int64_t causal_offset;
};

// Launches the MFMA attention kernel for bf16 / f16 with D == V in
// {64, 128, 256} (bi_sdpa_mfma.hip) on a device with `cus` compute units.
// Returns false when it is not built for the dtype and head dim (the caller
// then uses the VALU kernel).
bool sdpa_mfma_launch(const SdpaArgs& p, int dtype, int64_t D, int cus, hipStream_t stream);
