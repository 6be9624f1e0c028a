// Launch arguments and launch shapes shared by the attention kernels
// (bi_sdpa.hip: the VALU kernel for fp32 and the C entry points;
// bi_sdpa_mfma_kernel.h: the MFMA kernel for bf16 and f16).
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
  // The matrix-core kernels scale raw scores by |scale| * log2(e) and take a
  // negative scale as negated queries: qsign (0x80008000 then, else 0) is
  // XORed into every dword of q as it is loaded, which negates each score
  // exactly.
  float ascale2;
  uint32_t qsign;
  int mask_mode;
  int64_t causal_offset;
};

typedef void (*SdpaKernelFn)(SdpaArgs);

// Head-dim pairs (D for queries and keys, V for values) built for every
// element type. The reference accepts any multiples of 32
// (mlx_batch_invariant/_attention.py:224-227); these are the ones compiled.
#define BI_SDPA_DIM_PAIRS(X)                                                                   \
  X(32, 32) X(64, 64) X(96, 96) X(128, 128) X(160, 160) X(192, 192) X(224, 224) X(256, 256)     \
  X(288, 288) X(320, 320) X(352, 352) X(384, 384) X(416, 416) X(448, 448) X(480, 480)          \
  X(512, 512) X(192, 128) X(128, 64) X(64, 128) X(256, 128) X(128, 256) X(576, 512)

// Launch shapes of the MFMA kernel (bf16 / f16). None of them enters a
// column's arithmetic; they decide which workgroup, wave and lane evaluate a
// column and how operands travel.
//   SDPA_ROWS    several 16-column tiles per workgroup, one chain per wave
//   SDPA_TILE    one column tile, output dims whole (or split in two for V > 128)
//   SDPA_SPLITn  one column tile, output dims split over n workgroups (decode),
//                capped by the largest power of two that leaves each workgroup
//                a multiple of 16 dims; for D = V = 128 without an array mask,
//                4 more waves only issue the chains' loads
//   SDPA_SHARED  one 16-column tile per wave, every wave walking every key
//                block with all 4 chains' state of its columns: a key and value
//                block is loaded once into LDS for 4-8 column tiles (prefill;
//                D = V in {32, 64, 128})
enum SdpaShape { SDPA_ROWS = 0, SDPA_TILE = 1, SDPA_SPLIT2 = 2, SDPA_SPLIT4 = 3, SDPA_SPLIT8 = 4,
                 SDPA_SHARED = 5, SDPA_NUM_SHAPES = 6 };

// Heads wider than 128 carry more registers per column: one column tile per
// rows workgroup, no key prefetch, value dims always split at least in two.
constexpr bool sdpa_wide(int64_t D, int64_t V) { return D > 128 || V > 128; }
constexpr int sdpa_rows_tiles(int64_t D, int64_t V) { return sdpa_wide(D, V) ? 1 : 2; }
constexpr int sdpa_splits_max(int64_t V) {
  return (V / 16) % 8 == 0 ? 8 : (V / 16) % 4 == 0 ? 4 : (V / 16) % 2 == 0 ? 2 : 1;
}
constexpr int sdpa_splits_min(int64_t V) { return V > 128 ? 2 : 1; }
// SDPA_SHARED: built for D = V in {32, 64, 128}; its waves split the
// (D + V) / 16 loads of a key block evenly, at most 8 waves.
constexpr bool sdpa_shared_dims(int64_t D, int64_t V) {
  return D == V && (D == 32 || D == 64 || D == 128);
}
constexpr int sdpa_shared_waves(int64_t D, int64_t V) {
  return (D + V) / 16 >= 8 ? 8 : (int)((D + V) / 16);
}
constexpr int sdpa_shape_splits(int64_t V, int shape) {
  const int want = shape <= SDPA_TILE || shape == SDPA_SHARED ? 1 : 1 << (shape - 1);
  const int capped = want < sdpa_splits_max(V) ? want : sdpa_splits_max(V);
  return capped > sdpa_splits_min(V) ? capped : sdpa_splits_min(V);
}
constexpr int sdpa_shape_columns(int64_t D, int64_t V, int shape) {
  return shape == SDPA_ROWS     ? 16 * sdpa_rows_tiles(D, V)
         : shape == SDPA_SHARED ? 16 * sdpa_shared_waves(D, V)
                                : 16;
}
// The dim-split shapes for D = V = 128 without an array mask stage keys and
// values in LDS through loader waves, one beside each chain's wave.
constexpr bool sdpa_loaders(int64_t D, int64_t V, int shape, bool array_mask) {
  return !array_mask && D == 128 && V == 128 && shape >= SDPA_SPLIT2 && shape <= SDPA_SPLIT8;
}
// Threads per workgroup: 4 waves (one per chain), 8 with loader waves, or
// one wave per column tile.
constexpr int sdpa_shape_threads(int64_t D, int64_t V, int shape, bool array_mask) {
  return shape == SDPA_SHARED                        ? 64 * sdpa_shared_waves(D, V)
         : sdpa_loaders(D, V, shape, array_mask) ? 512
                                                     : 256;
}

// The MFMA kernel of one head-dim pair for (dtype, array mask or not, shape);
// nullptr for an element type it is not built for (bi_sdpa_mfma_d*.hip).
#define BI_SDPA_MFMA_DECLARE(D, V) \
  SdpaKernelFn sdpa_mfma_kernel_d##D##_v##V(int dtype, bool mask, int shape);
BI_SDPA_DIM_PAIRS(BI_SDPA_MFMA_DECLARE)
#undef BI_SDPA_MFMA_DECLARE
