// Device code of the batch-invariant GEMM (gfx950); included by the
// per-element-type translation units bi_gemm_{f32,f16,bf16}.hip.
//
// Restates the reference bi_gemm (mlx_batch_invariant/_gemm.py:29-130): one
// workgroup owns an output tile and the whole K reduction for it, the K-loop
// trip count depends on K alone, tiles are staged through LDS, and the bias is
// added to the fp32 accumulator before the single rounding to the element type
// (_gemm.py:115-129). No split-K, no atomics.
//
// Fixed per-element arithmetic (the invariance contract):
//   * K is consumed in chunk-steps q = 0, 1, 2, ... in ascending order,
//     ceil(K / 32) of them for bf16/f16 and ceil(K / 16) for fp32 -- a function
//     of K alone. Elements past K read as zero. The pipelined loop may run a
//     few more chunk-steps to finish its last round of stages; those see only
//     zeros in both operands, and adding exact zeros to an accumulator that
//     starts at +0.0 changes no bit (it can never hold -0.0, and x + 0 = x for
//     every other x, NaN and infinities included).
//       bf16/f16: chunk-step q is one v_mfma_f32_16x16x32_{bf16,f16}; lane
//                 group g = lane / 16 supplies k = 32q + 8g + t, t = 0..7.
//       fp32:     chunk-step q is four v_mfma_f32_16x16x4_f32, t = 0..3; lane
//                 group g supplies k = 16q + 4g + t. Chunk-step q accumulates
//                 into chain q mod 2 (two chains halve the length of each fp32
//                 accumulation) and acc = chain_0 + chain_1.
//     Every output element sees exactly this sequence of MFMAs on its own row
//     of A and column of B, each chain starting from +0.0.
//   * Epilogue: v = bias ? fma(alpha, acc, beta * bias[n]) : acc, then one
//     round-to-nearest-even to the element type.
// The workgroup footprint (rows x columns of C per workgroup, waves, pipeline
// depth, bytes staged per step) comes from a table of compile-time geometries
// that all run this same sequence per element; it only decides how many
// elements a workgroup owns and how their operands travel. An output row
// therefore has the same bits whatever M is, whatever rows surround it,
// whichever slot of a tile it lands in, and whichever geometry the launch
// picked.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "bi_internal.h"

namespace bi_gemm_dev {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;
typedef __attribute__((address_space(3))) void lds_void_t;

struct GemmArgs {
  const void* a;
  const void* b;
  const void* bias;
  void* out;
  int64_t M, N, K;
  int tiles_m, tiles_n;
  float alpha, beta;
  int vec_a, vec_b;  // rows of A / rows of B may be read as aligned 16-byte vectors
  // Affine-quantized B (quantized kernels only): B is the packed (N, K * bits
  // / 32) uint32 weight, qs / qz the (N, K / group) scales and biases in the
  // element type, group = 1 << qgroup_shift.
  const void* qs;
  const void* qz;
  int qgroup_shift;
};

// ---------------------------------------------------------------- element types

template <typename T> struct Elem;
template <> struct Elem<__bf16> {
  __device__ static float to_f32(__bf16 x) { return (float)x; }
  __device__ static __bf16 from_f32(float x) { return (__bf16)x; }  // RNE
};
template <> struct Elem<_Float16> {
  __device__ static float to_f32(_Float16 x) { return (float)x; }
  __device__ static _Float16 from_f32(float x) { return (_Float16)x; }  // RNE
};
template <typename T> struct IsBF16 { static constexpr bool value = false; };
template <> struct IsBF16<__bf16> { static constexpr bool value = true; };

template <> struct Elem<float> {
  __device__ static float to_f32(float x) { return x; }
  __device__ static float from_f32(float x) { return x; }
};

// One chunk-step of the fixed arithmetic for a 16x16 output block: `a` and
// `b` are this lane's 16-byte operand chunks.
__device__ inline f32x4_t chunk_step(__bf16, uint4 a, uint4 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
__device__ inline f32x4_t chunk_step(_Float16, uint4 a, uint4 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}
__device__ inline f32x4_t chunk_step(float, uint4 a, uint4 b, f32x4_t c) {
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.x), __uint_as_float(b.x), c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.y), __uint_as_float(b.y), c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.z), __uint_as_float(b.z), c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.w), __uint_as_float(b.w), c, 0, 0, 0);
  return c;
}

// 4 x 4 transpose of words across the lane groups g = lane / 16: afterwards
// register j of lane group g holds what register g of lane group j held.
// v_permlane32_swap exchanges the upper 32 lanes of its first operand with
// the lower 32 of its second; v_permlane16_swap the odd 16-lane rows of its
// first operand with the even rows of its second.
__device__ __forceinline__ void xpose_lane_groups(uint32_t (&r)[4]) {
  const auto s0 = __builtin_amdgcn_permlane32_swap(r[0], r[2], false, false);
  const auto s1 = __builtin_amdgcn_permlane32_swap(r[1], r[3], false, false);
  const auto t0 = __builtin_amdgcn_permlane16_swap(s0[0], s1[0], false, false);
  const auto t1 = __builtin_amdgcn_permlane16_swap(s0[1], s1[1], false, false);
  r[0] = t0[0];
  r[1] = t0[1];
  r[2] = t1[0];
  r[3] = t1[1];
}

// The 8 4-bit codes of word w (code t in bits 4t .. 4t + 3) as element-type
// integers, two per register, code 0 in the low half of the first. Codes 0-15
// in the low bits of a byte are the fp8 E4M3 values q * 2^-9 (subnormal for
// q < 8, then the first binade), so the scaled fp8 conversion with scale
// 2^9 yields q exactly, two codes per instruction: two byte permutes put
// codes 0-3 and 4-7 one per byte (each byte masked to its low nibble), and
// four conversions each take one 16-bit half.
template <typename T>
__device__ __forceinline__ uint4 codes_as_elems(uint32_t w) {
  const uint32_t v = w >> 4;
  const uint32_t lo = __builtin_amdgcn_perm(v, w, 0x05010400u) & 0x0F0F0F0Fu;  // codes 0 1 2 3
  const uint32_t hi = __builtin_amdgcn_perm(v, w, 0x07030602u) & 0x0F0F0F0Fu;  // codes 4 5 6 7
  uint4 r;
  if constexpr (IsBF16<T>::value) {
    r.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 512.0f, false));
    r.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 512.0f, true));
    r.z = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 512.0f, false));
    r.w = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 512.0f, true));
  } else {
    r.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 512.0f, false));
    r.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 512.0f, true));
    r.z = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 512.0f, false));
    r.w = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 512.0f, true));
  }
  return r;
}

// The 8 2-bit codes in the low 16 bits of v (code t in bits 2t, 2t + 1) as
// element-type integers, two per register, code 0 in the low half of the
// first. Each byte of codes spreads into four bytes by OR-ing shifted copies
// (u | u << 6 | u << 12 | u << 18 puts code i of u in bits 8i, 8i + 1 and
// no other code there; OR, not a sum, so nothing carries), masked to two bits;
// 0-3 read as fp8 E4M3 are q * 2^-9, so the scaled conversion with scale 2^9
// yields them exactly, two codes per instruction.
template <typename T>
__device__ __forceinline__ uint4 codes2_as_elems(uint32_t v) {
  const auto spread = [](uint32_t u) -> uint32_t {
    u = u | (u << 6);
    u = u | (u << 12);
    return u & 0x03030303u;
  };
  const uint32_t lo = spread(v & 0xFFu), hi = spread((v >> 8) & 0xFFu);
  uint4 r;
  if constexpr (IsBF16<T>::value) {
    r.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 512.0f, false));
    r.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 512.0f, true));
    r.z = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 512.0f, false));
    r.w = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 512.0f, true));
  } else {
    r.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 512.0f, false));
    r.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 512.0f, true));
    r.z = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 512.0f, false));
    r.w = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 512.0f, true));
  }
  return r;
}

// The 8 8-bit codes of words lo (codes 0-3, code t in byte t) and hi (codes
// 4-7) as element-type integers (0 .. 255 are exact in bf16 and f16), two per
// register, code 0 in the low half of the first: one v_cvt_f32_ubyte<b> per
// code and one pack per pair.
template <typename T>
__device__ __forceinline__ uint4 bytes_as_elems(uint32_t lo, uint32_t hi) {
  const auto pack = [](float c0, float c1) -> uint32_t {
    if constexpr (IsBF16<T>::value)  // the top halves of the fp32 values (exact: <= 8 bits)
      return __builtin_amdgcn_perm(__float_as_uint(c1), __float_as_uint(c0), 0x07060302u);
    else
      return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(c0, c1));
  };
  const auto byte = [](uint32_t d, int b) -> float { return (float)((d >> (8 * b)) & 0xFFu); };
  uint4 r;
  r.x = pack(byte(lo, 0), byte(lo, 1));
  r.y = pack(byte(lo, 2), byte(lo, 3));
  r.z = pack(byte(hi, 0), byte(hi, 1));
  r.w = pack(byte(hi, 2), byte(hi, 3));
  return r;
}

// Workgroups are dispatched round-robin over the 8 XCDs (each with its own L2).
// Remap so that consecutive logical tiles -- which share operand panels -- run
// on the same XCD.
__device__ inline int xcd_remap(int w, int total) {
  const int per = total >> 3;
  if (w < (per << 3)) return (w & 7) * per + (w >> 3);
  return w;
}

// Logical tile -> (row block, column block): groups of 4 row blocks, row
// blocks fastest within a group, then column blocks. The tiles an XCD runs
// at once then span about 4 row blocks of A and a few column blocks of B,
// which its L2 serves to each other (a tall column of row blocks would
// stream all of A through it). With 4 or fewer row blocks this is plain
// column-major order.
__device__ inline void tile_coords(int tile, int tiles_m, int tiles_n, int& mi, int& ni) {
  constexpr int kGroupM = 4;
  const int gsz = kGroupM * tiles_n;
  const int grp = tile / gsz, within = tile % gsz;
  const int rows = tiles_m - grp * kGroupM < kGroupM ? tiles_m - grp * kGroupM : kGroupM;
  mi = grp * kGroupM + within % rows;
  ni = within / rows;
}

// 16-byte chunk of row `row` of a row-major matrix with leading dimension
// `ld`, starting at element k, read element by element; elements of rows at
// or past `rows` or at or past column `limit` are zero. The path for operands
// the buffer path cannot take (unaligned, or panels of 2 GiB and more).
template <typename T>
__device__ inline uint4 load_chunk(const T* __restrict__ base, int64_t row, int64_t rows,
                                   int64_t ld, int64_t k, int64_t limit) {
  constexpr int E = 16 / sizeof(T);
  const bool row_ok = row < rows;
  union {
    uint4 u;
    T e[E];
  } r;
  const T* p = base + (row_ok ? row : 0) * ld;
#pragma unroll
  for (int i = 0; i < E; i++) r.e[i] = (row_ok && k + i < limit) ? p[k + i] : T(0);
  return r.u;
}

// Raw buffer resources (CDNA "V#"): loads whose byte offset is at or past
// num_records return zero in hardware, so out-of-range rows and K/N tails cost
// no branch. dword3 0x00020000 selects the untyped 32-bit format used by raw
// buffer accesses on the gfx9 family.
constexpr uint32_t kOutOfRange = 0x80000000u;  // >= every num_records used below
// The base and size are workgroup-uniform; readfirstlane states that to the
// compiler, which otherwise may wrap every buffer access in a loop over the
// distinct descriptors of the wave.
__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
  const int32_t n = bytes < (int64_t)kOutOfRange ? (int32_t)bytes : (int32_t)(kOutOfRange - 1);
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  void* ub = reinterpret_cast<void*>(((uint64_t)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(ub, (short)0, __builtin_amdgcn_readfirstlane(n),
                                           0x00020000);
}
__device__ inline uint4 buffer_chunk(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}

// Chunk swizzles: 16-byte chunk c of LDS row r is stored at chunk position
// c ^ swz(r) so that the MFMA operand reads spread over the LDS banks. The LDS
// has 64 banks of 4 bytes (256 bytes); by the bank-conflict counter, a 16-byte
// read serves lanes 0-7 and 16-23 in one pass (then 8-15 and 24-31, ...), i.e.
// rows 0-7 of a 16-row operand block at chunks 4j + g and 4j + g + 1. Rows of
// 8 chunks (128 bytes) put row parity in the bank half, so c ^ (r & 7) covers
// the 16 bank groups; rows of 16 or more chunks need c ^ 2 (r & 7), which sends
// the two chunks to even and odd bank groups (c ^ (r & 7) would give both chunk
// sets the same 8 bank groups: a 2-way conflict on every read).
template <int RC>
__device__ inline int swz_k(int r) {  // [rows][RC >= 4 chunks] tiles
  // Rows of 4 chunks (64 bytes): rows r and r + 4 share bank groups, so bit 2
  // of the row picks the chunk pair.
  return RC >= 16 ? (r & 7) << 1 : RC == 8 ? r & 7 : ((r >> 2) & 1) << 1;
}
// (K, N) B tiles are read with ds_read_b64_tr_b16: lane group g reads k-rows
// 8g + (0..3) (plus 4 for the second half), 32 bytes each. One pass serves
// groups 0 and 1 (then 2 and 3), 8 rows. 256-byte rows (16 chunks): the row's
// low two bits and bit 3 pick one of 8 chunk pairs. 128-byte rows (8 chunks):
// row parity picks the bank half, so bits 1 and 3 pick one of 4 chunk pairs.
template <typename T, int CPR>
__device__ inline int swz_nn(int k) {  // [k][CPR chunks] tiles (B in (K, N) layout)
  if constexpr (sizeof(T) == 2 && CPR == 8)
    return (((k >> 1) & 1) << 1) | (((k >> 3) & 1) << 2);
  else if constexpr (sizeof(T) == 2)
    return (((k & 3) << 1) | (((k >> 3) & 1) << 3)) & (CPR - 1);
  else
    return (((k >> 2) & 3) << 2) & (CPR - 1);
}

// s_waitcnt immediate (gfx9 encoding): wait until at most `vm` vector-memory
// operations of this wave are outstanding and all LDS operations completed.
constexpr int waitcnt_vm_lgkm0(int vm) {
  return (vm & 0xF) | ((vm >> 4) << 14) | (0x7 << 4) | (0x0 << 8);
}

// One workgroup computes a BM x BN tile of C over the whole of K.
//   WM x WN compute waves own (BM / WM) x (BN / WN) sub-tiles; NW >= WM * WN
//   waves in total, the extra waves only load. PL: the loading waves issue
//   every load and the compute waves none (a wave whose load issue stalls on
//   a busy memory pipeline then holds up no matrix products); otherwise all
//   NW waves share the loads.
//   KB: bytes of each A / B row staged per pipeline stage (a multiple of 128).
//   NS: stages in the LDS ring. Operands move global -> LDS with buffer loads
//       that write LDS directly (no VGPR staging, no ds_write); NS - 1 stages
//       are in flight while one is computed. One barrier per stage.
// The pipeline shape never changes what an output element computes: every
// geometry issues the same chunk-steps in the same order (see file header).
// One stage of the LDS ring: the A tile and the B tile, separate arrays.
struct Slot {
  uint4* a;
  uint4* b;
};
// One stage of the quantized kernel's two-slot ring: the A tile, the B tile
// (codes as element-type integers) and the stage's scale/bias entries.
struct QSlot {
  uint4* a;
  uint4* b;
  unsigned short* s16;
  unsigned short* z16;
};

template <typename T, int BM, int BN, int WM, int WN, int NW, int KB, int NS, bool TB, int QB = 0,
          bool PL = false, bool PP = false>
struct GemmTile {
  static constexpr int NT = 64 * NW;
  static constexpr int CW = WM * WN;                  // compute waves
  static constexpr int EPC = 16 / sizeof(T);          // elements per 16-byte chunk
  static constexpr int RC = KB / 16;                  // chunks per tile row per stage
  static constexpr int EPS = KB / sizeof(T);          // elements of K per stage
  static constexpr int CS = KB / 64;                  // chunk-steps per stage
  static constexpr int WTM = BM / WM, WTN = BN / WN;  // wave tile
  static constexpr int FM = WTM / 16, FN = WTN / 16;  // 16x16 MFMA blocks per wave
  static constexpr int A_CH = BM * RC;                // chunks per stage
  static constexpr int B_CH = BN * RC;
  static constexpr int LA = (A_CH + NT - 1) / NT;     // chunks per thread per stage (VGPR path)
  static constexpr int LB = (B_CH + NT - 1) / NT;
  static constexpr int NN_CPR = BN * (int)sizeof(T) / 16;  // chunks per k-row, (K, N) B tile
  static constexpr int STAGE_CH = A_CH + B_CH;
  static constexpr int LDW = PL ? NW - WM * WN : NW;  // waves that issue loads
  static constexpr int DMA = STAGE_CH / 64 / LDW;     // 1 KB LDS-DMA loads per loading wave per stage
  static constexpr int CHAINS = sizeof(T) == 4 ? 2 : 1;    // fp32: chain per chunk-step parity
  static_assert(CW <= NW && FM >= 1 && FN >= 1 && WTM % 16 == 0 && WTN % 16 == 0, "geometry");
  // fp32 alternates two chains by chunk-step parity, so its stages hold an
  // even number of chunk-steps.
  static_assert(KB % 64 == 0 && CS % CHAINS == 0 && (KB >= 128 || sizeof(T) == 2), "stage bytes");
  static_assert(TB || (NN_CPR >= 1 && (NN_CPR & (NN_CPR - 1)) == 0), "bad (K,N) tile width");
  static constexpr int DMA_A = A_CH / 64 / LDW;     // of which A loads (the rest load B)
  static_assert(LDW >= 1, "PL needs loading waves");
  static_assert(A_CH % (64 * LDW) == 0 && B_CH % (64 * LDW) == 0, "stage must split into 1 KB loads");
  static_assert(NS >= 2 && NS <= 8 && DMA * (NS - 2) <= 63, "ring depth");

  const T* __restrict__ A;
  const T* __restrict__ B;
  int64_t M, N, K, m0, n0;
  int tid, wave, lane, g, r16, wm, wn;
  // Buffer path: the A panel (rows m0.. of A), the B panel (rows n0.. of an
  // (N, K) B, or columns n0.. of a (K, N) B); bytes past the valid rows are
  // outside num_records.
  __amdgpu_buffer_rsrc_t ra_src, rb_src;
  // This lane's element offsets, within a stage's A and B arrays, of the
  // operand chunk of chunk-step j for the wave's first 16-row (16-column)
  // block; further blocks add 16 rows. Swizzles depend on the row mod 8 only,
  // so they are the same for every block. The empty asm hides how the offsets
  // were computed, which keeps each LDS read a short address chain off its
  // array: the compiler then attributes every read to its ring slot and knows
  // it does not depend on DMA still landing in other slots.
  int a_off[CS], b_off[CS];

  __device__ __forceinline__ void init_lds_offsets() {
#pragma unroll
    for (int j = 0; j < CS; j++) {
      int ao = (wm * WTM + r16) * RC + ((4 * j + g) ^ swz_k<RC>(r16));
      int bo = (wn * WTN + r16) * RC + ((4 * j + g) ^ swz_k<RC>(r16));
      asm("" : "+v"(ao));
      asm("" : "+v"(bo));
      a_off[j] = ao;
      b_off[j] = bo;
    }
  }

  __device__ __forceinline__ void init_buffers() {
    constexpr int64_t E = sizeof(T);
    ra_src = make_rsrc(A + m0 * K, min((int64_t)BM, M - m0) * K * E);
    if constexpr (TB)
      rb_src = make_rsrc(B + n0 * K, min((int64_t)BN, N - n0) * K * E);
    else
      rb_src = make_rsrc(B + n0, (K * N - n0) * E);
  }

  // Per-lane DMA addressing, fixed for the whole K loop. Load i of this wave
  // fills the 64 LDS chunks starting at chunk blk(i) * 64, one per lane; LDS
  // rows are swizzled, so the lane's position holds logical chunk
  // phys ^ swz(row). For stage s the lane loads panel byte offset
  // base[i] + s * step (step = EPS elements along K, or EPS rows of a (K, N)
  // B), provided its K index kidx[i] + s * EPS is below K (and, for a (K, N)
  // B, its column is inside N); otherwise it loads zeros.
  uint32_t dma_base[DMA];
  int32_t dma_kidx[DMA];

  __device__ __forceinline__ int dma_blk(int i) const {
    const int lw = PL ? wave - CW : wave;  // index among the loading waves
    return i < DMA_A ? i * LDW + lw : (i - DMA_A) * LDW + lw;
  }

  // Load addressing of 1 KB block `blk` of a stage's A (is_a) or B region:
  // this lane's panel byte offset for stage 0 and the K index that decides
  // whether it is inside the operand.
  __device__ __forceinline__ void dma_addr(bool is_a, int blk, uint32_t& base, int32_t& kidx) const {
    constexpr uint32_t E = sizeof(T);
    const int p = blk * 64 + lane;  // chunk position within the A or B region
    if (is_a || TB) {
      const int r = p / RC, c = (p % RC) ^ swz_k<RC>(r);
      base = (uint32_t)(r * K + c * EPC) * E;
      kidx = c * EPC;
    } else {
      const int kr = p / NN_CPR, c = (p % NN_CPR) ^ swz_nn<T, NN_CPR>(kr);
      const int n = c * EPC;
      base = (uint32_t)(kr * N + n) * E;
      // A column outside N never loads: push its K index out of range.
      kidx = (n0 + n < N) ? kr : INT32_MAX / 2;
    }
  }

  __device__ __forceinline__ void init_dma() {
#pragma unroll
    for (int i = 0; i < DMA; i++) dma_addr(i < DMA_A, dma_blk(i), dma_base[i], dma_kidx[i]);
  }

  // Issue this wave's LDS-DMA loads of stage s into `slot`.
  __device__ __forceinline__ void dma(int64_t s, Slot slot) const {
    constexpr uint32_t E = sizeof(T);
    const int32_t kleft = (int32_t)(K - s * EPS);  // K elements from this stage on
    const uint32_t a_step = (uint32_t)(s * EPS) * E;
    const uint32_t b_step = TB ? a_step : (uint32_t)(s * EPS * N) * E;
#pragma unroll
    for (int i = 0; i < DMA; i++) {
      const bool is_a = i < DMA_A;
      lds_void_t* dst = (lds_void_t*)((is_a ? slot.a : slot.b) + dma_blk(i) * 64);
      const uint32_t off = dma_kidx[i] < kleft ? dma_base[i] + (is_a ? a_step : b_step) : kOutOfRange;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(is_a ? ra_src : rb_src, dst, 16, off, 0, 0, 0);
    }
  }

  // Register-staged loads for operands the buffer path cannot take.
  __device__ __forceinline__ void gload_slow(int64_t s, uint4* ra, uint4* rb) const {
    const int64_t k0 = s * EPS;
#pragma unroll
    for (int i = 0; i < LA; i++) {
      const int q = tid + i * NT;
      if (A_CH % NT == 0 || q < A_CH)
        ra[i] = load_chunk<T>(A, m0 + q / RC, M, K, k0 + (q % RC) * EPC, K);
    }
#pragma unroll
    for (int i = 0; i < LB; i++) {
      const int q = tid + i * NT;
      if (B_CH % NT == 0 || q < B_CH) {
        if constexpr (TB)
          rb[i] = load_chunk<T>(B, n0 + q / RC, N, K, k0 + (q % RC) * EPC, K);
        else
          rb[i] = load_chunk<T>(B, k0 + q / NN_CPR, K, N, n0 + (q % NN_CPR) * EPC, N);
      }
    }
  }

  __device__ __forceinline__ void sstore(Slot sl, const uint4* ra, const uint4* rb) const {
    uint4* As = sl.a;
    uint4* Bs = sl.b;
#pragma unroll
    for (int i = 0; i < LA; i++) {
      const int q = tid + i * NT;
      if (A_CH % NT == 0 || q < A_CH) {
        const int r = q / RC, c = q % RC;
        As[r * RC + (c ^ swz_k<RC>(r))] = ra[i];
      }
    }
#pragma unroll
    for (int i = 0; i < LB; i++) {
      const int q = tid + i * NT;
      if (B_CH % NT == 0 || q < B_CH) {
        if constexpr (TB) {
          const int r = q / RC, c = q % RC;
          Bs[r * RC + (c ^ swz_k<RC>(r))] = rb[i];
        } else {
          const int r = q / NN_CPR, c = q % NN_CPR;
          Bs[r * NN_CPR + (c ^ swz_nn<T, NN_CPR>(r))] = rb[i];
        }
      }
    }
  }

  // B operand chunk for chunk-step j of the 16-column block at tile column nb.
  __device__ __forceinline__ uint4 load_b(const uint4* Bs, int j, int nb) const {
    if constexpr (TB) {
      return Bs[b_off[j] + nb * RC];
    } else if constexpr (sizeof(T) == 2) {
      // ds_read_tr16_b64: in each 16-lane group, lane i receives element
      // (row 4t + i/4, column i%4) of the 16 x (4 x 16-bit) rows addressed by
      // the group's lanes. Lane r16 addresses k-row kb + r16/4 at column
      // nb + 4 * (r16 % 4), so lane i receives B[kb + t][nb + i], t = 0..3.
      uint2 h[2];
#pragma unroll
      for (int half = 0; half < 2; half++) {
        const int kr = 32 * j + 8 * g + 4 * half + (r16 >> 2);
        const int col = wn * WTN + nb + 4 * (r16 & 3);
        const int chunk = (col >> 3) ^ swz_nn<T, NN_CPR>(kr);
        const char* addr =
            reinterpret_cast<const char*>(Bs) + (kr * NN_CPR + chunk) * 16 + (col & 7) * 2;
        i16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(addr));
        h[half] = __builtin_bit_cast(uint2, v);
      }
      return make_uint4(h[0].x, h[0].y, h[1].x, h[1].y);
    } else {
      // fp32: element t of the chunk is B[16j + 4g + t][nb + r16].
      const float* Bf = reinterpret_cast<const float*>(Bs);
      uint32_t e[4];
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const int kr = 16 * j + 4 * g + t;
        const int col = wn * WTN + nb + r16;
        const int chunk = (col >> 2) ^ swz_nn<T, NN_CPR>(kr);
        e[t] = __float_as_uint(Bf[(kr * NN_CPR + chunk) * 4 + (col & 3)]);
      }
      return make_uint4(e[0], e[1], e[2], e[3]);
    }
  }

  __device__ __forceinline__ void read_operands(Slot sl, int j, uint4 (&av)[FM],
                                                uint4 (&bv)[FN]) const {
    const uint4* As = sl.a;
    const uint4* Bs = sl.b;
#pragma unroll
    for (int i = 0; i < FM; i++) av[i] = As[a_off[j] + i * 16 * RC];
#pragma unroll
    for (int jn = 0; jn < FN; jn++) bv[jn] = load_b(Bs, j, jn * 16);
  }

  // All CS chunk-steps of the stage held in LDS at `As`, for every block of
  // this wave; operands of step j + 1 are read while step j's MFMAs run.
  __device__ __forceinline__ void compute_full(Slot As,
                                               f32x4_t (&acc)[CHAINS][FM][FN]) const {
    uint4 av[2][FM], bv[2][FN];
    read_operands(As, 0, av[0], bv[0]);
#pragma unroll
    for (int j = 0; j < CS; j++) {
      if (j + 1 < CS) read_operands(As, j + 1, av[(j + 1) & 1], bv[(j + 1) & 1]);
#pragma unroll
      for (int i = 0; i < FM; i++)
#pragma unroll
        for (int jn = 0; jn < FN; jn++)
          acc[j % CHAINS][i][jn] =
              chunk_step(T(0), av[j & 1][i], bv[j & 1][jn], acc[j % CHAINS][i][jn]);
    }
  }

  // The first `steps` (< CS) chunk-steps of the last stage.
  __device__ __forceinline__ void compute_part(Slot As, int steps,
                                               f32x4_t (&acc)[CHAINS][FM][FN]) const {
#pragma unroll
    for (int j = 0; j < CS - 1; j++) {
      if (j < steps) {
        uint4 av[FM], bv[FN];
        read_operands(As, j, av, bv);
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
          for (int jn = 0; jn < FN; jn++)
            acc[j % CHAINS][i][jn] = chunk_step(T(0), av[i], bv[jn], acc[j % CHAINS][i][jn]);
      }
    }
  }

  __device__ __forceinline__ void compute(Slot As, int steps,
                                          f32x4_t (&acc)[CHAINS][FM][FN]) const {
    if (steps == CS)
      compute_full(As, acc);
    else if (steps > 0)
      compute_part(As, steps, acc);
  }

  __device__ __forceinline__ int steps_of(int64_t nsteps, int64_t s) const {
    const int64_t left = nsteps - s * CS;
    return left <= 0 ? 0 : (left < CS ? (int)left : CS);
  }

  // Buffer path. The ring slots are distinct LDS arrays indexed at compile
  // time, which lets the compiler see that reading slot u does not depend on
  // the DMA still landing in the other slots. That relies on the per-array
  // alias scopes the compiler gives LDS accesses, so LDS pointers here carry
  // no __restrict__ (its scopes would replace the per-array ones) and reads
  // stay a short address chain off their array (see init_lds_offsets); either
  // mistake makes every read wait for all DMA in flight. The waits are explicit: before
  // computing stage s, this wave's loads of stages s+1 .. s+NS-2 may still be
  // in flight, then a barrier makes every wave's part of stage s visible and
  // guarantees the slot about to be refilled is no longer read.
  // The loop has no branches: whole rounds of NS stages, every stage computed
  // in full. Past K the stages hold zeros, which change no bit (file header).
  // A workgroup whose waves all compute runs only this loop: a wave whose
  // sub-tile lies outside C computes too and then stores nothing.
  template <bool COMPUTE, typename Slots>
  __device__ __forceinline__ void dma_rounds(const Slots& slots, int64_t nst,
                                             f32x4_t (&acc)[CHAINS][FM][FN]) const {
    for (int64_t s0 = 0; s0 < nst; s0 += NS) {
#pragma unroll
      for (int u = 0; u < NS; u++) {
        __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(DMA * (NS - 2)));
        asm volatile("s_barrier" ::: "memory");
        dma(s0 + u + NS - 1, slots((u + NS - 1) % NS));
        if constexpr (COMPUTE) compute_full(slots(u), acc);
      }
    }
  }

  template <typename Slots>
  __device__ __forceinline__ void main_loop_dma(const Slots& slots, int64_t nst, bool computes,
                                                f32x4_t (&acc)[CHAINS][FM][FN]) const {
    if constexpr (PL) {
      // The same rounds split by role: a loading wave waits for its own
      // loads of stage s (those of s+1 .. s+NS-2 may stay in flight) before
      // the barrier and refills the freed slot after it; a compute wave's
      // LDS reads of the previous stage have returned before it arrives.
      if (wave >= CW) {
#pragma unroll
        for (int u = 0; u < NS - 1; u++) dma(u, slots(u));
        for (int64_t s0 = 0; s0 < nst; s0 += NS) {
#pragma unroll
          for (int u = 0; u < NS; u++) {
            __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(DMA * (NS - 2)));
            asm volatile("s_barrier" ::: "memory");
            dma(s0 + u + NS - 1, slots((u + NS - 1) % NS));
          }
        }
      } else {
        for (int64_t s0 = 0; s0 < nst; s0 += NS) {
#pragma unroll
          for (int u = 0; u < NS; u++) {
            __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(63));
            asm volatile("s_barrier" ::: "memory");
            if (computes) compute_full(slots(u), acc);
          }
        }
      }
      return;
    }
#pragma unroll
    for (int u = 0; u < NS - 1; u++) dma(u, slots(u));
    if (NW == CW || computes)
      dma_rounds<true>(slots, nst, acc);
    else
      dma_rounds<false>(slots, nst, acc);
  }

  // ---- Ping-pong schedule (PP). The compute waves form two groups, waves
  // 0 .. CW/2 - 1 and CW/2 .. CW - 1; the hardware places wave w and wave
  // w + 4 of a workgroup on the same SIMD, so every SIMD holds waves of both
  // groups (CW/2 a multiple of 4). Chunk-step q takes two phases, separated
  // by workgroup barriers: group 0 reads q's operands from LDS in phase 2q
  // and runs q's MFMAs in phase 2q + 1; group 1 does the same one phase
  // later. In every phase one group's waves issue matrix products while the
  // other group's read LDS, so a SIMD's matrix core does not wait for its
  // own waves' operand reads, and each wave holds the operands of one
  // chunk-step only (16 waves of 64 x 64 wave tiles fit 128 registers). The
  // MFMAs per element and their order are those of every other footprint.
  // Loads: every stage holds one chunk-step; group 0 loads the A tiles and
  // group 1 the B tiles of the stage NS - 1 ahead, each right after issuing
  // its products (a load issue that stalls on a busy memory pipeline then
  // delays no operand read and no matrix product).
  static constexpr int PPG = CW / 2;                            // compute waves per group
  static constexpr int DMA_PA = PP ? A_CH / 64 / PPG : 1;  // A loads per group-0 wave per stage
  static constexpr int DMA_PB = PP ? B_CH / 64 / PPG : 1;  // B loads per group-1 wave per stage
  static constexpr int PPD = DMA_PA > DMA_PB ? DMA_PA : DMA_PB;
  static_assert(!PP || (!PL && CS == 1 && NS >= 3 && PPG % 4 == 0 && A_CH % (64 * PPG) == 0 &&
                        B_CH % (64 * PPG) == 0 && PPD * (NS - 2) <= 63),
                "ping-pong geometry");
  uint32_t pp_base[PPD];
  int32_t pp_kidx[PPD];

  __device__ __forceinline__ void init_dma_pp(int grp, int gw) {
    const int nd = grp == 0 ? DMA_PA : DMA_PB;
#pragma unroll
    for (int i = 0; i < PPD; i++)
      if (i < nd) dma_addr(grp == 0, i * PPG + gw, pp_base[i], pp_kidx[i]);
  }

  template <bool IS_A>
  __device__ __forceinline__ void dma_pp(int64_t s, Slot slot, int gw) const {
    constexpr uint32_t E = sizeof(T);
    constexpr int ND = IS_A ? DMA_PA : DMA_PB;
    const int32_t kleft = (int32_t)(K - s * EPS);
    const uint32_t step = (IS_A || TB) ? (uint32_t)(s * EPS) * E : (uint32_t)(s * EPS * N) * E;
#pragma unroll
    for (int i = 0; i < ND; i++) {
      lds_void_t* dst = (lds_void_t*)((IS_A ? slot.a : slot.b) + (i * PPG + gw) * 64);
      const uint32_t off = pp_kidx[i] < kleft ? pp_base[i] + step : kOutOfRange;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(IS_A ? ra_src : rb_src, dst, 16, off, 0, 0, 0);
    }
  }

  // Operand reads of the ping-pong schedule, issued as ds_read instructions
  // from one per-lane byte offset per operand block column plus the slot's
  // LDS address (a scalar, added right before the reads): the compiler would
  // otherwise keep a VGPR address per slot and block, which does not fit the
  // registers of 16 waves. The reads are waited for explicitly
  // (lgkmcnt(0) before the barrier that closes the read phase); the values
  // are first used after that barrier.
  uint32_t pa_off[CS], pb_off[CS][FN];

  __device__ __forceinline__ void init_lds_offsets_pp() {
#pragma unroll
    for (int j = 0; j < CS; j++) {
      pa_off[j] = (uint32_t)((wm * WTM + r16) * RC + ((4 * j + g) ^ swz_k<RC>(r16))) * 16;
#pragma unroll
      for (int jn = 0; jn < FN; jn++) {
        if constexpr (TB) {
          pb_off[j][jn] =
              (uint32_t)((wn * WTN + jn * 16 + r16) * RC + ((4 * j + g) ^ swz_k<RC>(r16))) * 16;
        } else {
          // As load_b: lane r16 of group g addresses k-row 32 j + 8 g + r16 / 4
          // at column 4 (r16 % 4) of the block; the second half (4 rows on)
          // has the same swizzle, so it is an immediate offset.
          const int kr = 32 * j + 8 * g + (r16 >> 2);
          const int col = wn * WTN + jn * 16 + 4 * (r16 & 3);
          const int chunk = (col >> 3) ^ swz_nn<T, NN_CPR>(kr);
          pb_off[j][jn] = (uint32_t)((kr * NN_CPR + chunk) * 16 + (col & 7) * 2);
        }
      }
    }
  }

  __device__ __forceinline__ static uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(lds_void_t*)p;
  }

  __device__ __forceinline__ void read_operands_pp(Slot sl, int j, uint4 (&av)[FM],
                                                   uint4 (&bv)[FN]) const {
    static_assert(sizeof(T) == 2, "ping-pong: 16-bit element types");
    uint32_t aa;
    asm volatile("v_add_u32 %0, %1, %2" : "=v"(aa) : "s"(lds_addr(sl.a)), "v"(pa_off[j]));
#pragma unroll
    for (int i = 0; i < FM; i++) {
      u32x4_t v;
      asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(aa), "n"(i * 16 * RC * 16));
      av[i] = __builtin_bit_cast(uint4, v);
    }
    const uint32_t bs = lds_addr(sl.b);
#pragma unroll
    for (int jn = 0; jn < FN; jn++) {
      uint32_t ba;
      asm volatile("v_add_u32 %0, %1, %2" : "=v"(ba) : "s"(bs), "v"(pb_off[j][jn]));
      if constexpr (TB) {
        u32x4_t v;
        asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(ba));
        bv[jn] = __builtin_bit_cast(uint4, v);
      } else {
        u32x2_t h0, h1;
        asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(h0) : "v"(ba));
        asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(h1) : "v"(ba), "n"(4 * NN_CPR * 16));
        bv[jn] = make_uint4(h0.x, h0.y, h1.x, h1.y);
      }
    }
  }

  // Waits for this wave's operand reads; tying the registers to the wait
  // keeps every use after it.
  __device__ __forceinline__ static void wait_operands(uint4 (&av)[FM], uint4 (&bv)[FN]) {
    u32x4_t a[FM], b[FN];
#pragma unroll
    for (int i = 0; i < FM; i++) a[i] = __builtin_bit_cast(u32x4_t, av[i]);
#pragma unroll
    for (int jn = 0; jn < FN; jn++) b[jn] = __builtin_bit_cast(u32x4_t, bv[jn]);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int i = 0; i < FM; i++) {
      asm volatile("" : "+v"(a[i]));
      av[i] = __builtin_bit_cast(uint4, a[i]);
    }
#pragma unroll
    for (int jn = 0; jn < FN; jn++) {
      asm volatile("" : "+v"(b[jn]));
      bv[jn] = __builtin_bit_cast(uint4, b[jn]);
    }
  }

  __device__ __forceinline__ static void pp_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  }

  __device__ __forceinline__ void pp_mfma(const uint4 (&av)[FM], const uint4 (&bv)[FN],
                                          f32x4_t (&acc)[CHAINS][FM][FN]) const {
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
      for (int jn = 0; jn < FN; jn++) acc[0][i][jn] = chunk_step(T(0), av[i], bv[jn], acc[0][i][jn]);
  }

  // One group's rounds (GRP 0 or 1; COMPUTE false for a wave whose sub-tile
  // lies outside C: it keeps the barriers and its share of the loads). Each
  // group runs a straight sequence of phases of its own, so its operands and
  // accumulators stay in the same registers from phase to phase. Phase p
  // opens with barrier B_p; stage s (= chunk-step s) is first read after
  // B_2s, and a wave that loads part of it waits for its own loads of it
  // before that barrier. Group 0 has issued the A tiles of stages up to
  // s + NS - 2 by then (in phase 2s - 1), group 1 the B tiles of stages up
  // to s + NS - 3 (in phase 2s - 2; its loads of phase 2s follow B_2s).
  // Stage s + NS - 1 refills the slot of stage s - 1, whose last reads
  // (group 1, phase 2s - 1) are complete before B_2s.
  template <int GRP, bool COMPUTE, typename Slots>
  __device__ __forceinline__ void pp_rounds(const Slots& slots, int64_t nst, int gw,
                                            f32x4_t (&acc)[CHAINS][FM][FN]) const {
    uint4 av[FM], bv[FN];
    if constexpr (GRP == 1) {
      __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(DMA_PB * (NS - 2)));
      pp_barrier();  // B_0: group 0 reads chunk-step 0
    }
    for (int64_t s0 = 0; s0 < nst; s0 += NS) {
#pragma unroll
      for (int u = 0; u < NS; u++) {
        if constexpr (GRP == 0) {
          // B_2s: read chunk-step s; B_2s+1: its products, then load the A
          // tiles of stage s + NS - 1.
          __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(DMA_PA * (NS - 2)));
          pp_barrier();
          if constexpr (COMPUTE) {
            read_operands_pp(slots(u), 0, av, bv);
            wait_operands(av, bv);
          }
          __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(63));
          pp_barrier();
          if constexpr (COMPUTE) pp_mfma(av, bv, acc);
          dma_pp<true>(s0 + u + NS - 1, slots((u + NS - 1) % NS), gw);
        } else {
          // B_2s+1: read chunk-step s; B_2s+2: its products, then load the B
          // tiles of stage s + NS - 1. Stage s + 1's B tiles must have landed
          // before B_2s+2.
          __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(63));
          pp_barrier();
          if constexpr (COMPUTE) {
            read_operands_pp(slots(u), 0, av, bv);
            wait_operands(av, bv);
          }
          __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(DMA_PB * (NS - 3)));
          pp_barrier();
          if constexpr (COMPUTE) pp_mfma(av, bv, acc);
          dma_pp<false>(s0 + u + NS - 1, slots((u + NS - 1) % NS), gw);
        }
      }
    }
    if constexpr (GRP == 0) {
      __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(63));
      pp_barrier();  // B_2Q: group 1's last products
    }
  }

  template <typename Slots>
  __device__ __forceinline__ void main_loop_pp(const Slots& slots, int64_t nst, bool computes,
                                               f32x4_t (&acc)[CHAINS][FM][FN]) {
    static_assert(CHAINS == 1, "ping-pong: 16-bit element types");
    const int grp = wave < PPG ? 0 : 1;
    const int gw = wave - grp * PPG;
    init_dma_pp(grp, gw);
    init_lds_offsets_pp();
    if (grp == 0) {
#pragma unroll
      for (int u = 0; u < NS - 1; u++) dma_pp<true>(u, slots(u), gw);
      if (computes) pp_rounds<0, true>(slots, nst, gw, acc);
      else pp_rounds<0, false>(slots, nst, gw, acc);
    } else {
#pragma unroll
      for (int u = 0; u < NS - 1; u++) dma_pp<false>(u, slots(u), gw);
      if (computes) pp_rounds<1, true>(slots, nst, gw, acc);
      else pp_rounds<1, false>(slots, nst, gw, acc);
    }
  }

  // ---- Affine-quantized B (QB bits per weight; 16-bit elements only).
  // Weight element k of row n is bits QB * (k % (32 / QB)) of uint32 word
  // k / (32 / QB) of that row (little-endian packing) and stands for
  // v = scale * q + bias with the scale and bias of its group k / group. The
  // product with the activation row x is formed per group, in fp32:
  //   P = sum_{k in group} x_k * q_k   (q_k as an element-type integer; exact
  //                                     products, fp32 MFMA sums)
  //   X = sum_{k in group} x_k         (the same MFMA against ones)
  //   acc = fma(scale, P, acc); acc = fma(bias, X, acc)
  // over groups in ascending order, acc starting at +0.0; P and X run the
  // group's chunk-steps (32 elements of K each, the dense kernel's lane
  // layout) from +0.0. That is sum_k x_k * (scale * q_k + bias) with fp32
  // roundings only -- the reference's fp32 product with its fp32 weights to
  // within fp32 accumulation error -- and a fixed sequence per output element.
  static constexpr int QP = NW == 8 ? 2 : 4;  // stages of loads in flight (registers)
  // Threads that load and stage the quantized operands: the waves that do
  // not compute, when there are such (the computing waves then only read LDS
  // and run the MFMAs and folds), else all.
  static constexpr int QNT = (QB != 0 && NW > CW) ? 64 * (NW - CW) : NT;
  static constexpr int QLA = (A_CH + QNT - 1) / QNT;
  static constexpr int GPS = EPS / 32;        // most groups that end in one stage
  static constexpr int QSB = BN * GPS;        // scale/bias entries staged per stage
  static constexpr int LSB = (QSB + QNT - 1) / QNT;
  // B is loaded in units of CPT consecutive chunks of a row: one aligned
  // dword (2 and 4 bits) or dword pair (8 bits) per unit.
  static constexpr int CPT = QB == 2 ? 2 : 1;  // (1 for the dense kernels, QB = 0)
  static constexpr int RCU = RC / CPT;        // units per tile row per stage
  static constexpr int B_U = BN * RCU;        // units per stage
  static constexpr int LBU = (B_U + QNT - 1) / QNT;
  static_assert(QB == 0 || (TB && sizeof(T) == 2 && (QB == 2 || QB == 4 || QB == 8)),
                "quantized B: (N, K) layout, 16-bit elements, 2/4/8 bits");
  static_assert(RC % CPT == 0, "stage holds whole units");
  // Staged loads are kept exactly as loaded -- no arithmetic on them, not
  // even a zero extension -- until the stage is stored: any would make the
  // wave wait for every load in flight, the prefetched stages with them.
  using QWord = typename std::conditional<QB == 8, uint2, uint32_t>::type;
  struct QStage {
    uint4 a[QLA];
    QWord w[LBU];                     // packed codes of unit i
    unsigned short sc[LSB], zb[LSB];  // scale and bias of entry i, element bits
  };
  __amdgpu_buffer_rsrc_t rs_src, rz_src;
  int64_t qrow_bytes;
  int qgshift;
  // Per-thread load addressing, fixed for the whole K loop: byte offsets of
  // the thread's A chunks, B units and scale/bias entries for stage 0, and
  // the K index (or group within the stage) that decides whether a load is
  // inside the operand. Stage s adds s * EPS elements (s * EPS * QB / 8 bytes
  // of B, glo(s) groups).
  uint32_t qa_off[QLA], qb_off[LBU], qs_off[LSB];
  int32_t qa_k[QLA], qb_k[LBU], qs_gi[LSB];
  int qtid;  // index among the QNT loading threads

  __device__ __forceinline__ void init_buffers_q(const GemmArgs& p) {
    constexpr int64_t E = sizeof(T);
    ra_src = make_rsrc(A + m0 * K, min((int64_t)BM, M - m0) * K * E);
    qrow_bytes = K * QB / 8;
    const int64_t rows = min((int64_t)BN, N - n0);
    rb_src = make_rsrc(reinterpret_cast<const char*>(B) + n0 * qrow_bytes, rows * qrow_bytes);
    qgshift = p.qgroup_shift;
    const int64_t G = K >> qgshift;  // groups per row
    rs_src = make_rsrc(static_cast<const T*>(p.qs) + n0 * G, rows * G * E);
    rz_src = make_rsrc(static_cast<const T*>(p.qz) + n0 * G, rows * G * E);
#pragma unroll
    for (int i = 0; i < QLA; i++) {
      const int q = qtid + i * QNT, r = q / RC, c = q % RC;
      qa_off[i] = (uint32_t)((r * K + c * EPC) * E);
      qa_k[i] = (A_CH % QNT == 0 || q < A_CH) ? c * EPC : INT32_MAX;
    }
#pragma unroll
    for (int i = 0; i < LBU; i++) {
      const int q = qtid + i * QNT, r = q / RCU, c = (q % RCU) * CPT;
      qb_off[i] = (uint32_t)(r * qrow_bytes + c * EPC * QB / 8);
      qb_k[i] = (B_U % QNT == 0 || q < B_U) ? c * EPC : INT32_MAX;
    }
#pragma unroll
    for (int i = 0; i < LSB; i++) {
      const int e = qtid + i * QNT, r = e / GPS, gi = e % GPS;
      qs_off[i] = (uint32_t)((r * G + gi) * E);
      qs_gi[i] = (QSB % QNT == 0 || e < QSB) ? gi : INT32_MAX;
    }
  }

  // Groups ending in stage s: [glo(s), glo(s + 1)). Stage and group sizes are
  // powers of two, so one divides the other.
  __device__ __forceinline__ int64_t glo(int64_t s) const { return (s * EPS) >> qgshift; }

  __device__ __forceinline__ void qload(int64_t s, QStage& st) const {
    constexpr uint32_t E = sizeof(T);
    const int32_t kleft = (int32_t)(K - s * EPS);  // K elements from this stage on
    const uint32_t a_step = (uint32_t)(s * EPS) * E;
    const uint32_t b_step = (uint32_t)(s * EPS) * QB / 8;
#pragma unroll
    for (int i = 0; i < QLA; i++)
      st.a[i] = buffer_chunk(ra_src, qa_k[i] < kleft ? qa_off[i] + a_step : kOutOfRange);
#pragma unroll
    for (int i = 0; i < LBU; i++) {
      const uint32_t wo = qb_k[i] < kleft ? qb_off[i] + b_step : kOutOfRange;
      if constexpr (QB == 8)
        st.w[i] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rb_src, (int)wo, 0, 0));
      else
        st.w[i] = __builtin_amdgcn_raw_buffer_load_b32(rb_src, (int)wo, 0, 0);
    }
    const int64_t g0 = glo(s);
    const int32_t gn = (int32_t)(glo(s + 1) - g0);  // groups ending in this stage
    const int32_t gleft = (int32_t)((K >> qgshift) - g0);
    const uint32_t s_step = (uint32_t)g0 * E;
#pragma unroll
    for (int i = 0; i < LSB; i++) {
      const bool in = qs_gi[i] < gn && qs_gi[i] < gleft;
      const uint32_t go = in ? qs_off[i] + s_step : kOutOfRange;
      st.sc[i] = __builtin_amdgcn_raw_buffer_load_b16(rs_src, (int)go, 0, 0);
      st.zb[i] = __builtin_amdgcn_raw_buffer_load_b16(rz_src, (int)go, 0, 0);
    }
  }

  __device__ __forceinline__ static float bits_to_f32(uint32_t b16) {
    return Elem<T>::to_f32(__builtin_bit_cast(T, (unsigned short)b16));
  }

  // Two integer codes (0 .. 255, exact in bf16 and f16) as a packed pair of
  // element-type values, low half first.
  __device__ __forceinline__ static uint32_t pack_codes(float c0, float c1) {
    if constexpr (IsBF16<T>::value)  // the top halves of the fp32 values (exact: <= 8 bits)
      return __builtin_amdgcn_perm(__float_as_uint(c1), __float_as_uint(c0), 0x07060302u);
    else
      return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(c0, c1));
  }

  // Codes of unit st.w[i] spread one per byte: byte b of d[j] holds code
  // b * SPREAD + j (2 and 4 bits), or byte b of word j holds code 4 j + b (8 bits).
  static constexpr int SPREAD = (QB == 8 || QB == 0) ? 1 : 8 / QB;
  static constexpr int ND = QB == 8 ? 2 : SPREAD;
  __device__ __forceinline__ static void spread_codes(QWord w, uint32_t (&d)[ND]) {
    if constexpr (QB == 8) {
      d[0] = w.x;
      d[1] = w.y;
    } else {
      constexpr uint32_t M = QB == 4 ? 0x0F0F0F0Fu : 0x03030303u;
#pragma unroll
      for (int j = 0; j < ND; j++) d[j] = (w >> (QB * j)) & M;
      // Opaque to the compiler: otherwise it folds the mask and the byte
      // select of code_at into one bit-field extract per code followed by a
      // byte-0 conversion (two instructions); kept apart, each code converts
      // with one v_cvt_f32_ubyte<b> (1-3 % faster at 256 rows, same bits).
#pragma unroll
      for (int j = 0; j < ND; j++) asm volatile("" : "+v"(d[j]));
    }
  }
  __device__ __forceinline__ static float code_at(const uint32_t (&d)[ND], int i) {
    const int j = QB == 8 ? i / 4 : i % SPREAD, b = QB == 8 ? i % 4 : i / SPREAD;
    return (float)((d[j] >> (8 * b)) & 0xFFu);  // v_cvt_f32_ubyte<b>
  }

  // Stage st into LDS: A as loaded, B's codes as element-type integers in the
  // dense (N, K) tile layout, and the stage's scale/bias entries.
  __device__ __forceinline__ void qstore(QSlot sl, const QStage& st) const {
#pragma unroll
    for (int i = 0; i < QLA; i++) {
      const int q = qtid + i * QNT;
      if (A_CH % QNT == 0 || q < A_CH) {
        const int r = q / RC, c = q % RC;
        sl.a[r * RC + (c ^ swz_k<RC>(r))] = st.a[i];
      }
    }
#pragma unroll
    for (int i = 0; i < LBU; i++) {
      const int q = qtid + i * QNT;
      if (B_U % QNT == 0 || q < B_U) {
        const int r = q / RCU, c = (q % RCU) * CPT;
        if constexpr (QB == 4) {
          // One unit is one chunk: eight codes, two per conversion.
          sl.b[r * RC + (c ^ swz_k<RC>(r))] = codes_as_elems<T>(st.w[i]);
          continue;
        }
        uint32_t d[ND];
        spread_codes(st.w[i], d);
#pragma unroll
        for (int cc = 0; cc < CPT; cc++) {
          uint4 v;
          v.x = pack_codes(code_at(d, 8 * cc + 0), code_at(d, 8 * cc + 1));
          v.y = pack_codes(code_at(d, 8 * cc + 2), code_at(d, 8 * cc + 3));
          v.z = pack_codes(code_at(d, 8 * cc + 4), code_at(d, 8 * cc + 5));
          v.w = pack_codes(code_at(d, 8 * cc + 6), code_at(d, 8 * cc + 7));
          sl.b[r * RC + ((c + cc) ^ swz_k<RC>(r))] = v;
        }
      }
    }
#pragma unroll
    for (int i = 0; i < LSB; i++) {
      const int e = qtid + i * QNT;
      if (QSB % QNT == 0 || e < QSB) {
        sl.s16[e] = st.sc[i];
        sl.z16[e] = st.zb[i];
      }
    }
  }

  // Fold group gi of the stage in `sl` (its scale and bias per column) into
  // acc; with `restart`, P and X start over from +0.0 (otherwise the next
  // group's first chunk-step starts them).
  __device__ __forceinline__ void q_fold(QSlot sl, int gi, bool restart, f32x4_t (&acc)[FM][FN],
                                         f32x4_t (&P)[FM][FN], f32x4_t (&X)[FM]) const {
#pragma unroll
    for (int jn = 0; jn < FN; jn++) {
      const int at = (wn * WTN + jn * 16 + r16) * GPS + gi;
      const float sc = bits_to_f32(sl.s16[at]), zb = bits_to_f32(sl.z16[at]);
#pragma unroll
      for (int i = 0; i < FM; i++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
          acc[i][jn][e] = __builtin_fmaf(sc, P[i][jn][e], acc[i][jn][e]);
          acc[i][jn][e] = __builtin_fmaf(zb, X[i][e], acc[i][jn][e]);
        }
    }
    if (restart) {
#pragma unroll
      for (int i = 0; i < FM; i++) {
        X[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int jn = 0; jn < FN; jn++) P[i][jn] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      }
    }
  }

  // One chunk-step into P and X; `first` (the group's first chunk-step)
  // starts them from +0.0.
  __device__ __forceinline__ void q_mfma(const uint4 (&av)[FM], const uint4 (&bv)[FN], bool first,
                                         f32x4_t (&P)[FM][FN], f32x4_t (&X)[FM]) const {
    constexpr uint32_t ONE = IsBF16<T>::value ? 0x3F803F80u : 0x3C003C00u;
    const uint4 ones = make_uint4(ONE, ONE, ONE, ONE);
    const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < FM; i++) {
      X[i] = chunk_step(T(0), av[i], ones, first ? zero : X[i]);
#pragma unroll
      for (int jn = 0; jn < FN; jn++)
        P[i][jn] = chunk_step(T(0), av[i], bv[jn], first ? zero : P[i][jn]);
    }
  }

  // Register sets for P and X: groups are independent until their folds, so
  // with groups no longer than a stage, NGR consecutive groups of a stage
  // each get their own P and X. Their MFMAs issue back to back and their
  // folds follow in ascending group order -- the same operations on the same
  // values as folding each group right after its last chunk-step, without
  // waiting for every group's products before the next group's MFMAs start.
  // A power of two, bounded by about 80 registers of P and X (the 64 x 64
  // footprint: two sets; four measured 7 % slower at group size 32).
  template <int GS>
  static constexpr int q_sets() {
    constexpr int ng = GS <= EPS ? EPS / GS : 1;
    constexpr int per = (FN + 1) * FM * 4;  // registers of one group's P and X
    int cap = 1;
    while (2 * cap * per <= 80) cap *= 2;
    return ng < cap ? ng : cap;
  }

  // All CS chunk-steps of stage s (held in `sl`), operands of step j + 1 read
  // while step j's MFMAs run. With groups no longer than a stage, round r of
  // the stage's groups (NGR of them) runs their chunk-steps into register
  // sets 0 .. NGR - 1 and then folds them in ascending order. GS (the group
  // size) is a compile-time constant, so the fold positions are too.
  template <int GS, int NGR>
  __device__ __forceinline__ void q_compute_full(QSlot sl, int64_t s, f32x4_t (&acc)[FM][FN],
                                                 f32x4_t (&P)[NGR][FM][FN],
                                                 f32x4_t (&X)[NGR][FM]) const {
    constexpr int CPG = GS / 32;  // chunk-steps per group
    uint4 av[2][FM], bv[2][FN];
    read_operands(Slot{sl.a, sl.b}, 0, av[0], bv[0]);
#pragma unroll
    for (int j = 0; j < CS; j++) {
      if (j + 1 < CS) read_operands(Slot{sl.a, sl.b}, j + 1, av[(j + 1) & 1], bv[(j + 1) & 1]);
      if constexpr (GS <= EPS) {
        // Inside a stage a group starts at every CPG-th chunk-step.
        const int gi = j / CPG;
        q_mfma(av[j & 1], bv[j & 1], j % CPG == 0, P[gi % NGR], X[gi % NGR]);
        if ((j + 1) % (CPG * NGR) == 0 || j + 1 == CS) {
#pragma unroll
          for (int q = gi - gi % NGR; q <= gi; q++) q_fold(sl, q, false, acc, P[q % NGR], X[q % NGR]);
        }
      } else {
        q_mfma(av[j & 1], bv[j & 1], false, P[0], X[0]);
      }
    }
    if constexpr (GS > EPS) {
      // Longer groups restart at the fold.
      if ((((s + 1) * EPS) & (GS - 1)) == 0) q_fold(sl, 0, true, acc, P[0], X[0]);
    }
  }

  // The first `steps` (< CS) chunk-steps of the last stage, one group at a
  // time in register set 0.
  template <int GS, int NGR>
  __device__ __forceinline__ void q_compute_part(QSlot sl, int64_t s, int steps,
                                                 f32x4_t (&acc)[FM][FN], f32x4_t (&P)[NGR][FM][FN],
                                                 f32x4_t (&X)[NGR][FM]) const {
#pragma unroll
    for (int j = 0; j < CS - 1; j++) {
      if (j < steps) {
        uint4 av[FM], bv[FN];
        read_operands(Slot{sl.a, sl.b}, j, av, bv);
        const int64_t k_beg = (s * CS + j) * 32, k_end = k_beg + 32;
        q_mfma(av, bv, (k_beg & (GS - 1)) == 0, P[0], X[0]);
        if ((k_end & (GS - 1)) == 0)
          q_fold(sl, (int)(k_end / GS - 1 - glo(s)), false, acc, P[0], X[0]);
      }
    }
  }

  template <int GS, int NGR>
  __device__ __forceinline__ void q_compute(QSlot sl, int64_t s, int steps, f32x4_t (&acc)[FM][FN],
                                            f32x4_t (&P)[NGR][FM][FN], f32x4_t (&X)[NGR][FM]) const {
    if (steps == CS)
      q_compute_full<GS, NGR>(sl, s, acc, P, X);
    else if (steps > 0)
      q_compute_part<GS, NGR>(sl, s, steps, acc, P, X);
  }

  // Loads run QP stages ahead in registers; each stage is converted into one
  // of two LDS slots one stage before it is computed (whole rounds of QP
  // stages, so ring indices are compile-time). Before a slot is rewritten,
  // the barrier guarantees every wave finished reading it (LDS reads retire
  // before the barrier: lgkmcnt(0)).
  template <bool COMPUTE, bool LOAD, int GS, int NGR, typename QSlots>
  __device__ __forceinline__ void q_rounds(const QSlots& slots, int64_t nst, int64_t nsteps,
                                           QStage (&q)[QP], f32x4_t (&acc)[FM][FN],
                                           f32x4_t (&P)[NGR][FM][FN], f32x4_t (&X)[NGR][FM]) const {
    for (int64_t s0 = 0; s0 < nst; s0 += QP) {
#pragma unroll
      for (int u = 0; u < QP; u++) {
        __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(63));
        asm volatile("s_barrier" ::: "memory");
        if constexpr (LOAD) {
          qstore(slots((u + 1) & 1), q[(u + 1) % QP]);
          qload(s0 + u + 1 + QP, q[(u + 1) % QP]);
        }
        if constexpr (COMPUTE)
          q_compute<GS, NGR>(slots(u & 1), s0 + u, steps_of(nsteps, s0 + u), acc, P, X);
      }
    }
  }

  template <int GS, typename QSlots>
  __device__ __forceinline__ void main_loop_q(const QSlots& slots, int64_t nst, int64_t nsteps,
                                              bool computes, f32x4_t (&acc)[FM][FN]) const {
    static_assert(QP % 2 == 0, "ring of two LDS slots");
    constexpr int NGR = q_sets<GS>();
    f32x4_t P[NGR][FM][FN], X[NGR][FM];
#pragma unroll
    for (int r = 0; r < NGR; r++)
#pragma unroll
      for (int i = 0; i < FM; i++) {
        X[r][i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int jn = 0; jn < FN; jn++) P[r][i][jn] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      }
    QStage q[QP];
    if constexpr (QNT < NT) {
      // Loading waves stage every operand; computing waves only compute.
      if (wave >= CW) {
#pragma unroll
        for (int u = 0; u < QP; u++) qload(u, q[u]);
        qstore(slots(0), q[0]);
        qload(QP, q[0]);
        q_rounds<false, true, GS, NGR>(slots, nst, nsteps, q, acc, P, X);
      } else if (computes) {
        q_rounds<true, false, GS, NGR>(slots, nst, nsteps, q, acc, P, X);
      } else {
        q_rounds<false, false, GS, NGR>(slots, nst, nsteps, q, acc, P, X);
      }
      return;
    }
#pragma unroll
    for (int u = 0; u < QP; u++) qload(u, q[u]);
    qstore(slots(0), q[0]);
    qload(QP, q[0]);
    if (computes)
      q_rounds<true, true, GS, NGR>(slots, nst, nsteps, q, acc, P, X);
    else
      q_rounds<false, true, GS, NGR>(slots, nst, nsteps, q, acc, P, X);
  }

  // Register-staged path (unaligned operands): two slots, double buffered.
  template <typename Slots>
  __device__ __forceinline__ void main_loop_slow(const Slots& slots, int64_t nst,
                                                 int64_t nsteps, bool computes,
                                                 f32x4_t (&acc)[CHAINS][FM][FN]) const {
    uint4 ra[LA], rb[LB];
    for (int64_t s = 0; s < nst; s++) {
      gload_slow(s, ra, rb);
      Slot slot = (s & 1) ? slots(1) : slots(0);
      sstore(slot, ra, rb);
      __syncthreads();
      if (computes) compute(slot, steps_of(nsteps, s), acc);
      __syncthreads();
    }
  }
};

template <typename T, int BM, int BN, int WM, int WN, int NW, int KB, int NS, bool TB, bool PL,
          bool PP>
__global__ void __launch_bounds__(64 * NW) gemm_kernel(GemmArgs p) {
  using Tile = GemmTile<T, BM, BN, WM, WN, NW, KB, NS, TB, 0, PL, PP>;
  constexpr int FM = Tile::FM, FN = Tile::FN, CHAINS = Tile::CHAINS;
  constexpr int AC = Tile::A_CH, BC = Tile::B_CH;
  // The LDS ring: NS stages, each an A and a B array (unused ones are a single chunk).
  __shared__ uint4 a0[AC], b0[BC], a1[AC], b1[BC];
  __shared__ uint4 a2[NS > 2 ? AC : 1], b2[NS > 2 ? BC : 1], a3[NS > 3 ? AC : 1], b3[NS > 3 ? BC : 1];
  __shared__ uint4 a4[NS > 4 ? AC : 1], b4[NS > 4 ? BC : 1], a5[NS > 5 ? AC : 1], b5[NS > 5 ? BC : 1];
  __shared__ uint4 a6[NS > 6 ? AC : 1], b6[NS > 6 ? BC : 1], a7[NS > 7 ? AC : 1], b7[NS > 7 ? BC : 1];
  // Slot u of the ring; u is a compile-time constant at every use (the loops
  // over it are unrolled), so each access names one LDS array.
  auto slots = [&](int u) -> Slot {
    switch (u) {
      case 0: return {a0, b0};
      case 1: return {a1, b1};
      case 2: return {a2, b2};
      case 3: return {a3, b3};
      case 4: return {a4, b4};
      case 5: return {a5, b5};
      case 6: return {a6, b6};
      default: return {a7, b7};
    }
  };

  Tile t;
  t.A = static_cast<const T*>(p.a);
  t.B = static_cast<const T*>(p.b);
  t.M = p.M;
  t.N = p.N;
  t.K = p.K;
  t.tid = threadIdx.x;
  t.lane = t.tid & 63;
  t.wave = __builtin_amdgcn_readfirstlane(t.tid >> 6);
  t.wm = (t.wave % Tile::CW) / WN;
  t.wn = (t.wave % Tile::CW) % WN;
  t.g = t.lane >> 4;
  t.r16 = t.lane & 15;
  const int tile = xcd_remap(blockIdx.x, p.tiles_m * p.tiles_n);
  int mi, ni;
  tile_coords(tile, p.tiles_m, p.tiles_n, mi, ni);
  t.m0 = (int64_t)mi * BM;
  t.n0 = (int64_t)ni * BN;

  const int64_t M = t.M, N = t.N, K = t.K;
  const int64_t nst = (K + Tile::EPS - 1) / Tile::EPS;
  // A chunk-step is 4 chunks of the row: 32 elements (16-bit) or 16 (fp32).
  const int64_t nsteps = (K + 4 * Tile::EPC - 1) / (4 * Tile::EPC);
  const int64_t wrow = t.m0 + t.wm * Tile::WTM, wcol = t.n0 + t.wn * Tile::WTN;
  // Waves whose whole sub-tile lies outside C load but do not compute.
  const bool computes = t.wave < Tile::CW && wrow < M && wcol < N;

  f32x4_t acc[CHAINS][FM][FN];
#pragma unroll
  for (int ch = 0; ch < CHAINS; ch++)
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
      for (int jn = 0; jn < FN; jn++) acc[ch][i][jn] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  t.init_lds_offsets();
  if (p.vec_a && p.vec_b) {
    t.init_buffers();
    if constexpr (PP) {
      t.main_loop_pp(slots, nst, computes, acc);
    } else {
      // With PL only the loading waves need the load addressing.
      if (!PL || t.wave >= Tile::CW) t.init_dma();
      t.main_loop_dma(slots, nst, computes, acc);
    }
  } else if constexpr (!PL && !PP) {
    // PL and PP footprints take 16-byte aligned operands only: the host
    // launches another footprint for the others (the slow path's registers
    // would make the whole kernel spill).
    t.main_loop_slow(slots, nst, nsteps, computes, acc);
  }

  // Epilogue: one rounding per element. A wave whose sub-tile lies wholly
  // inside C, with 16-byte aligned output rows, rounds its tile into LDS
  // (the ring is free once every wave is past the loop and no load is in
  // flight) and stores it back row by row with 16-byte stores, so each row
  // of the tile is written as whole cache lines. Otherwise (C's edges,
  // unaligned rows) each lane stores its own elements. Both store the same
  // values.
  constexpr int SWB = Tile::WTM * Tile::WTN * (int)sizeof(T);  // staged bytes per wave
  constexpr int WPA = AC * 16 / SWB;                            // waves per A array
  constexpr int WPB = BC * 16 / SWB;                            // waves per B array
  // The A arrays of the ring, or where they are too few, A and B arrays.
  constexpr bool STAGED_A = WPA >= 1 && WPA * NS >= Tile::CW;
  constexpr bool STAGED = STAGED_A || (WPA >= 1 && (WPA + WPB) * NS >= Tile::CW);
  if constexpr (STAGED) {
    __builtin_amdgcn_s_waitcnt(0);
    asm volatile("s_barrier" ::: "memory");
  }
  if (!computes) return;
  T* __restrict__ out = static_cast<T*>(p.out);
  const T* __restrict__ bias = static_cast<const T*>(p.bias);
  const float alpha = p.alpha, beta = p.beta;
  if constexpr (STAGED) {
    const bool whole = wrow + Tile::WTM <= M && wcol + Tile::WTN <= N &&
                       N % Tile::EPC == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0;
    if (whole) {
      T* stage;
      if constexpr (STAGED_A) {
        stage = reinterpret_cast<T*>(slots(t.wave / WPA).a) + (t.wave % WPA) * (SWB / (int)sizeof(T));
      } else {
        const int u = t.wave / (WPA + WPB), r = t.wave % (WPA + WPB);
        stage = r < WPA ? reinterpret_cast<T*>(slots(u).a) + r * (SWB / (int)sizeof(T))
                        : reinterpret_cast<T*>(slots(u).b) + (r - WPA) * (SWB / (int)sizeof(T));
      }
#pragma unroll
      for (int jn = 0; jn < FN; jn++) {
        const int c = jn * 16 + t.r16;
        const float bv = bias ? beta * Elem<T>::to_f32(bias[wcol + c]) : 0.f;
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
          for (int e = 0; e < 4; e++) {
            float v = acc[0][i][jn][e];
            if constexpr (CHAINS == 2) v = v + acc[1][i][jn][e];
            if (bias) v = __builtin_fmaf(alpha, v, bv);
            stage[(i * 16 + 4 * t.g + e) * Tile::WTN + c] = Elem<T>::from_f32(v);
          }
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      constexpr int CPRW = Tile::WTN * (int)sizeof(T) / 16;  // 16-byte chunks per tile row
      constexpr int RPI = 64 / CPRW;                          // rows per wave-wide pass
#pragma unroll
      for (int r0 = 0; r0 < Tile::WTM; r0 += RPI) {
        const int r = r0 + t.lane / CPRW, c = t.lane % CPRW;
        if (Tile::WTM % RPI == 0 || r < Tile::WTM) {
          const uint4 v = reinterpret_cast<const uint4*>(stage)[r * CPRW + c];
          *reinterpret_cast<uint4*>(out + (wrow + r) * N + wcol + c * Tile::EPC) = v;
        }
      }
      return;
    }
  }
#pragma unroll
  for (int jn = 0; jn < FN; jn++) {
    const int64_t col = wcol + jn * 16 + t.r16;
    if (col >= N) continue;
    const float bv = bias ? beta * Elem<T>::to_f32(bias[col]) : 0.f;
#pragma unroll
    for (int i = 0; i < FM; i++) {
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int64_t row = wrow + i * 16 + 4 * t.g + e;
        if (row < M) {
          float v = acc[0][i][jn][e];
          if constexpr (CHAINS == 2) v = v + acc[1][i][jn][e];
          if (bias) v = __builtin_fmaf(alpha, v, bv);
          out[row * N + col] = Elem<T>::from_f32(v);
        }
      }
    }
  }
}

// Quantized-B GEMM: the dense kernel's tile walk and chunk-step order over
// B's integer codes, with the per-group scale and bias folded into the fp32
// accumulator (GemmTile's quantized part). Every output element sees the same
// sequence of MFMAs and folds on its own row of A and column of B; the
// footprint only decides which elements a workgroup owns. One RNE rounding at
// the end.
template <typename T, int BM, int BN, int WM, int WN, int NW, int KB, int QB, int GS>
__global__ void __launch_bounds__(64 * NW) gemm_qkernel(GemmArgs p) {
  using Tile = GemmTile<T, BM, BN, WM, WN, NW, KB, 2, true, QB>;
  constexpr int FM = Tile::FM, FN = Tile::FN;
  constexpr int AC = Tile::A_CH, BC = Tile::B_CH, SB = Tile::QSB;
  __shared__ uint4 a0[AC], b0[BC], a1[AC], b1[BC];
  __shared__ unsigned short s0[SB], z0[SB], s1[SB], z1[SB];
  auto slots = [&](int u) -> QSlot {
    if (u == 0) return {a0, b0, s0, z0};
    return {a1, b1, s1, z1};
  };

  Tile t;
  t.A = static_cast<const T*>(p.a);
  t.B = static_cast<const T*>(p.b);
  t.M = p.M;
  t.N = p.N;
  t.K = p.K;
  t.tid = threadIdx.x;
  t.qtid = t.tid - (Tile::NT - Tile::QNT);
  t.lane = t.tid & 63;
  t.wave = __builtin_amdgcn_readfirstlane(t.tid >> 6);
  t.wm = (t.wave % Tile::CW) / WN;
  t.wn = (t.wave % Tile::CW) % WN;
  t.g = t.lane >> 4;
  t.r16 = t.lane & 15;
  const int tile = xcd_remap(blockIdx.x, p.tiles_m * p.tiles_n);
  int mi, ni;
  tile_coords(tile, p.tiles_m, p.tiles_n, mi, ni);
  t.m0 = (int64_t)mi * BM;
  t.n0 = (int64_t)ni * BN;

  const int64_t M = t.M, N = t.N, K = t.K;
  const int64_t nst = (K + Tile::EPS - 1) / Tile::EPS;
  const int64_t nsteps = (K + 4 * Tile::EPC - 1) / (4 * Tile::EPC);
  const int64_t wrow = t.m0 + t.wm * Tile::WTM, wcol = t.n0 + t.wn * Tile::WTN;
  const bool computes = t.wave < Tile::CW && wrow < M && wcol < N;

  f32x4_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int jn = 0; jn < FN; jn++) acc[i][jn] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  t.init_lds_offsets();
  // The host launches quantized kernels only with 16-byte aligned rows of A.
  t.init_buffers_q(p);
  t.template main_loop_q<GS>(slots, nst, nsteps, computes, acc);

  if (!computes) return;
  T* __restrict__ out = static_cast<T*>(p.out);
#pragma unroll
  for (int jn = 0; jn < FN; jn++) {
    const int64_t col = wcol + jn * 16 + t.r16;
    if (col >= N) continue;
#pragma unroll
    for (int i = 0; i < FM; i++) {
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int64_t row = wrow + i * 16 + 4 * t.g + e;
        if (row < M) out[row * N + col] = Elem<T>::from_f32(acc[i][jn][e]);
      }
    }
  }
}

// ------------------------------------------------------------------ geometries

// Footprints of C per workgroup. Every entry runs the same per-element
// arithmetic; the table only trades parallelism against operand reuse and
// latency hiding. Columns: id, BM, BN, WM, WN, NW (waves), KB (stage bytes),
// NS (LDS ring stages), PL (loading waves issue all loads), PP (1: ping-pong
// schedule of the compute waves; 2: the four-wave footprint of bi_gemm_w4.h,
// whose KB and NS describe its stage and its ring of 32 KB slots).
#define BI_GEOMETRIES(X)                     \
  X(0, 16, 16, 1, 1, 4, 512, 4, 0, 0)        \
  X(1, 64, 16, 4, 1, 4, 256, 4, 0, 0)        \
  X(2, 64, 64, 2, 2, 8, 256, 4, 0, 0)        \
  X(3, 128, 128, 4, 2, 8, 128, 4, 0, 0)      \
  X(4, 256, 128, 4, 2, 12, 128, 3, 1, 0)     \
  X(5, 64, 32, 4, 2, 8, 256, 3, 0, 0)        \
  X(6, 256, 256, 4, 4, 16, 64, 4, 0, 1)      \
  X(7, 256, 256, 2, 2, 4, 128, 5, 0, 2)

using KernelFn = void (*)(GemmArgs);

}  // namespace bi_gemm_dev

#include "bi_gemm_w4.h"
#include "bi_gemm_qdecode.h"

namespace bi_gemm_dev {

// Kernel for geometry g in the translation unit of element type T.
template <typename T>
KernelFn kernel_for(int g, bool trans_b) {
// fp32 carries two accumulator chains per element: with more than 8 waves
// (at most 168 registers each) the 64 x 64 wave tiles do not fit.
#define BI_GEO_CASE(id, bm, bn, wm, wn, nw, kb, ns, pl, pp)                             \
  case id:                                                                             \
    if constexpr (pp == 2) {                                                           \
      if constexpr (sizeof(T) == 2)                                                    \
        return trans_b ? gemm_w4_kernel<T, true> : gemm_w4_kernel<T, false>;           \
      else                                                                             \
        return nullptr;                                                                \
    } else if constexpr (sizeof(T) == 4 && (nw > 8 || pp)) {                           \
      return nullptr;                                                                  \
    } else {                                                                           \
      return trans_b ? gemm_kernel<T, bm, bn, wm, wn, nw, kb, ns, true, pl, pp != 0>   \
                     : gemm_kernel<T, bm, bn, wm, wn, nw, kb, ns, false, pl, pp != 0>; \
    }
  switch (g) { BI_GEOMETRIES(BI_GEO_CASE) }
#undef BI_GEO_CASE
  return nullptr;
}

// Quantized-B kernel for geometry g (16-bit element types; (N, K) packed B).
// Footprints above 128 x 128 and those whose loading waves issue every load
// (PL) are not built: the quantized kernel's loads land in registers of the
// computing waves, and larger tiles would spill them.
template <typename T, int BM, int BN, int WM, int WN, int NW, int KB, int QB>
KernelFn qkernel_gs(int group) {
  switch (group) {
    case 32: return gemm_qkernel<T, BM, BN, WM, WN, NW, KB, QB, 32>;
    case 64: return gemm_qkernel<T, BM, BN, WM, WN, NW, KB, QB, 64>;
    case 128: return gemm_qkernel<T, BM, BN, WM, WN, NW, KB, QB, 128>;
  }
  return nullptr;
}

template <typename T>
KernelFn qkernel_for(int g, int bits, int group) {
#define BI_QGEO_CASE(id, bm, bn, wm, wn, nw, kb, ns, pl, pp)                         \
  case id:                                                                          \
    if constexpr (bm * bn <= 128 * 128 && !pl && !pp) {                             \
      switch (bits) {                                                               \
        case 2: return qkernel_gs<T, bm, bn, wm, wn, nw, kb, 2>(group);             \
        case 4: return qkernel_gs<T, bm, bn, wm, wn, nw, kb, 4>(group);             \
        case 8: return qkernel_gs<T, bm, bn, wm, wn, nw, kb, 8>(group);             \
      }                                                                             \
    }                                                                               \
    return nullptr;
  switch (g) { BI_GEOMETRIES(BI_QGEO_CASE) }
#undef BI_QGEO_CASE
  return nullptr;
}

// The quantized decode footprint (2-, 4- or 8-bit codes, at most 8 rows) for
// group size `group` and `rows` rows of x, kQDecodeWaves waves per workgroup.
constexpr int kQDecodeWaves = 4;
template <typename T, int GS, int QB>
KernelFn qdecode_kernel_rows(int rows) {
  constexpr int NW = kQDecodeWaves;
  if (rows <= 1) return gemm_qdecode_kernel<T, GS, 1, NW, QB>;
  if (rows == 2) return gemm_qdecode_kernel<T, GS, 2, NW, QB>;
  if (rows <= 4) return gemm_qdecode_kernel<T, GS, 4, NW, QB>;
  return gemm_qdecode_kernel<T, GS, 8, NW, QB>;
}
template <typename T, int QB>
KernelFn qdecode_kernel_group(int group, int rows) {
  switch (group) {
    case 32: return qdecode_kernel_rows<T, 32, QB>(rows);
    case 64: return qdecode_kernel_rows<T, 64, QB>(rows);
    case 128: return qdecode_kernel_rows<T, 128, QB>(rows);
  }
  return nullptr;
}
template <typename T>
KernelFn qdecode_kernel_for(int group, int rows, int bits) {
  switch (bits) {
    case 2: return qdecode_kernel_group<T, 2>(group, rows);
    case 4: return qdecode_kernel_group<T, 4>(group, rows);
    case 8: return qdecode_kernel_group<T, 8>(group, rows);
  }
  return nullptr;
}

}  // namespace bi_gemm_dev

// Per-type kernel tables, defined in bi_gemm_{f32,f16,bf16}.hip.
bi_gemm_dev::KernelFn bi_gemm_kernel_f32(int g, bool trans_b);
bi_gemm_dev::KernelFn bi_gemm_kernel_f16(int g, bool trans_b);
bi_gemm_dev::KernelFn bi_gemm_kernel_bf16(int g, bool trans_b);
bi_gemm_dev::KernelFn bi_qgemm_kernel_f16(int g, int bits, int group);
bi_gemm_dev::KernelFn bi_qgemm_kernel_bf16(int g, int bits, int group);
bi_gemm_dev::KernelFn bi_qdecode_kernel_f16(int group, int rows, int bits);
bi_gemm_dev::KernelFn bi_qdecode_kernel_bf16(int group, int rows, int bits);
