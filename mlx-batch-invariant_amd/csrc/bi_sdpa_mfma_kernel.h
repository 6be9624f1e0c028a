// Batch-invariant single-pass attention on MFMA (gfx950), bf16 and f16: the
// kernel template, included by one instantiation unit per built head-dim pair
// (bi_sdpa_mfma_d*.hip); bi_sdpa.hip chooses the launch shape.
//
// Restates the reference bi_sdpa (mlx_batch_invariant/_attention.py:32-149)
// with matrix cores: one workgroup owns the whole key reduction for each of
// its query columns -- a column is one (query head, query row) pair; the
// columns of a workgroup share a batch index and a kv head, so they read the
// same keys and values -- with no split-KV, no second pass and no switch on
// query length or context length. The workgroup's 4 waves walk the keys in a
// fixed stride order (the reference's fixed per-simdgroup strides, :89) and
// their partial results are merged in a fixed order through LDS (:124-141).
// D is the query/key head dim and V the value head dim (both multiples of 32,
// reference :33-34, :224-227).
//
// Fixed per-column arithmetic (the invariance contract):
//   * Keys are taken in blocks of 32 (block b = keys 32b .. 32b + 31). Block b
//     belongs to chain b mod 4; each chain walks its blocks in ascending order.
//   * Score: raw_i = q . k_i as a chain of v_mfma_f32_16x16x32_{bf16,f16}
//     over the head dim in ascending 32-element chunks from +0.0 (exact
//     products, fp32 sums). With a = |scale| * log2 e (a negative scale
//     negates q's elements, which negates every raw_i exactly), the scaled
//     score is s_i = raw_i * a, plus mask_i * log2 e for an additive mask.
//   * Key i is used iff i < N, i <= row + causal_offset (causal) and
//     mask_i > -3e38 (array mask) (reference :92-96).
//   * Each chain runs an online softmax in base 2 over its blocks: with M the
//     largest used s_i of the block (without a mask taken as max_i(raw_i) * a,
//     the same value since rounding is monotonic; none used: the block leaves
//     the chain unchanged), m' = M > m + 8 ? M : m (a lazily moved base),
//     f = m' == m ? 1 : exp2(m - m'),
//     p_i = exp2(fma(raw_i, a, t_i)) with t_i = -m' (array mask:
//     mask_i * log2 e - m'; 0 for unused keys), l = fma(l, f, sum_i p_i) with
//     the block sum taken in a fixed tree; o = o * f + 0.0 (skipped when
//     f == 1, which changes no bits), then o += p . v as one
//     v_mfma_f32_16x16x32_{bf16,f16} over the block's 32 keys per 16-dim block,
//     p rounded once to T (round to nearest even); lane group g supplies
//     keys 4g .. 4g + 3 and 16 + 4g .. 16 + 4g + 3. m starts at the lowest
//     finite float and l at 0 (reference :76-79). A mask of zeros gives the
//     bits of no mask.
//   * Merge: a sink (reference :80-86, an extra denominator term exp(sink))
//     enters here as one more partial with m = sink * log2 e, l = 1, o = 0,
//     ahead of the chains: M = max of the sink's and the chains' m;
//     L = exp2(sink2 - M) (0 without a sink), O = +0.0; then for
//     c = 0, 1, 2, 3 in order, e_c = exp2(m_c - M), L = fma(l_c, e_c, L) and
//     O = fma(o_c, e_c, O); out = L == 0 ? O : O / L, one rounding to T.
//     (Seeding a chain's base with the sink, as the reference seeds its
//     simdgroup 0, would put a large sink's p below f16's range.)
// Every column, whatever workgroup or lane it lands in, however many rows or
// heads share its keys and whatever the launch shape (columns per workgroup,
// prefetch depths), runs exactly this sequence: an output row has the same
// bits for any batch, query length and context past its visible keys.
#pragma once

#include <hip/hip_runtime.h>
#include <float.h>
#include <math.h>
#include <stdint.h>

#include <type_traits>

#include "bi_internal.h"
#include "bi_sdpa_args.h"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// 16-byte copies as single vector loads / stores (a uint4 assignment is a
// struct copy, which would keep staged data in scratch memory).
__device__ __forceinline__ uint4 ld16(const void* p) {
  return __builtin_bit_cast(uint4, *reinterpret_cast<const u32x4_t*>(p));
}
__device__ __forceinline__ void st16(uint4* p, uint4 v) {
  *reinterpret_cast<u32x4_t*>(p) = __builtin_bit_cast(u32x4_t, v);
}

constexpr int kWaves = 4;  // = chains
constexpr int kThreads = 64 * kWaves;
constexpr int kBlk = 32;   // keys per block
constexpr float kLog2e = 1.4426950408889634f;

// s_waitcnt immediates (gfx9 encoding: vmcnt [3:0] + [15:14], expcnt [6:4],
// lgkmcnt [11:8]).
constexpr int lcm(int a, int b) {
  int x = a, y = b;
  while (y) {
    const int t = x % y;
    x = y;
    y = t;
  }
  return a / x * b;
}
constexpr int wait_vm(int vm) { return (vm & 0xF) | ((vm >> 4) << 14) | (0x7 << 4) | (0xF << 8); }
constexpr int kWaitAll = 0;
constexpr int kWaitLds = 0xF | (0x3 << 14) | (0x7 << 4);  // lgkmcnt(0) only

// 16x16x32: lane (r = lane % 16, g = lane / 16) supplies A[r][8g + t] and
// B[8g + t][r], t = 0..7; it receives C[4g + e][r], e = 0..3.
__device__ inline f32x4_t mma32(__bf16, uint4 a, uint4 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
__device__ inline f32x4_t mma32(_Float16, uint4 a, uint4 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}
// Two 4-element halves as one 8-element MFMA operand (elements 0-3 from lo).
__device__ inline uint4 join(uint2 lo, uint2 hi) { return make_uint4(lo.x, lo.y, hi.x, hi.y); }

// ds_read_b64_tr_b16 (in each 16-lane group, lane i receives element i of
// the four 4 x 16-bit rows its group addresses, one per row) as an asm
// statement. Values arrive in LDS through loads that write it directly; the
// compiler's tracking of those loads cannot always tell which slot an
// intrinsic read touches and then waits for every load in flight, including
// the next blocks' prefetch. As asm the read is ordered by the explicit waits
// only: the caller waits for the slot's loads before and for the read
// (lgkmcnt) after.
__device__ __forceinline__ u32x2_t ds_read_tr(uint32_t lds_addr) {
  u32x2_t v;
  asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(v) : "v"(lds_addr) : "memory");
  return v;
}
// A 16-byte LDS read as an asm statement, for the same reason.
__device__ __forceinline__ u32x4_t ds_read_b128(uint32_t lds_addr) {
  u32x4_t v;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(lds_addr) : "memory");
  return v;
}
// The same two reads at a lane address plus a constant (the instruction's
// 16-bit offset field), so that unrolled reads share one address register.
__device__ __forceinline__ u32x2_t ds_read_tr_at(uint32_t lds_addr, int off) {
  u32x2_t v;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(lds_addr), "i"(off) : "memory");
  return v;
}
__device__ __forceinline__ u32x4_t ds_read_b128_at(uint32_t lds_addr, int off) {
  u32x4_t v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(lds_addr), "i"(off) : "memory");
  return v;
}

template <typename T> __device__ inline unsigned short tbits(T x) {
  return __builtin_bit_cast(unsigned short, x);
}

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Four probabilities p (finite, >= 0) rounded to the element type (RNE),
// packed two per dword: element e in bits 16 (e % 2) of dword e / 2.
template <typename T>
__device__ __forceinline__ uint2 pack_p(const float (&pv)[4]) {
  uint32_t w[2];
#pragma unroll
  for (int j = 0; j < 2; j++) {
    if constexpr (__is_same(T, __bf16)) {
      const f32x2_t d = {pv[2 * j], pv[2 * j + 1]};
      w[j] = __builtin_bit_cast(uint32_t, __builtin_convertvector(d, bf16x2_t));
    } else {
      w[j] = (uint32_t)tbits((T)pv[2 * j]) | ((uint32_t)tbits((T)pv[2 * j + 1]) << 16);
    }
  }
  return make_uint2(w[0], w[1]);
}

// A query chunk with every element's sign flipped when qsign is 0x80008000
// (a negative scale), unchanged when it is 0.
__device__ __forceinline__ uint4 qneg(uint4 q, uint32_t qsign) {
  return make_uint4(q.x ^ qsign, q.y ^ qsign, q.z ^ qsign, q.w ^ qsign);
}

__device__ inline int xcd_remap(int w, int total) {
  const int per = total >> 3;
  if (w < (per << 3)) return (w & 7) * per + (w >> 3);
  return w;
}

// Buffer resource over [base, base + n) (wave-uniform, n below 2^31): loads
// past the end return zeros without touching memory. clamp31 caps a byte
// count that is never negative at 2^31 - 1 (the shifted count is truncated
// to 32 bits, so the test stays a 32-bit scalar compare).
__device__ inline __amdgpu_buffer_rsrc_t make_rsrc_n(const void* base, uint32_t n) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  void* ub = reinterpret_cast<void*>(((uint64_t)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(ub, (short)0, (int)__builtin_amdgcn_readfirstlane(n),
                                           0x00020000);
}
__device__ __forceinline__ uint32_t clamp31(int64_t bytes) {
  return (uint32_t)((uint64_t)bytes >> 31) != 0 ? 0x7FFFFFFFu : (uint32_t)bytes;
}

// Sum / max over the four lanes of a column (lanes r, r + 16, r + 32, r + 48,
// one per 16-lane row). permlane16_swap pairs rows (0, 1) and (2, 3),
// permlane32_swap the two halves; every lane adds its pair's operands in the
// same order (lower row first), so all four end with identical bits.
// The larger of two lanes' block maxima as a compare and select (fmaxf
// would first canonicalise both operands: two more instructions). The maxima
// are never NaN (fmaxf skips NaN scores), and which of +0 / -0 it keeps
// changes no probability's bits.
__device__ __forceinline__ float smax(float a, float b) { return a > b ? a : b; }
__device__ inline float row_pair(float x, bool is_max) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const float a = __uint_as_float(r[0]), b = __uint_as_float(r[1]);
  return is_max ? smax(a, b) : a + b;
}
__device__ inline float half_pair(float x, bool is_max) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const float a = __uint_as_float(r[0]), b = __uint_as_float(r[1]);
  return is_max ? smax(a, b) : a + b;
}
__device__ inline float col_sum(float x) { return half_pair(row_pair(x, false), false); }
__device__ inline float col_max(float x) { return half_pair(row_pair(x, true), true); }

// Launch shape: CT column tiles of 16 columns per workgroup, shared by the 4
// waves (one chain each); WS workgroups split a column tile's output dims
// (each computes the same scores and statistics, and o for V / WS dims); a
// wave's keys are loaded PK blocks ahead into registers (or, KL, into its
// LDS slots beside the values, by contiguous loads) and its values SV - 1
// blocks ahead into its own LDS slots; an array mask's values (MK) are
// loaded with the keys (MK = 1) or at the start of their own block (MK = 2,
// one register set). None of these enters a column's arithmetic.
template <typename T, int D, int V, int CT, int PK, int SV, int WS, int MK, bool KL>
struct Chain {
  static constexpr int NQ = D / 32;            // score MFMAs per 16 keys
  static constexpr int DW = V / WS;            // output dims per workgroup
  static constexpr int NB = DW / 16;           // 16-dim blocks of o held
  static constexpr int VCH = DW / 8;           // 16-byte chunks per value row held
  static constexpr int CH = D / 8;             // 16-byte chunks per key row
  static constexpr int NKL = (KL ? 0 : 2 * NQ) + (MK ? 8 * CT : 0);  // register loads per block
  static constexpr int DK = KL ? kBlk * CH / 64 : 0;  // key LDS-DMA loads per block
  static constexpr int DV = kBlk * VCH / 64;   // value LDS-DMA loads per block
  static constexpr int KSLOT = KL ? kBlk * CH : 0;  // uint4 of keys per slot
  static constexpr int VSLOT = KSLOT + kBlk * VCH;  // uint4 per slot (keys, then values)
  static constexpr int ARR_U4 = kWaves * VSLOT;  // one slot of every wave
  // LDS reads as asm statements (see ds_read_tr) except with 8 value loads
  // per block and keys in registers, where the compiler's own waits before
  // the intrinsic read were checked to be exactly VWAIT and it schedules the
  // products among the reads.
  static constexpr bool ASM_TR = KL || DV != 8;
  // Vector-memory operations issued after a block's value loads and before
  // its values are read: at least those of the SV - 1 blocks issued since
  // (the prologue issues the first SV - 1 value blocks before the first PK
  // key blocks, which keeps the count when PK >= SV - 2).
  static constexpr int VWAIT = (SV - 1) * (NKL + DK + DV);
  static_assert(SV >= 2 && SV <= 6 && PK >= 0 && (KL ? PK == 0 && !MK : PK >= SV - 2) &&
                    D % 32 == 0 && V % (16 * WS) == 0 && VCH >= 2 &&
                    (!KL || (CH & (CH - 1)) == 0),
                "shape");
  static_assert(VWAIT <= 63, "value loads in flight exceed the vmcnt range");
  static_assert(SV * ARR_U4 * 16 <= 160 * 1024, "LDS per workgroup");
  // The merge stages one column tile at a time: every chain's o fills one
  // slot array exactly and its (m, l) fit in another.
  static_assert(kWaves * NB * 64 <= ARR_U4 && kWaves * 64 / 2 <= ARR_U4, "merge staging");

  // Value slot: [32 keys][NPR chunk pairs], 32-byte pair j of key r stored at
  // pair (j + rot(r)) mod NPR. ds_read_tr16_b64: lane group g reads keys
  // 4g + (0..3), one pair (16 dims) each; by the bank-conflict counter one
  // pass serves groups 0 and 1 (then 2 and 3), i.e. 8 consecutive keys, so
  // those 8 pairs must fall in distinct 8-bank groups of the 64 banks of 4
  // bytes: key r's pair lands in group (r * NPR + pair) mod 8. With 2^t the
  // largest power of two (at most 8) dividing NPR, rot(r) = (r mod 8) >> (3 - t)
  // separates them for every NPR (checked exhaustively for NPR = 1..16).
  static constexpr int NPR = VCH / 2;
  static constexpr int ROT_SHIFT = NPR % 8 == 0 ? 0 : NPR % 4 == 0 ? 1 : NPR % 2 == 0 ? 2 : 3;
  __device__ __forceinline__ static int rot_v(int r) { return (r & 7) >> ROT_SHIFT; }
  // LDS chunk of value chunk c of key r, and the value chunk stored at LDS
  // chunk c of key r.
  __device__ __forceinline__ static int vchunk_lds(int r, int c) {
    return 2 * (((c >> 1) + rot_v(r)) % NPR) + (c & 1);
  }
  __device__ __forceinline__ static int vchunk_src(int r, int c) {
    return 2 * (((c >> 1) + NPR - rot_v(r)) % NPR) + (c & 1);
  }
  // Key slot (KL): [32 keys][CH chunks], chunk c of key r at c ^ swz_k(r): the
  // score MFMAs' A reads (16 keys, one chunk each) then hit distinct banks.
  __device__ __forceinline__ static int swz_k(int r) { return r & ((CH < 16 ? CH : 16) - 1); }

  // Key and value rows of the stream, and the batch's mask. Each block's
  // buffer resources start at the block's first row (first key for the mask),
  // so the lane offsets are the same for every block (and below 2^31: the
  // host bounds 32 * stride and the mask's extent); loads for blocks
  // i >= nit use an empty resource, which reads nothing and returns zeros.
  const T* kb;
  const T* vb;
  const T* mb;
  int64_t ks2, vs2, N, mext;
  int nit;
  int wave;
  // Lane byte offsets: key row 16kt + r16 at dims 8g ..; value chunk j;
  // mask keys 4g .. of the lane's row in each column tile. The other key and
  // mask loads add constants (immediate offsets, which the range check
  // includes; a scalar offset would not be checked).
  uint32_t koff[2], kdoff[KL ? DK : 1], voff[DV], moff[MK ? CT : 1];

  // mrow: this lane's mask row offset (elements from the batch's mask) per
  // column tile; kmax: keys that some column of the workgroup can see. The
  // key and value streams end there, so keys no column uses (past N, or past
  // every column's causal bound, e.g. the unwritten tail of a cache) read as
  // zeros: their p is +0 in every column, and their values never reach o,
  // whatever they hold (the reference never reads them, _attention.py:92-93).
  __device__ __forceinline__ void init(const SdpaArgs& p, int64_t b, int64_t kvh, int ws, int w,
                                       int n_it, int lane, const int64_t* mrow, int64_t kmax) {
    constexpr uint32_t E = sizeof(T);
    const int g = lane >> 4, r16 = lane & 15;
    kb = static_cast<const T*>(p.k) + b * p.ks[0] + kvh * p.ks[1];
    vb = static_cast<const T*>(p.v) + b * p.vs[0] + kvh * p.vs[1];  // row starts
    ks2 = p.ks[2];
    vs2 = p.vs[2];
    N = kmax;
    nit = n_it;
    wave = w;
    if constexpr (MK) {
      // Elements of the batch's mask that any (head, row) reaches.
      mb = static_cast<const T*>(p.mask) + b * p.ms[0];
      mext = (p.H - 1) * p.ms[1] + (p.qL - 1) * p.ms[2] + p.N;
#pragma unroll
      for (int ct = 0; ct < CT; ct++) moff[ct] = (uint32_t)((mrow[ct] + 4 * g) * E);
    }
#pragma unroll
    for (int kt = 0; kt < 2; kt++) koff[kt] = (uint32_t)(((16 * kt + r16) * ks2 + 8 * g) * E);
#pragma unroll
    for (int j = 0; j < DV; j++) {
      const int pos = j * 64 + lane, r = pos / VCH, c = vchunk_src(r, pos % VCH);
      voff[j] = (uint32_t)((r * vs2 + ws * DW + c * 8) * E);
    }
    if constexpr (KL) {
#pragma unroll
      for (int j = 0; j < DK; j++) {
        const int pos = j * 64 + lane, r = pos / CH, c = (pos % CH) ^ swz_k(r);
        kdoff[j] = (uint32_t)((r * ks2 + c * 8) * E);
      }
    }
  }
  // Rows key0 .. N - 1 of a stream whose rows hold `row` elements.
  // (Blocks i < nit start below N, so the byte count is at least one row.)
  __device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const T* base, int64_t stride, int row,
                                                         int i) const {
    const int64_t key0 = (int64_t)(wave + kWaves * i) * kBlk;
    const bool in = i < nit;
    return make_rsrc_n(base + (in ? key0 * stride : 0),
                       in ? clamp31(((N - key0 - 1) * stride + row) * (int64_t)sizeof(T)) : 0u);
  }
  // Keys of block i into the score MFMAs' A operands: lane (r16, g) holds
  // K[16kt + r16][32q + 8g .. + 7]. Mask values: those of the lane's keys
  // 16kt + 4g + e (j = 4kt + e) in each column tile.
  struct KRegs {
    uint4 k[2][NQ];
    unsigned short m[MK == 1 ? CT : 1][8];
  };
  struct MRegs {
    unsigned short m[CT][8];
  };
  __device__ __forceinline__ void mload(int i, unsigned short (&m)[CT][8]) const {
    const int64_t key0 = (int64_t)(wave + kWaves * i) * kBlk;
    const bool in = i < nit;  // then key0 < N <= mext
    const auto rm = make_rsrc_n(mb + (in ? key0 : 0), in ? clamp31((mext - key0) * (int64_t)sizeof(T)) : 0u);
#pragma unroll
    for (int ct = 0; ct < CT; ct++)
#pragma unroll
      for (int j = 0; j < 8; j++)
        m[ct][j] = __builtin_amdgcn_raw_buffer_load_b16(
            rm, (int)(moff[ct] + (16 * (j >> 2) + (j & 3)) * sizeof(T)), 0, 0);
  }
  __device__ __forceinline__ void kload(int i, KRegs& kr) const {
    if constexpr (!KL) {
      const auto rs = rsrc(kb, ks2, D, i);
#pragma unroll
      for (int kt = 0; kt < 2; kt++)
#pragma unroll
        for (int q = 0; q < NQ; q++)
          kr.k[kt][q] = __builtin_bit_cast(
              uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(koff[kt] + 32 * q * sizeof(T)),
                                                           0, 0));
    }
    if constexpr (MK == 1) mload(i, kr.m);
  }
  // Keys (KL) and values of block i into an LDS slot (loads that write LDS
  // directly; the keys of a slot first, then its values).
  __device__ __forceinline__ void vload(int i, uint4* dst) const {
    // The slot's previous reads have returned before new data lands.
    __builtin_amdgcn_s_waitcnt(kWaitLds);
    if constexpr (KL) {
      const auto rk = rsrc(kb, ks2, D, i);
#pragma unroll
      for (int j = 0; j < DK; j++)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_void_t*)(dst + j * 64), 16,
                                                 (int)kdoff[j], 0, 0, 0);
    }
    const auto rs = rsrc(vb, vs2, V, i);
#pragma unroll
    for (int j = 0; j < DV; j++)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t*)(dst + KSLOT + j * 64), 16,
                                               (int)voff[j], 0, 0, 0);
  }
};

// LW: 0, or kWaves loader waves (keys in LDS only). A loader wave issues the
// loads of one chain's blocks, so the chain wave's instruction stream holds
// no load issue (which stalls while the memory pipeline is busy).
template <typename T, int D, int V, int CT, int PK, int SV, int WS, int MK, bool KL, int LW>
__global__ void __launch_bounds__(kThreads + 64 * LW) sdpa_mfma_kernel(SdpaArgs p) {
  static_assert(LW == 0 || (LW == kWaves && KL && PK == 0 && SV >= 3), "loader waves: one per chain");
  using C = Chain<T, D, V, CT, PK, SV, WS, MK, KL>;
  constexpr int NQ = C::NQ, NB = C::NB, VCH = C::VCH;
  constexpr int COLS = 16 * CT;  // columns per workgroup
  // Value slot s of every wave is array s: an LDS read then names the one
  // array whose loads it waits for, and loads into the other slots stay in
  // flight.
  __shared__ uint4 va0[C::ARR_U4], va1[C::ARR_U4], va2[SV > 2 ? C::ARR_U4 : 1],
      va3[SV > 3 ? C::ARR_U4 : 1], va4[SV > 4 ? C::ARR_U4 : 1], va5[SV > 5 ? C::ARR_U4 : 1];
  auto arr = [&](int s) __attribute__((always_inline)) -> uint4* {
    return s == 0 ? va0 : s == 1 ? va1 : s == 2 ? va2 : s == 3 ? va3 : s == 4 ? va4 : va5;
  };

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool loader = LW != 0 && wv >= kWaves;  // wave kWaves + c loads chain c's blocks
  const int wave = loader ? wv - kWaves : wv;   // the chain
  const int g = lane >> 4, r16 = lane & 15;

  // Workgroup -> (batch, kv head, block of COLS of the G x qL columns of that
  // kv head -- column cc is row cc / G, head cc % G -- and slice of dims).
  const int64_t G = p.H / p.Hkv;
  const int64_t ncol = G * p.qL;
  const int64_t ncb = (ncol + COLS - 1) / COLS;
  int64_t t = xcd_remap(blockIdx.x, (int)(p.B * p.Hkv * ncb * WS));
  const int ws = (int)(t % WS);
  t /= WS;
  // Causal: the last column blocks see the most keys; they start first.
  const int64_t cb = p.mask_mode == BI_MASK_CAUSAL ? ncb - 1 - t % ncb : t % ncb;
  t /= ncb;
  const int64_t kvh = t % p.Hkv;
  const int64_t b = t / p.Hkv;
  const int64_t c0 = cb * COLS;

  // Keys of a column: [0, kend); the workgroup walks the blocks that its last
  // row can see.
  auto kend_of = [&](int64_t s) __attribute__((always_inline)) -> int64_t {
    if (p.mask_mode != BI_MASK_CAUSAL) return p.N;
    const int64_t last = s + p.causal_offset;
    return last < 0 ? 0 : (last + 1 < p.N ? last + 1 : p.N);
  };
  const int64_t last_cc = (c0 + COLS < ncol ? c0 + COLS : ncol) - 1;
  const int64_t kmax = kend_of(last_cc / G);  // keys some column of the workgroup sees
  // Block counts and indices fit in 32 bits (the host bounds N below
  // 2^31 - 1024), which keeps the loop's compares on the scalar unit.
  const int nblk = (int)((kmax + kBlk - 1) / kBlk);
  const int nfull = (int)(kend_of(c0 / G) / kBlk);  // blocks every column of the workgroup sees

  // This lane's column in each tile; its query as the B operand of the score
  // MFMAs (Q[col][32i + 8g ..]); its chain state.
  bool colv[CT];
  int64_t srow[CT], head[CT];
  int kend[CT];
  uint4 qt[CT][NQ];
  int64_t mrow[CT];
  float m[CT], l[CT];
  f32x4_t o[CT][NB];
#pragma unroll
  for (int ct = 0; ct < CT; ct++) {
    const int64_t cc = c0 + 16 * ct + r16;
    colv[ct] = cc < ncol;
    srow[ct] = colv[ct] ? cc / G : 0;
    head[ct] = kvh * G + (colv[ct] ? cc % G : 0);
    kend[ct] = colv[ct] ? (int)kend_of(srow[ct]) : 0;
    const T* qrow = static_cast<const T*>(p.q) + b * p.qs[0] + head[ct] * p.qs[1] + srow[ct] * p.qs[2];
#pragma unroll
    for (int i = 0; i < NQ; i++)
      qt[ct][i] = colv[ct] ? qneg(ld16(qrow + 32 * i + 8 * g), p.qsign) : make_uint4(0, 0, 0, 0);
    mrow[ct] = head[ct] * p.ms[1] + srow[ct] * p.ms[2];
    m[ct] = -FLT_MAX;
    l[ct] = 0.f;
#pragma unroll
    for (int i = 0; i < NB; i++) o[ct][i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  // Key and value rows of the stream; per-block buffer resources start at the
  // block's first row, so the lane offsets below are the same for every block
  // (and below 2^31: the host bounds 32 * stride).
  // This chain's blocks are wave + 4i, i < nit.
  const int nit = nblk > wave ? (nblk - wave + kWaves - 1) / kWaves : 0;
  const int wslot = wave * C::VSLOT;  // this wave's slot within each array
  C ld;
  ld.init(p, b, kvh, ws, wave, nit, lane, mrow, kmax);
  // With loader waves every wave runs the same number of steps (chain 0 has
  // the most blocks), one barrier each. PIPE (four slots or more): at step j
  // a chain wave reads and scores the keys of block j while it finishes block
  // j - 1, so there are nit0 + 1 steps and blocks are issued SV - 2 steps
  // ahead; otherwise step j computes block j, issued SV - 1 steps ahead
  // (two steps at the slot counts built, three and four).
  const int nit0 = nblk > 0 ? (nblk + kWaves - 1) / kWaves : 0;
  constexpr bool PIPE = LW != 0 && SV >= 4;
  constexpr int AHEAD = PIPE ? SV - 2 : SV - 1;
  const int steps = PIPE ? nit0 + 1 : nit0;
  if constexpr (LW != 0) {
    if (loader) {
      // Block j lands in slot j % SV. Before barrier j this wave waits for
      // its loads of block j (the AHEAD - 1 younger blocks may stay in
      // flight), so after the barrier the chain wave reads whole blocks. The
      // slot refilled after barrier j held block j + AHEAD - SV, which the
      // chain wave finished reading before it arrived (PIPE: block j - 2,
      // whose values were read at step j - 1; else block j - 1).
#pragma unroll
      for (int u = 0; u < AHEAD; u++) ld.vload(u, arr(u) + wslot);
      for (int j0 = 0; j0 < steps; j0 += SV) {
#pragma unroll
        for (int u = 0; u < SV; u++) {
          if (j0 + u >= steps) break;
          __builtin_amdgcn_s_waitcnt(wait_vm((AHEAD - 1) * (C::DK + C::DV)));
          asm volatile("s_barrier" ::: "memory");
          ld.vload(j0 + u + AHEAD, arr((u + AHEAD) % SV) + wslot);
        }
      }
      // The merge below reuses the slots: no load may still be landing
      // (those past the chain's blocks write zeros). Then the merge's barriers.
      __builtin_amdgcn_s_waitcnt(kWaitAll);
#pragma unroll
      for (int ct = 0; ct < CT; ct++) {
        asm volatile("s_barrier" ::: "memory");
        asm volatile("s_barrier" ::: "memory");
      }
      return;
    }
  }
  // Keys of slot `slot` (KL) into kl: lane (r16, g) reads chunk 4q + g of
  // key 16kt + r16. Issued only; the caller waits (lgkmcnt) before use.
  using KL_t = u32x4_t[KL ? 2 : 1][KL ? NQ : 1];
  auto kread = [&](int slot, KL_t& kl) __attribute__((always_inline)) {
    if constexpr (KL) {
      const uint32_t ks = (uint32_t)(uintptr_t)(lds_void_t*)(arr(slot) + wslot);
#pragma unroll
      for (int kt = 0; kt < 2; kt++)
#pragma unroll
        for (int i = 0; i < NQ; i++) {
          const int r = 16 * kt + r16;
          kl[kt][i] = ds_read_b128(ks + (r * C::CH + ((4 * i + g) ^ C::swz_k(r))) * 16);
        }
    }
  };
  // Scores: S^T tiles (16 keys x 16 columns); lane (g, r16) holds keys
  // 16kt + 4g + e of column r16. Keys from kr, or (KL) from kl once its reads
  // have returned.
  auto scores = [&](const typename C::KRegs& kr, KL_t& kl, f32x4_t (&sc)[CT][2])
                    __attribute__((always_inline)) {
    if constexpr (KL) {
#pragma unroll
      for (int kt = 0; kt < 2; kt++)
#pragma unroll
        for (int i = 0; i < NQ; i++) asm volatile("" : "+v"(kl[kt][i]));
    }
#pragma unroll
    for (int ct = 0; ct < CT; ct++)
#pragma unroll
      for (int kt = 0; kt < 2; kt++) {
        sc[ct][kt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < NQ; i++) {
          const uint4 a = KL ? __builtin_bit_cast(uint4, kl[KL ? kt : 0][KL ? i : 0]) : kr.k[kt][i];
          sc[ct][kt] = mma32(T(0), a, qt[ct][i], sc[ct][kt]);
        }
      }
  };
  // Values of slot `slot` transposed for the P.V products (issued only;
  // update() waits for them).
  using VA_t = u32x2_t[NB][2];
  auto vread = [&](int slot, VA_t& va) __attribute__((always_inline)) {
    uint4* const vslot = arr(slot) + wslot + C::KSLOT;
#pragma unroll
    for (int db = 0; db < NB; db++) {
#pragma unroll
      for (int kt = 0; kt < 2; kt++) {
        // V^T block (dims 16db .., keys 16kt + 4g ..): lane r16 addresses key
        // 16kt + 4g + r16 / 4 at dim col and receives V[16kt + 4g + t][16db + r16].
        const int kr = 16 * kt + 4 * g + (r16 >> 2);
        const int col = 16 * db + 4 * (r16 & 3);
        const int chunk = C::vchunk_lds(kr, col >> 3);
        const int off = (kr * VCH + chunk) * 16 + (col & 7) * 2;
        if constexpr (C::ASM_TR) {
          va[db][kt] = ds_read_tr((uint32_t)(uintptr_t)(lds_void_t*)vslot + off);
        } else {
          va[db][kt] = __builtin_bit_cast(
              u32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                           (lds_i16x4_t*)(reinterpret_cast<char*>(vslot) + off)));
        }
      }
    }
  };
  // Block blk of this chain given its scores: online softmax, rescale, and
  // o += P . V with the values in value slot `slot`, read into va here or,
  // VPRE, already issued by the caller (asm LDS reads only).
  constexpr int MKCT = MK ? CT : 1;
  auto update = [&](auto vpre, const f32x4_t (&sc)[CT][2], const unsigned short (&mk)[MKCT][8],
                    int slot, int blk, VA_t& va) __attribute__((always_inline)) {
    constexpr bool VPRE = decltype(vpre)::value;
    static_assert(!VPRE || C::ASM_TR, "values read ahead by asm reads only");
    // Key indices fit in 32 bits (the host checks N < 2^31).
    const int key0 = blk * kBlk + 4 * g;
    uint2 ph[CT][2];
    float f[CT];
    uint32_t used = 0;  // mask: bit 4kt + e set if this lane's column uses key 16kt + 4g + e
    // FULL: every column of the workgroup uses all 32 keys of the block (no
    // mask, below every causal bound), so the per-key bookkeeping drops out;
    // the arithmetic is the same.
    auto softmax = [&](auto full_tag) __attribute__((always_inline)) {
      constexpr bool FULL = decltype(full_tag)::value;
#pragma unroll
      for (int ct = 0; ct < CT; ct++) {
        // Raw scores r (q . k) and the exponent's addend t: p = exp2(fma(r,
        // a, t)) with a = |scale| * log2 e, t = -m' (or mask * log2 e - m').
        float r[2][4], t[2][4];
        bool use[2][4];
#pragma unroll
        for (int kt = 0; kt < 2; kt++)
#pragma unroll
          for (int e = 0; e < 4; e++) {
            r[kt][e] = sc[ct][kt][e];
            use[kt][e] = FULL || key0 + 16 * kt + e < kend[ct];
          }
        float bm = -INFINITY;
        if constexpr (MK) {  // keys past N read 0 and are unused
#pragma unroll
          for (int kt = 0; kt < 2; kt++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
              const float mv = (float)__builtin_bit_cast(T, mk[ct][4 * kt + e]);
              use[kt][e] = use[kt][e] && mv > -3.0e38f;
              t[kt][e] = mv * kLog2e;
              const float sv = r[kt][e] * p.ascale2 + t[kt][e];
              bm = use[kt][e] ? fmaxf(bm, sv) : bm;
              used |= use[kt][e] ? 1u << (4 * kt + e) : 0u;
            }
        } else {
          // Rounding is monotonic: the largest raw score, scaled, is the
          // largest scaled score.
#pragma unroll
          for (int kt = 0; kt < 2; kt++)
#pragma unroll
            for (int e = 0; e < 4; e++) bm = use[kt][e] ? fmaxf(bm, r[kt][e]) : bm;
        }
        // The base moves only when the block's largest score passes it by more
        // than 8 (p then stays <= 2^8): few rescales, the same result after o / l.
        // The column's largest score is one of its four lanes' maxima, so it
        // moves iff one of those lanes' own maxima (scaled) passes m + 8, by
        // the same product and compare; when no lane of the wave does, every
        // column keeps m and f = 1 without the cross-lane maximum.
        const float m8 = m[ct] + 8.f;
        float mn = m[ct];
        f[ct] = 1.f;
        if (__builtin_amdgcn_ballot_w64((MK ? bm : bm * p.ascale2) > m8) != 0) {  // wave-uniform
          bm = MK ? col_max(bm) : col_max(bm) * p.ascale2;
          const bool any = bm > -INFINITY;
          mn = (any && bm > m8) ? bm : m[ct];
          f[ct] = mn == m[ct] ? 1.f : __builtin_amdgcn_exp2f(m[ct] - mn);
        }
        float pv[2][4];
        float ps = 0.f;
#pragma unroll
        for (int kt = 0; kt < 2; kt++)
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const float tt = MK ? t[kt][e] - mn : -mn;
            pv[kt][e] = use[kt][e] ? __builtin_amdgcn_exp2f(__builtin_fmaf(r[kt][e], p.ascale2, tt)) : 0.f;
            ps = kt + e == 0 ? pv[0][0] : ps + pv[kt][e];  // p >= +0: the same as 0 + p
          }
        ps = col_sum(ps);
        l[ct] = __builtin_fmaf(l[ct], f[ct], ps);
        m[ct] = mn;
        // P^T as the B operand of the P.V MFMAs, rounded once to T.
#pragma unroll
        for (int kt = 0; kt < 2; kt++) ph[ct][kt] = pack_p<T>(pv[kt]);
      }
    };
    if (!MK && blk < nfull)
      softmax(std::true_type{});
    else
      softmax(std::false_type{});
    // Rescale; adding +0.0 turns an underflowed -0.0 into +0.0, so o is never
    // -0.0 and a column with no usable key in this block (f == 1, all p == 0)
    // keeps its o exactly through the products below.
#pragma unroll
    for (int ct = 0; ct < CT; ct++)
      if (f[ct] != 1.f) {
#pragma unroll
        for (int i = 0; i < NB; i++) o[ct][i] = o[ct][i] * f[ct] + 0.f;
      }
    // The block's values have landed in the slot (vector memory completes in
    // order: at most VWAIT younger operations may still be in flight).
    if constexpr (!KL) __builtin_amdgcn_s_waitcnt(wait_vm(C::VWAIT));
    asm volatile("" ::: "memory");
    if constexpr (!VPRE) vread(slot, va);
    if constexpr (C::ASM_TR) {
      // All of them have returned; the empty statements make every use of a
      // read's result come after the wait.
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
      for (int db = 0; db < NB; db++) asm volatile("" : "+v"(va[db][0]), "+v"(va[db][1]));
    }
    // With an array mask, values of keys that no column of the workgroup uses
    // are zeroed, as the reference never reads them (they may hold anything,
    // e.g. an unwritten cache slot behind a padding mask). Their p is +0 in
    // every column and o is never -0.0, so for finite values this changes no
    // bit. Lane group g holds keys 16kt + 4g + t, t = 0..3. (Without a mask,
    // keys at or past the workgroup's last visible key read as zeros: the
    // streams end there.)
    // OR over the 16 columns of the lane's row group (rotations by 1, 2, 4, 8
    // within each row of 16 lanes): bit 4kt + t set if some column uses key
    // 16kt + 4g + t.
    if constexpr (MK != 0) {
      used |= __builtin_amdgcn_mov_dpp((int)used, 0x121, 0xF, 0xF, false);  // row_ror:1
      used |= __builtin_amdgcn_mov_dpp((int)used, 0x122, 0xF, 0xF, false);  // row_ror:2
      used |= __builtin_amdgcn_mov_dpp((int)used, 0x124, 0xF, 0xF, false);  // row_ror:4
      used |= __builtin_amdgcn_mov_dpp((int)used, 0x128, 0xF, 0xF, false);  // row_ror:8
    }
    if (MK != 0 && __builtin_amdgcn_ballot_w64(used != 0xFFu) != 0) {  // wave-uniform
#pragma unroll
      for (int kt = 0; kt < 2; kt++) {
        uint32_t keep[4];
#pragma unroll
        for (int t = 0; t < 4; t++) keep[t] = (used >> (4 * kt + t)) & 1 ? 0xFFFFu : 0u;
        const u32x2_t vm = {keep[0] | (keep[1] << 16), keep[2] | (keep[3] << 16)};
#pragma unroll
        for (int db = 0; db < NB; db++) va[db][kt] &= vm;
      }
    }
    // o += P . V over the block's 32 keys: A = V^T (16 dims x 32 keys), lane
    // (r16, g) holding keys 4g + t and 16 + 4g + t of dim 16db + r16; B = P^T
    // with the same keys of column r16 -- the 16x16x32 operand layout with K
    // slots 0-3 and 4-7 of lane group g taken by those two key quads.
#pragma unroll
    for (int db = 0; db < NB; db++) {
      const uint4 vt = join(__builtin_bit_cast(uint2, va[db][0]), __builtin_bit_cast(uint2, va[db][1]));
#pragma unroll
      for (int ct = 0; ct < CT; ct++) {
        o[ct][db] = mma32(T(0), vt, join(ph[ct][0], ph[ct][1]), o[ct][db]);
      }
    }
  };
  // One block of this chain: keys in kr (or, KL, in slot `slot` beside the
  // values, landed with at most VWAIT younger operations in flight).
  auto compute = [&](const typename C::KRegs& kr, const unsigned short (&mk)[MKCT][8], int slot,
                     int blk) __attribute__((always_inline)) {
    KL_t kl;
    if constexpr (KL) {
      __builtin_amdgcn_s_waitcnt(wait_vm(C::VWAIT));
      kread(slot, kl);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    f32x4_t sc[CT][2];
    scores(kr, kl, sc);
    VA_t va;
    update(std::false_type{}, sc, mk, slot, blk, va);
  };

  // Block i of the chain: keys loaded at step i - PK, values at step
  // i - SV + 1 into slot i % SV. The loop is unrolled over U steps (the
  // least common multiple of the two rotations) so that register and slot
  // indices are compile-time.
  constexpr int U = lcm(PK + 1, SV);
  typename C::KRegs kr[PK + 1];
  typename C::MRegs mcur;  // MK == 2: this step's mask values
  if constexpr (PIPE) {
    // Step j: after the barrier blocks up to j are in their slots. The keys
    // of block j are read and scored while block j - 1 (whose scores the
    // previous step left in sp) finishes: the two are independent, so each
    // hides the other's latency. Every product is the one compute() makes.
    f32x4_t sp[CT][2];
    for (int j0 = 0; j0 < steps; j0 += SV) {
#pragma unroll
      for (int u = 0; u < SV; u++) {
        const int j = j0 + u;
        if (j >= steps) break;
        asm volatile("s_barrier" ::: "memory");
        // From step nit on, the slot's stale keys are read and scored too
        // (unconditionally, so no copies of the registers): those scores
        // are never used.
        KL_t kl;
        kread(u, kl);
        if (j >= 1 && j <= nit) {
          // Block j - 1's values are read before its softmax, which hides
          // their latency.
          VA_t va;
          vread((u + SV - 1) % SV, va);
          update(std::true_type{}, sp, kr[0].m, (u + SV - 1) % SV, wave + kWaves * (j - 1), va);
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        scores(kr[0], kl, sp);
      }
    }
  } else if constexpr (LW != 0) {
    // Step j: after the barrier block j is in slot j % SV.
    for (int j0 = 0; j0 < steps; j0 += SV) {
#pragma unroll
      for (int u = 0; u < SV; u++) {
        const int j = j0 + u;
        if (j >= steps) break;
        asm volatile("s_barrier" ::: "memory");
        if (j < nit) compute(kr[0], kr[0].m, u, wave + kWaves * j);
      }
    }
  } else {
#pragma unroll
    for (int u = 0; u < SV - 1; u++) ld.vload(u, arr(u) + wslot);
#pragma unroll
    for (int u = 0; u < PK; u++) ld.kload(u, kr[u]);
    for (int i0 = 0; i0 < nit; i0 += U) {
#pragma unroll
      for (int u = 0; u < U; u++) {
        const int i = i0 + u;
        if constexpr (MK == 2) ld.mload(i, mcur.m);
        ld.kload(i + PK, kr[(u + PK) % (PK + 1)]);
        ld.vload(i + SV - 1, arr((u + SV - 1) % SV) + wslot);
        if (i < nit) {
          if constexpr (MK == 2)
            compute(kr[u % (PK + 1)], mcur.m, u % SV, wave + kWaves * i);
          else
            compute(kr[u % (PK + 1)], kr[u % (PK + 1)].m, u % SV, wave + kWaves * i);
        }
      }
    }
  }

  // Merge the 4 chains in order through LDS, one column tile at a time: o of
  // chain c in va0, (m, l) in va1 (the value slots are free once every
  // wave's loads and reads have completed).
  uint4* const mo = va0;
  float2* const ml = reinterpret_cast<float2*>(va1);
#pragma unroll
  for (int ct = 0; ct < CT; ct++) {
    __builtin_amdgcn_s_waitcnt(kWaitAll);
    asm volatile("s_barrier" ::: "memory");
#pragma unroll
    for (int db = 0; db < NB; db++)
      st16(mo + (wave * NB + db) * 64 + lane, __builtin_bit_cast(uint4, o[ct][db]));
    ml[wave * 64 + lane] = make_float2(m[ct], l[ct]);
    __builtin_amdgcn_s_waitcnt(kWaitAll);
    asm volatile("s_barrier" ::: "memory");
    float mc[kWaves], lc[kWaves], ec[kWaves];
    // The sink (base 2) first: -FLT_MAX without one.
    const float sk = p.sinks ? (float)static_cast<const T*>(p.sinks)[head[ct]] * kLog2e : -FLT_MAX;
    float M = sk;
#pragma unroll
    for (int c = 0; c < kWaves; c++) {
      const float2 v = ml[c * 64 + lane];
      mc[c] = v.x;
      lc[c] = v.y;
      M = fmaxf(M, mc[c]);
    }
    float L = p.sinks ? __builtin_amdgcn_exp2f(sk - M) : 0.f;  // the sink's l = 1
#pragma unroll
    for (int c = 0; c < kWaves; c++) {
      ec[c] = __builtin_amdgcn_exp2f(mc[c] - M);
      L = __builtin_fmaf(lc[c], ec[c], L);
    }
    T* __restrict__ out =
        static_cast<T*>(p.out) + ((b * p.H + head[ct]) * p.qL + srow[ct]) * V + ws * C::DW;
    // Wave w writes out the dim blocks w, w + 4, ... of this workgroup.
#pragma unroll
    for (int k = 0; k < (NB + kWaves - 1) / kWaves; k++) {
      const int db = wave + kWaves * k;
      if (db >= NB) break;
      f32x4_t O = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < kWaves; c++) {
        const f32x4_t oc = __builtin_bit_cast(f32x4_t, ld16(mo + (c * NB + db) * 64 + lane));
#pragma unroll
        for (int e = 0; e < 4; e++) O[e] = __builtin_fmaf(oc[e], ec[c], O[e]);
      }
      unsigned short ob[4];
#pragma unroll
      for (int e = 0; e < 4; e++) ob[e] = tbits((T)(L == 0.f ? O[e] : O[e] / L));
      if (colv[ct])
        *reinterpret_cast<uint2*>(out + 16 * db + 4 * g) =
            make_uint2(ob[0] | ((uint32_t)ob[1] << 16), ob[2] | ((uint32_t)ob[3] << 16));
    }
  }
}

// f(integral_constant<I>) for I = I0 .. N - 1 while it returns true.
template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F& f) {
  if constexpr (I < N) {
    if (f(std::integral_constant<int, I>{})) static_for<I + 1, N>(f);
  }
}

// Launch shape SDPA_SHARED (prefill without an array mask): NW waves, each
// owning one tile of 16 columns, and every wave walks every key block of the
// workgroup in ascending order, block b updating the state of chain b mod 4
// that the wave keeps for its columns. A column's 4 chains, their blocks and
// their arithmetic are those of the other shapes (the steps below are the
// same operations in the same order as sdpa_mfma_kernel's), only evaluated
// by one wave: a key and value block is loaded once, into LDS slots that all
// waves read, for 16 * NW columns instead of 16 or 32.
//
// The slots form two groups of GP. The waves synchronise once per group:
// at group g's barrier every wave's loads of group g have landed and every
// wave has finished group g - 1, whose slots then take group g + 1's loads.
// Between barriers the waves drift apart, so one wave's softmax overlaps
// another's products on the same SIMD.
template <typename T, int D, int V, int NW, int GP, int NG>
struct Shared {
  static constexpr int NQ = D / 32;        // score MFMAs per 16 keys
  static constexpr int NB = V / 16;        // 16-dim blocks of o
  static constexpr int CH = D / 8;         // 16-byte chunks per key row
  static constexpr int VCH = V / 8;        // 16-byte chunks per value row
  static constexpr int KSLOT = kBlk * CH;  // uint4 of keys per slot
  static constexpr int SLOT = KSLOT + kBlk * VCH;  // uint4 per slot (keys, then values)
  static constexpr int NL = SLOT / 64;     // LDS-DMA loads per block
  static constexpr int LPW = NL / NW;      // of them issued by each wave
  static constexpr int S = NG * GP;        // slots
  static constexpr int HALF = GP * SLOT * 16;  // bytes of one group's slots
  // Lane address registers: one per 64 KB of slots (LDS read offsets are
  // 16-bit immediates; a slot starts at most 48 KB into its window and its
  // reads stay within 16 KB of that).
  static constexpr int NBASE = (S * SLOT * 16 + 65535) / 65536;
  static_assert(NL % NW == 0 && (CH & (CH - 1)) == 0 && (VCH & (VCH - 1)) == 0 && D <= 128 &&
                    V <= 128 && VCH >= 4 && (4 % GP == 0 || GP % 4 == 0),
                "shape");
  static_assert(NG >= 2 && (NG - 1) * GP * LPW <= 63, "loads in flight exceed the vmcnt range");
  static_assert(S * SLOT * 16 <= 160 * 1024 && HALF <= 65536 && SLOT * 16 <= 16384,
                "LDS per workgroup");
  // Key rows: chunk c of key r at c ^ (r mod CH), so that the 16 keys of a
  // score operand read distinct banks. Value rows: 32-byte pair j of key r at
  // pair (j + rot(r)) mod NPR, rot(r) = (r mod 8) >> (3 - t) with 2^t the
  // largest power of two (at most 8) dividing NPR: the transposed reads of 8
  // consecutive keys fall in distinct 8-bank groups.
  static constexpr int NPR = VCH / 2;
  static constexpr int ROT_SHIFT = NPR % 8 == 0 ? 0 : NPR % 4 == 0 ? 1 : NPR % 2 == 0 ? 2 : 3;
  __device__ __forceinline__ static int swz_k(int r) { return r & (CH < 16 ? CH - 1 : 15); }
  __device__ __forceinline__ static int rot_v(int r) { return (r & 7) >> ROT_SHIFT; }
  __device__ __forceinline__ static int vchunk_lds(int r, int c) {
    return 2 * (((c >> 1) + rot_v(r)) % NPR) + (c & 1);
  }
  __device__ __forceinline__ static int vchunk_src(int r, int c) {
    return 2 * (((c >> 1) + NPR - rot_v(r)) % NPR) + (c & 1);
  }

  // Loads of a block: NL of 64 lanes x 16 bytes, load j filling slot uint4s
  // 64j .. 64j + 63 (keys for j < KSLOT / 64, then values); wave w issues
  // loads w * LPW .. + LPW - 1. Lane byte offsets count from the block's
  // first row (below 2^31: the host bounds 32 * stride). Block i's rows end
  // at kmax, so keys no column of the workgroup sees read as zeros whatever
  // the memory holds; blocks past nblk - 1 read nothing. (Member functions
  // rather than lambdas in the kernel: a lambda there that makes buffer
  // resources cost the kernel its host stub.)
  struct Loads {
    // A wave's loads all fall in one stream, keys or values (the key loads
    // are a whole number of waves' shares), so it keeps one stream's state:
    // the next block's first row, the bytes from there to the end of the
    // last row some column sees, 32 rows in bytes, and the blocks left to
    // load (issue() walks the blocks in order).
    static_assert((KSLOT / 64) % LPW == 0, "a wave's loads lie in one stream");
    const char* sp;
    int64_t srem, sstep;
    int left;
    uint32_t loff[LPW];
    __device__ __forceinline__ void init(const SdpaArgs& p, int64_t b, int64_t kvh, int64_t kmax,
                                         int nblk, int wave, int lane) {
      constexpr uint32_t E = sizeof(T);
      const bool keys = wave * LPW < KSLOT / 64;  // wave-uniform
      const int64_t s2 = keys ? p.ks[2] : p.vs[2];
      const T* base = keys ? static_cast<const T*>(p.k) + b * p.ks[0] + kvh * p.ks[1]
                           : static_cast<const T*>(p.v) + b * p.vs[0] + kvh * p.vs[1];
      sp = reinterpret_cast<const char*>(base);
      srem = ((kmax - 1) * s2 + (keys ? D : V)) * E;
      sstep = kBlk * s2 * E;
      left = nblk;
#pragma unroll
      for (int u = 0; u < LPW; u++) {
        const int j = wave * LPW + u;
        if (keys) {
          const int pos = j * 64 + lane, r = pos / CH, c = (pos % CH) ^ swz_k(r);
          loff[u] = (uint32_t)((r * s2 + c * 8) * E);
        } else {
          const int pos = (j - KSLOT / 64) * 64 + lane, r = pos / VCH, c = vchunk_src(r, pos % VCH);
          loff[u] = (uint32_t)((r * s2 + c * 8) * E);
        }
      }
    }
    // This wave's loads of the next block into the slot at dst (the slot's
    // first uint4 plus this wave's first load). While blocks are left, the
    // remaining byte count is at least one row (D or V elements).
    __device__ __forceinline__ void issue(uint4* dst) {
      const auto rs = make_rsrc_n(sp, left > 0 ? clamp31(srem) : 0u);
#pragma unroll
      for (int u = 0; u < LPW; u++)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t*)(dst + u * 64), 16, (int)loff[u],
                                                 0, 0, 0);
      sp += sstep;
      srem -= sstep;
      left--;
    }
  };
};

template <typename T, int D, int V, int NW, int GP, int NG>
__global__ void __launch_bounds__(64 * NW) sdpa_shared_kernel(SdpaArgs p) {
  using C = Shared<T, D, V, NW, GP, NG>;
  constexpr int NQ = C::NQ, NB = C::NB, CH = C::CH, VCH = C::VCH, LPW = C::LPW;
  constexpr int COLS = 16 * NW;  // columns per workgroup
  __shared__ uint4 ring[C::S * C::SLOT];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, r16 = lane & 15;

  // Workgroup -> (batch, kv head, block of COLS of the G x qL columns of that
  // kv head -- column cc is row cc / G, head cc % G).
  const int64_t G = p.H / p.Hkv;
  const int64_t ncol = G * p.qL;
  const int64_t ncb = (ncol + COLS - 1) / COLS;
  int64_t t = xcd_remap(blockIdx.x, (int)(p.B * p.Hkv * ncb));
  // Causal: the last column blocks see the most keys; they start first.
  const int64_t cb = p.mask_mode == BI_MASK_CAUSAL ? ncb - 1 - t % ncb : t % ncb;
  t /= ncb;
  const int64_t kvh = t % p.Hkv;
  const int64_t b = t / p.Hkv;
  const int64_t c0 = cb * COLS;

  auto kend_of = [&](int64_t s) __attribute__((always_inline)) -> int64_t {
    if (p.mask_mode != BI_MASK_CAUSAL) return p.N;
    const int64_t last = s + p.causal_offset;
    return last < 0 ? 0 : (last + 1 < p.N ? last + 1 : p.N);
  };
  const int64_t last_cc = (c0 + COLS < ncol ? c0 + COLS : ncol) - 1;
  const int64_t kmax = kend_of(last_cc / G);  // keys some column of the workgroup sees
  // Block counts and indices fit in 32 bits (the host bounds N below
  // 2^31 - 1024), which keeps the loop's compares on the scalar unit.
  const int nblk = (int)((kmax + kBlk - 1) / kBlk);
  // This wave's columns w0 .. w0 + 15: the blocks holding a key the last of
  // them sees, and the blocks whose keys every one of them sees.
  const int64_t w0 = c0 + 16 * wave;
  const bool wany = w0 < ncol;
  const int64_t wlast = (w0 + 16 < ncol ? w0 + 16 : ncol) - 1;
  const int nvis_w = wany ? (int)((kend_of(wlast / G) + kBlk - 1) / kBlk) : 0;
  const int nfull_w = wany ? (int)(kend_of(w0 / G) / kBlk) : 0;

  // This lane's column, its query as the B operand of the score MFMAs
  // (Q[col][32i + 8g ..]), and the 4 chains' state.
  const int64_t cc = w0 + r16;
  const bool colv = cc < ncol;
  const int64_t srow = colv ? cc / G : 0;
  const int64_t head = kvh * G + (colv ? cc % G : 0);
  const int kend = colv ? (int)kend_of(srow) : 0;
  uint4 qt[NQ];
  {
    const T* qrow = static_cast<const T*>(p.q) + b * p.qs[0] + head * p.qs[1] + srow * p.qs[2];
#pragma unroll
    for (int i = 0; i < NQ; i++)
      qt[i] = colv ? qneg(ld16(qrow + 32 * i + 8 * g), p.qsign) : make_uint4(0, 0, 0, 0);
  }
  float m[4], l[4];
  f32x4_t o[4][NB];
#pragma unroll
  for (int c = 0; c < 4; c++) {
    m[c] = -FLT_MAX;
    l[c] = 0.f;
#pragma unroll
    for (int i = 0; i < NB; i++) o[c][i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  typename C::Loads ld;
  ld.init(p, b, kvh, kmax, nblk, wave, lane);
  // The next block (blocks are issued in order; block i of group h,
  // 0 .. NG - 1, goes to slot h * GP + i mod GP).
  auto issue = [&](int slot) __attribute__((always_inline)) {
    ld.issue(ring + slot * C::SLOT + wave * LPW * 64);
  };

  // LDS lane addresses in slot 0 of each group: lane (r16, g) reads chunk
  // 4i + g of key r16 as the A operand of the score MFMAs (key 16 + r16:
  // + 16 rows, the same swizzle); lane r16 of group g addresses value key
  // 4g + r16 / 4 at dim 16db + 4 (r16 mod 4) for the transposed reads (key
  // + 16: + 16 rows). Slots within a group and key halves are constant
  // offsets. The empty asm keeps each an opaque register, so the unrolled
  // reads do not each recompute theirs.
  constexpr int NBASE = C::NBASE;
  uint32_t kofs[NBASE][NQ], vofs[NBASE][NB];
  {
    const uint32_t rb = (uint32_t)(uintptr_t)(lds_void_t*)ring;
    const int kr = 4 * g + (r16 >> 2);
#pragma unroll
    for (int h = 0; h < NBASE; h++) {
#pragma unroll
      for (int i = 0; i < NQ; i++) {
        kofs[h][i] = rb + h * 65536 + (r16 * CH + ((4 * i + g) ^ C::swz_k(r16))) * 16;
        asm volatile("" : "+v"(kofs[h][i]));
      }
#pragma unroll
      for (int db = 0; db < NB; db++) {
        const int col = 16 * db + 4 * (r16 & 3);
        vofs[h][db] = rb + h * 65536 + C::KSLOT * 16 +
                      (kr * VCH + C::vchunk_lds(kr, col >> 3)) * 16 + (col & 7) * 2;
        asm volatile("" : "+v"(vofs[h][db]));
      }
    }
  }

  // One block of chain c from slot `slot` (its loads have landed for every
  // wave: the caller waited and synchronised).
  auto compute = [&](auto slot_c, auto chain, int blk) __attribute__((always_inline)) {
    constexpr int c = decltype(chain)::value;
    constexpr int slot = decltype(slot_c)::value;
    constexpr int h = slot * C::SLOT * 16 / 65536;
    constexpr int SOFF = slot * C::SLOT * 16 % 65536;
    // Scores: S^T tiles (16 keys x 16 columns); lane (g, r16) holds keys
    // 16kt + 4g + e of column r16.
    // Both key halves' reads are issued first; the first half's products run
    // while the second half's reads are in flight.
    f32x4_t sc[2];
    {
      u32x4_t kl[2][NQ];
#pragma unroll
      for (int kt = 0; kt < 2; kt++)
#pragma unroll
        for (int i = 0; i < NQ; i++) kl[kt][i] = ds_read_b128_at(kofs[h][i], SOFF + kt * 16 * CH * 16);
      asm volatile("s_waitcnt lgkmcnt(%0)" ::"i"(NQ) : "memory");
#pragma unroll
      for (int i = 0; i < NQ; i++) asm volatile("" : "+v"(kl[0][i]));
      sc[0] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < NQ; i++)
        sc[0] = mma32(T(0), __builtin_bit_cast(uint4, kl[0][i]), qt[i], sc[0]);
      // sc[0] as an operand keeps the first half's MFMAs ahead of this wait
      // (the compiler does not order MFMAs against asm statements otherwise).
      asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(sc[0]) :: "memory");
#pragma unroll
      for (int i = 0; i < NQ; i++) asm volatile("" : "+v"(kl[1][i]));
      sc[1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < NQ; i++)
        sc[1] = mma32(T(0), __builtin_bit_cast(uint4, kl[1][i]), qt[i], sc[1]);
    }
    // V^T blocks (dims 16db .., keys 16kt + 4g ..): lane r16 receives
    // V[16kt + 4g + t][16db + r16]. Read before the softmax, which hides
    // their latency.
    u32x2_t va[NB][2];
#pragma unroll
    for (int db = 0; db < NB; db++)
#pragma unroll
      for (int kt = 0; kt < 2; kt++)
        va[db][kt] = ds_read_tr_at(vofs[h][db], SOFF + kt * 16 * VCH * 16);
    // Softmax of chain c over the block (the per-column steps of
    // sdpa_mfma_kernel, in the same order).
    const int key0 = blk * kBlk + 4 * g;
    uint2 ph[2];
    float f;
    auto softmax = [&](auto full_tag) __attribute__((always_inline)) {
      constexpr bool FULL = decltype(full_tag)::value;
      bool use[2][4];
      float bm = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 2; kt++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
          use[kt][e] = FULL || key0 + 16 * kt + e < kend;
          bm = use[kt][e] ? fmaxf(bm, sc[kt][e]) : bm;
        }
      // The column's maximum is one of its four lanes' maxima, so the column
      // moves its base iff one of its lanes' own scaled maxima exceeds
      // m + 8 (the same product, the same compare). When no lane of the
      // wave does, every column keeps m and f = 1 without the cross-lane
      // maximum; otherwise the full step runs, with the same result.
      const float m8 = m[c] + 8.f;
      float mn = m[c];
      f = 1.f;
      if (__builtin_amdgcn_ballot_w64(bm * p.ascale2 > m8) != 0) {  // wave-uniform
        bm = col_max(bm) * p.ascale2;
        const bool any = bm > -INFINITY;
        mn = (any && bm > m8) ? bm : m[c];
        f = mn == m[c] ? 1.f : __builtin_amdgcn_exp2f(m[c] - mn);
      }
      float pv[2][4];
      float ps = 0.f;
#pragma unroll
      for (int kt = 0; kt < 2; kt++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
          pv[kt][e] = use[kt][e] ? __builtin_amdgcn_exp2f(__builtin_fmaf(sc[kt][e], p.ascale2, -mn)) : 0.f;
          ps = kt + e == 0 ? pv[0][0] : ps + pv[kt][e];  // p >= +0: the same as 0 + p
        }
      ps = col_sum(ps);
      l[c] = __builtin_fmaf(l[c], f, ps);
      m[c] = mn;
#pragma unroll
      for (int kt = 0; kt < 2; kt++) ph[kt] = pack_p<T>(pv[kt]);
    };
    if (blk < nfull_w)
      softmax(std::true_type{});
    else
      softmax(std::false_type{});
    // Rescale (+0.0: o is never -0.0).
    if (f != 1.f) {
#pragma unroll
      for (int i = 0; i < NB; i++) o[c][i] = o[c][i] * f + 0.f;
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int db = 0; db < NB; db++) asm volatile("" : "+v"(va[db][0]), "+v"(va[db][1]));
    // o += P . V over the block's 32 keys.
#pragma unroll
    for (int db = 0; db < NB; db++) {
      const uint4 vt =
          join(__builtin_bit_cast(uint2, va[db][0]), __builtin_bit_cast(uint2, va[db][1]));
      o[c][db] = mma32(T(0), vt, join(ph[0], ph[1]), o[c][db]);
    }
  };

  // Group q holds blocks q * GP .. + GP - 1 in slots (q mod NG) * GP ..;
  // groups q + 1 .. q + NG - 1 load while group q is computed. A wave skips
  // a block none of its columns can see (for them it changes nothing).
  // Unrolled over UG groups (UG * GP a multiple of 4, UG a multiple of NG),
  // so slot and chain indices are compile-time.
  constexpr int UG = lcm(NG, GP >= 4 ? 1 : 4 / GP);
#pragma unroll
  for (int u = 0; u < (NG - 1) * GP; u++) issue(u);
  int q0 = 0;
  auto group = [&](auto qc) __attribute__((always_inline)) -> bool {
    constexpr int uq = decltype(qc)::value;
    const int q = q0 + uq;
    if (q * GP >= nblk) return false;  // the same for every wave
    // This wave's loads of group q have landed (those of the NG - 2 groups
    // after it may not have); after the barrier every wave's have, and
    // every wave has finished group q - 1, whose slots take group q + NG - 1.
    __builtin_amdgcn_s_waitcnt(wait_vm((NG - 2) * GP * LPW));
    asm volatile("s_barrier" ::: "memory");
#pragma unroll
    for (int u = 0; u < GP; u++) issue(((uq + NG - 1) % NG) * GP + u);
    auto blockstep = [&](auto bc) __attribute__((always_inline)) -> bool {
      constexpr int u = decltype(bc)::value;
      const int i = q * GP + u;
      if (i >= nblk) return false;
      if (i < nvis_w)
        compute(std::integral_constant<int, (uq % NG) * GP + u>{},
                std::integral_constant<int, (uq * GP + u) % 4>{}, i);
      return true;
    };
    static_for<0, GP>(blockstep);
    return true;
  };
  for (; q0 * GP < nblk; q0 += UG) static_for<0, UG>(group);
  // The loads issued past the last block (they read nothing but still write
  // their slots) complete before the workgroup's LDS is released.
  __builtin_amdgcn_s_waitcnt(kWaitAll);

  // Merge the 4 chains in order, in registers (the sink first: -FLT_MAX
  // without one).
  const float sk = p.sinks ? (float)static_cast<const T*>(p.sinks)[head] * kLog2e : -FLT_MAX;
  float M = sk;
#pragma unroll
  for (int c = 0; c < 4; c++) M = fmaxf(M, m[c]);
  float L = p.sinks ? __builtin_amdgcn_exp2f(sk - M) : 0.f;  // the sink's l = 1
  float ec[4];
#pragma unroll
  for (int c = 0; c < 4; c++) {
    ec[c] = __builtin_amdgcn_exp2f(m[c] - M);
    L = __builtin_fmaf(l[c], ec[c], L);
  }
  T* __restrict__ out = static_cast<T*>(p.out) + ((b * p.H + head) * p.qL + srow) * V;
#pragma unroll
  for (int db = 0; db < NB; db++) {
    f32x4_t O = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 4; c++)
#pragma unroll
      for (int e = 0; e < 4; e++) O[e] = __builtin_fmaf(o[c][db][e], ec[c], O[e]);
    unsigned short ob[4];
#pragma unroll
    for (int e = 0; e < 4; e++) ob[e] = tbits((T)(L == 0.f ? O[e] : O[e] / L));
    if (colv)
      *reinterpret_cast<uint2*>(out + 16 * db + 4 * g) =
          make_uint2(ob[0] | ((uint32_t)ob[1] << 16), ob[2] | ((uint32_t)ob[3] << 16));
  }
}

// Slots of a loader-wave shape: four (a block lands two steps before its
// keys are read) where they fit the 160 KB of LDS, else three (one step).
constexpr int sdpa_loader_slots(int D, int V, int WS) {
  return 4 * kWaves * (kBlk * D / 8 + kBlk * (V / WS) / 8) * 16 <= 160 * 1024 ? 4 : 3;
}

// Kernel of launch shape `SHAPE` (SdpaShape) for head dims (D, V). The rows
// shape with an array mask loads the mask values at the start of their own
// block and no keys ahead, which keeps two workgroups per CU within the
// registers; the split shapes without a mask at D = V = 128 load the keys
// through LDS by contiguous loads (sdpa_loader_slots). Wide heads (D or V above
// 128) load no keys ahead. Keys one block ahead and values in two slots
// otherwise: deeper prefetch measured no faster.
template <typename T, int D, int V, bool MASK, int SHAPE>
constexpr SdpaKernelFn mfma_kernel() {
  constexpr int MK = MASK ? 1 : 0;
  constexpr int PK = sdpa_wide(D, V) ? 0 : 1;
  constexpr int WS = sdpa_shape_splits(V, SHAPE);
  if constexpr (SHAPE == SDPA_SHARED) {
    if constexpr (sdpa_shared_dims(D, V) && !MASK)
      return sdpa_shared_kernel<T, D, V, sdpa_shared_waves(D, V), 2, 2>;
    else
      return nullptr;
  } else if constexpr (SHAPE == SDPA_ROWS) {
    return sdpa_mfma_kernel<T, D, V, sdpa_rows_tiles(D, V), MASK ? 0 : PK, 2, WS, MASK ? 2 : 0,
                            false, 0>;
  } else if constexpr (SHAPE == SDPA_TILE) {
    return sdpa_mfma_kernel<T, D, V, 1, PK, 2, WS, MK, false, 0>;
  } else {
    // Keys in LDS with loader waves (sdpa_loaders: the host launches 8 waves).
    constexpr bool KLS = sdpa_loaders(D, V, SHAPE, MASK);
    return sdpa_mfma_kernel<T, D, V, 1, KLS ? 0 : PK, KLS ? sdpa_loader_slots(D, V, WS) : 2, WS, MK, KLS,
                            KLS ? kWaves : 0>;
  }
}

template <typename T, int D, int V, bool MASK>
SdpaKernelFn mfma_kernel_shape(int shape) {
  switch (shape) {
    case SDPA_ROWS: return mfma_kernel<T, D, V, MASK, SDPA_ROWS>();
    case SDPA_TILE: return mfma_kernel<T, D, V, MASK, SDPA_TILE>();
    case SDPA_SPLIT2: return mfma_kernel<T, D, V, MASK, SDPA_SPLIT2>();
    case SDPA_SPLIT4: return mfma_kernel<T, D, V, MASK, SDPA_SPLIT4>();
    case SDPA_SPLIT8: return mfma_kernel<T, D, V, MASK, SDPA_SPLIT8>();
    case SDPA_SHARED: return mfma_kernel<T, D, V, MASK, SDPA_SHARED>();
  }
  return nullptr;
}

template <int D, int V>
SdpaKernelFn mfma_kernel_for(int dtype, bool mask, int shape) {
  if (dtype == BI_BF16)
    return mask ? mfma_kernel_shape<__bf16, D, V, true>(shape)
                : mfma_kernel_shape<__bf16, D, V, false>(shape);
  if (dtype == BI_F16)
    return mask ? mfma_kernel_shape<_Float16, D, V, true>(shape)
                : mfma_kernel_shape<_Float16, D, V, false>(shape);
  return nullptr;
}

}  // namespace

// Defines the lookup of one head-dim pair's kernels (declared in
// bi_sdpa_args.h); each instantiation unit expands it once.
#define BI_SDPA_MFMA_DEFINE(D, V)                                                   \
  SdpaKernelFn sdpa_mfma_kernel_d##D##_v##V(int dtype, bool mask, int shape) {      \
    return mfma_kernel_for<D, V>(dtype, mask, shape);                               \
  }
