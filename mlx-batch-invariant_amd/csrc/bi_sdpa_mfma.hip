// Batch-invariant single-pass attention on MFMA (gfx950), bf16 and f16.
//
// Restates the reference bi_sdpa (mlx_batch_invariant/_attention.py:32-149)
// with matrix cores: one workgroup owns the whole key reduction for each of
// its query columns -- a column is one (query head, query row) pair; the
// columns of a workgroup share a batch index and a kv head, so they read the
// same keys and values -- with no split-KV, no second pass and no switch on
// query length or context length. Which columns share a workgroup, and where
// a column sits in it, never changes the column's arithmetic.
//
// Fixed per-column arithmetic (the invariance contract):
//   * Keys are consumed in blocks of 32 (keys 32b .. 32b + 31), ascending.
//   * Score: raw_i = q . k_i as a chain of v_mfma_f32_16x16x32_{bf16,f16}
//     over the head dim in ascending 32-element chunks from +0.0 (exact
//     products, fp32 sums); s_i = raw_i * (scale * log2 e), plus
//     mask_i * log2 e for an additive mask.
//   * Key i is used iff i < N, i <= row + causal_offset (causal) and
//     mask_i > -3e38 (array mask) (reference :92-96).
//   * Online softmax in base 2, one chain per column over the blocks: with M
//     the largest used score of the block (none: the block leaves the column
//     unchanged), m' = max(m, M), f = m' == m ? 1 : exp2(m - m'),
//     p_i = exp2(s_i - m') (0 for unused keys), l = fma(l, f, sum_i p_i) with
//     the block sum taken in a fixed tree; o = o * f (skipped when f == 1,
//     which changes no bits), then o += p . v as v_mfma_f32_16x16x16 with p
//     split into hi = T(p) and lo = T(p - hi): for each 16-dim block, keys
//     0-15 hi, keys 0-15 lo, keys 16-31 hi, keys 16-31 lo. m starts at the
//     lowest finite float and l at 0; a sink starts them at
//     sink * log2 e and 1 (reference :80-86).
//   * out = l == 0 ? o : o / l, one rounding to T.
// Every column, whatever workgroup, wave or lane it lands in and however many
// rows or heads share its keys, runs exactly this sequence: an output row has
// the same bits for any batch, query length, context past its visible keys,
// and launch shape.
#include <hip/hip_runtime.h>
#include <float.h>
#include <math.h>
#include <stdint.h>

#include "bi_internal.h"
#include "bi_sdpa_args.h"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// 16-byte copies as single vector loads / stores (a uint4 assignment is a
// struct copy, which would keep staged data in scratch memory).
__device__ __forceinline__ uint4 ld16(const void* p) {
  return __builtin_bit_cast(uint4, *reinterpret_cast<const u32x4_t*>(p));
}
__device__ __forceinline__ void st16(uint4* p, uint4 v) {
  *reinterpret_cast<u32x4_t*>(p) = __builtin_bit_cast(u32x4_t, v);
}

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kCols = 16 * kWaves;  // query columns per workgroup
constexpr int kBlk = 32;            // keys per block
constexpr float kLog2e = 1.4426950408889634f;
// s_waitcnt immediate (gfx9 encoding): vmcnt 63 (no wait), expcnt 7, lgkmcnt 0.
constexpr int kWaitLdsOnly = 0xF | (0x3 << 14) | (0x7 << 4);

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
// 16x16x16: lane (r, g) supplies A[r][4g + t] and B[4g + t][r], t = 0..3;
// it receives C[4g + e][r].
__device__ inline f32x4_t mma16(__bf16, uint2 a, uint2 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4_t, a),
                                                   __builtin_bit_cast(i16x4_t, b), c, 0, 0, 0);
}
__device__ inline f32x4_t mma16(_Float16, uint2 a, uint2 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4_t, a),
                                               __builtin_bit_cast(f16x4_t, b), c, 0, 0, 0);
}

template <typename T> __device__ inline unsigned short tbits(T x) {
  return __builtin_bit_cast(unsigned short, x);
}
template <typename T> __device__ inline float tval(unsigned short b) {
  return (float)__builtin_bit_cast(T, b);
}

__device__ inline int xcd_remap(int w, int total) {
  const int per = total >> 3;
  if (w < (per << 3)) return (w & 7) * per + (w >> 3);
  return w;
}

// Sum / max over the four lanes of a column (lanes r, r + 16, r + 32, r + 48,
// one per 16-lane row). permlane16_swap pairs rows (0, 1) and (2, 3),
// permlane32_swap the two halves; every lane adds its pair's operands in the
// same order (lower row first), so all four end with identical bits.
__device__ inline float row_pair(float x, bool is_max) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const float a = __uint_as_float(r[0]), b = __uint_as_float(r[1]);
  return is_max ? fmaxf(a, b) : a + b;
}
__device__ inline float half_pair(float x, bool is_max) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const float a = __uint_as_float(r[0]), b = __uint_as_float(r[1]);
  return is_max ? fmaxf(a, b) : a + b;
}
__device__ inline float col_sum(float x) { return half_pair(row_pair(x, false), false); }
__device__ inline float col_max(float x) { return half_pair(row_pair(x, true), true); }

// Launch shape: CT column tiles of 16 columns per workgroup; the 4 / CT waves
// of a column tile split its output dims, NB 16-dim blocks each, so a
// workgroup covers DW = (4 / CT) * NB * 16 dims and D / DW workgroups share a
// column tile's dims. Waves that share a column tile compute its scores and
// softmax statistics identically. The shape changes which wave does what,
// never a column's arithmetic.
template <typename T, int D, int CT, int NB>
struct Attn {
  static constexpr int DS = kWaves / CT;           // waves per column tile
  static constexpr int DW = DS * NB * 16;          // output dims per workgroup
  static constexpr int WS = D / DW;                // workgroups per column tile
  static constexpr int CH = D / 8;                 // 16-byte chunks per key row
  static constexpr int VCH = DW / 8;               // value chunks per row held
  static constexpr int NQ = D / 32;                // score MFMAs per 16 keys
  static constexpr int SB = D == 256 ? 1 : 2;      // blocks per stage (one barrier)
  static constexpr int SK = SB * kBlk;             // keys per stage
  static constexpr int KCH = SK * CH;              // chunks per K tile
  static constexpr int VTCH = SK * VCH;            // chunks per V tile
  static constexpr int LK = KCH / kThreads;        // K chunks per thread per stage
  static constexpr int LV = (VTCH + kThreads - 1) / kThreads;
  static constexpr int QP = 2;                     // stages of loads in flight
  static_assert(QP % 2 == 0, "the two LDS slots alternate within a round of QP stages");
  static_assert(KCH % kThreads == 0 && D % DW == 0 && NB >= 1, "shape");

  // K tile: [SK keys][CH chunks], chunk c of key r at c ^ swz_k(r): the score
  // MFMA's A reads (16 keys, one chunk each) then hit distinct banks.
  __device__ __forceinline__ static int swz_k(int r) { return r & ((CH < 16 ? CH : 16) - 1); }
  // V tile: [SK keys][VCH chunks] read transposed by ds_read_tr16_b64 (four
  // consecutive keys, 32 bytes each): rows k .. k + 3 land on distinct banks.
  __device__ __forceinline__ static int swz_v(int r) {
    return ((((r & 3) << 1) | (((r >> 3) & 1) << 3))) & (VCH - 1);
  }

  struct Stage {
    uint4 k[LK], v[LV];
  };
  struct Slot {
    uint4* k;
    uint4* v;
  };

  const T* kb;
  const T* vb;  // first of this workgroup's value dims
  int64_t ks2, vs2;
  int klast, tid;

  // Loads of stage s (keys past the last usable one reload it: the values
  // go unused). Loaded registers are left untouched until stored.
  __device__ __forceinline__ void load(int64_t s, Stage& st) const {
#pragma unroll
    for (int i = 0; i < LK; i++) {
      const int q = tid + i * kThreads, r = q / CH, c = q % CH;
      int key = (int)s * SK + r;
      key = key < klast ? key : klast;
      st.k[i] = ld16(kb + (int64_t)key * ks2 + c * 8);
    }
#pragma unroll
    for (int i = 0; i < LV; i++) {
      const int q = tid + i * kThreads;
      if (VTCH % kThreads == 0 || q < VTCH) {
        const int r = q / VCH, c = q % VCH;
        int key = (int)s * SK + r;
        key = key < klast ? key : klast;
        st.v[i] = ld16(vb + (int64_t)key * vs2 + c * 8);
      }
    }
  }
  __device__ __forceinline__ void store(Slot sl, const Stage& st) const {
#pragma unroll
    for (int i = 0; i < LK; i++) {
      const int q = tid + i * kThreads, r = q / CH, c = q % CH;
      st16(sl.k + r * CH + (c ^ swz_k(r)), st.k[i]);
    }
#pragma unroll
    for (int i = 0; i < LV; i++) {
      const int q = tid + i * kThreads;
      if (VTCH % kThreads == 0 || q < VTCH) {
        const int r = q / VCH, c = q % VCH;
        st16(sl.v + r * VCH + (c ^ swz_v(r)), st.v[i]);
      }
    }
  }

  __device__ __forceinline__ void prologue(Stage (&st)[QP], Slot first) const {
#pragma unroll
    for (int u = 0; u < QP; u++) load(u, st[u]);
    store(first, st[0]);
    load(QP, st[0]);
  }

  // Stages s0 .. s0 + QP - 1: before computing stage s0 + u from one LDS
  // slot, stage s0 + u + 1 (loaded QP stages earlier) is stored to the other
  // and stage s0 + u + 1 + QP is loaded in its registers.
  template <typename Slots, typename Compute>
  __device__ __forceinline__ void round(int64_t s0, Stage (&st)[QP], const Slots& slots,
                                        const Compute& compute) const {
#pragma unroll
    for (int u = 0; u < QP; u++) {
      // LDS writes and reads of the previous block retired, then the
      // barrier; the global loads in flight are not waited for.
      __builtin_amdgcn_s_waitcnt(kWaitLdsOnly);
      asm volatile("s_barrier" ::: "memory");
      store(slots((u + 1) & 1), st[(u + 1) % QP]);
      load(s0 + u + 1 + QP, st[(u + 1) % QP]);
      compute(slots(u & 1), s0 + u);
    }
  }
};

template <typename T, int D, int CT, int NB>
__global__ void __launch_bounds__(kThreads) sdpa_mfma_kernel(SdpaArgs p) {
  using A = Attn<T, D, CT, NB>;
  constexpr int CH = A::CH, VCH = A::VCH, NQ = A::NQ, QP = A::QP, DS = A::DS, WS = A::WS;
  constexpr int COLS = 16 * CT;  // columns per workgroup
  __shared__ uint4 k0s[A::KCH], v0s[A::VTCH], k1s[A::KCH], v1s[A::VTCH];
  auto slots = [&](int u) __attribute__((always_inline)) -> typename A::Slot {
    if (u == 0) return {k0s, v0s};
    return {k1s, v1s};
  };

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, r16 = lane & 15;
  const int ct = wave % CT, ds = wave / CT;

  // Workgroup -> (batch, kv head, block of COLS of the G x qL columns of that
  // kv head -- column cc is row cc / G, head cc % G -- and slice of DW dims).
  const int64_t G = p.H / p.Hkv;
  const int64_t ncol = G * p.qL;
  const int64_t ncb = (ncol + COLS - 1) / COLS;
  int64_t t = xcd_remap(blockIdx.x, (int)(p.B * p.Hkv * ncb * WS));
  const int ws = (int)(t % WS);
  t /= WS;
  const int64_t cb = t % ncb;
  t /= ncb;
  const int64_t kvh = t % p.Hkv;
  const int64_t b = t / p.Hkv;
  const int64_t c0 = cb * COLS;
  const int64_t cc = c0 + ct * 16 + r16;  // this lane's column
  const bool colv = cc < ncol;
  const int64_t srow = colv ? cc / G : 0;
  const int64_t head = kvh * G + (colv ? cc % G : 0);
  const bool wave_cols = c0 + ct * 16 < ncol;  // wave-uniform: any column here
  const int dw0 = ws * A::DW + ds * NB * 16;    // first output dim of this wave

  // Keys of a column: [0, kend); the workgroup walks the blocks that its last
  // row can see.
  auto kend_of = [&](int64_t s) __attribute__((always_inline)) -> int64_t {
    if (p.mask_mode != BI_MASK_CAUSAL) return p.N;
    const int64_t last = s + p.causal_offset;
    return last < 0 ? 0 : (last + 1 < p.N ? last + 1 : p.N);
  };
  const int64_t last_cc = (c0 + COLS < ncol ? c0 + COLS : ncol) - 1;
  const int64_t kmax = kend_of(last_cc / G);
  const int kend = colv ? (int)kend_of(srow) : 0;
  const int nkeys = (int)p.N;
  const int64_t nblk = (kmax + kBlk - 1) / kBlk;
  const int64_t nst = (nblk + A::SB - 1) / A::SB;

  // The column's query as the B operand of the score MFMAs: Q[col][32t + 8g ..].
  uint4 qt[NQ];
  {
    const T* qrow = static_cast<const T*>(p.q) + b * p.qs[0] + head * p.qs[1] + srow * p.qs[2];
#pragma unroll
    for (int i = 0; i < NQ; i++)
      qt[i] = colv ? ld16(qrow + 32 * i + 8 * g) : make_uint4(0, 0, 0, 0);
  }
  float m = -FLT_MAX, l = 0.f;
  if (p.sinks && colv) {
    m = (float)static_cast<const T*>(p.sinks)[head] * kLog2e;
    l = 1.f;
  }
  f32x4_t o[NB];
#pragma unroll
  for (int i = 0; i < NB; i++) o[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // Array mask row of the column (lanes without a column read the first row).
  const bool has_mask = p.mask_mode == BI_MASK_ARRAY;
  const T* mrow = has_mask ? static_cast<const T*>(p.mask) + b * p.ms[0] + head * p.ms[1] +
                                 srow * p.ms[2]
                           : nullptr;

  A at;
  at.kb = static_cast<const T*>(p.k) + b * p.ks[0] + kvh * p.ks[1];
  at.vb = static_cast<const T*>(p.v) + b * p.vs[0] + kvh * p.vs[1] + ws * A::DW;
  at.ks2 = p.ks[2];
  at.vs2 = p.vs[2];
  at.klast = (int)p.N - 1;
  at.tid = tid;

  // Block blk (rows 32j .. 32j + 31 of the stage tiles in sl) for this wave's
  // 16 columns and NB dim blocks.
  auto compute = [&](typename A::Slot sl, int j, int64_t blk) __attribute__((always_inline)) {
    // Scores: S^T tiles (16 keys x 16 columns); lane (g, r16) holds keys
    // 16kt + 4g + e of column r16.
    f32x4_t sc[2];
#pragma unroll
    for (int kt = 0; kt < 2; kt++) {
      sc[kt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      const int kr = kBlk * j + 16 * kt + r16;
#pragma unroll
      for (int i = 0; i < NQ; i++)
        sc[kt] = mma32(T(0), ld16(sl.k + kr * CH + ((4 * i + g) ^ A::swz_k(kr))), qt[i], sc[kt]);
    }
    // Key indices fit in 32 bits (the host checks N < 2^31).
    const int key0 = (int)blk * kBlk + 4 * g;
    float s[2][4];
    bool use[2][4];
#pragma unroll
    for (int kt = 0; kt < 2; kt++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        s[kt][e] = sc[kt][e] * p.scale2;
        use[kt][e] = key0 + 16 * kt + e < kend;
      }
    if (has_mask) {  // wave-uniform; every lane loads (in bounds), unused lanes ignore it
#pragma unroll
      for (int kt = 0; kt < 2; kt++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int key = key0 + 16 * kt + e;
          const float mv = (float)mrow[key < nkeys ? key : 0];
          use[kt][e] = use[kt][e] && mv > -3.0e38f;
          s[kt][e] = s[kt][e] + mv * kLog2e;
        }
    }
    float bm = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; kt++)
#pragma unroll
      for (int e = 0; e < 4; e++) bm = use[kt][e] ? fmaxf(bm, s[kt][e]) : bm;
    bm = col_max(bm);
    const bool any = bm > -INFINITY;
    const float mn = any ? fmaxf(m, bm) : m;
    const float f = mn == m ? 1.f : __builtin_amdgcn_exp2f(m - mn);
    float pv[2][4];
    float ps = 0.f;
#pragma unroll
    for (int kt = 0; kt < 2; kt++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        pv[kt][e] = use[kt][e] ? __builtin_amdgcn_exp2f(s[kt][e] - mn) : 0.f;
        ps = ps + pv[kt][e];
      }
    ps = col_sum(ps);
    l = __builtin_fmaf(l, f, ps);
    m = mn;
    // P^T as the B operand of the 16x16x16 MFMAs, split into two planes.
    uint2 ph[2], pl[2];
#pragma unroll
    for (int kt = 0; kt < 2; kt++) {
      unsigned short hb[4], lb[4];
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const T hi = (T)pv[kt][e];
        hb[e] = tbits(hi);
        lb[e] = tbits((T)(pv[kt][e] - (float)hi));
      }
      ph[kt] = make_uint2(hb[0] | ((uint32_t)hb[1] << 16), hb[2] | ((uint32_t)hb[3] << 16));
      pl[kt] = make_uint2(lb[0] | ((uint32_t)lb[1] << 16), lb[2] | ((uint32_t)lb[3] << 16));
    }
    if (f != 1.f) {
#pragma unroll
      for (int i = 0; i < NB; i++) o[i] = o[i] * f;
    }
    // A column with no usable key in this block keeps its o exactly (adding
    // the zero products could still turn a -0.0 into +0.0).
    const bool keep = colv && !any;
    f32x4_t saved[NB];
    const bool slow = __builtin_amdgcn_ballot_w64(keep) != 0;
    if (slow) {
#pragma unroll
      for (int i = 0; i < NB; i++) saved[i] = o[i];
    }
#pragma unroll
    for (int db = 0; db < NB; db++) {
#pragma unroll
      for (int kt = 0; kt < 2; kt++) {
        // V^T block (this wave's dim block db, keys 16kt + 4g ..): lane r16
        // addresses key 16kt + 4g + r16 / 4 at tile dim col and receives
        // V[16kt + 4g + t][col0 + r16], t = 0..3.
        const int kr = kBlk * j + 16 * kt + 4 * g + (r16 >> 2);
        const int col = 16 * (ds * NB + db) + 4 * (r16 & 3);
        const int chunk = (col >> 3) ^ A::swz_v(kr);
        const char* addr = reinterpret_cast<const char*>(sl.v) + (kr * VCH + chunk) * 16 + (col & 7) * 2;
        const uint2 va = __builtin_bit_cast(
            uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(addr)));
        o[db] = mma16(T(0), va, ph[kt], o[db]);
        o[db] = mma16(T(0), va, pl[kt], o[db]);
      }
    }
    if (slow && keep) {
#pragma unroll
      for (int i = 0; i < NB; i++) o[i] = saved[i];
    }
  };

  if (nst > 0) {
    typename A::Stage st[QP];
    at.prologue(st, slots(0));
    for (int64_t s0 = 0; s0 < nst; s0 += QP)
      at.round(s0, st, slots, [&](typename A::Slot sl, int64_t stg) __attribute__((always_inline)) {
        if (wave_cols) {
#pragma unroll
          for (int j = 0; j < A::SB; j++)
            if (stg * A::SB + j < nblk) compute(sl, j, stg * A::SB + j);
        }
      });
  }

  if (!colv) return;
  T* __restrict__ out = static_cast<T*>(p.out) + ((b * p.H + head) * p.qL + srow) * D + dw0;
#pragma unroll
  for (int db = 0; db < NB; db++) {
    unsigned short ob[4];
#pragma unroll
    for (int e = 0; e < 4; e++) ob[e] = tbits((T)(l == 0.f ? o[db][e] : o[db][e] / l));
    *reinterpret_cast<uint2*>(out + 16 * db + 4 * g) =
        make_uint2(ob[0] | ((uint32_t)ob[1] << 16), ob[2] | ((uint32_t)ob[3] << 16));
  }
}

using Fn = void (*)(SdpaArgs);

// Shapes: "wide" (4 column tiles, each wave all dims) whenever its
// workgroups fill the GPU or a kv head has more than 16 columns (prefill);
// "narrow" (1 column tile, dims split over the 4 waves and over workgroups)
// for small decode batches, where the wide grid would leave compute units
// idle.
struct Shape {
  Fn fn;
  int cols, ws;
};

template <typename T, int D>
Shape shape_for(int64_t ncol, int64_t streams, int cus) {
  constexpr int NDB = D / 16;
  const int64_t wide_wgs = streams * ((ncol + 63) / 64);
  if (ncol > 16 || wide_wgs >= cus) return {sdpa_mfma_kernel<T, D, 4, NDB>, 64, 1};
  using N = Attn<T, D, 1, 1>;
  return {sdpa_mfma_kernel<T, D, 1, 1>, 16, N::WS};
}

template <typename T>
Shape shape_for_dims(int64_t D, int64_t ncol, int64_t streams, int cus) {
  switch (D) {
    case 64: return shape_for<T, 64>(ncol, streams, cus);
    case 128: return shape_for<T, 128>(ncol, streams, cus);
    case 256: return shape_for<T, 256>(ncol, streams, cus);
  }
  return {nullptr, 0, 0};
}

}  // namespace

bool sdpa_mfma_launch(const SdpaArgs& p, int dtype, int64_t D, int cus, hipStream_t stream) {
  const int64_t ncol = (p.H / p.Hkv) * p.qL;
  const int64_t streams = p.B * p.Hkv;
  const Shape sh = dtype == BI_BF16 ? shape_for_dims<__bf16>(D, ncol, streams, cus)
                 : dtype == BI_F16  ? shape_for_dims<_Float16>(D, ncol, streams, cus)
                                    : Shape{nullptr, 0, 0};
  if (!sh.fn) return false;
  const int64_t ncb = (ncol + sh.cols - 1) / sh.cols;
  const int64_t blocks = streams * ncb * sh.ws;
  hipLaunchKernelGGL(sh.fn, dim3((unsigned)blocks), dim3(kThreads), 0, stream, p);
  return true;
}
