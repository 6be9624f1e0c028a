// Batch-invariant single-pass scaled dot product attention for gfx950: the
// fp32 kernel (bf16 and f16 run on matrix cores, bi_sdpa_mfma_kernel.h), and the
// C entry point bi_sdpa that validates arguments and launches either.
//
// Restates the reference bi_sdpa (mlx_batch_invariant/_attention.py:32-149):
// one workgroup owns the whole reduction over the key sequence for a query
// row of a few heads (the query heads of one kv head that share its keys
// under grouped-query attention); keys are split over a fixed number of
// partial online softmaxes by key index; the partials are combined in a fixed
// order. There is no split-KV, no second pass and no route switch on query
// length or context length. How many heads share a workgroup changes only
// which loads are shared, never a head's arithmetic.
//
// Fixed per-row arithmetic (the invariance contract):
//   * 256 threads = 4 waves x 8 groups of 8 lanes = 32 partials. Key i belongs
//     to partial p = i mod 32 (wave p / 8, group p % 8) and each partial walks
//     its keys in ascending order (reference _attention.py:89, 32 simdgroups).
//   * Lane r of a group owns the 16-byte chunks r, r + 8, ... of the head dim.
//     q is pre-multiplied once by scale * log2(e) in fp32 (reference :68-71
//     scales q first); a key's score is the lane's chunk-ordered fma dot
//     product, summed over the 8 lanes by three commutative exchanges, so all 8
//     lanes hold the same bits; plus mask * log2(e).
//   * Online softmax in base 2 with v_exp_f32: the running max starts at the
//     lowest finite float (reference :76-79), f = exp2(m - m'), p = exp2(s - m'),
//     l = fma(l, f, p), o = fma(p, v, o * f). A sink seeds partial 0 with
//     m = sink * log2(e), l = 1 (reference :80-86).
//   * Keys with mask value <= -3e38 are skipped (reference :94-96); a causal
//     key i is used iff i <= s + causal_offset (reference :92-93 with
//     causal_offset = N - qL).
//   * Combine: M = max of the 32 partial maxima, then for p = 0..31 in order
//     L = fma(l_p, exp2(m_p - M), L) and o = fma(o_p, exp2(m_p - M), o);
//     out = L == 0 ? o : o / L (reference :124-141), one rounding to T.
#include <hip/hip_runtime.h>
#include <float.h>
#include <atomic>
#include <stdint.h>

#include <type_traits>

#include "bi_internal.h"
#include "bi_sdpa_args.h"

namespace {

constexpr int kThreads = 256;
constexpr int64_t kMaskSlack = 64;  // keys a block may read past N
constexpr int kPartials = 32;
constexpr int kGroupLanes = 8;
constexpr float kLog2e = 1.4426950408889634f;

template <typename T> __device__ inline float to_f32(T x) { return (float)x; }
// A mask element held as its zero-extended bits (16-bit types) or as itself
// (fp32).
template <typename T, typename R> __device__ inline float raw_to_f32(R x) {
  if constexpr (sizeof(T) == 4)
    return x;
  else
    return (float)__builtin_bit_cast(T, (unsigned short)x);
}
template <typename T> __device__ inline T from_f32(float x) { return (T)x; }  // RNE

template <int CTRL>
__device__ inline float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, false));
}

// Sum over the 8 lanes of a group. Each exchange pairs two lanes that add the
// same two operands (a + b and b + a are the same bits), so every lane of the
// group ends with an identical value.
__device__ inline float group_sum8(float x) {
  x = x + dpp<0xB1>(x);   // quad_perm [1,0,3,2]: lane ^ 1
  x = x + dpp<0x4E>(x);   // quad_perm [2,3,0,1]: lane ^ 2
  x = x + dpp<0x141>(x);  // row_half_mirror: lane i <-> 7 - i within 8 lanes
  return x;
}

__device__ inline int xcd_remap(int w, int total) {
  const int per = total >> 3;
  if (w < (per << 3)) return (w & 7) * per + (w >> 3);
  return w;
}

// This lane's 16-byte chunks r, r + 8, ... of a row of N_ELEM elements.
template <typename T, int N_ELEM>
__device__ inline void load_raw(const T* __restrict__ row, int r, uint4* dst) {
  constexpr int CE = 16 / sizeof(T);
  constexpr int NC = N_ELEM / CE / kGroupLanes;
#pragma unroll
  for (int i = 0; i < NC; i++)
    dst[i] = *reinterpret_cast<const uint4*>(row + (r + kGroupLanes * i) * CE);
}

// Emits nothing, but the values count as produced here and memory accesses
// may not move across: they are computed before any later load is issued.
template <int NE>
__device__ inline void settle(float* x) {
  static_assert(NE % 4 == 0, "groups of four");
#pragma unroll
  for (int e = 0; e < NE; e += 4)
    asm volatile("" : "+v"(x[e]), "+v"(x[e + 1]), "+v"(x[e + 2]), "+v"(x[e + 3]) :: "memory");
}

template <typename T, int NC>
__device__ inline void to_floats(const uint4* src, float* dst) {
  constexpr int CE = 16 / sizeof(T);
#pragma unroll
  for (int i = 0; i < NC; i++) {
    const T* e = reinterpret_cast<const T*>(&src[i]);
#pragma unroll
    for (int t = 0; t < CE; t++) dst[i * CE + t] = to_f32<T>(e[t]);
  }
}

// One workgroup per (batch, kv head, group of GC query heads of that kv head,
// query row). Every key and value row is loaded (and converted) once and used
// by the GC heads, which share it under grouped-query attention; each head
// keeps its own partial softmax state and runs exactly the per-row arithmetic
// described above, so the result of a head does not depend on GC. The key
// rows of the next PF keys of each partial are loaded ahead of their use.
template <typename T, int D, int V, int GC, int PF>
__global__ void __launch_bounds__(kThreads) sdpa_kernel(SdpaArgs p) {
  constexpr int CE = 16 / sizeof(T);
  constexpr int EQ = D / kGroupLanes;  // q/k elements per lane
  constexpr int EV = V / kGroupLanes;  // v/o elements per lane
  constexpr int NCK = EQ / CE, NCV = EV / CE;  // 16-byte chunks per lane
  static_assert(D % (CE * kGroupLanes) == 0 && V % (CE * kGroupLanes) == 0, "head dim");

  __shared__ float part_m[kPartials], part_l[kPartials];
  __shared__ float part_o[kPartials * V];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int part = (tid >> 6) * 8 + (lane >> 3);  // wave * 8 + group
  const int r = lane & 7;

  const int64_t G = p.H / p.Hkv;
  const int64_t NHC = G / GC;  // head groups per kv head
  int64_t t = xcd_remap(blockIdx.x, (int)(p.B * p.Hkv * NHC * p.qL));
  const int64_t hc = t % NHC;
  t /= NHC;
  const int64_t s = t % p.qL;
  t /= p.qL;
  const int64_t kvh = t % p.Hkv;
  const int64_t b = t / p.Hkv;
  const int64_t h0 = kvh * G + hc * GC;  // first query head of this workgroup

  const T* __restrict__ kb = static_cast<const T*>(p.k) + b * p.ks[0] + kvh * p.ks[1];
  const T* __restrict__ vb = static_cast<const T*>(p.v) + b * p.vs[0] + kvh * p.vs[1];

  float q2[GC][EQ];
  float m[GC], l[GC];
  float o[GC][EV];
#pragma unroll
  for (int g = 0; g < GC; g++) {
    const T* __restrict__ qrow =
        static_cast<const T*>(p.q) + b * p.qs[0] + (h0 + g) * p.qs[1] + s * p.qs[2];
    uint4 qc[NCK];
    load_raw<T, D>(qrow, r, qc);
    to_floats<T, NCK>(qc, q2[g]);
#pragma unroll
    for (int e = 0; e < EQ; e++) q2[g][e] = q2[g][e] * p.scale2;
    m[g] = -FLT_MAX;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < EV; e++) o[g][e] = 0.f;
    if (p.sinks && part == 0) {
      m[g] = to_f32<T>(static_cast<const T*>(p.sinks)[h0 + g]) * kLog2e;
      l[g] = 1.f;
    }
  }

  int64_t kend = p.N;
  if (p.mask_mode == BI_MASK_CAUSAL) {
    const int64_t last = s + p.causal_offset;  // last usable key
    kend = last < 0 ? 0 : (last + 1 < p.N ? last + 1 : p.N);
  }
  const T* __restrict__ mbase = nullptr;
  if (p.mask_mode == BI_MASK_ARRAY)
    mbase = static_cast<const T*>(p.mask) + b * p.ms[0] + h0 * p.ms[1] + s * p.ms[2];

  // Key i of this partial: the raw chunks (and raw mask values) of the PF
  // keys ahead live in kq/vq/mq. Loads are unconditional -- a key past the
  // last usable one reloads that key, and its values go unused -- and stay
  // untouched until the key is used: a load under a branch, or arithmetic on
  // a loaded register right after it is issued, would make the wave wait for
  // every load in flight, the prefetched keys included.
  // Mask elements: 16-bit ones are held zero-extended in a register of their
  // own (two in one register would need a merge that waits for the load).
  using MRaw = typename std::conditional<sizeof(T) == 4, float, unsigned short>::type;
  using MReg = typename std::conditional<sizeof(T) == 4, float, uint32_t>::type;
  const MRaw* __restrict__ mraw = reinterpret_cast<const MRaw*>(mbase);
  const int64_t klast = kend - 1;
  uint4 kq[PF][NCK], vq[PF][NCV];
  MReg mq[PF][GC];
  if (kend > 0) {
#pragma unroll
    for (int u = 0; u < PF; u++) {
      const int64_t i0 = part + (int64_t)kPartials * u;
      const int64_t i = i0 < klast ? i0 : klast;
      load_raw<T, D>(kb + i * p.ks[2], r, kq[u]);
      load_raw<T, V>(vb + i * p.vs[2], r, vq[u]);
      if (mraw) {
#pragma unroll
        for (int g = 0; g < GC; g++) mq[u][g] = mraw[g * p.ms[1] + i];
      }
    }
  }
  for (int64_t i0 = part; i0 < kend; i0 += (int64_t)kPartials * PF) {
#pragma unroll
    for (int u = 0; u < PF; u++) {
      const int64_t i = i0 + (int64_t)kPartials * u;
      float kf[EQ], vf[EV], mv[GC];
      to_floats<T, NCK>(kq[u], kf);
      to_floats<T, NCV>(vq[u], vf);
      if (mraw) {
#pragma unroll
        for (int g = 0; g < GC; g++) mv[g] = raw_to_f32<T>(mq[u][g]);
      }
      // Finish converting before the reload below is issued: converted lazily
      // after it, the old and new raw values would need two register sets
      // and a copy that waits for the reload.
      settle<EQ>(kf);
      settle<EV>(vf);
      const int64_t in0 = i + (int64_t)kPartials * PF;
      const int64_t inext = in0 < klast ? in0 : klast;
      load_raw<T, D>(kb + inext * p.ks[2], r, kq[u]);
      load_raw<T, V>(vb + inext * p.vs[2], r, vq[u]);
      if (mraw) {
#pragma unroll
        for (int g = 0; g < GC; g++) mq[u][g] = mraw[g * p.ms[1] + inext];
      }
      if (i < kend) {
#pragma unroll
        for (int g = 0; g < GC; g++) {
          float bias2 = 0.f;
          bool use = true;
          if (mraw) {
            use = mv[g] > -3.0e38f;
            bias2 = mv[g] * kLog2e;
          }
          if (use) {
            float d = 0.f;
#pragma unroll
            for (int e = 0; e < EQ; e++) d = __builtin_fmaf(q2[g][e], kf[e], d);
            const float sc = group_sum8(d) + bias2;
            const float nm = fmaxf(m[g], sc);
            const float f = __builtin_amdgcn_exp2f(m[g] - nm);
            const float pe = __builtin_amdgcn_exp2f(sc - nm);
            m[g] = nm;
            l[g] = __builtin_fmaf(l[g], f, pe);
            // o * f is o exactly when f == 1 (the running max did not move,
            // the usual case after the first keys): skipping the product
            // then changes no bits.
            if (f != 1.f) {
#pragma unroll
              for (int e = 0; e < EV; e++) o[g][e] = o[g][e] * f;
            }
#pragma unroll
            for (int e = 0; e < EV; e++) o[g][e] = __builtin_fmaf(pe, vf[e], o[g][e]);
          }
        }
      }
    }
  }

  // Fixed-order combine of the 32 partials, one head at a time.
#pragma unroll
  for (int g = 0; g < GC; g++) {
    if (r == 0) {
      part_m[part] = m[g];
      part_l[part] = l[g];
    }
#pragma unroll
    for (int i = 0; i < EV / CE; i++)
#pragma unroll
      for (int e = 0; e < CE; e++)
        part_o[part * V + (r + kGroupLanes * i) * CE + e] = o[g][i * CE + e];
    __syncthreads();

    T* __restrict__ out = static_cast<T*>(p.out) + ((b * p.H + h0 + g) * p.qL + s) * V;
    for (int e = tid; e < V; e += kThreads) {
      float mx = part_m[0];
#pragma unroll
      for (int q = 1; q < kPartials; q++) mx = fmaxf(mx, part_m[q]);
      float L = 0.f, acc = 0.f;
#pragma unroll
      for (int q = 0; q < kPartials; q++) {
        const float f = __builtin_amdgcn_exp2f(part_m[q] - mx);
        L = __builtin_fmaf(part_l[q], f, L);
        acc = __builtin_fmaf(part_o[q * V + e], f, acc);
      }
      out[e] = from_f32<T>(L == 0.f ? acc : acc / L);
    }
    __syncthreads();
  }
}

// Compute units of the current device, read once per device.
int device_cus() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// ---------------------------------------------------------------- fp32 shapes
// Shape s of the fp32 kernel groups GC = 2^s query heads per workgroup
// (s = 0..3). The choice only decides which loads are shared.

// Largest heads-per-workgroup built for the head dims: the per-head state
// (q and the output accumulator) grows with them.
int f32_max_group(int64_t D, int64_t V) {
  const int64_t w = D > V ? D : V;
  return w <= 64 ? 8 : w <= 128 ? 4 : 2;
}

// Heads per workgroup: the largest count that divides the query-head group
// and still leaves about two workgroups per compute unit (`rows` query rows in
// all). For D = 128, four heads share one kv stream's loads (decode is
// bandwidth-bound), but need 278 registers, one wave per SIMD; prefill (more
// than 16 query rows) takes two, at 200 registers and twice the waves
// (L = 2048 causal: 1.96 -> 1.38 ms).
int f32_pick_shape(int64_t G, int64_t D, int64_t V, int64_t rows, int64_t qL, int cus) {
  int cap = f32_max_group(D, V);
  if (cap == 4 && qL > 16) cap = 2;
  const int64_t want = 2 * (int64_t)cus;
  int s = 0;
  for (int gc = cap; gc > 1; gc >>= 1)
    if (G % gc == 0 && rows / gc >= want) {
      while ((1 << s) < gc) s++;
      return s;
    }
  return 0;
}

template <typename T, int D, int V>
SdpaKernelFn f32_kernel_for_group(int gc) {
  constexpr int PF = 2;
  constexpr int W = D > V ? D : V;
  switch (gc) {
    case 1: return sdpa_kernel<T, D, V, 1, PF>;
    case 2: return sdpa_kernel<T, D, V, 2, PF>;
    case 4:
      if constexpr (W <= 128) return sdpa_kernel<T, D, V, 4, PF>;
      break;
    case 8:
      if constexpr (W <= 64) return sdpa_kernel<T, D, V, 8, PF>;
      break;
  }
  return nullptr;
}

SdpaKernelFn f32_kernel(int64_t D, int64_t V, int shape) {
  if (shape < 0 || shape > 3) return nullptr;
#define BI_F32_CASE(d, v) \
  if (D == d && V == v) return f32_kernel_for_group<float, d, v>(1 << shape);
  BI_SDPA_DIM_PAIRS(BI_F32_CASE)
#undef BI_F32_CASE
  return nullptr;
}

// ---------------------------------------------------------------- MFMA shapes

SdpaKernelFn mfma_kernel(int64_t D, int64_t V, int dtype, bool mask, int shape) {
#define BI_MFMA_CASE(d, v) \
  if (D == d && V == v) return sdpa_mfma_kernel_d##d##_v##v(dtype, mask, shape);
  BI_SDPA_DIM_PAIRS(BI_MFMA_CASE)
#undef BI_MFMA_CASE
  return nullptr;
}

// Prefill (a kv head has more than 16 columns): "shared" for D = V = 128
// without an array mask when its grid of 128-column workgroups (one per
// compute unit at a time) covers at least 4/5 of the compute units and fills
// at least 3/4 of its rounds over them, or gives every compute unit two
// (L = 2048 causal: 113 -> 88 us; B = 1, 1024 query rows over 4200 keys:
// rows 166 us, shared 129 us; at 192 workgroups the two tie, at 320 rows
// wins; at D = 64 and 32 shared measured slower), else "rows" when that
// grid fills the compute units. Otherwise one
// column tile, with the output dims split over 2, 4 or 8 workgroups when the
// grid of column tiles would leave compute units idle: decode, and short
// chunks of prefill such as 16 query rows.
int mfma_pick_shape(int64_t D, int64_t V, int64_t ncol, int64_t streams, bool array_mask,
                    int cus) {
  // Shared needs its workgroups at least half full: with a few query rows
  // per kv head (B = 64, qL = 5 or 8: 20 or 32 of 128 columns) most of its
  // waves would idle while the others walk every block (rows 360 us against
  // 387 us at N = 8192); from 64 columns it leads (qL = 17: 416 against 579 us).
  const int sc = sdpa_shape_columns(D, V, SDPA_SHARED);
  if (2 * ncol >= sc && D == 128 && V == 128 && !array_mask) {
    const int64_t w = streams * ((ncol + sc - 1) / sc);
    const int64_t rounds = (w + cus - 1) / cus;
    if (w >= 2 * (int64_t)cus || (5 * w >= 4 * (int64_t)cus && 4 * w >= 3 * rounds * cus))
      return SDPA_SHARED;
  }
  const int rc = sdpa_shape_columns(D, V, SDPA_ROWS);
  if (ncol > 16 && streams * ((ncol + rc - 1) / rc) >= cus) return SDPA_ROWS;
  const int64_t tiles = streams * ((ncol + 15) / 16);  // workgroups at one column tile
  // The fewest rounds of workgroups over the CUs, counting one dim-split
  // workgroup and two one-tile workgroups per CU at a time, then the most
  // workgroups per column tile. A half-used round costs a whole one (decode
  // B=6, N=8192, D=128: 8-way split in 384 workgroups 68 us, 4-way in 192
  // 37 us; B=24: 2-way 156 us, one tile 137 us; the same at D=64 and 256
  // and with an array mask).
  int best = SDPA_TILE;
  int64_t best_rounds = (tiles * sdpa_shape_splits(V, SDPA_TILE) + 2 * (int64_t)cus - 1) /
                        (2 * (int64_t)cus);
  for (int s = SDPA_SPLIT2; s <= SDPA_SPLIT8; s++) {
    const int64_t r = (tiles * sdpa_shape_splits(V, s) + cus - 1) / cus;
    if (r <= best_rounds) {
      best = s;
      best_rounds = r;
    }
  }
  return best;
}

bool dims_built(int64_t D, int64_t V) {
#define BI_DIMS_CASE(d, v) \
  if (D == d && V == v) return true;
  BI_SDPA_DIM_PAIRS(BI_DIMS_CASE)
#undef BI_DIMS_CASE
  return false;
}

int pick_shape(int64_t B, int64_t H, int64_t Hkv, int64_t qL, int64_t D, int64_t V, int dtype,
               int mask_mode, int cus) {
  if (dtype == BI_F32) return f32_pick_shape(H / Hkv, D, V, B * H * qL, qL, cus);
  return mfma_pick_shape(D, V, (H / Hkv) * qL, B * Hkv, mask_mode == BI_MASK_ARRAY, cus);
}

// Columns (query heads for fp32, (head, row) columns otherwise) and output-dim
// splits per workgroup of a shape; false if it is not built.
bool shape_geometry(int64_t D, int64_t V, int dtype, int shape, int* columns, int* splits) {
  if (dtype == BI_F32) {
    if (!f32_kernel(D, V, shape)) return false;
    *columns = 1 << shape;
    *splits = 1;
    return true;
  }
  if (shape < 0 || shape >= SDPA_NUM_SHAPES || !mfma_kernel(D, V, dtype, false, shape))
    return false;
  *columns = sdpa_shape_columns(D, V, shape);
  *splits = sdpa_shape_splits(V, shape);
  return true;
}

// Validates, packs the arguments and launches shape `shape` (-1: the shape
// bi_sdpa picks).
int sdpa_run(const void* q, const void* k, const void* v, const void* mask,
             const int64_t* mask_strides, const void* sinks, void* out, int64_t B, int64_t H,
             int64_t Hkv, int64_t qL, int64_t N, int64_t D, int64_t V,
             const int64_t* qkv_strides, float scale, int mask_mode, int64_t causal_offset,
             int dtype, int shape, void* hip_stream) {
  const int esz = bi::elem_size(dtype);
  if (!esz) return bi::fail(BI_EINVAL, "bi_sdpa: unknown dtype %d", dtype);
  if (B < 0 || H <= 0 || Hkv <= 0 || qL < 0 || N < 0 || D <= 0 || V <= 0)
    return bi::fail(BI_EINVAL, "bi_sdpa: bad sizes B=%lld H=%lld Hkv=%lld qL=%lld N=%lld D=%lld V=%lld",
                    (long long)B, (long long)H, (long long)Hkv, (long long)qL, (long long)N,
                    (long long)D, (long long)V);
  if (H % Hkv) return bi::fail(BI_EINVAL, "bi_sdpa: H=%lld is not a multiple of Hkv=%lld",
                               (long long)H, (long long)Hkv);
  if (mask_mode != BI_MASK_NONE && mask_mode != BI_MASK_CAUSAL && mask_mode != BI_MASK_ARRAY)
    return bi::fail(BI_EINVAL, "bi_sdpa: unknown mask mode %d", mask_mode);
  if (mask_mode == BI_MASK_ARRAY && (!mask || !mask_strides))
    return bi::fail(BI_EINVAL, "bi_sdpa: array mask needs a mask pointer and strides");
  if (!dims_built(D, V))
    return bi::fail(BI_EUNSUPPORTED, "bi_sdpa: head dims D=%lld V=%lld are not built "
                    "(supported: D == V in {32, 64, ..., 512}; (D, V) in {(192, 128), (128, 64), "
                    "(64, 128), (256, 128), (128, 256), (576, 512)})",
                    (long long)D, (long long)V);
  const int64_t rows = B * H * qL;
  if (rows == 0) return BI_OK;
  if (rows > INT32_MAX) return bi::fail(BI_EINVAL, "bi_sdpa: B*H*qL too large");
  if (N > INT32_MAX - 1024) return bi::fail(BI_EINVAL, "bi_sdpa: N=%lld keys is too many", (long long)N);
  if (!q || !out || (N > 0 && (!k || !v)))
    return bi::fail(BI_EINVAL, "bi_sdpa: null tensor pointer");

  SdpaArgs p;
  p.q = q;
  p.k = k;
  p.v = v;
  p.mask = mask_mode == BI_MASK_ARRAY ? mask : nullptr;
  p.sinks = sinks;
  p.out = out;
  p.B = B;
  p.H = H;
  p.Hkv = Hkv;
  p.qL = qL;
  p.N = N;
  if (qkv_strides) {
    for (int i = 0; i < 3; i++) {
      p.qs[i] = qkv_strides[i];
      p.ks[i] = qkv_strides[3 + i];
      p.vs[i] = qkv_strides[6 + i];
    }
  } else {
    p.qs[0] = H * qL * D, p.qs[1] = qL * D, p.qs[2] = D;
    p.ks[0] = Hkv * N * D, p.ks[1] = N * D, p.ks[2] = D;
    p.vs[0] = Hkv * N * V, p.vs[1] = N * V, p.vs[2] = V;
  }
  const int ce = 16 / esz;
  for (int i = 0; i < 3; i++) {
    if (p.qs[i] % ce || p.ks[i] % ce || p.vs[i] % ce)
      return bi::fail(BI_EINVAL, "bi_sdpa: q/k/v strides must be multiples of %d elements", ce);
  }
  if ((uintptr_t)q % 16 || (N > 0 && ((uintptr_t)k % 16 || (uintptr_t)v % 16)))
    return bi::fail(BI_EINVAL, "bi_sdpa: q, k and v must be 16-byte aligned");
  for (int i = 0; i < 3; i++) p.ms[i] = (mask_mode == BI_MASK_ARRAY) ? mask_strides[i] : 0;
  p.scale2 = scale * 1.4426950408889634f;
  p.ascale2 = (scale < 0.f ? -scale : scale) * 1.4426950408889634f;
  p.qsign = scale < 0.f ? 0x80008000u : 0u;
  p.mask_mode = mask_mode;
  p.causal_offset = mask_mode == BI_MASK_CAUSAL ? causal_offset : 0;

  // The MFMA kernel addresses 32 key / value rows from a block's first row,
  // and a batch's mask, with 32-bit byte offsets.
  if (dtype != BI_F32) {
    const int64_t st = p.ks[2] > p.vs[2] ? p.ks[2] : p.vs[2];
    if ((32 * st + (D > V ? D : V)) * esz > INT32_MAX)
      return bi::fail(BI_EUNSUPPORTED, "bi_sdpa: key/value row stride %lld is too large",
                      (long long)st);
    if (mask_mode == BI_MASK_ARRAY &&
        ((H - 1) * p.ms[1] + (qL - 1) * p.ms[2] + N + kMaskSlack) * esz > INT32_MAX)
      return bi::fail(BI_EUNSUPPORTED, "bi_sdpa: the mask of one batch entry is too large");
  }
  if (shape < 0) shape = pick_shape(B, H, Hkv, qL, D, V, dtype, mask_mode, device_cus());
  int columns = 0, splits = 0;
  if (!shape_geometry(D, V, dtype, shape, &columns, &splits))
    return bi::fail(BI_EINVAL, "bi_sdpa: launch shape %d is not built for dtype %d D=%lld V=%lld",
                    shape, dtype, (long long)D, (long long)V);
  // fp32 runs on the VALU kernel above; bf16 and f16 on matrix cores
  // (bi_sdpa_mfma_kernel.h). Each is the only arithmetic for its element type.
  SdpaKernelFn fn;
  int64_t blocks;
  if (dtype == BI_F32) {
    if ((H / Hkv) % columns)
      return bi::fail(BI_EINVAL, "bi_sdpa: %d heads per workgroup do not divide the %lld query "
                      "heads of a kv head", columns, (long long)(H / Hkv));
    fn = f32_kernel(D, V, shape);
    blocks = rows / columns;
  } else {
    fn = mfma_kernel(D, V, dtype, mask_mode == BI_MASK_ARRAY, shape);
    const int64_t ncol = (H / Hkv) * qL;
    blocks = B * Hkv * ((ncol + columns - 1) / columns) * splits;
  }
  if (blocks > INT32_MAX) return bi::fail(BI_EINVAL, "bi_sdpa: grid too large");
  if (!fn)
    return bi::fail(BI_EINVAL, "bi_sdpa: launch shape %d is not built for this mask", shape);
  const int threads =
      dtype == BI_F32 ? kThreads : sdpa_shape_threads(D, V, shape, mask_mode == BI_MASK_ARRAY);
  hipLaunchKernelGGL(fn, dim3((unsigned)blocks), dim3(threads), 0,
                     static_cast<hipStream_t>(hip_stream), p);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return bi::launch_error(e, "bi_sdpa launch");
  return BI_OK;
}

}  // namespace

extern "C" int bi_sdpa(const void* q, const void* k, const void* v, const void* mask,
                       const int64_t* mask_strides, const void* sinks, void* out, int64_t B,
                       int64_t H, int64_t Hkv, int64_t qL, int64_t N, int64_t D, int64_t V,
                       const int64_t* qkv_strides, float scale, int mask_mode,
                       int64_t causal_offset, int dtype, void* hip_stream) {
  return sdpa_run(q, k, v, mask, mask_strides, sinks, out, B, H, Hkv, qL, N, D, V, qkv_strides,
                  scale, mask_mode, causal_offset, dtype, -1, hip_stream);
}

extern "C" int bi_sdpa_with_shape(const void* q, const void* k, const void* v, const void* mask,
                                  const int64_t* mask_strides, const void* sinks, void* out,
                                  int64_t B, int64_t H, int64_t Hkv, int64_t qL, int64_t N,
                                  int64_t D, int64_t V, const int64_t* qkv_strides, float scale,
                                  int mask_mode, int64_t causal_offset, int dtype, int shape,
                                  void* hip_stream) {
  if (shape < 0) return bi::fail(BI_EINVAL, "bi_sdpa_with_shape: shape %d", shape);
  return sdpa_run(q, k, v, mask, mask_strides, sinks, out, B, H, Hkv, qL, N, D, V, qkv_strides,
                  scale, mask_mode, causal_offset, dtype, shape, hip_stream);
}

extern "C" int bi_sdpa_pick_shape(int64_t B, int64_t H, int64_t Hkv, int64_t qL, int64_t D,
                                  int64_t V, int dtype, int mask_mode, int cus) {
  if (!bi::elem_size(dtype)) return bi::fail(BI_EINVAL, "bi_sdpa_pick_shape: unknown dtype %d", dtype);
  if (B <= 0 || H <= 0 || Hkv <= 0 || qL <= 0 || H % Hkv || cus < 0)
    return bi::fail(BI_EINVAL, "bi_sdpa_pick_shape: bad sizes");
  if (mask_mode != BI_MASK_NONE && mask_mode != BI_MASK_CAUSAL && mask_mode != BI_MASK_ARRAY)
    return bi::fail(BI_EINVAL, "bi_sdpa_pick_shape: unknown mask mode %d", mask_mode);
  if (!dims_built(D, V))
    return bi::fail(BI_EUNSUPPORTED, "bi_sdpa_pick_shape: head dims D=%lld V=%lld are not built",
                    (long long)D, (long long)V);
  return pick_shape(B, H, Hkv, qL, D, V, dtype, mask_mode, cus > 0 ? cus : device_cus());
}

extern "C" int bi_sdpa_shape_info(int64_t D, int64_t V, int dtype, int shape, int* columns,
                                  int* splits) {
  int c = 0, w = 0;
  if (!bi::elem_size(dtype) || !shape_geometry(D, V, dtype, shape, &c, &w))
    return bi::fail(BI_EINVAL, "bi_sdpa_shape_info: no shape %d for dtype %d D=%lld V=%lld",
                    shape, dtype, (long long)D, (long long)V);
  if (columns) *columns = c;
  if (splits) *splits = w;
  return BI_OK;
}
