// Batch-invariant GEMM for gfx950 (MI355X).
//
// Restates the reference bi_gemm (mlx_batch_invariant/_gemm.py:29-130): one
// workgroup owns an output tile and the whole K reduction for it, the K-loop
// trip count depends on K alone, tiles are staged through LDS, and the bias is
// added to the fp32 accumulator before the single rounding to the element type
// (_gemm.py:115-129). No split-K, no atomics.
//
// Fixed per-element arithmetic (the invariance contract):
//   * K is walked in stages of 128 bytes per row: 64 elements for bf16/f16,
//     32 for fp32. Stage s is zero-padded past K; the number of stages is
//     ceil(K / stage), a function of K only.
//   * A stage is two chunk-steps j = 0, 1. In chunk-step j, lane group
//     g = lane / 16 of an MFMA holds the 16-byte chunk c = 4j + g of its row.
//       bf16/f16: one v_mfma_f32_16x16x32_{bf16,f16} per chunk-step; lane group
//                 g supplies k = 64s + 32j + 8g + t, t = 0..7.
//       fp32:     four v_mfma_f32_16x16x4_f32 per chunk-step, t = 0..3; lane
//                 group g supplies k = 32s + 16j + 4g + t. Chunk-step j
//                 accumulates into its own chain acc_j (two chains halve the
//                 length of each fp32 accumulation), and acc = acc_0 + acc_1.
//     Every output element sees exactly this sequence of MFMAs on its own row
//     of A and column of B, each chain starting from +0.0.
//   * Epilogue: v = bias ? fma(alpha, acc, beta * bias[n]) : acc, then one
//     round-to-nearest-even to the element type.
// The workgroup footprint (rows x columns of C per workgroup, waves per
// workgroup) is a table of compile-time geometries that all run this same
// sequence per element; it only decides how many elements a workgroup owns.
// An output row therefore has the same bits whatever M is, whatever rows
// surround it, whichever slot of a tile it lands in, and whichever geometry
// the launch picked.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "bi_internal.h"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;

constexpr int kRowBytes = 128;              // bytes of K per tile row per stage
constexpr int kChunks = kRowBytes / 16;     // 16-byte chunks per tile row

struct GemmArgs {
  const void* a;
  const void* b;
  const void* bias;
  void* out;
  int64_t M, N, K;
  int tiles_m, tiles_n;
  float alpha, beta;
  int vec_a, vec_b;  // rows of A / rows of B may be read as aligned 16-byte vectors
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

// Workgroups are dispatched round-robin over the 8 XCDs (each with its own L2).
// Remap so that consecutive logical tiles -- which share operand panels -- run
// on the same XCD.
__device__ inline int xcd_remap(int w, int total) {
  const int per = total >> 3;
  if (w < (per << 3)) return (w & 7) * per + (w >> 3);
  return w;
}

// 16 bytes of a K-contiguous row starting at element k; elements at or past
// `limit` read as zero.
template <typename T>
__device__ inline uint4 load_row_chunk(const T* row, int64_t k, int64_t limit, bool vec) {
  constexpr int E = 16 / sizeof(T);
  if (vec && k + E <= limit) return *reinterpret_cast<const uint4*>(row + k);
  union {
    uint4 u;
    T e[E];
  } r;
#pragma unroll
  for (int i = 0; i < E; i++) r.e[i] = (k + i < limit) ? row[k + i] : T(0);
  return r.u;
}

// Chunk swizzles: 16-byte chunk c of LDS row r is stored at chunk position
// c ^ swz(r) so that the MFMA operand reads of 16 consecutive rows spread over
// the LDS banks.
__device__ inline int swz_k(int r) { return r & 7; }  // [rows][8 chunks] tiles
template <typename T, int CPR>
__device__ inline int swz_nn(int k) {  // [k][CPR chunks] tiles (B in (K, N) layout)
  if constexpr (sizeof(T) == 2)
    return (((k & 3) << 1) | (((k >> 3) & 1) << 3)) & (CPR - 1);
  else
    return (((k >> 2) & 3) << 2) & (CPR - 1);
}

template <typename T, int BM, int BN, int WM, int WN, bool TB>
__global__ void __launch_bounds__(64 * WM * WN) gemm_kernel(GemmArgs p) {
  constexpr int NT = 64 * WM * WN;
  constexpr int EPC = 16 / sizeof(T);          // elements per 16-byte chunk
  constexpr int EPS = kRowBytes / sizeof(T);   // elements of K per stage
  constexpr int WTM = BM / WM, WTN = BN / WN;  // wave tile
  constexpr int FM = WTM / 16, FN = WTN / 16;  // 16x16 MFMA blocks per wave
  constexpr int A_CH = BM * kChunks;           // chunks per stage
  constexpr int B_CH = BN * kChunks;
  constexpr int LA = (A_CH + NT - 1) / NT;     // chunks per thread per stage
  constexpr int LB = (B_CH + NT - 1) / NT;
  constexpr int NN_CPR = BN * (int)sizeof(T) / 16;  // chunks per k-row of a (K, N) B tile
  constexpr int STAGE_CH = A_CH + B_CH;
  static_assert(FM >= 1 && FN >= 1 && WTM % 16 == 0 && WTN % 16 == 0, "bad geometry");
  static_assert(TB || (NN_CPR >= 1 && (NN_CPR & (NN_CPR - 1)) == 0), "bad (K,N) tile width");

  __shared__ uint4 smem[2 * STAGE_CH];

  const T* __restrict__ A = static_cast<const T*>(p.a);
  const T* __restrict__ B = static_cast<const T*>(p.b);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int g = lane >> 4, r16 = lane & 15;

  const int tile = xcd_remap(blockIdx.x, p.tiles_m * p.tiles_n);
  const int64_t m0 = (int64_t)(tile % p.tiles_m) * BM;
  const int64_t n0 = (int64_t)(tile / p.tiles_m) * BN;
  const int64_t M = p.M, N = p.N, K = p.K;
  const int64_t nst = (K + EPS - 1) / EPS;
  const bool vec_a = p.vec_a, vec_b = p.vec_b;

  // 16-row / 16-column blocks of this wave that hold at least one valid output.
  const int64_t wrow = m0 + wm * WTM, wcol = n0 + wn * WTN;
  const int fm_valid = (int)max((int64_t)0, min((int64_t)FM, (M - wrow + 15) / 16));
  const int fn_valid = (int)max((int64_t)0, min((int64_t)FN, (N - wcol + 15) / 16));

  uint4 ra[LA], rb[LB];

  auto gload = [&](int64_t s) {
    const int64_t k0 = s * EPS;
#pragma unroll
    for (int i = 0; i < LA; i++) {
      const int q = tid + i * NT;
      if (A_CH % NT == 0 || q < A_CH) {
        const int r = q / kChunks, c = q % kChunks;
        const int64_t gr = m0 + r;
        ra[i] = (gr < M) ? load_row_chunk<T>(A + gr * K, k0 + c * EPC, K, vec_a)
                         : make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int i = 0; i < LB; i++) {
      const int q = tid + i * NT;
      if (B_CH % NT == 0 || q < B_CH) {
        if constexpr (TB) {
          const int r = q / kChunks, c = q % kChunks;
          const int64_t gn = n0 + r;
          rb[i] = (gn < N) ? load_row_chunk<T>(B + gn * K, k0 + c * EPC, K, vec_b)
                           : make_uint4(0, 0, 0, 0);
        } else {
          const int r = q / NN_CPR, c = q % NN_CPR;
          const int64_t gk = k0 + r;
          rb[i] = (gk < K) ? load_row_chunk<T>(B + gk * N, n0 + c * EPC, N, vec_b)
                           : make_uint4(0, 0, 0, 0);
        }
      }
    }
  };

  auto sstore = [&](int buf) {
    uint4* As = smem + buf * STAGE_CH;
    uint4* Bs = As + A_CH;
#pragma unroll
    for (int i = 0; i < LA; i++) {
      const int q = tid + i * NT;
      if (A_CH % NT == 0 || q < A_CH) {
        const int r = q / kChunks, c = q % kChunks;
        As[r * kChunks + (c ^ swz_k(r))] = ra[i];
      }
    }
#pragma unroll
    for (int i = 0; i < LB; i++) {
      const int q = tid + i * NT;
      if (B_CH % NT == 0 || q < B_CH) {
        if constexpr (TB) {
          const int r = q / kChunks, c = q % kChunks;
          Bs[r * kChunks + (c ^ swz_k(r))] = rb[i];
        } else {
          const int r = q / NN_CPR, c = q % NN_CPR;
          Bs[r * NN_CPR + (c ^ swz_nn<T, NN_CPR>(r))] = rb[i];
        }
      }
    }
  };

  // B operand chunk for chunk-step j of 16-column block starting at tile column nb.
  auto load_b = [&](const uint4* Bs, int j, int nb) -> uint4 {
    if constexpr (TB) {
      const int r = nb + r16;
      return Bs[r * kChunks + ((4 * j + g) ^ swz_k(r))];
    } else if constexpr (sizeof(T) == 2) {
      // ds_read_tr16_b64: in each 16-lane group, lane i receives element
      // (row 4t + i/4, column i%4) of the 16 x (4 x 16-bit) rows addressed by
      // the group's lanes. Lane r16 addresses k-row kb + r16/4 at column
      // nb + 4 * (r16 % 4), so lane i receives B[kb + t][nb + i], t = 0..3.
      uint2 h[2];
#pragma unroll
      for (int half = 0; half < 2; half++) {
        const int kr = 32 * j + 8 * g + 4 * half + (r16 >> 2);
        const int col = nb + 4 * (r16 & 3);
        const int chunk = (col >> 3) ^ swz_nn<T, NN_CPR>(kr);
        const char* addr = reinterpret_cast<const char*>(Bs) + (kr * NN_CPR + chunk) * 16 + (col & 7) * 2;
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
        const int col = nb + r16;
        const int chunk = (col >> 2) ^ swz_nn<T, NN_CPR>(kr);
        e[t] = __float_as_uint(Bf[(kr * NN_CPR + chunk) * 4 + (col & 3)]);
      }
      return make_uint4(e[0], e[1], e[2], e[3]);
    }
  };

  // fp32 keeps one accumulator chain per chunk-step j; 16-bit types one chain.
  constexpr int CHAINS = sizeof(T) == 4 ? 2 : 1;
  f32x4_t acc[CHAINS][FM][FN];
#pragma unroll
  for (int ch = 0; ch < CHAINS; ch++)
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
      for (int jn = 0; jn < FN; jn++) acc[ch][i][jn] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  if (nst > 0) {
    gload(0);
    sstore(0);
  }
  __syncthreads();

  for (int64_t s = 0; s < nst; ++s) {
    const int buf = (int)(s & 1);
    if (s + 1 < nst) gload(s + 1);
    const uint4* As = smem + buf * STAGE_CH;
    const uint4* Bs = As + A_CH;
#pragma unroll
    for (int j = 0; j < 2; j++) {
      uint4 av[FM], bv[FN];
#pragma unroll
      for (int i = 0; i < FM; i++) {
        if (i < fm_valid) {
          const int r = wm * WTM + i * 16 + r16;
          av[i] = As[r * kChunks + ((4 * j + g) ^ swz_k(r))];
        }
      }
#pragma unroll
      for (int jn = 0; jn < FN; jn++)
        if (jn < fn_valid) bv[jn] = load_b(Bs, j, wn * WTN + jn * 16);
#pragma unroll
      for (int i = 0; i < FM; i++)
        if (i < fm_valid)
#pragma unroll
          for (int jn = 0; jn < FN; jn++)
            if (jn < fn_valid)
              acc[j % CHAINS][i][jn] = chunk_step(T(0), av[i], bv[jn], acc[j % CHAINS][i][jn]);
    }
    if (s + 1 < nst) sstore(buf ^ 1);
    __syncthreads();
  }

  // Epilogue: one rounding per element.
  T* __restrict__ out = static_cast<T*>(p.out);
  const T* __restrict__ bias = static_cast<const T*>(p.bias);
  const float alpha = p.alpha, beta = p.beta;
#pragma unroll
  for (int i = 0; i < FM; i++) {
    if (i >= fm_valid) continue;
#pragma unroll
    for (int jn = 0; jn < FN; jn++) {
      if (jn >= fn_valid) continue;
      const int64_t col = wcol + jn * 16 + r16;
      if (col >= N) continue;
      const float bv = bias ? beta * Elem<T>::to_f32(bias[col]) : 0.f;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int64_t row = wrow + i * 16 + 4 * g + e;
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

// ------------------------------------------------------------------ geometries

struct Geometry {
  int bm, bn, waves;
};

// Footprints of C per workgroup. Every entry runs the same per-element
// arithmetic; the table only trades parallelism against operand reuse.
constexpr Geometry kGeometries[] = {
    {16, 16, 1},    // 0: decode, 1 wave
    {64, 16, 1},    // 1: small M, 1 wave
    {64, 64, 4},    // 2: 4 waves of 32x32
    {128, 64, 4},   // 3: 4 waves of 64x32
    {128, 128, 4},  // 4: 4 waves of 64x64
    {256, 128, 8},  // 5: 8 waves of 64x64
};
constexpr int kNumGeometries = sizeof(kGeometries) / sizeof(kGeometries[0]);

using KernelFn = void (*)(GemmArgs);

template <typename T, bool TB>
KernelFn kernel_for(int g) {
  switch (g) {
    case 0: return gemm_kernel<T, 16, 16, 1, 1, TB>;
    case 1: return gemm_kernel<T, 64, 16, 1, 1, TB>;
    case 2: return gemm_kernel<T, 64, 64, 2, 2, TB>;
    case 3: return gemm_kernel<T, 128, 64, 2, 2, TB>;
    case 4: return gemm_kernel<T, 128, 128, 2, 2, TB>;
    case 5: return gemm_kernel<T, 256, 128, 4, 2, TB>;
  }
  return nullptr;
}

KernelFn select_kernel(int dtype, int trans_b, int g) {
  switch (dtype) {
    case BI_F32: return trans_b ? kernel_for<float, true>(g) : kernel_for<float, false>(g);
    case BI_F16: return trans_b ? kernel_for<_Float16, true>(g) : kernel_for<_Float16, false>(g);
    case BI_BF16: return trans_b ? kernel_for<__bf16, true>(g) : kernel_for<__bf16, false>(g);
  }
  return nullptr;
}

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

int pick_geometry(int64_t M, int64_t N) {
  constexpr int64_t kCUs = 256;
  if (M <= 16) return 0;
  if (M <= 64) return ceil_div(N, 64) >= kCUs ? 2 : 1;
  // Largest footprint that still gives every CU a workgroup.
  for (int g : {5, 4, 3}) {
    const Geometry& G = kGeometries[g];
    if (ceil_div(M, G.bm) * ceil_div(N, G.bn) >= kCUs) return g;
  }
  return 2;
}

int validate(const void* a, const void* b, void* out, int64_t M, int64_t N, int64_t K,
             int dtype, int trans_b) {
  if (dtype != BI_F32 && dtype != BI_F16 && dtype != BI_BF16)
    return bi::fail(BI_EINVAL, "bi_gemm: unknown dtype %d", dtype);
  if (trans_b != 0 && trans_b != 1) return bi::fail(BI_EINVAL, "bi_gemm: trans_b must be 0 or 1");
  if (M < 0 || N < 0 || K < 0)
    return bi::fail(BI_EINVAL, "bi_gemm: negative size M=%lld N=%lld K=%lld", (long long)M,
                    (long long)N, (long long)K);
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX)
    return bi::fail(BI_EINVAL, "bi_gemm: dimension too large");
  if (M == 0 || N == 0) return BI_OK;
  if (!out || (K > 0 && (!a || !b)))
    return bi::fail(BI_EINVAL, "bi_gemm: null operand pointer");
  const int64_t tiles = ceil_div(M, 16) * ceil_div(N, 16);
  if (tiles > INT32_MAX) return bi::fail(BI_EINVAL, "bi_gemm: output too large");
  return BI_OK;
}

int launch(const void* a, const void* b, const void* bias, void* out, int64_t M, int64_t N,
           int64_t K, int dtype, int trans_b, float alpha, float beta, int g, void* stream) {
  const Geometry& G = kGeometries[g];
  GemmArgs p;
  p.a = a;
  p.b = b;
  p.bias = bias;
  p.out = out;
  p.M = M;
  p.N = N;
  p.K = K;
  p.tiles_m = (int)ceil_div(M, G.bm);
  p.tiles_n = (int)ceil_div(N, G.bn);
  p.alpha = alpha;
  p.beta = beta;
  const int esz = bi::elem_size(dtype);
  const int epc = 16 / esz;
  p.vec_a = (K % epc == 0) && ((uintptr_t)a % 16 == 0);
  p.vec_b = (trans_b ? (K % epc == 0) : (N % epc == 0)) && ((uintptr_t)b % 16 == 0);
  const int64_t blocks = (int64_t)p.tiles_m * p.tiles_n;
  if (blocks > INT32_MAX) return bi::fail(BI_EINVAL, "bi_gemm: too many tiles");
  KernelFn fn = select_kernel(dtype, trans_b, g);
  hipLaunchKernelGGL(fn, dim3((unsigned)blocks), dim3(64 * G.waves), 0,
                     static_cast<hipStream_t>(stream), p);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return bi::launch_error(e, "bi_gemm launch");
  return BI_OK;
}

}  // namespace

extern "C" int bi_gemm(const void* a, const void* b, const void* bias, void* out, int64_t M,
                       int64_t N, int64_t K, int dtype, int trans_b, float alpha, float beta,
                       void* hip_stream) {
  const int rc = validate(a, b, out, M, N, K, dtype, trans_b);
  if (rc != BI_OK || M == 0 || N == 0) return rc;
  return launch(a, b, bias, out, M, N, K, dtype, trans_b, alpha, beta, pick_geometry(M, N),
                hip_stream);
}

extern "C" int bi_gemm_num_geometries(void) { return kNumGeometries; }

extern "C" int bi_gemm_geometry_info(int g, int* block_m, int* block_n, int* waves) {
  if (g < 0 || g >= kNumGeometries) return bi::fail(BI_EINVAL, "unknown geometry %d", g);
  if (block_m) *block_m = kGeometries[g].bm;
  if (block_n) *block_n = kGeometries[g].bn;
  if (waves) *waves = kGeometries[g].waves;
  return BI_OK;
}

extern "C" int bi_gemm_pick_geometry(int64_t M, int64_t N, int64_t K, int dtype, int trans_b) {
  (void)K;
  (void)dtype;
  (void)trans_b;
  return pick_geometry(M, N);
}

extern "C" int bi_gemm_with_geometry(const void* a, const void* b, const void* bias, void* out,
                                     int64_t M, int64_t N, int64_t K, int dtype, int trans_b,
                                     float alpha, float beta, int g, void* hip_stream) {
  if (g < 0 || g >= kNumGeometries) return bi::fail(BI_EINVAL, "unknown geometry %d", g);
  const int rc = validate(a, b, out, M, N, K, dtype, trans_b);
  if (rc != BI_OK || M == 0 || N == 0) return rc;
  return launch(a, b, bias, out, M, N, K, dtype, trans_b, alpha, beta, g, hip_stream);
}

namespace {
__global__ void wavefront_size_kernel(int* out) {
  if (threadIdx.x == 0) out[0] = __builtin_amdgcn_wavefrontsize();
}
}  // namespace

extern "C" int bi_device_wavefront_size(int* out) {
  if (!out) return bi::fail(BI_EINVAL, "bi_device_wavefront_size: null output");
  int* d = nullptr;
  hipError_t e = hipMalloc(&d, sizeof(int));
  if (e != hipSuccess) return bi::launch_error(e, "hipMalloc");
  hipLaunchKernelGGL(wavefront_size_kernel, dim3(1), dim3(64), 0, 0, d);
  e = hipMemcpy(out, d, sizeof(int), hipMemcpyDeviceToHost);
  hipFree(d);
  if (e != hipSuccess) return bi::launch_error(e, "wavefront size probe");
  return BI_OK;
}
