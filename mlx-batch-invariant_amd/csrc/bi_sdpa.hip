// Batch-invariant single-pass scaled dot product attention for gfx950.
//
// Restates the reference bi_sdpa (mlx_batch_invariant/_attention.py:32-149):
// one workgroup per (batch, query head, query row) owns the whole reduction
// over the key sequence; keys are split over a fixed number of partial online
// softmaxes by key index; the partials are combined in a fixed order. There
// is no split-KV, no second pass and no route switch on query length or
// context length.
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
#include <stdint.h>

#include "bi_internal.h"

namespace {

constexpr int kThreads = 256;
constexpr int kPartials = 32;
constexpr int kGroupLanes = 8;
constexpr float kLog2e = 1.4426950408889634f;

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

template <typename T> __device__ inline float to_f32(T x) { return (float)x; }
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

template <typename T, int N_ELEM>
__device__ inline void load_chunks(const T* __restrict__ row, int r, float* dst) {
  constexpr int CE = 16 / sizeof(T);
  constexpr int NC = N_ELEM / CE / kGroupLanes;  // chunks per lane
#pragma unroll
  for (int i = 0; i < NC; i++) {
    const uint4 u = *reinterpret_cast<const uint4*>(row + (r + kGroupLanes * i) * CE);
    const T* e = reinterpret_cast<const T*>(&u);
#pragma unroll
    for (int t = 0; t < CE; t++) dst[i * CE + t] = to_f32<T>(e[t]);
  }
}

template <typename T, int D, int V>
__global__ void __launch_bounds__(kThreads) sdpa_kernel(SdpaArgs p) {
  constexpr int CE = 16 / sizeof(T);
  constexpr int EQ = D / kGroupLanes;  // q/k elements per lane
  constexpr int EV = V / kGroupLanes;  // v/o elements per lane
  static_assert(D % (CE * kGroupLanes) == 0 && V % (CE * kGroupLanes) == 0, "head dim");

  __shared__ float part_m[kPartials], part_l[kPartials];
  __shared__ float part_o[kPartials * V];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int part = (tid >> 6) * 8 + (lane >> 3);  // wave * 8 + group
  const int r = lane & 7;

  const int64_t G = p.H / p.Hkv;
  int64_t t = xcd_remap(blockIdx.x, (int)(p.B * p.H * p.qL));
  const int64_t hg = t % G;
  t /= G;
  const int64_t s = t % p.qL;
  t /= p.qL;
  const int64_t kvh = t % p.Hkv;
  const int64_t b = t / p.Hkv;
  const int64_t h = kvh * G + hg;

  const T* __restrict__ qrow = static_cast<const T*>(p.q) + b * p.qs[0] + h * p.qs[1] + s * p.qs[2];
  const T* __restrict__ kb = static_cast<const T*>(p.k) + b * p.ks[0] + kvh * p.ks[1];
  const T* __restrict__ vb = static_cast<const T*>(p.v) + b * p.vs[0] + kvh * p.vs[1];

  float q2[EQ];
  load_chunks<T, D>(qrow, r, q2);
#pragma unroll
  for (int e = 0; e < EQ; e++) q2[e] = q2[e] * p.scale2;

  float m = -FLT_MAX, l = 0.f;
  float o[EV];
#pragma unroll
  for (int e = 0; e < EV; e++) o[e] = 0.f;
  if (p.sinks && part == 0) {
    m = to_f32<T>(static_cast<const T*>(p.sinks)[h]) * kLog2e;
    l = 1.f;
  }

  int64_t kend = p.N;
  if (p.mask_mode == BI_MASK_CAUSAL) {
    const int64_t last = s + p.causal_offset;  // last usable key
    kend = last < 0 ? 0 : (last + 1 < p.N ? last + 1 : p.N);
  }
  const T* __restrict__ mrow = nullptr;
  if (p.mask_mode == BI_MASK_ARRAY)
    mrow = static_cast<const T*>(p.mask) + b * p.ms[0] + h * p.ms[1] + s * p.ms[2];

  for (int64_t i = part; i < kend; i += kPartials) {
    float bias2 = 0.f;
    bool use = true;
    if (mrow) {
      const float mv = to_f32<T>(mrow[i]);
      use = mv > -3.0e38f;
      bias2 = mv * kLog2e;
    }
    if (use) {
      float kf[EQ], vf[EV];
      load_chunks<T, D>(kb + i * p.ks[2], r, kf);
      load_chunks<T, V>(vb + i * p.vs[2], r, vf);
      float d = 0.f;
#pragma unroll
      for (int e = 0; e < EQ; e++) d = __builtin_fmaf(q2[e], kf[e], d);
      const float sc = group_sum8(d) + bias2;
      const float nm = fmaxf(m, sc);
      const float f = __builtin_amdgcn_exp2f(m - nm);
      const float pe = __builtin_amdgcn_exp2f(sc - nm);
      m = nm;
      l = __builtin_fmaf(l, f, pe);
#pragma unroll
      for (int e = 0; e < EV; e++) o[e] = __builtin_fmaf(pe, vf[e], o[e] * f);
    }
  }

  // Fixed-order combine of the 32 partials.
  if (r == 0) {
    part_m[part] = m;
    part_l[part] = l;
  }
#pragma unroll
  for (int i = 0; i < EV / CE; i++)
#pragma unroll
    for (int e = 0; e < CE; e++) part_o[part * V + (r + kGroupLanes * i) * CE + e] = o[i * CE + e];
  __syncthreads();

  T* __restrict__ out = static_cast<T*>(p.out) + ((b * p.H + h) * p.qL + s) * V;
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
}

using SdpaFn = void (*)(SdpaArgs);

template <typename T>
SdpaFn kernel_for_dims(int64_t D, int64_t V) {
  if (D != V) return nullptr;
  switch (D) {
    case 64: return sdpa_kernel<T, 64, 64>;
    case 128: return sdpa_kernel<T, 128, 128>;
    case 256: return sdpa_kernel<T, 256, 256>;
  }
  return nullptr;
}

SdpaFn select_kernel(int dtype, int64_t D, int64_t V) {
  switch (dtype) {
    case BI_F32: return kernel_for_dims<float>(D, V);
    case BI_F16: return kernel_for_dims<_Float16>(D, V);
    case BI_BF16: return kernel_for_dims<__bf16>(D, V);
  }
  return nullptr;
}

}  // namespace

extern "C" int bi_sdpa(const void* q, const void* k, const void* v, const void* mask,
                       const int64_t* mask_strides, const void* sinks, void* out, int64_t B,
                       int64_t H, int64_t Hkv, int64_t qL, int64_t N, int64_t D, int64_t V,
                       const int64_t* qkv_strides, float scale, int mask_mode,
                       int64_t causal_offset, int dtype, void* hip_stream) {
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
  SdpaFn fn = select_kernel(dtype, D, V);
  if (!fn)
    return bi::fail(BI_EUNSUPPORTED, "bi_sdpa: head dims D=%lld V=%lld are not built "
                    "(supported: D == V in {64, 128, 256})", (long long)D, (long long)V);
  const int64_t rows = B * H * qL;
  if (rows == 0) return BI_OK;
  if (rows > INT32_MAX) return bi::fail(BI_EINVAL, "bi_sdpa: B*H*qL too large");
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
  p.mask_mode = mask_mode;
  p.causal_offset = mask_mode == BI_MASK_CAUSAL ? causal_offset : 0;

  hipLaunchKernelGGL(fn, dim3((unsigned)rows), dim3(kThreads), 0,
                     static_cast<hipStream_t>(hip_stream), p);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return bi::launch_error(e, "bi_sdpa launch");
  return BI_OK;
}
