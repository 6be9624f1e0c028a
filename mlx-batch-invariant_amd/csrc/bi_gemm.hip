// Host side of the batch-invariant GEMM: geometry table, geometry choice,
// argument validation and the C ABI entry points of include/bi.h and
// include/bi_testing.h. The kernels and their arithmetic contract are in
// bi_gemm_kernel.h.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "bi_gemm_kernel.h"

namespace {

using bi_gemm_dev::GemmArgs;
using bi_gemm_dev::KernelFn;

struct Geometry {
  int bm, bn, waves;
  bool pl;  // loading waves issue every load, or the ping-pong schedule: 16-byte
            // aligned operands only
};

#define BI_GEO_ENTRY(id, bm, bn, wm, wn, nw, kb, ns, pl, pp) {bm, bn, nw, pl != 0 || pp != 0},
constexpr Geometry kGeometries[] = {BI_GEOMETRIES(BI_GEO_ENTRY)};
#undef BI_GEO_ENTRY
constexpr int kNumGeometries = sizeof(kGeometries) / sizeof(kGeometries[0]);

KernelFn select_kernel(int dtype, int trans_b, int g) {
  switch (dtype) {
    case BI_F32: return bi_gemm_kernel_f32(g, trans_b != 0);
    case BI_F16: return bi_gemm_kernel_f16(g, trans_b != 0);
    case BI_BF16: return bi_gemm_kernel_bf16(g, trans_b != 0);
  }
  return nullptr;
}

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Geometry for an (M, N) output: decode footprints for small M (they stream
// the weight once, with loader waves keeping the ring full); otherwise the
// footprint that moves the fewest operand bytes per CU while its tiles still
// cover (nearly) every CU. The thresholds come from a grid of this table on
// MI355X (M = 1..256, N = 4096..32000, K = 4096, 11008, 14336); since every
// geometry computes the same bits, they only move time.
int pick_geometry_f32(int64_t M, int64_t N) {
  // fp32 runs closer to its (8x lower) MFMA peak, so whole tiles per CU
  // weigh more than bytes per CU: at M = 256, N = 11008 64 x 64 tiles take
  // 226 us and 128 x 128 ones (172 of them) 253 us. The 256 x 128 footprint
  // (12 waves, at most 168 registers each) is not built for fp32's two
  // accumulator chains.
  if (M <= 16) return 0;
  const int64_t t128 = ceil_div(M, 128) * ceil_div(N, 128);
  if (M <= 64) {
    if (ceil_div(N, 128) >= 160) return 2;
    if (ceil_div(N, 64) >= 160) return 1;
    return M <= 32 ? 0 : 1;
  }
  if (ceil_div(M, 64) * ceil_div(N, 64) < 64) return 1;
  if (M <= 128) {
    if (t128 >= 200) return 3;
    return ceil_div(M, 64) * ceil_div(N, 32) >= 256 ? 5 : 1;
  }
  if (t128 >= (M <= 256 ? 200 : 160)) return 3;
  return 2;
}

int pick_geometry(int64_t M, int64_t N, int dtype, int trans_b) {
  const int64_t t128 = ceil_div(M, 128) * ceil_div(N, 128);  // 128 x 128 tiles
  const int64_t t64 = ceil_div(M, 64) * ceil_div(N, 64);     // 64 x 64 tiles
  // Decode: 16 x 16 tiles in a 64 KB ring, two workgroups per CU, so one
  // workgroup's ramp-up overlaps another's streaming (M = 1: 6.8 TB/s on a
  // 4096 x 32000 (N, K) weight). A (K, N) weight gives a 16-column tile 32
  // bytes of each weight row, so wide ones take wider tiles (N = 32000,
  // M = 1: 128 x 128 40 us, 16 x 16 52 us).
  if (M <= 16) {
    if (trans_b || dtype == BI_F32) return 0;
    return t128 >= 160 ? 3 : t64 >= 160 ? 2 : 0;
  }
  if (dtype == BI_F32) return pick_geometry_f32(M, N);
  if (M <= 64) {
    // 17..64 rows: the widest tile that still covers most CUs (N = 32000,
    // M = 64: 128 x 128 41 us, 64 x 32 49 us); 16 x 16 tiles for up to 32
    // rows of a narrow weight, 64 x 16 above.
    if (t128 >= 160) return 3;
    if (t64 >= 160) return 2;
    if (ceil_div(N, 32) >= (M <= 24 ? 256 : 192)) return 5;
    return M <= 32 ? 0 : 1;
  }
  // Small outputs (e.g. 256 x 512): 64 x 64 tiles would leave most CUs idle.
  if (t64 < 64) return 1;
  if (M <= 128) {
    // 65..128 rows: 128 x 128 tiles on wide weights (a 256-row tile would be
    // mostly padding), 64 x 32 on narrow ones.
    if (t128 >= 80) return 3;
    return t64 >= 192 ? 2 : 5;
  }
  if (M <= 256) {
    // 256 x 128 once its tiles cover most CUs (N = 22016, M = 192: 45 us
    // against 56 us for 128 x 128).
    if (ceil_div(N, 128) >= 160) return 4;
    return t128 >= 160 ? 3 : 2;
  }
  // More rows: the least estimated time per CU, in whole rounds of 256
  // workgroups (a few tiles past a multiple of the CU count cost a round:
  // N = 11008, M = 768 takes 95 us in 258 tiles of 256 x 128 and 87 us in
  // 516 of 128 x 128) times the rows and columns a tile streams, weighted
  // per footprint (time per streamed row, x1000, measured at M = 4096). The
  // 256 x 256 ping-pong footprint halves the operand bytes per product of
  // 128 x 128 (M = 4096: 1.19-1.33 PFLOP/s against 1.06-1.10 for 256 x 128
  // on (K, N) weights), but needs tiles for most CUs (M = 2048, N = 4096:
  // 128 of them, 92 us against 63 us for 256 x 128). On (N, K) weights the
  // four-wave 256 x 256 footprint takes its place: equal or faster on every
  // measured cell (M = 512..4096, N = 4096..32000, K = 4096..14336; M = 4096,
  // K = 11008, N = 4096: 260 against 298 us), 7 % faster on average.
  struct Cand { int g, bm, bn, w; };
  const Cand kCands[] = {{2, 64, 64, 129},
                         {3, 128, 128, 136},
                         {4, 256, 128, 144},
                         trans_b ? Cand{7, 256, 256, 180} : Cand{6, 256, 256, 192}};
  int best = 2;
  int64_t best_cost = -1;
  for (const Cand& c : kCands) {
    const int64_t cost = ceil_div(ceil_div(M, c.bm) * ceil_div(N, c.bn), 256) * (c.bm + c.bn) * c.w;
    if (best_cost < 0 || cost < best_cost) {
      best = c.g;
      best_cost = cost;
    }
  }
  return best;
}

// The quantized kernel's footprints, from a grid of every footprint over
// M = 1..512 and N = 4096..32000 (4-bit, group 64): 16 x 16 for decode and
// for 17..64 rows of a narrow weight; 64 x 64 for 17..64 rows of a wide one
// (N = 32000, M = 32: 37 us against 86 us for 64 x 16); above that the
// dense rules, except that 128 x 128 must fill the CUs (its workgroups
// dequantize twice the columns: N = 11008, M = 256: 64 x 64 61 us, 128 x 128
// 70 us).
// Id of the quantized decode footprint (bi_gemm_qdecode.h: 2-, 4- or 8-bit
// codes, at most 8 rows), one past the dense table.
constexpr int kQDecode = kNumGeometries;

int pick_qgeometry(int64_t M, int64_t N, int64_t K, int bits) {
  // The decode footprint. 2- and 4-bit: up to 4 rows everywhere; 5-8 rows
  // (an LDS share and register count that fit one workgroup per CU) only
  // while the column blocks fit one round over the 256 CUs (4-bit, N = 4096,
  // M = 8: 7.3 against 9.3 us; N = 11008: 18.5 against 13.6 us; 2-bit,
  // N = 4096, M = 8: 7.5 against 10.3 us; N = 11008: 19.0 against 14.1 us).
  // 8-bit: one row
  // everywhere (N = 32000: 29.5 against 33.1 us); up to 8 rows only with one
  // round of column blocks and of K (N = K = 4096, M = 8: 8.5 against 9.4 us;
  // K = 11008, M = 4: 21.3 against 19.8 us).
  const bool one_round = ceil_div(N, 16) <= 256;
  if ((bits == 4 || bits == 2) && (M <= 4 || (M <= 8 && one_round))) return kQDecode;
  if (bits == 8 && (M == 1 || (M <= 8 && one_round && K <= 4096))) return kQDecode;
  if (M <= 16) return 0;
  const int64_t t64 = ceil_div(M, 64) * ceil_div(N, 64);
  const int64_t t128 = ceil_div(M, 128) * ceil_div(N, 128);
  if (M <= 64) return ceil_div(N, 64) >= 160 ? 2 : 0;
  if (t64 < 64) return 1;
  if (M <= 128) {
    if (t128 >= 160) return 3;
    return t64 >= 192 ? 2 : 5;
  }
  return (M <= 256 ? t128 : ceil_div(N, 128)) >= 200 ? 3 : 2;
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

// 16-byte vector loads need 16-byte aligned bases and row lengths that are
// multiples of a chunk (K for A and (N, K) B; N for (K, N) B). The buffer
// path also needs every panel to fit a buffer resource (< 2 GiB).
struct VecFlags {
  bool a, b;
};
VecFlags vec_flags(const void* a, const void* b, int64_t N, int64_t K, int dtype, int trans_b,
                   const Geometry& G) {
  const int esz = bi::elem_size(dtype);
  const int epc = 16 / esz;
  const int64_t lim = (int64_t)1 << 31;
  VecFlags v;
  v.a = (K % epc == 0) && ((uintptr_t)a % 16 == 0) && (int64_t)G.bm * K * esz < lim;
  v.b = (trans_b ? (K % epc == 0) && (int64_t)G.bn * K * esz < lim
                 : (N % epc == 0) && K * N * esz < lim) &&
        ((uintptr_t)b % 16 == 0);
  return v;
}

// The geometry bi_gemm launches: pick_geometry's, unless that one takes
// aligned operands only and these are not; then the 128 x 128 footprint.
int pick_for(const void* a, const void* b, int64_t M, int64_t N, int64_t K, int dtype, int trans_b) {
  int g = pick_geometry(M, N, dtype, trans_b);
  if (kGeometries[g].pl) {
    const VecFlags v = vec_flags(a, b, N, K, dtype, trans_b, kGeometries[g]);
    if (!(v.a && v.b)) g = 3;
  }
  return g;
}

// start/stop (optional): hipEvents that receive the dispatch's own start and
// end timestamps (hipExtLaunchKernelGGL), so timing a launch adds no marker
// packets around it.
int launch(const void* a, const void* b, const void* bias, void* out, int64_t M, int64_t N,
           int64_t K, int dtype, int trans_b, float alpha, float beta, int g, void* stream,
           void* start = nullptr, void* stop = nullptr) {
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
  const VecFlags v = vec_flags(a, b, N, K, dtype, trans_b, G);
  if (G.pl && !(v.a && v.b))
    return bi::fail(BI_EUNSUPPORTED, "bi_gemm: geometry %d takes 16-byte aligned operands only", g);
  p.vec_a = v.a;
  p.vec_b = v.b;
  const int64_t blocks = (int64_t)p.tiles_m * p.tiles_n;
  if (blocks > INT32_MAX) return bi::fail(BI_EINVAL, "bi_gemm: too many tiles");
  KernelFn fn = select_kernel(dtype, trans_b, g);
  if (!fn) return bi::fail(BI_EUNSUPPORTED, "bi_gemm: geometry %d not built for this dtype", g);
  if (start || stop)
    hipExtLaunchKernelGGL(fn, dim3((unsigned)blocks), dim3(64 * G.waves), 0,
                          static_cast<hipStream_t>(stream), static_cast<hipEvent_t>(start),
                          static_cast<hipEvent_t>(stop), 0, p);
  else
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
  return launch(a, b, bias, out, M, N, K, dtype, trans_b, alpha, beta,
                pick_for(a, b, M, N, K, dtype, trans_b), hip_stream);
}

extern "C" int bi_gemm_timed(const void* a, const void* b, const void* bias, void* out,
                             int64_t M, int64_t N, int64_t K, int dtype, int trans_b, float alpha,
                             float beta, void* start_event, void* stop_event, void* hip_stream) {
  const int rc = validate(a, b, out, M, N, K, dtype, trans_b);
  if (rc != BI_OK || M == 0 || N == 0) return rc;
  return launch(a, b, bias, out, M, N, K, dtype, trans_b, alpha, beta,
                pick_for(a, b, M, N, K, dtype, trans_b), hip_stream, start_event, stop_event);
}

// ------------------------------------------------------------------ feed probe

namespace {

// The operand feed of a 256 x 256 footprint without its arithmetic: each
// workgroup (4 waves; its 128 KB of LDS leave room for one per CU) streams
// `stages` stages of 32 KB through a 4-slot LDS ring by direct-to-LDS loads,
// 8 of 1 KB per wave per stage with two stages in flight and a barrier per
// stage, as the GEMM's ring does, and does nothing with them. Workgroup w
// reads panel w % panels (panel_bytes, a power of two) of src; stage s starts
// at byte 32768 s of its panel, modulo the panel.
__global__ void __launch_bounds__(256) feed_probe_kernel(const char* src, int64_t panel_bytes,
                                                         int panels, int stages) {
  __shared__ uint4 ring[4][2048];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const __amdgpu_buffer_rsrc_t r =
      bi_gemm_dev::make_rsrc(src + (int64_t)(blockIdx.x % panels) * panel_bytes, panel_bytes);
  const uint64_t mask = (uint64_t)panel_bytes - 1;
  auto issue = [&](int64_t s, int slot) {
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int blk = i * 4 + w;
      const uint32_t off = (uint32_t)(((uint64_t)s * 32768 + blk * 1024 + lane * 16) & mask);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (bi_gemm_dev::lds_void_t*)(&ring[slot][blk * 64]),
                                               16, off, 0, 0, 0);
    }
  };
  issue(0, 0);
  issue(1, 1);
  issue(2, 2);
  for (int64_t s0 = 0; s0 < stages; s0 += 4) {
#pragma unroll
    for (int u = 0; u < 4; u++) {
      __builtin_amdgcn_s_waitcnt(bi_gemm_dev::waitcnt_vm_lgkm0(16));
      asm volatile("s_barrier" ::: "memory");
      issue(s0 + u + 3, (u + 3) & 3);
    }
  }
  // No load may still be landing in the LDS when the workgroup ends.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
}

}  // namespace

extern "C" int bi_feed_probe(const void* src, int64_t panel_bytes, int panels, int stages,
                             int workgroups, void* start_event, void* stop_event,
                             void* hip_stream) {
  if (!src) return bi::fail(BI_EINVAL, "bi_feed_probe: null source");
  if (panel_bytes < 32768 || panel_bytes > ((int64_t)1 << 30) || (panel_bytes & (panel_bytes - 1)))
    return bi::fail(BI_EINVAL, "bi_feed_probe: panel_bytes must be a power of two in [32 KiB, 1 GiB]");
  if (panels < 1 || stages < 1 || workgroups < 1)
    return bi::fail(BI_EINVAL, "bi_feed_probe: panels, stages and workgroups must be positive");
  hipExtLaunchKernelGGL(feed_probe_kernel, dim3((unsigned)workgroups), dim3(256), 0,
                        static_cast<hipStream_t>(hip_stream), static_cast<hipEvent_t>(start_event),
                        static_cast<hipEvent_t>(stop_event), 0, static_cast<const char*>(src),
                        panel_bytes, panels, stages);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return bi::launch_error(e, "bi_feed_probe launch");
  return BI_OK;
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
  return pick_geometry(M, N, dtype, trans_b);
}

extern "C" int bi_gemm_with_geometry(const void* a, const void* b, const void* bias, void* out,
                                     int64_t M, int64_t N, int64_t K, int dtype, int trans_b,
                                     float alpha, float beta, int g, void* hip_stream) {
  if (g < 0 || g >= kNumGeometries) return bi::fail(BI_EINVAL, "unknown geometry %d", g);
  const int rc = validate(a, b, out, M, N, K, dtype, trans_b);
  if (rc != BI_OK || M == 0 || N == 0) return rc;
  return launch(a, b, bias, out, M, N, K, dtype, trans_b, alpha, beta, g, hip_stream);
}

// ------------------------------------------------------------------ quantized

namespace {

KernelFn select_qkernel(int dtype, int g, int bits, int group) {
  switch (dtype) {
    case BI_F16: return bi_qgemm_kernel_f16(g, bits, group);
    case BI_BF16: return bi_qgemm_kernel_bf16(g, bits, group);
  }
  return nullptr;
}

int group_shift(int group_size) {
  switch (group_size) {
    case 32: return 5;
    case 64: return 6;
    case 128: return 7;
  }
  return -1;
}

int qvalidate(const void* x, const void* w, const void* scales, const void* biases, void* out,
              int64_t M, int64_t N, int64_t K, int group_size, int bits, int dtype) {
  if (dtype != BI_F32 && dtype != BI_F16 && dtype != BI_BF16)
    return bi::fail(BI_EINVAL, "bi_qgemm: unknown dtype %d", dtype);
  if (bits != 2 && bits != 4 && bits != 8)
    return bi::fail(BI_EINVAL, "bi_qgemm: bits must be one of (2, 4, 8), got %d", bits);
  if (group_shift(group_size) < 0)
    return bi::fail(BI_EINVAL, "bi_qgemm: group size must be 32, 64 or 128, got %d", group_size);
  if (M < 0 || N < 0 || K < 0)
    return bi::fail(BI_EINVAL, "bi_qgemm: negative size M=%lld N=%lld K=%lld", (long long)M,
                    (long long)N, (long long)K);
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX)
    return bi::fail(BI_EINVAL, "bi_qgemm: dimension too large");
  if (K % group_size)
    return bi::fail(BI_EINVAL, "bi_qgemm: group size %d does not divide K=%lld", group_size,
                    (long long)K);
  if (dtype == BI_F32)
    return bi::fail(BI_EUNSUPPORTED,
                    "bi_qgemm: quantized weights are built for float16/bfloat16 activations");
  if (M == 0 || N == 0) return BI_OK;
  if (!out || (K > 0 && (!x || !w || !scales || !biases)))
    return bi::fail(BI_EINVAL, "bi_qgemm: null operand pointer");
  if ((uintptr_t)x % 16 || (uintptr_t)w % 16 || (uintptr_t)scales % 2 || (uintptr_t)biases % 2)
    return bi::fail(BI_EINVAL, "bi_qgemm: x and the packed weight must be 16-byte aligned");
  const int64_t tiles = ceil_div(M, 16) * ceil_div(N, 16);
  if (tiles > INT32_MAX) return bi::fail(BI_EINVAL, "bi_qgemm: output too large");
  return BI_OK;
}

// The decode footprint: one workgroup per 16 output columns.
int qlaunch_decode(const void* x, const void* w, const void* scales, const void* biases,
                   void* out, int64_t M, int64_t N, int64_t K, int group_size, int bits,
                   int dtype, void* stream) {
  if (M > 8) return bi::fail(BI_EUNSUPPORTED, "bi_qgemm: the decode footprint takes at most 8 rows");
  const int64_t lim = (int64_t)1 << 31;
  if (M * K * 2 >= lim || 16 * K * bits / 8 >= lim)
    return bi::fail(BI_EUNSUPPORTED, "bi_qgemm: operand panel of 2 GiB or more");
  GemmArgs p = {};
  p.a = x;
  p.b = w;
  p.out = out;
  p.M = M;
  p.N = N;
  p.K = K;
  p.qs = scales;
  p.qz = biases;
  p.qgroup_shift = group_shift(group_size);
  const int64_t blocks = ceil_div(N, 16);
  if (blocks > INT32_MAX) return bi::fail(BI_EINVAL, "bi_qgemm: too many tiles");
  KernelFn fn = dtype == BI_F16 ? bi_qdecode_kernel_f16(group_size, (int)M, bits)
                                : bi_qdecode_kernel_bf16(group_size, (int)M, bits);
  if (!fn) return bi::fail(BI_EUNSUPPORTED, "bi_qgemm: decode footprint not built");
  hipLaunchKernelGGL(fn, dim3((unsigned)blocks), dim3(64 * bi_gemm_dev::kQDecodeWaves),
                     0, static_cast<hipStream_t>(stream), p);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return bi::launch_error(e, "bi_qgemm launch");
  return BI_OK;
}

int qlaunch(const void* x, const void* w, const void* scales, const void* biases, void* out,
            int64_t M, int64_t N, int64_t K, int group_size, int bits, int dtype, int g,
            void* stream) {
  if (g == kQDecode)
    return qlaunch_decode(x, w, scales, biases, out, M, N, K, group_size, bits, dtype, stream);
  const Geometry& G = kGeometries[g];
  const int64_t lim = (int64_t)1 << 31;
  if ((int64_t)G.bm * K * 2 >= lim || (int64_t)G.bn * K * bits / 8 >= lim)
    return bi::fail(BI_EUNSUPPORTED, "bi_qgemm: operand panel of 2 GiB or more");
  GemmArgs p = {};
  p.a = x;
  p.b = w;
  p.bias = nullptr;
  p.out = out;
  p.M = M;
  p.N = N;
  p.K = K;
  p.tiles_m = (int)ceil_div(M, G.bm);
  p.tiles_n = (int)ceil_div(N, G.bn);
  p.alpha = 1.f;
  p.beta = 1.f;
  p.vec_a = 1;
  p.vec_b = 1;
  p.qs = scales;
  p.qz = biases;
  p.qgroup_shift = group_shift(group_size);
  const int64_t blocks = (int64_t)p.tiles_m * p.tiles_n;
  if (blocks > INT32_MAX) return bi::fail(BI_EINVAL, "bi_qgemm: too many tiles");
  KernelFn fn = select_qkernel(dtype, g, bits, group_size);
  if (!fn) return bi::fail(BI_EUNSUPPORTED, "bi_qgemm: geometry %d not built", g);
  hipLaunchKernelGGL(fn, dim3((unsigned)blocks), dim3(64 * G.waves), 0,
                     static_cast<hipStream_t>(stream), p);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return bi::launch_error(e, "bi_qgemm launch");
  return BI_OK;
}

}  // namespace

extern "C" int bi_qgemm(const void* x, const void* w, const void* scales, const void* biases,
                        void* out, int64_t M, int64_t N, int64_t K, int group_size, int bits,
                        int dtype, void* hip_stream) {
  const int rc = qvalidate(x, w, scales, biases, out, M, N, K, group_size, bits, dtype);
  if (rc != BI_OK || M == 0 || N == 0) return rc;
  return qlaunch(x, w, scales, biases, out, M, N, K, group_size, bits, dtype,
                 pick_qgeometry(M, N, K, bits), hip_stream);
}

extern "C" int bi_qgemm_num_geometries(void) { return kQDecode + 1; }

extern "C" int bi_qgemm_pick_geometry(int64_t M, int64_t N, int64_t K, int bits) {
  if (bits != 2 && bits != 4 && bits != 8)
    return bi::fail(BI_EINVAL, "bi_qgemm: bits must be 2, 4 or 8, got %d", bits);
  return pick_qgeometry(M, N, K, bits);
}

extern "C" int bi_qgemm_with_geometry(const void* x, const void* w, const void* scales,
                                      const void* biases, void* out, int64_t M, int64_t N,
                                      int64_t K, int group_size, int bits, int dtype, int g,
                                      void* hip_stream) {
  if (g < 0 || g > kQDecode) return bi::fail(BI_EINVAL, "unknown geometry %d", g);
  const int rc = qvalidate(x, w, scales, biases, out, M, N, K, group_size, bits, dtype);
  if (rc != BI_OK || M == 0 || N == 0) return rc;
  return qlaunch(x, w, scales, biases, out, M, N, K, group_size, bits, dtype, g, hip_stream);
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
  (void)hipFree(d);
  if (e != hipSuccess) return bi::launch_error(e, "wavefront size probe");
  return BI_OK;
}
