/*
 * bi_testing.h -- introspection entry points of libbi.so used by the test
 * suite and the benchmark. They have no counterpart in the reference, whose
 * GEMM has a single output tile (reference _gemm.py:25-27).
 *
 * libbi.so builds its GEMM as a small table of workgroup output footprints
 * ("geometries": rows x columns of C per workgroup, waves per workgroup). All
 * of them execute the same per-element arithmetic: the same MFMA instruction
 * on the same K-chunks in the same ascending order, then the same epilogue.
 * bi_gemm picks a geometry from (M, N), the element type and the weight
 * layout (never from the values or the row's position). These entry
 * points let a test run one input through every geometry and compare bits,
 * which is the direct proof that the footprint choice cannot change a result.
 */
#ifndef BI_TESTING_H
#define BI_TESTING_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Number of GEMM geometries built into the library. */
int bi_gemm_num_geometries(void);

/* Describes geometry `g`: rows and columns of C per workgroup and waves per
 * workgroup. Returns BI_EINVAL for an unknown g. */
int bi_gemm_geometry_info(int g, int* block_m, int* block_n, int* waves);

/* The geometry bi_gemm would launch for this problem with 16-byte aligned
 * operands (for others it replaces a footprint that takes aligned operands
 * only, the 256 x 128 one, by 128 x 128). */
int bi_gemm_pick_geometry(int64_t M, int64_t N, int64_t K, int dtype, int trans_b);

/* bi_gemm with the geometry forced to `g` (same arguments and semantics);
 * BI_EUNSUPPORTED where g is not built for the dtype or takes aligned
 * operands only and these are not. */
int bi_gemm_with_geometry(const void* a, const void* b, const void* bias, void* out,
                          int64_t M, int64_t N, int64_t K, int dtype, int trans_b,
                          float alpha, float beta, int g, void* hip_stream);

/* bi_gemm (same arguments, semantics and kernel), with the kernel's own start
 * and end timestamps recorded into `start_event` and `stop_event` (hipEvent_t,
 * created by the caller; either may be NULL). A benchmark can then time one
 * launch with no marker packets between kernels; a hipEventRecord on each side
 * of a launch idles the GPU for several microseconds per record on this stack.
 * The reference times host-side (bench/bench.py:32-49) and has no counterpart. */
int bi_gemm_timed(const void* a, const void* b, const void* bias, void* out, int64_t M,
                  int64_t N, int64_t K, int dtype, int trans_b, float alpha, float beta,
                  void* start_event, void* stop_event, void* hip_stream);

/* Feed probe: the operand stream of a 256 x 256 GEMM footprint with no
 * arithmetic. `workgroups` workgroups of 256 threads each stream `stages`
 * stages of 32 KB through a 4-slot LDS ring by direct-to-LDS loads (8 of
 * 1 KB per wave per stage, two stages in flight, a barrier per stage, as in
 * the GEMM). Workgroup w reads panel w % panels of panel_bytes (a power of two,
 * 32 KiB .. 1 GiB) at src; the caller provides panels * panel_bytes bytes.
 * With one panel every pass after the first is served by the L2, so the rate
 * is the per-CU operand feed from L2 that bounds the large-M GEMM. Timed like
 * bi_gemm_timed (events may be NULL). No counterpart in the reference. */
int bi_feed_probe(const void* src, int64_t panel_bytes, int panels, int stages, int workgroups,
                  void* start_event, void* stop_event, void* hip_stream);

/* Number of geometries bi_qgemm_with_geometry accepts: the GEMM geometries
 * (bi_gemm_num_geometries()), then the quantized decode footprint, id
 * bi_gemm_num_geometries(): 16 output columns per workgroup whose waves split
 * K by groups (at most 8 rows of x; otherwise
 * BI_EUNSUPPORTED). No counterpart in the reference. */
int bi_qgemm_num_geometries(void);

/* The geometry bi_qgemm would launch for this problem (an id as for
 * bi_qgemm_with_geometry); BI_EINVAL for bits other than 2, 4 and 8. No
 * counterpart in the reference. */
int bi_qgemm_pick_geometry(int64_t M, int64_t N, int64_t K, int bits);

/* bi_qgemm with the geometry forced to `g` (same arguments and semantics). */
int bi_qgemm_with_geometry(const void* x, const void* w, const void* scales,
                           const void* biases, void* out, int64_t M, int64_t N, int64_t K,
                           int group_size, int bits, int dtype, int g, void* hip_stream);

/*
 * Attention launch shapes. bi_sdpa picks a launch shape from the grid alone:
 * for BI_F16 / BI_BF16 (matrix cores) how many 16-column tiles a workgroup
 * holds (a column is one (query head, query row) pair of a kv head) and over
 * how many workgroups the output dims are split; for BI_F32 how many query
 * heads share a workgroup's key and value loads. The reference has a single
 * launch shape (reference _attention.py:241-250: one threadgroup per row);
 * every shape here runs the same per-column arithmetic, and these entry
 * points let a test run one input through every shape and compare bits.
 *
 * Shapes of BI_F16 / BI_BF16: 0 "rows" (prefill: 2 column tiles per
 * workgroup, 1 for head dims above 128), 1 one tile, 2 / 3 / 4 one tile with
 * the output dims split over 2 / 4 / 8 workgroups (fewer where the value
 * head dim does not allow it), 5 "shared" (prefill without an array mask,
 * D and V in {32, 64, 128}: one column tile per wave, 4 or 8 waves reading
 * each key and value block once from LDS). Shapes of BI_F32: s = 0..3, 2^s
 * query heads per workgroup.
 */

/* The shape bi_sdpa picks for this problem (mask_mode as for bi_sdpa) on a
 * GPU of `cus` compute units (0: the current device's). Returns the shape
 * (>= 0) or a negative status. */
int bi_sdpa_pick_shape(int64_t B, int64_t H, int64_t Hkv, int64_t qL, int64_t D, int64_t V,
                       int dtype, int mask_mode, int cus);

/* Columns (BI_F32: query heads) and output-dim splits per workgroup of a
 * shape; BI_EINVAL if that shape is not built for the head dims. */
int bi_sdpa_shape_info(int64_t D, int64_t V, int dtype, int shape, int* columns, int* splits);

/* bi_sdpa with the launch shape forced to `shape` (same arguments and
 * semantics). BI_F32 shapes must divide the query heads of a kv head. */
int bi_sdpa_with_shape(const void* q, const void* k, const void* v,
                       const void* mask, const int64_t* mask_strides,
                       const void* sinks, void* out,
                       int64_t B, int64_t H, int64_t Hkv, int64_t qL, int64_t N,
                       int64_t D, int64_t V,
                       const int64_t* qkv_strides,
                       float scale, int mask_mode, int64_t causal_offset,
                       int dtype, int shape, void* hip_stream);

/* Wavefront width the kernels were compiled for (64 on gfx950); the fixed
 * reduction shapes assume it. Reads a device-side constant: needs a GPU. */
int bi_device_wavefront_size(int* out);

#ifdef __cplusplus
}
#endif

#endif /* BI_TESTING_H */
