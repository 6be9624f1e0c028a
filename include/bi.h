/*
 * bi.h -- C ABI of libbi.so, the MI355X (gfx950) batch-invariant GEMM and
 * attention kernels.
 *
 * The reference launches its two Metal kernels through MLX's
 * `mx.fast.metal_kernel` callables; each entry point below replaces exactly one
 * of those launches (cited per function). Plain C types only: no torch, no C++
 * types, no exceptions and no allocation cross this boundary. The caller owns
 * every buffer (device pointers), allocates the output, and passes the HIP
 * stream to launch on (NULL = the default stream). Every call is asynchronous
 * on that stream and safe to record into a HIP graph: the launch path makes no
 * allocation, no host synchronisation and no choice other than the grid that
 * depends on the shape.
 *
 * Every function returns BI_OK (0) or a negative status; bi_last_error() then
 * returns a thread-local message describing the failure. Arguments are
 * validated before any HIP call is made, so argument errors are reported the
 * same way on a machine without a GPU.
 */
#ifndef BI_H
#define BI_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BI_ABI_VERSION 1

/* Element types; the compute is always fp32 accumulate. */
enum bi_dtype { BI_F32 = 0, BI_F16 = 1, BI_BF16 = 2 };

enum bi_status {
  BI_OK = 0,
  BI_EINVAL = -1,       /* bad argument: null pointer, negative size, bad mode */
  BI_EUNSUPPORTED = -2, /* valid but not built: e.g. an attention head dim */
  BI_ELAUNCH = -3       /* the HIP launch itself failed */
};

/* Attention masks (reference _attention.py:173-202, MASK_MODE at :92-97). */
enum bi_mask_mode {
  BI_MASK_NONE = 0,
  BI_MASK_CAUSAL = 1, /* key i is used by query row s iff i <= s + causal_offset */
  BI_MASK_ARRAY = 2   /* additive mask in the element type; <= -3e38 skips the key */
};

/* ABI revision of the loaded library (BI_ABI_VERSION at build time). */
int bi_abi_version(void);

/* Thread-local message for the most recent non-zero return on this thread. */
const char* bi_last_error(void);

/*
 * out[m, n] = T( bias ? alpha * acc + beta * bias[n] : acc ),
 * acc = sum_k a[m, k] * B[k, n] accumulated in fp32.
 *
 * Replaces the bi_gemm launch `_KERNEL(inputs=[a2, b, bias_arr, coef], ...)`
 * at reference mlx_batch_invariant/_gemm.py:212-221 (kernel body
 * _gemm.py:29-130, B load :152-157, grid :210).
 *
 *   a     (M, K) row-major, element type `dtype`
 *   b     trans_b == 0: (K, N) row-major  (bi.matmul / bi.addmm layout)
 *         trans_b == 1: (N, K) row-major  (bi.linear / nn.Linear layout)
 *   bias  (N,) or NULL; alpha and beta are used only when bias is non-NULL
 *   out   (M, N) row-major
 *
 * One workgroup owns the whole K reduction of its output tile. The per-element
 * arithmetic (MFMA instruction, K-chunk order, epilogue) is fixed at compile
 * time and does not depend on M, N, the batch neighbours of a row, its position
 * inside a tile, or whether the call was captured in a graph. M == 0 or
 * N == 0 is a no-op. K == 0 yields the epilogue applied to a zero accumulator.
 */
int bi_gemm(const void* a, const void* b, const void* bias, void* out,
            int64_t M, int64_t N, int64_t K, int dtype, int trans_b,
            float alpha, float beta, void* hip_stream);

/*
 * Single-pass scaled dot product attention; one workgroup owns the whole key
 * reduction of a query row (for the query heads of one kv head together).
 *
 * Replaces the bi_sdpa launch `_KERNEL(inputs=[q, k, v, m, mstride, scale,
 * sinks], ...)` at reference mlx_batch_invariant/_attention.py:241-250 (kernel
 * body _attention.py:32-149).
 *
 *   q     (B, H, qL, D)      element strides qkv_strides[0..2] for (b, h, s)
 *   k     (B, Hkv, N, D)     strides qkv_strides[3..5] for (b, h, n)
 *   v     (B, Hkv, N, V)     strides qkv_strides[6..8] for (b, h, n)
 *         the last dimension of q, k and v is contiguous; qkv_strides == NULL
 *         means all three are fully contiguous
 *   mask  BI_MASK_ARRAY only: element type `dtype`, last dim (N) contiguous,
 *         element strides mask_strides[0..2] for (b, h, s); 0 broadcasts
 *   sinks (H,) logits in `dtype` or NULL (an extra denominator term per head)
 *   out   (B, H, qL, V) contiguous
 *   scale multiplies q.k; H must be a multiple of Hkv (GQA: head h reads
 *         kv head h / (H / Hkv))
 *
 * One fixed reduction per element type. BI_F32: key i is owned by partial
 * (i mod 32) and walked in ascending order; the 32 partials are combined in a
 * fixed order. BI_F16 / BI_BF16 (matrix cores): keys are taken in blocks of
 * 32, block b owned by chain (b mod 4) and walked in ascending order; the 4
 * chains are combined in a fixed order. Nothing in the reduction depends on
 * B, qL, the other query rows, or N beyond which keys exist, so growing the
 * context with masked keys leaves earlier results bitwise unchanged. A query
 * row whose keys are all masked yields 0. A sink enters the fixed-order
 * combine as one more partial (m = sink, l = 1, o = 0).
 * Keys that no query row can see -- past every row's causal bound (e.g. an
 * unwritten cache tail) or hidden by an array mask from every query sharing a
 * workgroup -- never reach the output, whatever they hold (the reference skips
 * them, _attention.py:92-98). The matrix-core path multiplies the values of a
 * key that is visible to another query row of the same 32-key block, but not
 * to this one, by zero; a NaN or infinity there, which reaches that other
 * row's output in any case, may also reach this row's, as an all-NaN row,
 * depending on the launch shape and on which rows share its workgroup. Bit
 * parity across launch shapes, batch sizes and query lengths therefore holds
 * for finite values of every key that some query row of the call can see.
 * Supported head dims (D, V): D == V in {32, 64, 96, ..., 512} (every multiple
 * of 32 up to 512) and (192, 128), (128, 64), (64, 128), (256, 128), (128, 256),
 * (576, 512); other multiples of 32 return BI_EUNSUPPORTED (each pair is a
 * compiled kernel set). fp32 heads above 352 keep part of their state in
 * scratch memory (correct, slower).
 */
int bi_sdpa(const void* q, const void* k, const void* v,
            const void* mask, const int64_t* mask_strides,
            const void* sinks, void* out,
            int64_t B, int64_t H, int64_t Hkv, int64_t qL, int64_t N,
            int64_t D, int64_t V,
            const int64_t* qkv_strides,
            float scale, int mask_mode, int64_t causal_offset,
            int dtype, void* hip_stream);

/*
 * out = x @ dequantize(w).T for an affine-quantized weight, without
 * materialising the dequantized matrix.
 *
 * Replaces the bi_qgemm launch `_QKERNEL(inputs=[x, w, scales, qbias, ...])`
 * at reference mlx_batch_invariant/_gemm.py:275-284 (quantized_linear
 * :243-285; the kernel's dequantizing B load :163-177).
 *
 *   x       (M, K) row-major, dtype BI_F16 or BI_BF16, 16-byte aligned
 *   w       (N, K * bits / 32) uint32, 16-byte aligned: weight element k of
 *           row n is bits bits * (k % (32 / bits)) .. of word k / (32 / bits)
 *           of that row (little-endian packing, the MLX affine layout)
 *   scales, (N, K / group_size) in the element type of x; element k of row n
 *   biases  dequantizes to the fp32 value
 *           v = fp32(scales[n][k/group] * q + biases[n][k/group])
 *   out     (M, N) row-major
 *   bits in {2, 4, 8}; group_size in {32, 64, 128} and dividing K.
 *
 * As in the reference kernel (a float B tile, _gemm.py:46, :170-173), v is
 * not rounded to the element type. The product is formed per group in fp32:
 * P = sum x_k * q_k and X = sum x_k over the group's 32-element chunks of K
 * (MFMAs with exact products), then acc = fma(scale, P, acc) and
 * acc = fma(bias, X, acc), groups in ascending order; the output is rounded
 * once. This is sum_k x_k * v_k with fp32 roundings only, the same sequence
 * for every output element: nothing depends on M or on a row's batch
 * neighbours. BI_F32 activations return BI_EUNSUPPORTED.
 */
int bi_qgemm(const void* x, const void* w, const void* scales, const void* biases, void* out,
             int64_t M, int64_t N, int64_t K, int group_size, int bits, int dtype,
             void* hip_stream);

#ifdef __cplusplus
}
#endif

#endif /* BI_H */
