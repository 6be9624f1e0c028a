/*
 * oracle.c -- CPU restatement of the reference's two kernels in fixed-order
 * fp32. TEST INFRASTRUCTURE ONLY: used by tests/ as an independent checker and
 * by bench.py as the timed CPU baseline; never linked into libbi.so.
 *
 * Inputs arrive as float32 arrays already decoded from the element type (bf16
 * and f16 are exact in fp32); outputs are the fp32 values right before the
 * final rounding, which the Python side applies (oracle/bits.py).
 *
 * Built with -ffp-contract=off: every fused multiply-add below is an explicit
 * fmaf(), everything else rounds after each operation.
 */
#include <float.h>
#include <math.h>
#include <stdint.h>

/*
 * Reference mlx_batch_invariant/_gemm.py:62-129. For each output element the
 * reference walks k0 = 0, 16, 32, ... and within it kk = 0, 8 with an 8x8x8
 * simdgroup MMA into an fp32 accumulator (:62-104); Apple's internal order of
 * the 8 products is not specified, so it is restated here as ascending k with
 * one fmaf per term. B is read as b[k * N + n] or, when trans_b,
 * b[n * K + k] (:152-157). Epilogue (:118-129): the bias is applied to the
 * fp32 accumulator as alpha * acc + beta * bias (restated as
 * fmaf(alpha, acc, beta * bias)) before the single rounding.
 * Rows are independent, so rows are split over OpenMP threads; each element's
 * order is fixed.
 */
void oracle_gemm(const float* a, const float* b, const float* bias, float* out,
                 int64_t M, int64_t N, int64_t K, int trans_b, float alpha, float beta) {
#pragma omp parallel for schedule(static)
  for (int64_t m = 0; m < M; m++) {
    const float* arow = a + m * K;
    for (int64_t n = 0; n < N; n++) {
      float acc = 0.0f;
      if (trans_b) {
        const float* brow = b + n * K;
        for (int64_t k = 0; k < K; k++) acc = fmaf(arow[k], brow[k], acc);
      } else {
        for (int64_t k = 0; k < K; k++) acc = fmaf(arow[k], b[k * N + n], acc);
      }
      if (bias) acc = fmaf(alpha, acc, beta * bias[n]);
      out[m * N + n] = acc;
    }
  }
}

/* Same as oracle_gemm for trans_b == 0 but with B pre-transposed into bt
 * (N, K) so the inner loop is contiguous -- the layout the CPU baseline times. */
void oracle_gemm_bt(const float* a, const float* bt, float* out, int64_t M, int64_t N,
                    int64_t K) {
#pragma omp parallel for schedule(static) collapse(2)
  for (int64_t m = 0; m < M; m++) {
    for (int64_t n = 0; n < N; n++) {
      const float* arow = a + m * K;
      const float* brow = bt + n * K;
      float acc = 0.0f;
      for (int64_t k = 0; k < K; k++) acc = fmaf(arow[k], brow[k], acc);
      out[m * N + n] = acc;
    }
  }
}

#define SDPA_BN 32 /* partials = stride over keys; reference _attention.py:29 */
#define SDPA_BD 32 /* lanes of a simdgroup; reference _attention.py:30 */

/*
 * Reference mlx_batch_invariant/_attention.py:32-149, one query row per call of
 * the inner body. q (B,H,qL,D), k (B,Hkv,N,D), v (B,Hkv,N,V) contiguous;
 * mask (optional, mode 2) read at mask[b*ms0 + h*ms1 + s*ms2 + i]; sinks (H,)
 * optional. mode 1 (causal): key i is used iff i <= s + causal_offset
 * (reference :92-93 uses causal_offset = N - qL).
 *
 *   qv = scale * q                                           (:68-71)
 *   per partial sg = 0..31: max = -FLT_MAX, sum = 0          (:78-79)
 *     sink in partial 0: max = sink, sum = 1                 (:80-86)
 *     keys i = sg, sg + 32, ...                              (:89)
 *       mask value <= -3e38 skips the key                    (:94-96)
 *       score = sum over 32 lanes of the lane's D/32 products (lane-sequential
 *               fmaf), lanes added as a pairwise tree (simd_sum; Apple's tree
 *               is unspecified) + mask value                 (:99-106)
 *       new = max(max, score); f = exp(max - new); p = exp(score - new)
 *       sum = sum * f + p; o = o * f + p * v                 (:108-115)
 *   combine (:124-141): M = max of maxima; f_sg = exp(max_sg - M);
 *     sum = sum_sg sum_sg * f_sg, o = sum_sg o_sg * f_sg (ascending sg);
 *     out = sum == 0 ? o : o / sum.
 * The reference's `fast::exp` is restated as expf. The C products/sums use
 * explicit fmaf where the restatement fuses.
 */
void oracle_sdpa(const float* q, const float* k, const float* v, const float* mask,
                 int64_t ms0, int64_t ms1, int64_t ms2, const float* sinks, float* out,
                 int64_t B, int64_t H, int64_t Hkv, int64_t qL, int64_t N, int64_t D,
                 int64_t V, float scale, int mode, int64_t causal_offset) {
  const int64_t gqa = H / Hkv;
#pragma omp parallel for schedule(dynamic) collapse(3)
  for (int64_t b = 0; b < B; b++) {
    for (int64_t h = 0; h < H; h++) {
      for (int64_t s = 0; s < qL; s++) {
        const int64_t kvh = h / gqa;
        const float* qp = q + ((b * H + h) * qL + s) * D;
        const float* kp = k + (b * Hkv + kvh) * N * D;
        const float* vp = v + (b * Hkv + kvh) * N * V;
        float qv[1024];
        float o[SDPA_BN][1024];
        float mx[SDPA_BN], sm[SDPA_BN];
        for (int64_t j = 0; j < D; j++) qv[j] = scale * qp[j];
        const int64_t per = D / SDPA_BD;
        for (int sg = 0; sg < SDPA_BN; sg++) {
          mx[sg] = -FLT_MAX;
          sm[sg] = 0.0f;
          for (int64_t j = 0; j < V; j++) o[sg][j] = 0.0f;
          if (sinks && sg == 0) {
            mx[sg] = sinks[h];
            sm[sg] = 1.0f;
          }
          for (int64_t i = sg; i < N; i += SDPA_BN) {
            float bias = 0.0f;
            if (mode == 1 && !(i <= s + causal_offset)) continue;
            if (mode == 2) {
              bias = mask[b * ms0 + h * ms1 + s * ms2 + i];
              if (!(bias > -3.0e38f)) continue;
            }
            float lanes[SDPA_BD];
            for (int l = 0; l < SDPA_BD; l++) {
              float acc = 0.0f;
              for (int64_t j = 0; j < per; j++)
                acc = fmaf(qv[l * per + j], kp[i * D + l * per + j], acc);
              lanes[l] = acc;
            }
            for (int w = SDPA_BD / 2; w >= 1; w /= 2)
              for (int l = 0; l < w; l++) lanes[l] = lanes[l] + lanes[l + w];
            const float score = lanes[0] + bias;
            const float nm = fmaxf(mx[sg], score);
            const float f = expf(mx[sg] - nm);
            const float p = expf(score - nm);
            mx[sg] = nm;
            sm[sg] = fmaf(sm[sg], f, p);
            for (int64_t j = 0; j < V; j++) o[sg][j] = fmaf(p, vp[i * V + j], o[sg][j] * f);
          }
        }
        float M = mx[0];
        for (int sg = 1; sg < SDPA_BN; sg++) M = fmaxf(M, mx[sg]);
        float fac[SDPA_BN];
        float L = 0.0f;
        for (int sg = 0; sg < SDPA_BN; sg++) {
          fac[sg] = expf(mx[sg] - M);
          L = fmaf(sm[sg], fac[sg], L);
        }
        float* op = out + ((b * H + h) * qL + s) * V;
        for (int64_t j = 0; j < V; j++) {
          float acc = 0.0f;
          for (int sg = 0; sg < SDPA_BN; sg++) acc = fmaf(o[sg][j], fac[sg], acc);
          op[j] = (L == 0.0f) ? acc : acc / L;
        }
      }
    }
  }
}
