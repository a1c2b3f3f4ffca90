/*
 * okf_oracle.h -- CPU restatement of ChatOKF's quantized weight x activation
 * path.  TEST INFRASTRUCTURE ONLY: the checker for the HIP library and the
 * timed CPU baseline.  Nothing in the product (chatokf_amd/, include/) links,
 * loads or calls it.
 *
 * Every function follows one reference function (file:line relative to the
 * reference checkout).  Arithmetic keeps the reference's fp32 evaluation
 * order; the file is compiled with -O2 -ffp-contract=off -fno-fast-math so
 * that no multiply-add is fused and no sum is reassociated.
 *
 * Pinning (the evidence that this restatement is right):
 *   - okf_ref_dequant: hand-built known-answer blocks per format, the IQ2_XXS
 *     tables against the reference's two copies (Swift grid and the Metal
 *     header), and an independent numpy decoder (tests/test_oracle.py).
 *   - okf_ref_matvec / okf_ref_matmul: float64 brute-force dot over the
 *     dequantized weights (agreement ~1e-6 relative), the closed form of the
 *     Q2_0 lo/hi/sum identity, linearity in x, and matmul == N x matvec.
 *   - Unpinned assumption (no Swift toolchain exists to run the original):
 *     that Swift emitted no FMA contraction or reassociation in GQ.matvec;
 *     the fp32 evaluation order below is the one the Swift source spells out.
 */
#ifndef OKF_ORACLE_H
#define OKF_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids, LLM/Base/GGUF.swift:3-14 */
enum {
    OKF_REF_Q4_0 = 2,
    OKF_REF_Q8_0 = 8,
    OKF_REF_IQ4_NL = 20,
    OKF_REF_Q4_K = 12,
    OKF_REF_Q5_K = 13,
    OKF_REF_Q6_K = 14,
    OKF_REF_IQ4_XS = 23,
    OKF_REF_IQ2_XS = 17,
    OKF_REF_IQ3_XXS = 18,
    OKF_REF_IQ1_S = 19,
    OKF_REF_IQ3_S = 21,
    OKF_REF_IQ2_S = 22,
    OKF_REF_IQ1_M = 29,
    OKF_REF_F32 = 0,
    OKF_REF_F16 = 1,
    OKF_REF_BF16 = 30,
    OKF_REF_Q2_K = 10,
    OKF_REF_Q3_K = 11,
    OKF_REF_IQ2_XXS = 16,
    OKF_REF_Q2_0 = 42,
};

/* GGUF.rowByteCount, LLM/Base/GGUF.swift:160-188.  0 on success, -1 for an
 * unsupported type or an n that is not a whole number of blocks. */
int okf_ref_row_bytes(int32_t type, uint64_t n, uint64_t *out);

/* IEEE binary16 bits -> float, exact (Float(Float16) in Swift). */
float okf_ref_f16_to_f32(uint16_t h);

/* GQ.gather(row:from:0,count:n), LLM/Gemma/Gemma4Quant.swift:330-364:
 * unpack n weights starting at p (a row start) into out. */
int okf_ref_dequant(int32_t type, const uint8_t *p, uint64_t n, float *out);

/* GQ.matvec, LLM/Gemma/Gemma4Quant.swift:89-148 (Q2_0 arm:
 * LLM/Base/Quant.swift:28-65).  W is M rows of rowBytes(K), x[K] -> y[M].
 * threads <= 0 uses every usable core. */
int okf_ref_matvec(int32_t type, const uint8_t *w, uint32_t K, uint32_t M,
                   const float *x, float *y, int threads);

/* GQ.matmul, LLM/Gemma/Gemma4Quant.swift:150-170: X[N][K] -> Y[N][M].
 * Q8_0 uses the block-reuse matmul (:172-223); Q2_0, Q4_K and IQ2_XXS run N
 * sequential matvecs (:159-169). */
int okf_ref_matmul(int32_t type, const uint8_t *w, uint32_t K, uint32_t M,
                   const float *X, uint32_t N, float *Y, int threads);

/* Cores this process may run on (sched_getaffinity). */
int okf_ref_usable_cores(void);

/* silu(a) * b elementwise into out: silu(x) = x / (1 + expf(-x)) as Swift's
 * silu (LLM/Base/Kernels.swift:3) and the Metal silu_mul kernel
 * (LLM/metal/Kernels.metal:7, :3280-3285). */
void okf_ref_silu_mul(const float *a, const float *b, uint32_t n, float *out);

/* Per row of n: x += r (r may be NULL: no add), then
 * y = x * (1 / sqrt(sum(x^2) / n + eps)) * w, sequential fp32 sum, as
 * Kern.rmsnorm (LLM/Base/Kernels.swift:12-20) applied to the residual sum
 * that add_rmsnorm_batch forms (LLM/metal/Kernels.metal:2839-2862). */
void okf_ref_add_rmsnorm(float *x, const float *r, const float *w, float *y, uint32_t n, uint32_t rows,
                         float eps);

/* Per row of n: the index of the largest value, ties to the lower index, NaN
 * skipped, 0 when nothing exceeds -inf (argmax_rows,
 * LLM/metal/Kernels.metal:2756-2795; Vectors.argmax,
 * LLM/Base/Vectors.swift:11-18, scans the same way from a finite floor). */
void okf_ref_argmax_rows(const float *x, uint32_t n, uint32_t rows, int32_t *out);

#ifdef __cplusplus
}
#endif
#endif
