/*
 * imq_oracle.h -- CPU restatement of the MLX-format affine 4-bit quantized
 * linear path, used ONLY as the checker (tests, smoke, bench cpu_baseline).
 * Nothing in the product library links or calls this code.
 *
 * Format (Sources/ImarelloDirect/DirectTEEncoder.swift:106-123,
 *         Sources/ImarelloDirect/DirectDiTStep.swift:853):
 *   w       uint32 [N, K/8]   eight 4-bit codes per word, low nibble first:
 *                             code k of row n = (w[n][k/8] >> (4*(k%8))) & 0xF
 *   scales  bf16   [N, K/64]  one scale per 64 consecutive K elements
 *   biases  bf16   [N, K/64]
 *   deq(W)[n][k] = RNE_bf16( fl32( s[n][k/64] * q[n][k] + b[n][k/64] ) )
 *   Y[M, N]      = X[M, K] . deq(W)^T    (MLX quantizedMM with transpose=true,
 *                                         Sources/ImarelloDirect/DirectQmmSpike.swift:55-58)
 *
 * All bf16 values travel as raw uint16 bit patterns.
 */
#ifndef IMQ_ORACLE_H
#define IMQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* bf16 -> f32: bits << 16 (DirectTEEncoder.swift:44-46). */
float oracle_bf16_to_f32(uint16_t h);

/* f32 -> bf16 round-to-nearest-even, integer form with no NaN special case,
 * exactly as DirectTEEncoder.swift:39-43. */
uint16_t oracle_f32_to_bf16(float v);

/* Dequantize rows [0, n) of a packed matrix to bf16 bit patterns,
 * out[n][k] (row-major).  Follows DirectTEEncoder.embedRow
 * (DirectTEEncoder.swift:106-123) for every row.  Returns 0, or -1 on a
 * shape the format does not allow (k % 64 != 0, non-positive sizes). */
int oracle_dequantize(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                      uint16_t* out, int64_t n, int64_t k);

/* Dequant-then-matmul:  y[m][n] = RNE_bf16( sum_k x[m][k] * deq(W)[n][k] )
 * with the sum accumulated in double (so the result is the correctly rounded
 * bf16 of a near-exact dot product).  x and y are bf16 bit patterns.
 * `threads` > 0 caps the OpenMP thread count; 0 uses the runtime default.
 * Returns 0, or -1 on a bad shape. */
int oracle_qmm_t(const uint16_t* x, const uint32_t* w, const uint16_t* scales,
                 const uint16_t* biases, uint16_t* y, int64_t m, int64_t n, int64_t k,
                 int threads);

/* Same contraction with fp32 accumulation in natural k order and bf16 output:
 * the arithmetic of a CPU quantized matmul (on-the-fly dequant to bf16, f32
 * accumulate, bf16 out).  Used as the timed CPU baseline; it is not the
 * parity reference (oracle_qmm_t is). */
int oracle_qmm_t_f32acc(const uint16_t* x, const uint32_t* w, const uint16_t* scales,
                        const uint16_t* biases, uint16_t* y, int64_t m, int64_t n, int64_t k,
                        int threads);

/* IEEE binary16 <-> f32: exact widening, and RNE narrowing (overflow to inf).
 * f16 is the element type of the reference's DiT kernels
 * (DirectDiTStep.swift:82-85, scales precast by TransformerWeights.swift:40-54). */
float oracle_f16_to_f32(uint16_t h);
uint16_t oracle_f32_to_f16(float v);
/* The two conversions over arrays of n elements. */
void oracle_f16_to_f32_n(const uint16_t* in, float* out, int64_t n);
void oracle_f32_to_f16_n(const float* in, uint16_t* out, int64_t n);

/* oracle_dequantize for T = bf16 (dtype 0) or f16 (dtype 1): scales, biases
 * and out are T bit patterns; out = RNE_T(fl32(fl32(s*q) + b)). */
int oracle_dequantize_t(int dtype, const uint32_t* w, const uint16_t* scales,
                        const uint16_t* biases, uint16_t* out, int64_t n, int64_t k);

/* y[m][n] = sum_k x[m][k] * deq_T(W)[n][k], accumulated in double and NOT
 * rounded (the caller rounds once to T); x, scales, biases are T bit
 * patterns, T = bf16 (dtype 0) or f16 (dtype 1).  For checks on a few rows of
 * large problems: each weight row is dequantized once for all m rows. */
int oracle_qmm_t_f64(int dtype, const uint16_t* x, const uint32_t* w, const uint16_t* scales,
                     const uint16_t* biases, double* y, int64_t m, int64_t n, int64_t k,
                     int threads);

/* Number of OpenMP threads a parallel region would use (for reporting). */
int oracle_max_threads(void);

#ifdef __cplusplus
}
#endif
#endif
