/*
 * imq_oracle.c -- CPU restatement of the affine 4-bit quantized linear path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP library.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.  The
 * product library never links, loads or falls back to this code.
 *
 * Every function cites the reference file:line whose behaviour it restates.
 */
#include "imq_oracle.h"

#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* DirectTEEncoder.swift:44-46  (bf16ToF32: UInt32(u) << 16). */
float oracle_bf16_to_f32(uint16_t h) {
    uint32_t bits = (uint32_t)h << 16;
    float f;
    memcpy(&f, &bits, sizeof f);
    return f;
}

/* DirectTEEncoder.swift:39-43  (f32ToBF16: bits + 0x7FFF + ((bits >> 16) & 1), >> 16;
 * wrapping add, no NaN special case). */
uint16_t oracle_f32_to_bf16(float v) {
    uint32_t bits;
    memcpy(&bits, &v, sizeof bits);
    uint32_t rounded = bits + 0x7FFFu + ((bits >> 16) & 1u);
    return (uint16_t)(rounded >> 16);
}

/* One row of DirectTEEncoder.embedRow (DirectTEEncoder.swift:106-123):
 * for each group g of 64: scale, bias = bf16 -> f32; for each packed word of
 * the group, for each nibble n (low first): out = f32ToBF16(scale * q + bias).
 * two rounded f32 operations.  scale * q is exact in f32 (8-bit significand
 * times a 4-bit integer) unless it overflows to +-inf, so the rounding that
 * matters is the addition's; the product is kept a separate operation so that
 * the overflow case matches too. */
static void dequant_row(const uint32_t* wrow, const uint16_t* srow, const uint16_t* brow,
                        uint16_t* out, int64_t k) {
    const int64_t groups = k / 64;
    for (int64_t g = 0; g < groups; ++g) {
        const float scale = oracle_bf16_to_f32(srow[g]);
        const float bias = oracle_bf16_to_f32(brow[g]);
        const int64_t col_base = g * 64;
        for (int64_t wd = 0; wd < 8; ++wd) {
            const uint32_t packed = wrow[col_base / 8 + wd];
            for (int nib = 0; nib < 8; ++nib) {
                const float q = (float)((packed >> (4u * (uint32_t)nib)) & 0xFu);
                volatile float prod = scale * q; /* exact; keep the two steps explicit */
                out[col_base + wd * 8 + nib] = oracle_f32_to_bf16(prod + bias);
            }
        }
    }
}

/* Correctly rounded double -> bf16 (RNE).  A plain (float) cast followed by
 * RNE to bf16 rounds twice; rounding to odd at f32 first (24 >= 8 + 2 bits)
 * makes the second RNE give the correctly rounded result. */
static uint16_t f64_to_bf16(double v) {
    float f = (float)v;
    if ((double)f != v && f == f) {
        uint32_t bits;
        memcpy(&bits, &f, sizeof bits);
        const double af = f < 0 ? -(double)f : (double)f;
        const double av = v < 0 ? -v : v;
        if (af > av) bits -= 1u;  /* step toward zero: truncation */
        bits |= 1u;               /* sticky bit: round to odd */
        memcpy(&f, &bits, sizeof f);
    }
    return oracle_f32_to_bf16(f);
}

static int shape_ok(int64_t n, int64_t k) { return n > 0 && k > 0 && (k % 64) == 0; }

int oracle_dequantize(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                      uint16_t* out, int64_t n, int64_t k) {
    if (!shape_ok(n, k) || !w || !scales || !biases || !out) return -1;
    const int64_t wpr = k / 8, gpr = k / 64;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < n; ++r)
        dequant_row(w + r * wpr, scales + r * gpr, biases + r * gpr, out + r * k, k);
    return 0;
}

static void set_threads(int threads) {
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#else
    (void)threads;
#endif
}

int oracle_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* Dequant-then-matmul with transpose=true (DirectQmmSpike.swift:55-58: y = x . deq(w)^T),
 * the contraction MLX's affine_qmm_t computes (Docs/ENGINE_RESEARCH.md:236: f32
 * accumulation).  The oracle accumulates in double so that its only rounding
 * that matters is the final RNE to bf16. */
int oracle_qmm_t(const uint16_t* x, const uint32_t* w, const uint16_t* scales,
                 const uint16_t* biases, uint16_t* y, int64_t m, int64_t n, int64_t k,
                 int threads) {
    if (m <= 0 || !shape_ok(n, k) || !x || !w || !scales || !biases || !y) return -1;
    set_threads(threads);
    double* xd = (double*)malloc((size_t)(m * k) * sizeof(double));
    if (!xd) return -1;
    for (int64_t i = 0; i < m * k; ++i) xd[i] = (double)oracle_bf16_to_f32(x[i]);
    const int64_t wpr = k / 8, gpr = k / 64;
    int failed = 0;
#pragma omp parallel
    {
        uint16_t* row = (uint16_t*)malloc((size_t)k * sizeof(uint16_t));
        double* rowd = (double*)malloc((size_t)k * sizeof(double));
        if (!row || !rowd) {
#pragma omp atomic write
            failed = 1;
        } else {
#pragma omp for schedule(static)
            for (int64_t c = 0; c < n; ++c) {
                dequant_row(w + c * wpr, scales + c * gpr, biases + c * gpr, row, k);
                for (int64_t i = 0; i < k; ++i) rowd[i] = (double)oracle_bf16_to_f32(row[i]);
                for (int64_t r = 0; r < m; ++r) {
                    const double* xr = xd + r * k;
                    double acc = 0.0;
                    for (int64_t i = 0; i < k; ++i) acc += xr[i] * rowd[i];
                    y[r * n + c] = f64_to_bf16(acc);
                }
            }
        }
        free(row);
        free(rowd);
    }
    free(xd);
    return failed ? -1 : 0;
}

/* CPU quantized matmul in the shape of MLX's CPU qmm: dequantize a weight row
 * to bf16 values, multiply-accumulate in f32, round the output to bf16. */
int oracle_qmm_t_f32acc(const uint16_t* x, const uint32_t* w, const uint16_t* scales,
                        const uint16_t* biases, uint16_t* y, int64_t m, int64_t n, int64_t k,
                        int threads) {
    if (m <= 0 || !shape_ok(n, k) || !x || !w || !scales || !biases || !y) return -1;
    set_threads(threads);
    float* xf = (float*)malloc((size_t)(m * k) * sizeof(float));
    if (!xf) return -1;
    for (int64_t i = 0; i < m * k; ++i) xf[i] = oracle_bf16_to_f32(x[i]);
    const int64_t wpr = k / 8, gpr = k / 64;
    int failed = 0;
#pragma omp parallel
    {
        uint16_t* row = (uint16_t*)malloc((size_t)k * sizeof(uint16_t));
        float* rowf = (float*)malloc((size_t)k * sizeof(float));
        if (!row || !rowf) {
#pragma omp atomic write
            failed = 1;
        } else {
#pragma omp for schedule(static)
            for (int64_t c = 0; c < n; ++c) {
                dequant_row(w + c * wpr, scales + c * gpr, biases + c * gpr, row, k);
                for (int64_t i = 0; i < k; ++i) rowf[i] = oracle_bf16_to_f32(row[i]);
                for (int64_t r = 0; r < m; ++r) {
                    const float* xr = xf + r * k;
                    float acc = 0.0f;
#pragma omp simd reduction(+ : acc)
                    for (int64_t i = 0; i < k; ++i) acc += xr[i] * rowf[i];
                    y[r * n + c] = oracle_f32_to_bf16(acc);
                }
            }
        }
        free(row);
        free(rowf);
    }
    free(xf);
    return failed ? -1 : 0;
}
