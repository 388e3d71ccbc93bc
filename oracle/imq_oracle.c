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

/* IEEE binary16 bits -> f32 (exact: every f16 value is an f32 value).  The f16
 * element type of the reference's DiT kernels (affine_qmm_t_float16_t,
 * DirectDiTStep.swift:82-85) with its scales precast to f16
 * (TransformerWeights.swift:40-54). */
float oracle_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    uint32_t u;
    if (e == 0x1Fu) {
        u = sign | 0x7F800000u | (m << 13);
    } else if (e != 0) {
        u = sign | ((e + 112u) << 23) | (m << 13);
    } else {
        const float v = (float)m * 0x1p-24f; /* subnormal (or zero): m * 2^-24, exact */
        return sign ? -v : v;
    }
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

/* f32 -> IEEE binary16 bits, round to nearest even (overflow to inf, NaN kept
 * quiet), by integer arithmetic on the f32 pattern. */
uint16_t oracle_f32_to_f16(float v) {
    uint32_t u;
    memcpy(&u, &v, sizeof u);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    const uint32_t a = u & 0x7FFFFFFFu;
    if (a >= 0x7F800000u) /* inf, NaN */
        return (uint16_t)(sign | 0x7C00u | (a > 0x7F800000u ? 0x200u | ((a >> 13) & 0x3FFu) : 0u));
    if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520: rounds to inf */
    if (a >= 0x38800000u) {                                   /* normal f16: >= 2^-14 */
        const uint32_t r = a - 0x38000000u;                    /* exponent bias 127 -> 15 */
        return (uint16_t)(sign | ((r + 0xFFFu + ((r >> 13) & 1u)) >> 13));
    }
    if (a < 0x33000000u) return sign; /* <= 2^-25: zero (2^-25 itself ties to even 0) */
    /* subnormal f16: m = RNE(value * 2^24) */
    const uint32_t mant = (a & 0x7FFFFFu) | 0x800000u;
    const int shift = 126 - (int)(a >> 23);                   /* 14 .. 24 */
    uint32_t m = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (m & 1u))) ++m;
    return (uint16_t)(sign | m);
}

void oracle_f16_to_f32_n(const uint16_t* in, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = oracle_f16_to_f32(in[i]);
}

void oracle_f32_to_f16_n(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = oracle_f32_to_f16(in[i]);
}

/* T = bf16 (dtype 0) or f16 (dtype 1) bit patterns. */
static float t_to_f32(int dtype, uint16_t h) {
    return dtype == 0 ? oracle_bf16_to_f32(h) : oracle_f16_to_f32(h);
}

/* dequant_row in T: RNE_T(fl32(fl32(s * q) + b)) with s, b given in T
 * (DirectTEEncoder.swift:106-123 for bf16; the f16 DiT pack for f16). */
static void dequant_row_t(int dtype, const uint32_t* wrow, const uint16_t* srow,
                          const uint16_t* brow, uint16_t* out, int64_t k) {
    for (int64_t g = 0; g < k / 64; ++g) {
        const float scale = t_to_f32(dtype, srow[g]);
        const float bias = t_to_f32(dtype, brow[g]);
        for (int64_t wd = 0; wd < 8; ++wd) {
            const uint32_t packed = wrow[g * 8 + wd];
            for (int nib = 0; nib < 8; ++nib) {
                const float q = (float)((packed >> (4u * (uint32_t)nib)) & 0xFu);
                volatile float prod = scale * q;
                volatile float sum = prod + bias;
                out[g * 64 + wd * 8 + nib] =
                    dtype == 0 ? oracle_f32_to_bf16(sum) : oracle_f32_to_f16(sum);
            }
        }
    }
}

int oracle_dequantize_t(int dtype, const uint32_t* w, const uint16_t* scales,
                        const uint16_t* biases, uint16_t* out, int64_t n, int64_t k) {
    if ((dtype != 0 && dtype != 1) || !shape_ok(n, k) || !w || !scales || !biases || !out)
        return -1;
    const int64_t wpr = k / 8, gpr = k / 64;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < n; ++r)
        dequant_row_t(dtype, w + r * wpr, scales + r * gpr, biases + r * gpr, out + r * k, k);
    return 0;
}

/* Unrounded y[m][n] = sum_k x[m][k] * deq_T(W)[n][k] accumulated in double, in
 * k order: the contraction of quantizedMM(transpose: true)
 * (DirectQmmSpike.swift:55-58) before the output rounding, which the caller
 * applies (RNE to T once, from double). */
int oracle_qmm_t_f64(int dtype, const uint16_t* x, const uint32_t* w, const uint16_t* scales,
                     const uint16_t* biases, double* y, int64_t m, int64_t n, int64_t k,
                     int threads) {
    if ((dtype != 0 && dtype != 1) || m <= 0 || !shape_ok(n, k) || !x || !w || !scales ||
        !biases || !y)
        return -1;
    set_threads(threads);
    double* xd = (double*)malloc((size_t)(m * k) * sizeof(double));
    if (!xd) return -1;
    for (int64_t i = 0; i < m * k; ++i) xd[i] = (double)t_to_f32(dtype, x[i]);
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
                dequant_row_t(dtype, w + c * wpr, scales + c * gpr, biases + c * gpr, row, k);
                for (int64_t i = 0; i < k; ++i) rowd[i] = (double)t_to_f32(dtype, row[i]);
                for (int64_t r = 0; r < m; ++r) {
                    const double* xr = xd + r * k;
                    double acc = 0.0;
                    for (int64_t i = 0; i < k; ++i) acc += xr[i] * rowd[i];
                    y[r * n + c] = acc;
                }
            }
        }
        free(row);
        free(rowd);
    }
    free(xd);
    return failed ? -1 : 0;
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
