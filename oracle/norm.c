/*
 * Norm family + gated residual for the CPU oracle (test infrastructure only;
 * see oracle.h).  Every function restates device/cpu/layernorm/compute.go.
 *
 * Reductions run sequentially in index order (the Generic Go kernels,
 * device/cpu/dot/bf16_generic.go:9-21, device/cpu/reduction/bf16_kernels.go:40-51,
 * device/cpu/layernorm/f32_generic.go:3-12).  The amd64 build of the reference
 * reaches AVX-512 versions of the f32 dot/sum with another summation order; the
 * difference is bounded by a few f32 ulp of the sum.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>

#define LAYERNORM_EPS 1e-5 /* compute.go:11 */

/* dot of a row with itself, f32 accumulate; 16-bit formats round the result
 * to their own format (dot/bf16_generic.go:9-21, dot/compute.go:17-22) */
static float row_sumsq(const void *in, size_t off, int64_t n, int dtype) {
    float s = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
        float v = or_load(in, off + (size_t)i, dtype);
        s += v * v;
    }
    if (dtype == OR_BF16) return or_bf16_to_f32(or_f32_to_bf16(s));
    if (dtype == OR_F16) return or_f16_to_f32(or_f32_to_f16(s));
    return s;
}

static float row_sum(const void *in, size_t off, int64_t n, int dtype) {
    float s = 0.0f;
    for (int64_t i = 0; i < n; ++i) s += or_load(in, off + (size_t)i, dtype);
    return s;
}

/* applyRMSRowF32 compute.go:350-363 / applyRMSRowBF16 :365-374 / applyRMSRowF16 :376-385 */
static void rms_row(const void *in, const void *scale, void *out, size_t off, int64_t n,
                    double eps, int dtype) {
    float ss = row_sumsq(in, off, n, dtype);
    if (dtype == OR_F32) {
        double mean_square = (double)ss / (double)n;
        float inv = (float)(1.0 / sqrt(mean_square + eps));
        for (int64_t i = 0; i < n; ++i) {
            float combined = inv * ((const float *)scale)[i];
            ((float *)out)[off + (size_t)i] = ((const float *)in)[off + (size_t)i] * combined;
        }
        return;
    }
    float mean_square = ss / (float)n;
    float inv = (float)(1.0 / sqrt((double)mean_square + eps));
    for (int64_t i = 0; i < n; ++i) {
        float v = or_load(in, off + (size_t)i, dtype) * inv * or_load(scale, (size_t)i, dtype);
        or_store(out, off + (size_t)i, v, dtype);
    }
}

int or_rmsnorm(const void *input, const void *scale, void *output,
               int64_t rows, int64_t last_dim, double epsilon, int dtype) {
    if (rows == 0 || last_dim == 0) return 0;           /* compute.go:41-43 */
    if (!(epsilon > 0)) return -6;                      /* device/config.go:86-92 */
    if (dtype != OR_F32 && dtype != OR_BF16 && dtype != OR_F16) return -6;
#pragma omp parallel for schedule(static) num_threads(oracle_get_threads())
    for (int64_t r = 0; r < rows; ++r)
        rms_row(input, scale, output, (size_t)(r * last_dim), last_dim, epsilon, dtype);
    return 0;
}

/* runLayerNormF32 compute.go:109-127 + computeRowMean/Variance :335-343,
 * LayerNormApplyRowGeneric f32_generic.go:14-24;
 * applyLayerNormRowBF16 :484-497 (bf16-rounded sum, f32 variance, f32 eps add);
 * applyLayerNormRowF16 :499-511 (sequential f32 mean, no rounding) */
static void layernorm_row(const void *in, const void *scale, const void *bias, void *out,
                          size_t off, int64_t n, int dtype) {
    if (dtype == OR_F32) {
        const float *x = (const float *)in + off;
        double mean = (double)row_sum(in, off, n, OR_F32) / (double)n;
        float mean32 = (float)mean;
        float sq = 0.0f;
        for (int64_t i = 0; i < n; ++i) {
            float d = x[i] - mean32;
            sq += d * d;
        }
        double variance = (double)sq / (double)n;
        double inv = 1.0 / sqrt(variance + LAYERNORM_EPS);
        float inv32 = (float)inv;
        for (int64_t i = 0; i < n; ++i) {
            float d = x[i] - mean32;
            d *= inv32;
            d *= ((const float *)scale)[i];
            ((float *)out)[off + (size_t)i] = d + ((const float *)bias)[i];
        }
        return;
    }
    float mean;
    if (dtype == OR_BF16) {
        float s = row_sum(in, off, n, dtype);
        mean = or_bf16_to_f32(or_f32_to_bf16(s)) / (float)n;
    } else {
        mean = row_sum(in, off, n, dtype) / (float)n;
    }
    float variance = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
        float d = or_load(in, off + (size_t)i, dtype) - mean;
        variance += d * d;
    }
    variance = variance / (float)n;
    float inv = (float)(1.0 / sqrt((double)(variance + (float)LAYERNORM_EPS)));
    for (int64_t i = 0; i < n; ++i) {
        float normalized = (or_load(in, off + (size_t)i, dtype) - mean) * inv;
        float v = normalized * or_load(scale, (size_t)i, dtype) + or_load(bias, (size_t)i, dtype);
        or_store(out, off + (size_t)i, v, dtype);
    }
}

int or_layernorm(const void *input, const void *scale, const void *bias, void *output,
                 int64_t rows, int64_t last_dim, int dtype) {
    if (rows == 0 || last_dim == 0) return 0;           /* compute.go:19-21 */
    if (dtype != OR_F32 && dtype != OR_BF16 && dtype != OR_F16) return -6;
#pragma omp parallel for schedule(static) num_threads(oracle_get_threads())
    for (int64_t r = 0; r < rows; ++r)
        layernorm_row(input, scale, bias, output, (size_t)(r * last_dim), last_dim, dtype);
    return 0;
}

/* adaptiveRMSNormMeanSquare* compute.go:435-482: 256 strided lanes, then a
 * halving tree over the lanes */
static float adaptive_mean_square(const void *in, size_t off, int64_t n, int dtype) {
    float partial[256] = {0};
    for (int lane = 0; lane < 256; ++lane)
        for (int64_t c = lane; c < n; c += 256) {
            float v = or_load(in, off + (size_t)c, dtype);
            partial[lane] += v * v;
        }
    for (int stride = 128; stride > 0; stride >>= 1)
        for (int lane = 0; lane < stride; ++lane) partial[lane] += partial[lane + stride];
    return partial[0] / (float)n;
}

/* validateAdaptiveRMSNorm compute.go:624-644; rows compute.go:387-433 */
int or_adaptive_rmsnorm(const void *input, const void *modulation, void *output,
                        int64_t rows, int64_t last_dim, int64_t rows_per_batch,
                        int64_t modulation_cols, double epsilon, int dtype) {
    if (rows == 0 || last_dim == 0) return 0;
    if (!(epsilon > 0)) return -6;
    if (rows_per_batch <= 0 || rows % rows_per_batch != 0) return -6;
    if (modulation_cols < 2 * last_dim) return -6;
    if (dtype != OR_F32 && dtype != OR_BF16 && dtype != OR_F16) return -6;
#pragma omp parallel for schedule(static) num_threads(oracle_get_threads())
    for (int64_t r = 0; r < rows; ++r) {
        size_t off = (size_t)(r * last_dim);
        size_t moff = (size_t)((r / rows_per_batch) * modulation_cols);
        float ms = adaptive_mean_square(input, off, last_dim, dtype);
        float inv = (float)(1.0 / sqrt((double)ms + epsilon));
        for (int64_t c = 0; c < last_dim; ++c) {
            float normalized = or_load(input, off + (size_t)c, dtype) * inv;
            float sc = or_load(modulation, moff + (size_t)c, dtype);
            float sh = or_load(modulation, moff + (size_t)(last_dim + c), dtype);
            or_store(output, off + (size_t)c, normalized * (1 + sc) + sh, dtype);
        }
    }
    return 0;
}

/* validateModulatedLayerNorm compute.go:604-622, offsets :646-660, rows :513-570.
 * Shift at set*3H, scale at set*3H + H. */
int or_modulated_layernorm(const void *input, const void *modulation, void *output,
                           int64_t rows, int64_t last_dim, int64_t rows_per_batch,
                           int64_t modulation_cols, double epsilon, int set, int dtype) {
    if (rows == 0 || last_dim == 0) return 0;
    if (!(epsilon > 0) || set < 0) return -6;
    if (rows_per_batch <= 0 || rows % rows_per_batch != 0) return -6;
    if (modulation_cols < ((int64_t)set * 3 + 2) * last_dim) return -6;
    if (dtype != OR_F32 && dtype != OR_BF16 && dtype != OR_F16) return -6;
#pragma omp parallel for schedule(static) num_threads(oracle_get_threads())
    for (int64_t r = 0; r < rows; ++r) {
        size_t off = (size_t)(r * last_dim);
        size_t moff = (size_t)((r / rows_per_batch) * modulation_cols + (int64_t)set * last_dim * 3);
        float mean, inv;
        if (dtype == OR_F32) {
            const float *x = (const float *)input + off;
            double mean64 = (double)row_sum(input, off, last_dim, OR_F32) / (double)last_dim;
            float m32 = (float)mean64;
            float sq = 0.0f;
            for (int64_t i = 0; i < last_dim; ++i) {
                float d = x[i] - m32;
                sq += d * d;
            }
            double variance = (double)sq / (double)last_dim;
            inv = (float)(1.0 / sqrt(variance + epsilon));
            mean = m32;
        } else {
            if (dtype == OR_BF16)
                mean = or_bf16_to_f32(or_f32_to_bf16(row_sum(input, off, last_dim, dtype))) /
                       (float)last_dim;
            else
                mean = row_sum(input, off, last_dim, dtype) / (float)last_dim;
            float variance = 0.0f;
            for (int64_t i = 0; i < last_dim; ++i) {
                float d = or_load(input, off + (size_t)i, dtype) - mean;
                variance += d * d;
            }
            variance = variance / (float)last_dim;
            inv = (float)(1.0 / sqrt((double)variance + epsilon));
        }
        for (int64_t c = 0; c < last_dim; ++c) {
            float normalized = (or_load(input, off + (size_t)c, dtype) - mean) * inv;
            float sh = or_load(modulation, moff + (size_t)c, dtype);
            float sc = or_load(modulation, moff + (size_t)(last_dim + c), dtype);
            or_store(output, off + (size_t)c, normalized * (1 + sc) + sh, dtype);
        }
    }
    return 0;
}

/* copyGatedResidualFloat32 execution/math_gated_residual_intrinsic.go:206-223
 * (layout check :131-139).  16-bit formats compute in f32 and store in the
 * tensor dtype, as the only device implementation does
 * (device/metal/layernorm/layernorm.metal:152-174). */
int or_gated_residual(const void *residual, const void *branch, const void *modulation,
                      void *output, int64_t rows, int64_t last_dim, int64_t rows_per_batch,
                      int64_t modulation_cols, int set, int dtype) {
    if (rows == 0 || last_dim == 0) return 0;
    if (rows_per_batch <= 0 || rows % rows_per_batch != 0) return -6;
    if (set < 0 || modulation_cols < ((int64_t)set * 3 + 3) * last_dim) return -6;
    if (dtype != OR_F32 && dtype != OR_BF16 && dtype != OR_F16) return -6;
#pragma omp parallel for schedule(static) num_threads(oracle_get_threads())
    for (int64_t r = 0; r < rows; ++r) {
        size_t off = (size_t)(r * last_dim);
        size_t moff = (size_t)((r / rows_per_batch) * modulation_cols +
                               (int64_t)set * last_dim * 3 + last_dim * 2);
        for (int64_t c = 0; c < last_dim; ++c) {
            float res = or_load(residual, off + (size_t)c, dtype);
            float gate = or_load(modulation, moff + (size_t)c, dtype);
            float br = or_load(branch, off + (size_t)c, dtype);
            or_store(output, off + (size_t)c, res + gate * br, dtype);
        }
    }
    return 0;
}
