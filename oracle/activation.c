/*
 * Gated activations for the CPU oracle (test infrastructure only; see oracle.h).
 * Restates device/cpu/activation/gated.go:10-136 (tensor and packed forms),
 * dispatchGatedPacked / dispatchGatedTensors compute.go:72-176 and the scalar
 * math of device/cpu/math/f32.go:88-105, math/activation.go:26-57,290-308,
 * math/extra_activation.go:84-90.
 */
#include "oracle.h"

#include <math.h>

#define GELU_TANH_ALPHA 0.7978845608028654 /* math/constant.go:20 */
#define GELU_TANH_BETA 0.044715            /* math/constant.go:21 */
#define SQRT_TWO_OVER_TWO 0.7071067811865475 /* math/activation.go:15 */

static float sigmoid32(float v) { /* FastSigmoid32 f32.go:88-95 */
    if (v >= 0) return 1 / (1 + or_fast_exp32(-v));
    float e = or_fast_exp32(v);
    return e / (1 + e);
}
static float silu32(float v) { return v / (1 + or_fast_exp32(-v)); } /* f32.go:97-99 */
static float gelu32(float v) { /* FastGelu32 activation.go:54-57 */
    double x = (double)v;
    return (float)(0.5 * x * (1 + erf(x * SQRT_TWO_OVER_TWO)));
}
static float tanh_pade32(float x) { /* FastTanh32 f32.go:74-86 */
    if (x > 4.92f) return 1.0f;
    if (x < -4.92f) return -1.0f;
    float x2 = x * x;
    float num = x * (135135.0f + x2 * (17325.0f + x2 * (378.0f + x2)));
    float den = 135135.0f + x2 * (62370.0f + x2 * (3150.0f + x2 * 28.0f));
    return num / den;
}
static float gelu_tanh32(float v) { /* FastGeluTanh32 f32.go:101-105 */
    double x = (double)v;
    double inner = GELU_TANH_ALPHA * (x + GELU_TANH_BETA * x * x * x);
    return (float)(0.5 * x * (1 + (double)tanh_pade32((float)inner)));
}

static float combine(int kind, float g, float u) {
    switch (kind) {
    case OR_GATE_SWIGLU: return silu32(g) * u;            /* FastSwiGLU32 activation.go:294-296 */
    case OR_GATE_GEGLU: return g * gelu32(u);             /* FastGeGLU32 activation.go:290-292 */
    case OR_GATE_GEGLU_TANH: return g * gelu_tanh32(u);   /* FastGeGLUTanh32 activation.go:306-308 */
    case OR_GATE_SIGLU: return sigmoid32(g) * u;          /* FastSiGLU32 activation.go:302-304 */
    case OR_GATE_GLU: return g * sigmoid32(u);            /* FastGLU32 activation.go:286-288 */
    case OR_GATE_REGLU: return g * (u > 0 ? u : 0);       /* FastReGLU32 activation.go:298-300 */
    case OR_GATE_LINGLU: return g * u;                    /* FastLinGLU32 extra_activation.go:84-86 */
    default: return NAN;
    }
}

static int gated_dtype_ok(int dtype) { return dtype == OR_F32 || dtype == OR_F16 || dtype == OR_BF16; }

int or_gated_tensors(int kind, void *dst, const void *gate, const void *up,
                     int64_t count, int dtype) {
    if (count == 0) return 0;
    if (!gated_dtype_ok(dtype) || kind < 0 || kind > OR_GATE_LINGLU) return -6;
#pragma omp parallel for schedule(static) num_threads(oracle_get_threads())
    for (int64_t i = 0; i < count; ++i)
        or_store(dst, (size_t)i, combine(kind, or_load(gate, (size_t)i, dtype),
                                         or_load(up, (size_t)i, dtype)), dtype);
    return 0;
}

/* packed rows [gate(half) | up(half)] -> [half], compute.go:72-116 */
int or_gated_packed(int kind, void *dst, const void *packed,
                    int64_t batch, int64_t half_count, int dtype) {
    if (batch == 0 || half_count == 0) return 0;
    if (!gated_dtype_ok(dtype) || kind < 0 || kind > OR_GATE_LINGLU) return -6;
#pragma omp parallel for schedule(static) num_threads(oracle_get_threads())
    for (int64_t b = 0; b < batch; ++b) {
        size_t row = (size_t)(b * half_count * 2), out = (size_t)(b * half_count);
        for (int64_t i = 0; i < half_count; ++i) {
            float g = or_load(packed, row + (size_t)i, dtype);
            float u = or_load(packed, row + (size_t)(half_count + i), dtype);
            or_store(dst, out + (size_t)i, combine(kind, g, u), dtype);
        }
    }
    return 0;
}

/* unary Silu / Gelu (activation/ops.go:37-51): per-element FastSilu32 /
 * FastGelu32; the 16-bit LUT paths tabulate the same scalar function */
int or_unary(int kind, void *dst, const void *src, int64_t count, int dtype) {
    if (count == 0) return 0;
    if (!gated_dtype_ok(dtype) || (kind != OR_UNARY_SILU && kind != OR_UNARY_GELU)) return -6;
#pragma omp parallel for schedule(static) num_threads(oracle_get_threads())
    for (int64_t i = 0; i < count; ++i) {
        float v = or_load(src, (size_t)i, dtype);
        or_store(dst, (size_t)i, kind == OR_UNARY_SILU ? silu32(v) : gelu32(v), dtype);
    }
    return 0;
}
