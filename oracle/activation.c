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
/* FastExp64 math/f64.go:10-32: the 2^f polynomial in float64, scaled by ldexp */
static double fast_exp64(double x) {
    if (x < -708.3964185322641) return 0.0;
    if (x > 709.782712893384) return 0x1p1023 * (1 + (1 - 0x1p-52));
    double z = x * 1.4426950408889634;
    int64_t k = (int64_t)z;
    if (z < 0) k--;
    double f = z - (double)k;
    double poly = 1.0 + f * (0.6931471805599453 + f * (0.2402265069591007 + f * (0.05550410706910451 +
                  f * (0.009618127167766223 + f * 0.001333899727232439))));
    return ldexp(poly, (int)k);
}
double or_fast_exp64(double x) { return fast_exp64(x); }
/* FastSilu64 math/f64.go:90-92, narrowed to float32 as the 16-bit tables are
 * filled (activation/lut.go:14-62: lut[bits] = narrow(float32(op(float64(x))))) */
static float silu64(float v) {
    double x = (double)v;
    return (float)(x / (1 + fast_exp64(-x)));
}
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
float or_fast_tanh32(float x) { return tanh_pade32(x); }
float or_fast_sigmoid32(float x) { return sigmoid32(x); }
float or_fast_silu64(float x) { return silu64(x); }
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
    case OR_GATE_SEGLU: return u * sigmoid32(g);          /* FastSeGLU32 extra_activation.go:88-90 */
    default: return NAN;
    }
}

static int gated_dtype_ok(int dtype) { return dtype == OR_F32 || dtype == OR_F16 || dtype == OR_BF16; }

int or_gated_tensors(int kind, void *dst, const void *gate, const void *up,
                     int64_t count, int dtype) {
    if (count == 0) return 0;
    if (!gated_dtype_ok(dtype) || kind < 0 || kind > OR_GATE_SEGLU) return -6;
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
    if (!gated_dtype_ok(dtype) || kind < 0 || kind > OR_GATE_SEGLU) return -6;
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

/* unary Silu / Gelu (activation/ops.go:37-51, dispatchActivation f32_apply.go:128-148):
 * f32 runs FastSilu32 / FastGelu32 per element (f32_generic.go:72-97); f16 / bf16
 * look each input up in a table filled with narrow(float32(FastSilu64 /
 * FastGelu64(x))) (lut.go:14-62).  float32(FastGelu64(x)) is gelu32's own
 * arithmetic; FastSilu64 differs from FastSilu32 (float64 exp and division). */
int or_unary(int kind, void *dst, const void *src, int64_t count, int dtype) {
    if (count == 0) return 0;
    if (!gated_dtype_ok(dtype) || (kind != OR_UNARY_SILU && kind != OR_UNARY_GELU)) return -6;
#pragma omp parallel for schedule(static) num_threads(oracle_get_threads())
    for (int64_t i = 0; i < count; ++i) {
        float v = or_load(src, (size_t)i, dtype);
        float y = kind == OR_UNARY_SILU ? (dtype == OR_F32 ? silu32(v) : silu64(v)) : gelu32(v);
        or_store(dst, (size_t)i, y, dtype);
    }
    return 0;
}
