/*
 * Integer (de)quantisation and the remaining convert/ casts (int8, int4, f64).
 *
 * TEST INFRASTRUCTURE ONLY: the checker for puter_amd/csrc/quant.hip; nothing
 * in the shipped library links or calls it.
 *
 * Semantics followed (reference file:line):
 *   Dequant   device/cpu/dequant/ops.go:11-37 -> dequantInt8Generic
 *             device/cpu/dequant/int8_generic.go:3-7:
 *             dst = float32(int32(src) - int32(zeroPoint)) * scale
 *   Dequant4  device/cpu/dequant/ops.go:39-58 -> dequantInt4Generic
 *             device/cpu/dequant/int4_generic.go:5-10:
 *             dst = float32(int(nibble) - int(zeroPoint)) * scale
 *   Quant     device/cpu/quant/ops.go:10-37 -> quantInt8Generic
 *             device/cpu/quant/int8_generic.go:5-18:
 *             scaled = math.Round(float64(value / scale)) + float64(zeroPoint),
 *             saturated to [-128, 127]
 *   casts     convert/int_f32.go:14-25 (Int8ToFloat32), :30-52 (Float32ToInt8:
 *             saturate, else truncate toward zero), :59-77 (Int4ToFloat32),
 *             convert/f32_f64.go:8-17 (Float32ToFloat64 / Float64ToFloat32).
 *
 * Int4 layout: Int4Vector / Int4Pair live in github.com/theapemachine/manifesto
 * (absent here).  The reference's own SIMD kernel states it and its parity
 * tests hold it against Int4Vector.Get: element 2k is the low nibble of byte k,
 * element 2k+1 the high nibble, each a signed 4-bit value
 * (device/cpu/dequant/dequant_int4_neon_arm64.s:4-6; the x86 macros
 * x86_int4_macros.inc:6-14 sign-extend the same way).
 *
 * Quant follows the generic kernel (the parity tests' reference function,
 * quant_int8_generic_parity_test.go:13-25): an f32 division and
 * round-half-away-from-zero.  The AVX-512 kernel the reference dispatches to
 * on amd64 (int8_avx512_amd64.s:27-35) multiplies by 1/scale and rounds ties
 * to even; the two agree except on exact .5 ties and where x * (1/scale)
 * rounds differently from x / scale, which the reference's tests never hit
 * (scale 0.125, Gaussian inputs).
 *
 * NaN: Go's int8(NaN) is implementation-defined; on amd64 the conversion
 * (CVTTSD2SL / CVTTSS2SL, low byte kept) yields 0, which is the rule used for
 * Quant and Float32ToInt8 (parity unpinned by the reference's tests).
 *
 * f32 <-> f64: plain C conversions, which on x86-64 compile to CVTSS2SD /
 * CVTSD2SS exactly as Go's conversions do on amd64 (round to nearest even,
 * signalling NaNs quieted, the payload's top bits kept).
 */
#include <math.h>
#include <string.h>

#include "oracle.h"

float or_dequant_int8_one(int8_t code, float scale, int8_t zero_point) {
    return (float)((int32_t)code - (int32_t)zero_point) * scale;
}

int or_int4_nibble(const uint8_t *src, size_t index) {
    const uint8_t b = src[index >> 1];
    const int v = (index & 1) ? (b >> 4) : (b & 15);
    return v >= 8 ? v - 16 : v;
}

int8_t or_quant_int8_one(float value, float scale, int8_t zero_point) {
    const float quotient = value / scale;  /* f32 division, as Go's value/scale */
    const double scaled = round((double)quotient) + (double)zero_point;
    if (scaled > 127.0) return 127;
    if (scaled < -128.0) return -128;
    if (isnan(scaled)) return 0;
    return (int8_t)scaled;
}

int8_t or_f32_to_int8(float value) {
    if (value < -128.0f) return -128;
    if (value > 127.0f) return 127;
    if (isnan(value)) return 0;
    return (int8_t)(int)value;  /* truncation toward zero */
}

int or_dequant_int8(float *dst, const int8_t *src, size_t count, float scale, int zero_point) {
    if (zero_point < -128 || zero_point > 127) return -6;
    for (size_t i = 0; i < count; ++i) dst[i] = or_dequant_int8_one(src[i], scale, (int8_t)zero_point);
    return 0;
}

int or_dequant_int4(float *dst, const uint8_t *src, size_t count, float scale, int zero_point) {
    if (zero_point < -128 || zero_point > 127) return -6;
    for (size_t i = 0; i < count; ++i)
        dst[i] = (float)(or_int4_nibble(src, i) - zero_point) * scale;
    return 0;
}

int or_quant_int8(int8_t *dst, const float *src, size_t count, float scale, int zero_point) {
    if (zero_point < -128 || zero_point > 127) return -6;
    for (size_t i = 0; i < count; ++i) dst[i] = or_quant_int8_one(src[i], scale, (int8_t)zero_point);
    return 0;
}

/* Int8ToFloat32, Float32ToInt8, Int4ToFloat32, Float32ToFloat64, Float64ToFloat32 */
int or_cast_ext(void *dst, int dst_dtype, const void *src, int src_dtype, size_t count) {
    if (src_dtype == OR_I8 && dst_dtype == OR_F32) {
        for (size_t i = 0; i < count; ++i) ((float *)dst)[i] = (float)((const int8_t *)src)[i];
    } else if (src_dtype == OR_F32 && dst_dtype == OR_I8) {
        for (size_t i = 0; i < count; ++i) ((int8_t *)dst)[i] = or_f32_to_int8(((const float *)src)[i]);
    } else if (src_dtype == OR_I4 && dst_dtype == OR_F32) {
        for (size_t i = 0; i < count; ++i) ((float *)dst)[i] = (float)or_int4_nibble((const uint8_t *)src, i);
    } else if (src_dtype == OR_F32 && dst_dtype == OR_F64) {
        for (size_t i = 0; i < count; ++i) ((double *)dst)[i] = (double)((const float *)src)[i];
    } else if (src_dtype == OR_F64 && dst_dtype == OR_F32) {
        for (size_t i = 0; i < count; ++i) ((float *)dst)[i] = (float)((const double *)src)[i];
    } else {
        return -6;
    }
    return 0;
}

/* shape.cast between two float formats without an f32 side
 * (execution/shape_cast_intrinsic.go:56-115): every source value widened to
 * float64 (convert.BytesToFloat64; exact for bf16 / f16 / fp8 / f64), then
 * float32(v) narrowed to the target (NewBfloat16FromFloat32(float32(v)),
 * Fromfloat32(float32(v)), NewF8E4M3/E5M2FromFloat32(float32(v))), or the
 * float64 kept for an f64 target.  Same format: the input unchanged (:35-41). */
static int or_float_fmt(int dt) { return dt == OR_F16 || dt == OR_BF16 || dt == OR_F8E4M3 || dt == OR_F8E5M2 || dt == OR_F64; }
int or_cast_pair(void *dst, int dst_dtype, const void *src, int src_dtype, size_t count) {
    if (!or_float_fmt(src_dtype) || !or_float_fmt(dst_dtype)) return -6;
    for (size_t i = 0; i < count; ++i) {
        double v = src_dtype == OR_F64 ? ((const double *)src)[i] : (double)or_load(src, i, src_dtype);
        if (dst_dtype == OR_F64) {
            ((double *)dst)[i] = v;
        } else if (src_dtype == dst_dtype) {
            size_t es = dst_dtype == OR_F16 || dst_dtype == OR_BF16 ? 2 : 1;
            memcpy((char *)dst + i * es, (const char *)src + i * es, es);
        } else {
            or_store(dst, i, (float)v, dst_dtype);
        }
    }
    return 0;
}
