/*
 * Scalar dtype codecs and FastExp32 for the CPU oracle (test infrastructure
 * only; see oracle.h).
 *
 * Reference call sites: convert/bf16_f32.go:26,34; convert/f16_f32.go:30,38;
 * convert/fp8_f32.go:14,30,45,61; device/cpu/rope/dtype_load.go:9-28;
 * device/cpu/activation/compute.go:17-36.  The scalar converters themselves live
 * in github.com/theapemachine/manifesto/dtype (go.mod:5 replaces it by a local
 * path that is not shipped, go.mod:17 names v1.2.3), so the rules below are
 * restated from the documents and hand-written code that the reference does hold:
 *
 *  bf16 narrow: round-to-nearest-even via (u + 0x7FFF + ((u >> 16) & 1)) >> 16,
 *    the reference's own AVX-512 pack (device/cpu/avx512_bf16_macros.inc:47-59).
 *    NaN -> quiet NaN keeping sign and top payload bits (u >> 16 | 0x0040); the
 *    asm has no NaN branch, so NaN encoding is parity unpinned.
 *  f16 narrow: IEEE binary16 round-to-nearest-even with subnormals
 *    (convert/f16_f32.go:14-16).  The F16 API (Fromfloat32/Frombits/Bits) is the
 *    x448/float16 one, whose NaN rule (sign | 0x7C00 | 0x0200 | mant >> 13) is
 *    used here.
 *  fp8 narrow: "saturating round-to-nearest-even" (convert/fp8_f32.go:20-23,51-54).
 *    E4M3FN: bias 7, no infinities, NaN = S.1111.111 (0x7F/0xFF,
 *    device/cpu/elementwise/fp8_test.go:24-29,131-133), max finite 448.
 *    E5M2: bias 15, exponent 0x1F = Inf/NaN (fp8_test.go:46), max finite 57344.
 *    Any |x| at or above the largest finite value, infinities included,
 *    saturates to +-max finite; NaN -> 0x7F|s (E4M3FN) and 0x7E|s (E5M2).
 *  widening: bf16 = bits << 16; f16 exact (NaN keeps payload, x448 rule);
 *    fp8 per the OCP 8-bit floating point specification (NaN -> sign|0x7FC00000).
 *
 * FastExp32 follows device/cpu/math/f32.go:21-46 operation by operation.
 */
#include "oracle.h"

#include <math.h>
#include <string.h>

static inline uint32_t f2u(float v) { uint32_t u; memcpy(&u, &v, 4); return u; }
static inline float u2f(uint32_t u) { float v; memcpy(&v, &u, 4); return v; }

float or_bf16_to_f32(uint16_t bits) { return u2f((uint32_t)bits << 16); }

uint16_t or_f32_to_bf16(float value) {
    uint32_t u = f2u(value);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x0040u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float or_f16_to_f32(uint16_t bits) {
    uint32_t sign = (uint32_t)(bits & 0x8000u) << 16;
    uint32_t exp = (bits >> 10) & 0x1Fu;
    uint32_t man = bits & 0x3FFu;
    if (exp == 0x1F) return u2f(sign | 0x7F800000u | (man << 13));
    if (exp == 0) {
        /* subnormal or zero: man * 2^-24, exact in f32 */
        float mag = (float)man * 0x1p-24f;
        return u2f(sign | f2u(mag));
    }
    return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t or_f32_to_f16(float value) {
    uint32_t u = f2u(value);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7FFFFFFFu;
    if (a >= 0x7F800000u) {
        if (a == 0x7F800000u) return sign | 0x7C00u;
        return (uint16_t)(sign | 0x7C00u | 0x0200u | ((a & 0x7FFFFFu) >> 13));
    }
    if (a >= 0x477FF000u) return sign | 0x7C00u; /* rounds to >= 65536: overflow to Inf */
    if (a >= 0x38800000u) {
        /* normal in f16: rebias exponent (127 -> 15) and round 13 bits */
        uint32_t t = a - (112u << 23);
        t += 0x0FFFu + ((t >> 13) & 1u);
        return (uint16_t)(sign | (t >> 13));
    }
    /* subnormal in f16: magnitude * 2^24 rounded to an integer (RNE) */
    float scaled = u2f(a) * 0x1p24f;
    float r = nearbyintf(scaled);
    return (uint16_t)(sign | (uint16_t)r);
}

float or_e4m3_to_f32(uint8_t bits) {
    uint32_t sign = (uint32_t)(bits & 0x80u) << 24;
    uint32_t exp = (bits >> 3) & 0xFu;
    uint32_t man = bits & 0x7u;
    if (exp == 0xF && man == 0x7) return u2f(sign | 0x7FC00000u);
    if (exp == 0) return u2f(sign | f2u((float)man * 0x1p-9f));
    return u2f(sign | ((exp + 120u) << 23) | (man << 20));
}

uint8_t or_f32_to_e4m3(float value) {
    uint32_t u = f2u(value);
    uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
    uint32_t a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return sign | 0x7Fu;
    if (a >= 0x43E00000u) return sign | 0x7Eu; /* >= 448 (and Inf): saturate */
    if (a >= 0x3C800000u) {                    /* >= 2^-6: normal */
        uint32_t t = a - (120u << 23);
        t += 0x7FFFFu + ((t >> 20) & 1u);
        return (uint8_t)(sign | (t >> 20));
    }
    float r = nearbyintf(u2f(a) * 0x1p9f);
    return (uint8_t)(sign | (uint8_t)r);
}

float or_e5m2_to_f32(uint8_t bits) {
    uint32_t sign = (uint32_t)(bits & 0x80u) << 24;
    uint32_t exp = (bits >> 2) & 0x1Fu;
    uint32_t man = bits & 0x3u;
    if (exp == 0x1F) return man ? u2f(sign | 0x7FC00000u) : u2f(sign | 0x7F800000u);
    if (exp == 0) return u2f(sign | f2u((float)man * 0x1p-16f));
    return u2f(sign | ((exp + 112u) << 23) | (man << 21));
}

uint8_t or_f32_to_e5m2(float value) {
    uint32_t u = f2u(value);
    uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
    uint32_t a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return sign | 0x7Eu;
    if (a >= 0x47600000u) return sign | 0x7Bu; /* >= 57344 (and Inf): saturate */
    if (a >= 0x38800000u) {                    /* >= 2^-14: normal */
        uint32_t t = a - (112u << 23);
        t += 0xFFFFFu + ((t >> 21) & 1u);
        return (uint8_t)(sign | (t >> 21));
    }
    float r = nearbyintf(u2f(a) * 0x1p16f);
    return (uint8_t)(sign | (uint8_t)r);
}

/* device/cpu/math/f32.go:21-46 */
float or_fast_exp32(float x) {
    if (x < -87.33654f) return 0.0f;
    if (x > 88.72283f) return 0x1p127f * (1.0f + (1.0f - 0x1p-23f));
    float z = x * 1.4426950408889634f;
    int32_t k = (int32_t)z;
    if (z < 0) k--;
    volatile float kf = (float)k; /* fastExp32Fraction is //go:noinline: plain subtract */
    float f = z - kf;
    float poly = 1.0f + f * (0.69314718f + f * (0.24022650f + f * (0.05550410f +
                 f * (0.00961812f + f * 0.00133389f))));
    uint32_t bits = f2u(poly);
    bits += (uint32_t)k << 23;
    return u2f(bits);
}

float or_load(const void *base, size_t index, int dtype) {
    switch (dtype) {
    case OR_F32: return ((const float *)base)[index];
    case OR_F16: return or_f16_to_f32(((const uint16_t *)base)[index]);
    case OR_BF16: return or_bf16_to_f32(((const uint16_t *)base)[index]);
    case OR_F8E4M3: return or_e4m3_to_f32(((const uint8_t *)base)[index]);
    case OR_F8E5M2: return or_e5m2_to_f32(((const uint8_t *)base)[index]);
    default: return NAN;
    }
}

void or_store(void *base, size_t index, float value, int dtype) {
    switch (dtype) {
    case OR_F32: ((float *)base)[index] = value; break;
    case OR_F16: ((uint16_t *)base)[index] = or_f32_to_f16(value); break;
    case OR_BF16: ((uint16_t *)base)[index] = or_f32_to_bf16(value); break;
    case OR_F8E4M3: ((uint8_t *)base)[index] = or_f32_to_e4m3(value); break;
    case OR_F8E5M2: ((uint8_t *)base)[index] = or_f32_to_e5m2(value); break;
    default: break;
    }
}

static int valid_float_dtype(int dtype) { return dtype >= OR_F32 && dtype <= OR_F8E5M2; }

int or_cast_to_f32(float *dst, const void *src, size_t count, int src_dtype) {
    if (!valid_float_dtype(src_dtype)) return -6;
#pragma omp parallel for schedule(static) num_threads(oracle_get_threads())
    for (long i = 0; i < (long)count; ++i) dst[i] = or_load(src, (size_t)i, src_dtype);
    return 0;
}

int or_cast_from_f32(void *dst, const float *src, size_t count, int dst_dtype) {
    if (!valid_float_dtype(dst_dtype)) return -6;
#pragma omp parallel for schedule(static) num_threads(oracle_get_threads())
    for (long i = 0; i < (long)count; ++i) or_store(dst, (size_t)i, src[i], dst_dtype);
    return 0;
}

static int g_threads = 1;
void oracle_set_threads(int threads) { g_threads = threads > 0 ? threads : 1; }
int oracle_get_threads(void) { return g_threads; }
