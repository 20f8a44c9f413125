// Integer (de)quantisation and the int8 / int4 / f64 casts.
//
// Reference semantics:
//   Dequant   device/interface.go:197 -> device/cpu/dequant/ops.go:11-37,
//             dequantInt8Generic int8_generic.go:3-7:
//             dst = float32(int32(src) - int32(zeroPoint)) * scale  (F32 <- Int8 only)
//   Dequant4  device/interface.go:198 -> dequant/ops.go:39-58, int4_generic.go:5-10:
//             dst = float32(int(nibble) - int(zeroPoint)) * scale  (F32 <- Int4 only)
//   Quant     device/interface.go:580-582 -> device/cpu/quant/ops.go:10-37,
//             quantInt8Generic int8_generic.go:5-18:
//             round-half-away(float64(value / scale)) + zeroPoint, saturated to int8
//   casts     convert/int_f32.go:14-77 (Int8ToFloat32, Float32ToInt8 saturating
//             then truncating, Int4ToFloat32), convert/f32_f64.go:8-17.
// Int4 streams hold two signed nibbles per byte, element 2k in the low nibble
// of byte k and element 2k+1 in the high nibble
// (device/cpu/dequant/dequant_int4_neon_arm64.s:4-6).
// Quant follows the generic kernel (an f32 division, ties away from zero); a
// NaN input, which Go's int8 conversion leaves implementation-defined, gives 0
// as Go's conversion does on amd64.  f64 <-> f32 is done on the integer bits:
// round to nearest even with gradual underflow, signalling NaNs quieted and
// the payload's top bits kept (what CVTSS2SD / CVTSD2SS do for Go on amd64),
// independent of the GPU's float mode registers.
//
// HBM-bound streaming kernels: one grid-strided map kernel per conversion.
// A unit is a small fixed group of elements sized so that lane l's unit
// (u = base + k*256 + l) keeps both sides of every wave-wide load and store
// contiguous (e.g. 4 int8 = 4 bytes in, 16 bytes of f32 out); each thread issues
// kUnroll units' loads before it converts and stores them.  Unaligned buffers and
// the ragged tail go element by element.
#include "common.hpp"
#include <algorithm>
#include <cmath>

namespace puter {

constexpr int kQuantUnroll = 4;

// ---- element rules --------------------------------------------------------
__device__ __forceinline__ float dequant_one(int code, float scale, int zp) {
    return (float)(code - zp) * scale;
}
__device__ __forceinline__ int int4_nibble(uint32_t byte, int high) {
    const int v = high ? (int)((byte >> 4) & 15u) : (int)(byte & 15u);
    return v >= 8 ? v - 16 : v;
}
__device__ __forceinline__ uint32_t quant_one(float value, float scale, int zp) {
    const float q = __fdiv_rn(value, scale);
    float r = truncf(q);
    if (fabsf(q - r) >= 0.5f) r += copysignf(1.0f, q);  // math.Round: ties away from zero
    const float scaled = r + (float)zp;                  // exact below 2^24, saturates above
    if (scaled > 127.0f) return 0x7Fu;
    if (scaled < -128.0f) return 0x80u;
    if (scaled != scaled) return 0u;
    return (uint32_t)(int)scaled & 0xFFu;
}
// Quant without the division on the common path.  With inv = RN(1/scale) a
// normal number (the launcher checks 2^-125 <= |scale| <= 2^125), qa =
// RN(value * inv) is within 1.5 * 2^-23 |value/scale| (< 2^-22.4 |qa|) of
// q = RN(value / scale): three roundings of at most 2^-24 each.  Rounding half
// away from zero gives the same integer for qa and q unless a half-integer
// lies within that distance, so the result is exact whenever qa is more than
// 2^-21 |qa| from a tie; |qa| >= 256 saturates on its sign either way
// (|zero point| <= 128).  Branch-free; returns false (NaN, or near a tie) when
// the exact division must decide.
__device__ __forceinline__ bool quant_try(float value, float inv, int zp, uint32_t &out) {
    const float qa = value * inv;
    const float aq = fabsf(qa);
    const float t = truncf(qa);
    const float frac = fabsf(qa - t);
    const float r = frac > 0.5f ? t + copysignf(1.0f, qa) : t;
    const float scaled = fminf(fmaxf(r + (float)zp, -128.0f), 127.0f);  // integral: exact saturation
    out = (uint32_t)(int)scaled & 0xFFu;
    return aq >= 256.0f || fabsf(frac - 0.5f) > aq * 0x1p-21f;
}
__device__ __forceinline__ uint32_t f32_to_i8(float v) {
    if (v < -128.0f) return 0x80u;
    if (v > 127.0f) return 0x7Fu;
    if (v != v) return 0u;
    return (uint32_t)(int)v & 0xFFu;  // truncation toward zero
}

// ---- conversions as unit / element operations ------------------------------
struct DequantI8Op {  // also Int8ToFloat32 (scale 1, zero point 0: exact)
    static constexpr int N = 4;
    using In = uint32_t;
    float *dst;
    const uint8_t *src;
    float scale;
    int zp;
    __device__ In load(size_t u) const { return __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(src) + u); }
    __device__ void store(size_t u, In w) const {
        float f[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) f[i] = dequant_one((int)(int8_t)(w >> (8 * i)), scale, zp);
        st_stream(make_uint4(__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]), __float_as_uint(f[3])),
                  reinterpret_cast<uint4 *>(dst) + u);
    }
    __device__ void elem(size_t i) const { dst[i] = dequant_one((int)(int8_t)src[i], scale, zp); }
};

struct DequantI4Op {  // also Int4ToFloat32
    static constexpr int N = 4;
    using In = uint32_t;  // 16 bits used: 4 nibbles
    float *dst;
    const uint8_t *src;
    float scale;
    int zp;
    __device__ In load(size_t u) const { return reinterpret_cast<const uint16_t *>(src)[u]; }
    __device__ void store(size_t u, In w) const {
        float f[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) f[i] = dequant_one(int4_nibble(w >> (8 * (i >> 1)), i & 1), scale, zp);
        st_stream(make_uint4(__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]), __float_as_uint(f[3])),
                  reinterpret_cast<uint4 *>(dst) + u);
    }
    __device__ void elem(size_t i) const { dst[i] = dequant_one(int4_nibble(src[i >> 1], (int)(i & 1)), scale, zp); }
};

template <bool QUANT>  // QUANT: Quant (scale, zero point); else Float32ToInt8
struct ToI8Op {
    static constexpr int N = 4;
    using In = uint4;
    uint8_t *dst;
    const float *src;
    float scale;
    int zp;
    float inv;     // RN(1 / scale) when fast, see quant_one_fast
    int fast;
    __device__ uint32_t one(float v) const {
        if constexpr (!QUANT) return f32_to_i8(v);
        else return quant_one(v, scale, zp);
    }
    __device__ In load(size_t u) const { return ld_stream(reinterpret_cast<const uint4 *>(src) + u); }
    __device__ void store(size_t u, In w) const {
        const float v[4] = {__uint_as_float(w.x), __uint_as_float(w.y), __uint_as_float(w.z), __uint_as_float(w.w)};
        uint32_t b = 0;
        bool exact = true;
        if constexpr (QUANT) {
            if (fast) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    uint32_t r;
                    exact = quant_try(v[i], inv, zp, r) && exact;
                    b |= r << (8 * i);
                }
            } else {
                exact = false;
            }
        }
        if (!QUANT || __any(!exact)) {  // wave-uniform: the exact rule for the whole unit
            b = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) b |= one(v[i]) << (8 * i);
        }
        __builtin_nontemporal_store(b, reinterpret_cast<uint32_t *>(dst) + u);
    }
    __device__ void elem(size_t i) const { dst[i] = (uint8_t)one(src[i]); }
};

struct F32ToF64Op {
    static constexpr int N = 2;
    using In = uint2;
    uint64_t *dst;
    const uint32_t *src;
    __device__ In load(size_t u) const {
        typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
        const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(src) + u);
        return make_uint2(v.x, v.y);
    }
    __device__ void store(size_t u, In w) const {
        const uint64_t a = f32_to_f64_bits(w.x), b = f32_to_f64_bits(w.y);
        st_stream(make_uint4((uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b, (uint32_t)(b >> 32)),
                  reinterpret_cast<uint4 *>(dst) + u);
    }
    __device__ void elem(size_t i) const { dst[i] = f32_to_f64_bits(src[i]); }
};

struct F64ToF32Op {
    static constexpr int N = 2;
    using In = uint4;
    uint32_t *dst;
    const uint64_t *src;
    __device__ In load(size_t u) const { return ld_stream(reinterpret_cast<const uint4 *>(src) + u); }
    __device__ void store(size_t u, In w) const {
        typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
        u32x2 t = {f64_to_f32_bits(((uint64_t)w.y << 32) | w.x), f64_to_f32_bits(((uint64_t)w.w << 32) | w.z)};
        __builtin_nontemporal_store(t, reinterpret_cast<u32x2 *>(dst) + u);
    }
    __device__ void elem(size_t i) const { dst[i] = f64_to_f32_bits(src[i]); }
};

template <class Op>
__global__ __launch_bounds__(256) void map_kernel(Op op, int64_t count, int vectorised) {
    const size_t tid = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t gstride = (size_t)gridDim.x * 256;
    size_t body = 0;
    if (vectorised) {
        const size_t units = (size_t)count / Op::N;
        for (size_t base = (size_t)blockIdx.x * 256 * kQuantUnroll + threadIdx.x; base < units;
             base += gstride * kQuantUnroll) {
            typename Op::In in[kQuantUnroll];
#pragma unroll
            for (int k = 0; k < kQuantUnroll; ++k)
                if (base + k * 256 < units) in[k] = op.load(base + k * 256);
#pragma unroll
            for (int k = 0; k < kQuantUnroll; ++k)
                if (base + k * 256 < units) op.store(base + k * 256, in[k]);
        }
        body = units * Op::N;
    }
    for (size_t i = body + tid; i < (size_t)count; i += gstride) op.elem(i);
}

template <class Op>
static int launch_map(const Op &op, int64_t count, bool vectorised, hipStream_t s, const char *what) {
    const int64_t per_block = vectorised ? 256LL * Op::N * kQuantUnroll : 256;
    const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>((count + per_block - 1) / per_block, 8192));
    map_kernel<Op><<<(unsigned)blocks, 256, 0, s>>>(op, count, vectorised ? 1 : 0);
    return check_launch(what);
}

static int check_config(int64_t count, const void *dst, const void *src, int zero_point, const char *what) {
    if (count < 0) return fail(PUTER_ERR_INVALID, "%s: negative count", what);
    if (zero_point < -128 || zero_point > 127) return fail(PUTER_ERR_INVALID, "%s: zero point %d outside int8", what, zero_point);
    if (count > 0 && (!dst || !src)) return fail(PUTER_ERR_NIL, "%s: nil buffer", what);
    return PUTER_OK;
}

// int8 / int4 / f64 legs of puter_hip_cast (one side is F32)
int cast_ext(void *dst, int dst_dtype, const void *src, int src_dtype, int64_t count, hipStream_t s) {
    const bool vec = aligned16(dst) && aligned16(src);
    if (src_dtype == PUTER_I8 && dst_dtype == PUTER_F32)
        return launch_map(DequantI8Op{static_cast<float *>(dst), static_cast<const uint8_t *>(src), 1.0f, 0}, count, vec, s, "cast");
    if (src_dtype == PUTER_I4 && dst_dtype == PUTER_F32)
        return launch_map(DequantI4Op{static_cast<float *>(dst), static_cast<const uint8_t *>(src), 1.0f, 0}, count, vec, s, "cast");
    if (src_dtype == PUTER_F32 && dst_dtype == PUTER_I8)
        return launch_map(ToI8Op<false>{static_cast<uint8_t *>(dst), static_cast<const float *>(src), 1.0f, 0, 1.0f, 0}, count, vec, s, "cast");
    if (src_dtype == PUTER_F32 && dst_dtype == PUTER_F64)
        return launch_map(F32ToF64Op{static_cast<uint64_t *>(dst), static_cast<const uint32_t *>(src)}, count, vec, s, "cast");
    if (src_dtype == PUTER_F64 && dst_dtype == PUTER_F32)
        return launch_map(F64ToF32Op{static_cast<uint32_t *>(dst), static_cast<const uint64_t *>(src)}, count, vec, s, "cast");
    return fail(PUTER_ERR_INVALID, "cast: unsupported pair %d -> %d", src_dtype, dst_dtype);
}

}  // namespace puter

using namespace puter;

extern "C" {

int puter_hip_dequant(void *dst, const void *src, int64_t count, float scale, int32_t zero_point,
                      int dst_dtype, int src_dtype, void *stream) {
    int rc = check_config(count, dst, src, zero_point, "dequant");
    if (rc) return rc;
    if (count == 0) return PUTER_OK;
    if (dst_dtype != PUTER_F32 || src_dtype != PUTER_I8)  // "dequant: Dequant unsupported dtype pair"
        return fail(PUTER_ERR_INVALID, "dequant: unsupported dtype pair %d -> %d", src_dtype, dst_dtype);
    return launch_map(DequantI8Op{static_cast<float *>(dst), static_cast<const uint8_t *>(src), scale, zero_point},
                      count, aligned16(dst) && aligned16(src), as_stream(stream), "dequant");
}

int puter_hip_dequant4(void *dst, const void *src, int64_t pair_count, float scale, int32_t zero_point,
                       int dst_dtype, int src_dtype, void *stream) {
    int rc = check_config(pair_count, dst, src, zero_point, "dequant4");
    if (rc) return rc;
    if (pair_count == 0) return PUTER_OK;
    if (dst_dtype != PUTER_F32 || src_dtype != PUTER_I4)
        return fail(PUTER_ERR_INVALID, "dequant4: unsupported dtype pair %d -> %d", src_dtype, dst_dtype);
    return launch_map(DequantI4Op{static_cast<float *>(dst), static_cast<const uint8_t *>(src), scale, zero_point},
                      pair_count, aligned16(dst) && aligned16(src), as_stream(stream), "dequant4");
}

int puter_hip_quant(void *dst, const void *src, int64_t count, float scale, int32_t zero_point,
                    int dst_dtype, int src_dtype, void *stream) {
    int rc = check_config(count, dst, src, zero_point, "quant");
    if (rc) return rc;
    if (count == 0) return PUTER_OK;
    if (dst_dtype != PUTER_I8 || src_dtype != PUTER_F32)  // "quant: Quant unsupported dtype pair"
        return fail(PUTER_ERR_INVALID, "quant: unsupported dtype pair %d -> %d", src_dtype, dst_dtype);
    // the reciprocal fast path needs 1/scale normal and finite
    const float mag = std::fabs(scale);
    const int fast = mag >= 0x1p-125f && mag <= 0x1p125f;
    const float inv = fast ? 1.0f / scale : 0.0f;
    return launch_map(ToI8Op<true>{static_cast<uint8_t *>(dst), static_cast<const float *>(src), scale, zero_point, inv, fast},
                      count, aligned16(dst) && aligned16(src), as_stream(stream), "quant");
}

}  // extern "C"
