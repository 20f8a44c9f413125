// Shared device helpers for the gfx950 kernels: bit-exact dtype codecs, wave64
// reductions, 16-byte vector access, launch/error plumbing for the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>
#include <cstdio>
#include <string>

#include "../../include/puter_hip.h"

namespace puter {

// ---------------------------------------------------------------- errors --
void set_error(const char *fmt, ...);
int fail(int status, const char *fmt, ...);
int check_launch(const char *what);
inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }
// compute units of the current device, cached per device (256 when the query fails)
int device_cus();

// The library's scratch buffer on the current device (split-K partials of Matmul
// and of one-row attention), held for one call's launches: the constructor orders
// the call's stream after the buffer's last user on another stream and grows the
// buffer if needed; finish() records the call's completion on its stream.  The
// device's lock is held from construction to destruction.  On a stream that is
// capturing a graph the lease neither grows, orders nor records: it hands out the
// buffer it finds (never freed afterwards) or fails with PUTER_ERR_INVALID when
// that is too small.
struct SplitScratch;
class ScratchLease {
public:
    ScratchLease(size_t bytes, hipStream_t s);
    ScratchLease(const ScratchLease &) = delete;
    ScratchLease &operator=(const ScratchLease &) = delete;
    int status() const { return status_; }
    void *ptr() const { return ptr_; }
    int finish();  // call once, after the launches that use ptr()
private:
    SplitScratch *sc_ = nullptr;
    std::unique_lock<std::mutex> lock_;
    hipStream_t s_;
    void *ptr_ = nullptr;
    int status_ = 0;
    bool captured_ = false;
};

inline bool is_float_dtype(int dt) { return dt >= PUTER_F32 && dt <= PUTER_F8E5M2; }
inline bool is_norm_dtype(int dt) { return dt == PUTER_F32 || dt == PUTER_F16 || dt == PUTER_BF16; }
inline int dtype_bytes(int dt) {
    switch (dt) {
    case PUTER_F32: return 4;
    case PUTER_F16: case PUTER_BF16: return 2;
    case PUTER_F8E4M3: case PUTER_F8E5M2: return 1;
    case PUTER_I32: return 4;
    default: return 0;
    }
}
inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

constexpr int kWave = 64;

// ---------------------------------------------------------------- codecs --
// Element rules are stated in include/puter_hip.h (casts) and match the CPU
// oracle bit for bit: RNE narrowing, fp8 saturating, NaN kept as NaN.

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
    return __uint_as_float(bits16 << 16);
}
// Round-to-nearest-even narrowing, NaN kept as NaN with its payload's top
// bits and the quiet bit set.  gfx950's v_cvt_pk_bf16_f32 implements exactly
// this rule: checked against the software statement
//   NaN -> (bits >> 16) | 0x40, else (bits + 0x7FFF + ((bits >> 16) & 1)) >> 16
// for all 2^32 inputs on MI355X.
// The empty asm hides v's origin so the compiler emits the plain conversion
// and never folds a preceding multiply into a mixed-precision FMA (whose
// implicit +0.0 addend would turn -0.0 into +0.0).
__device__ __forceinline__ uint32_t f32_to_bf16(float v) {
    asm("" : "+v"(v));
    return __builtin_bit_cast(uint16_t, (__bf16)v);
}
__device__ __forceinline__ float f16_to_f32(uint32_t h) {
    uint32_t sign = (h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    if (exp == 0x1Fu) return __uint_as_float(sign | 0x7F800000u | (man << 13));
    if (exp == 0u) return __uint_as_float(sign | __float_as_uint((float)man * 0x1p-24f));
    return __uint_as_float(sign | ((exp + 112u) << 23) | (man << 13));
}
// IEEE binary16 round-to-nearest-even narrowing (overflow to infinity,
// gradual underflow, NaN quieted with its payload's top bits).  gfx950's
// v_cvt_f16_f32 matches the bit-level software statement of this rule for
// all 2^32 inputs on MI355X.  (The widening above stays in software: the
// hardware widening quiets signalling NaNs.)
__device__ __forceinline__ uint32_t f32_to_f16(float v) {
    asm("" : "+v"(v));
    return __builtin_bit_cast(uint16_t, (_Float16)v);
}

__device__ __forceinline__ float e4m3_to_f32(uint32_t b) {
    uint32_t sign = (b & 0x80u) << 24;
    uint32_t exp = (b >> 3) & 0xFu;
    uint32_t man = b & 0x7u;
    if (exp == 0xFu && man == 0x7u) return __uint_as_float(sign | 0x7FC00000u);
    if (exp == 0u) return __uint_as_float(sign | __float_as_uint((float)man * 0x1p-9f));
    return __uint_as_float(sign | ((exp + 120u) << 23) | (man << 20));
}
__device__ __forceinline__ uint32_t f32_to_e4m3(float v) {
    uint32_t u = __float_as_uint(v);
    uint32_t sign = (u >> 24) & 0x80u;
    uint32_t a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return sign | 0x7Fu;
    if (a >= 0x43E00000u) return sign | 0x7Eu;
    if (a >= 0x3C800000u) {
        uint32_t t = a - (120u << 23);
        t += 0x7FFFFu + ((t >> 20) & 1u);
        return sign | (t >> 20);
    }
    return sign | (uint32_t)__builtin_rintf(__uint_as_float(a) * 0x1p9f);
}

__device__ __forceinline__ float e5m2_to_f32(uint32_t b) {
    uint32_t sign = (b & 0x80u) << 24;
    uint32_t exp = (b >> 2) & 0x1Fu;
    uint32_t man = b & 0x3u;
    if (exp == 0x1Fu) return __uint_as_float(sign | (man ? 0x7FC00000u : 0x7F800000u));
    if (exp == 0u) return __uint_as_float(sign | __float_as_uint((float)man * 0x1p-16f));
    return __uint_as_float(sign | ((exp + 112u) << 23) | (man << 21));
}
__device__ __forceinline__ uint32_t f32_to_e5m2(float v) {
    uint32_t u = __float_as_uint(v);
    uint32_t sign = (u >> 24) & 0x80u;
    uint32_t a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return sign | 0x7Eu;
    if (a >= 0x47600000u) return sign | 0x7Bu;
    if (a >= 0x38800000u) {
        uint32_t t = a - (112u << 23);
        t += 0xFFFFFu + ((t >> 21) & 1u);
        return sign | (t >> 21);
    }
    return sign | (uint32_t)__builtin_rintf(__uint_as_float(a) * 0x1p16f);
}

// f32 <-> f64 on the integer bits (independent of the float mode registers):
// widening is exact (signalling NaNs quieted, payload kept); narrowing rounds to
// nearest even with gradual underflow, as Go's float32(f64) / float64(f32)
// conversions (convert/f32_f64.go:8-17).
__device__ __forceinline__ uint64_t f32_to_f64_bits(uint32_t x) {
    const uint64_t sign = (uint64_t)(x & 0x80000000u) << 32;
    const uint32_t e = (x >> 23) & 0xFFu, m = x & 0x7FFFFFu;
    if (e == 0xFFu) {
        if (m == 0) return sign | 0x7FF0000000000000ull;
        return sign | 0x7FF8000000000000ull | ((uint64_t)m << 29);  // quiet, payload kept
    }
    if (e == 0) {
        if (m == 0) return sign;
        const int p = 31 - __clz(m);                                 // top set bit of the denormal
        return sign | ((uint64_t)(p + 874) << 52) | (((uint64_t)m << (52 - p)) & 0xFFFFFFFFFFFFFull);
    }
    return sign | ((uint64_t)(e + 896) << 52) | ((uint64_t)m << 29);
}
__device__ __forceinline__ uint32_t f64_to_f32_bits(uint64_t x) {
    const uint32_t sign = (uint32_t)(x >> 32) & 0x80000000u;
    const int e = (int)((x >> 52) & 0x7FF);
    const uint64_t m = x & 0xFFFFFFFFFFFFFull;
    if (e == 0x7FF) {
        if (m == 0) return sign | 0x7F800000u;
        return sign | 0x7FC00000u | (uint32_t)(m >> 29);  // quiet, top payload bits
    }
    if (e == 0) return sign;  // f64 denormals lie far below half the least f32 denormal
    int exp = e - 896;        // biased f32 exponent of the value before rounding
    if (exp >= 0xFF) return sign | 0x7F800000u;
    const uint64_t sig = m | (1ull << 52);
    int shift = 29;
    if (exp < 1) {
        shift = 30 - exp;     // gradual underflow: fewer significant bits kept
        if (shift > 54) return sign;
    }
    uint64_t keep = sig >> shift;
    const uint64_t rem = sig & ((1ull << shift) - 1), half = 1ull << (shift - 1);
    if (rem > half || (rem == half && (keep & 1))) ++keep;   // round to nearest even
    if (exp < 1) return sign | (uint32_t)keep;               // 2^23 becomes the least normal
    if (keep >> 24) { keep >>= 1; ++exp; }
    if (exp >= 0xFF) return sign | 0x7F800000u;
    return sign | ((uint32_t)exp << 23) | ((uint32_t)keep & 0x7FFFFFu);
}

// Typed element access.  Storage types: float, uint16_t (bf16/f16), uint8_t (fp8).
template <int DT> struct Elem;
template <> struct Elem<PUTER_F32> {
    using T = float;
    static __device__ __forceinline__ float load(T v) { return v; }
    static __device__ __forceinline__ T store(float v) { return v; }
};
template <> struct Elem<PUTER_BF16> {
    using T = uint16_t;
    static __device__ __forceinline__ float load(T v) { return bf16_to_f32(v); }
    static __device__ __forceinline__ T store(float v) { return (T)f32_to_bf16(v); }
};
template <> struct Elem<PUTER_F16> {
    using T = uint16_t;
    static __device__ __forceinline__ float load(T v) { return f16_to_f32(v); }
    static __device__ __forceinline__ T store(float v) { return (T)f32_to_f16(v); }
};
template <> struct Elem<PUTER_F8E4M3> {
    using T = uint8_t;
    static __device__ __forceinline__ float load(T v) { return e4m3_to_f32(v); }
    static __device__ __forceinline__ T store(float v) { return (T)f32_to_e4m3(v); }
};
template <> struct Elem<PUTER_F8E5M2> {
    using T = uint8_t;
    static __device__ __forceinline__ float load(T v) { return e5m2_to_f32(v); }
    static __device__ __forceinline__ T store(float v) { return (T)f32_to_e5m2(v); }
};

// The reference rounds 16-bit dot / sum results to the 16-bit format
// (device/cpu/dot/bf16_generic.go:9-21, reduction/bf16_kernels.go:40-51).
template <int DT> __device__ __forceinline__ float round_reduction(float s) {
    if constexpr (DT == PUTER_BF16) return bf16_to_f32(f32_to_bf16(s));
    else if constexpr (DT == PUTER_F16) return f16_to_f32(f32_to_f16(s));
    else return s;
}

// 16-byte vector of elements.
template <int DT> struct Vec {
    using T = typename Elem<DT>::T;
    static constexpr int N = 16 / sizeof(T);
};

__device__ __forceinline__ void unpack(const uint4 &v, float (&f)[8], int dt_bf16) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (dt_bf16) {
            f[2 * i] = __uint_as_float(w[i] << 16);
            f[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
        } else {
            f[2 * i] = f16_to_f32(w[i] & 0xFFFFu);
            f[2 * i + 1] = f16_to_f32(w[i] >> 16);
        }
    }
}

// Convert one 16-byte vector of elements into floats.
template <int DT>
__device__ __forceinline__ void unpack_vec(const uint4 &v, float (&f)[Vec<DT>::N]) {
    if constexpr (DT == PUTER_F32) {
        f[0] = __uint_as_float(v.x); f[1] = __uint_as_float(v.y);
        f[2] = __uint_as_float(v.z); f[3] = __uint_as_float(v.w);
    } else if constexpr (DT == PUTER_BF16 || DT == PUTER_F16) {
        unpack(v, f, DT == PUTER_BF16);
    } else {
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 16; ++i) f[i] = Elem<DT>::load((uint8_t)(w[i >> 2] >> (8 * (i & 3))));
    }
}

// Load/convert N contiguous elements (16 bytes) into floats.
template <int DT>
__device__ __forceinline__ void load_vec(const void *base, size_t vec_index, float (&f)[Vec<DT>::N]) {
    unpack_vec<DT>(reinterpret_cast<const uint4 *>(base)[vec_index], f);
}

template <int DT>
__device__ __forceinline__ uint4 pack_vec(const float (&f)[Vec<DT>::N]) {
    uint4 v;
    if constexpr (DT == PUTER_F32) {
        v.x = __float_as_uint(f[0]); v.y = __float_as_uint(f[1]);
        v.z = __float_as_uint(f[2]); v.w = __float_as_uint(f[3]);
    } else if constexpr (DT == PUTER_BF16 || DT == PUTER_F16) {
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            w[i] = (uint32_t)Elem<DT>::store(f[2 * i]) | ((uint32_t)Elem<DT>::store(f[2 * i + 1]) << 16);
        v.x = w[0]; v.y = w[1]; v.z = w[2]; v.w = w[3];
    } else {
        uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 16; ++i) w[i >> 2] |= (uint32_t)Elem<DT>::store(f[i]) << (8 * (i & 3));
        v.x = w[0]; v.y = w[1]; v.z = w[2]; v.w = w[3];
    }
    return v;
}

// Streaming (non-temporal) 16-byte access: data touched once bypasses the
// cache hierarchy's retention so resident tables (gamma, gate rows) stay hot.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_stream(const uint4 *p) {
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st_stream(uint4 v, uint4 *p) {
    u32x4_t t = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(t, reinterpret_cast<u32x4_t *>(p));
}

// ----------------------------------------------------- wave64 reductions --
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
    return v;
}

// ------------------------------------------------------------ FastExp32 --
// device/cpu/math/f32.go:21-46, evaluated operation by operation (no FMA):
// clamps, z = x*log2(e), k = trunc(z) (one less below 0), f = z - k, a
// degree-5 polynomial for 2^f, then k added to the exponent field.
__device__ __forceinline__ float fast_exp32(float x) {
    if (x < -87.33654f) return 0.0f;
    if (x > 88.72283f) return 0x1p127f * (1.0f + (1.0f - 0x1p-23f));
    const float z = __fmul_rn(x, 1.4426950408889634f);
    int32_t k = (int32_t)z;
    if (z < 0) k--;
    const float f = __fsub_rn(z, (float)k);
    float p = __fmul_rn(f, 0.00133389f);
    p = __fmul_rn(f, __fadd_rn(0.00961812f, p));
    p = __fmul_rn(f, __fadd_rn(0.05550410f, p));
    p = __fmul_rn(f, __fadd_rn(0.24022650f, p));
    p = __fmul_rn(f, __fadd_rn(0.69314718f, p));
    p = __fadd_rn(1.0f, p);
    return __uint_as_float(__float_as_uint(p) + ((uint32_t)k << 23));
}

}  // namespace puter
