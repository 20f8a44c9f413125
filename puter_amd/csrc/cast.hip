// dtype casts between f32 and bf16 / f16 / fp8-E4M3FN / fp8-E5M2, and between
// any two of bf16 / f16 / fp8 / f64 in one pass (the int8, int4 and f32 <-> f64
// pairs are in quant.hip).
// Reference: convert/bf16_f32.go:11-38, convert/f16_f32.go:10-42,
// convert/fp8_f32.go:8-65 (slice-to-slice, len(dst) == len(src)).
//
// HBM-bound streaming kernel.  The unit of work is four elements: one 16-byte
// f32 vector and its 8-byte (bf16/f16) or 4-byte (fp8) narrow image.  Lane l of
// a block handles units base + u*256 + l, so every wave-wide load and store is
// one contiguous burst on both sides (1 KiB of f32, 512 B / 256 B narrow).  Each
// thread issues kUnroll units' loads before converting and storing them, the
// grid strides over the array, and the ragged tail (< 4 elements, or unaligned
// pointers) goes element by element.  Rounding is integer-exact (common.hpp).
#include "common.hpp"

namespace puter {

constexpr int kUnroll = 4;

typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

template <int ES> struct Narrow;            // the narrow side's 4-element image
template <> struct Narrow<2> {
    using T = uint2;
    static __device__ __forceinline__ T load(const void *p, size_t i) {
        const u32x2_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t *>(p) + i);
        return make_uint2(v.x, v.y);
    }
    static __device__ __forceinline__ void store(void *p, size_t i, T v) {
        u32x2_t t = {v.x, v.y};
        __builtin_nontemporal_store(t, reinterpret_cast<u32x2_t *>(p) + i);
    }
};
template <> struct Narrow<1> {
    using T = uint32_t;
    static __device__ __forceinline__ T load(const void *p, size_t i) {
        return __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(p) + i);
    }
    static __device__ __forceinline__ void store(void *p, size_t i, T v) {
        __builtin_nontemporal_store(v, reinterpret_cast<uint32_t *>(p) + i);
    }
};

template <int DT>
__device__ __forceinline__ void widen4(uint2 w, float (&f)[4]) {
    f[0] = Elem<DT>::load((uint16_t)(w.x & 0xFFFFu));
    f[1] = Elem<DT>::load((uint16_t)(w.x >> 16));
    f[2] = Elem<DT>::load((uint16_t)(w.y & 0xFFFFu));
    f[3] = Elem<DT>::load((uint16_t)(w.y >> 16));
}
template <int DT>
__device__ __forceinline__ void widen4(uint32_t w, float (&f)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) f[i] = Elem<DT>::load((uint8_t)(w >> (8 * i)));
}
template <int DT>
__device__ __forceinline__ void narrow4(const float (&f)[4], uint2 &w) {
    w.x = (uint32_t)Elem<DT>::store(f[0]) | ((uint32_t)Elem<DT>::store(f[1]) << 16);
    w.y = (uint32_t)Elem<DT>::store(f[2]) | ((uint32_t)Elem<DT>::store(f[3]) << 16);
}
template <int DT>
__device__ __forceinline__ void narrow4(const float (&f)[4], uint32_t &w) {
    w = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) w |= (uint32_t)Elem<DT>::store(f[i]) << (8 * i);
}

// NARROW_DT is the non-f32 side; TO_F32 selects the direction.
template <int NARROW_DT, bool TO_F32>
__global__ __launch_bounds__(256) void cast_kernel(void *__restrict__ dst,
                                                   const void *__restrict__ src, int64_t count,
                                                   int vectorised) {
    constexpr int ES = sizeof(typename Elem<NARROW_DT>::T);
    using NT = Narrow<ES>;
    using W = typename NT::T;
    const size_t tid = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t gstride = (size_t)gridDim.x * 256;
    size_t body = 0;
    if (vectorised) {
        const size_t units = (size_t)count / 4;
        for (size_t base = (size_t)blockIdx.x * 256 * kUnroll + threadIdx.x; base < units;
             base += gstride * kUnroll) {
            if constexpr (TO_F32) {
                W in[kUnroll];
#pragma unroll
                for (int u = 0; u < kUnroll; ++u)
                    if (base + u * 256 < units) in[u] = NT::load(src, base + u * 256);
#pragma unroll
                for (int u = 0; u < kUnroll; ++u)
                    if (base + u * 256 < units) {
                        float f[4];
                        widen4<NARROW_DT>(in[u], f);
                        st_stream(make_uint4(__float_as_uint(f[0]), __float_as_uint(f[1]),
                                             __float_as_uint(f[2]), __float_as_uint(f[3])),
                                  reinterpret_cast<uint4 *>(dst) + base + u * 256);
                    }
            } else {
                uint4 in[kUnroll];
#pragma unroll
                for (int u = 0; u < kUnroll; ++u)
                    if (base + u * 256 < units) in[u] = ld_stream(reinterpret_cast<const uint4 *>(src) + base + u * 256);
#pragma unroll
                for (int u = 0; u < kUnroll; ++u)
                    if (base + u * 256 < units) {
                        const float f[4] = {__uint_as_float(in[u].x), __uint_as_float(in[u].y),
                                            __uint_as_float(in[u].z), __uint_as_float(in[u].w)};
                        W w;
                        narrow4<NARROW_DT>(f, w);
                        NT::store(dst, base + u * 256, w);
                    }
            }
        }
        body = units * 4;
    }
    using N = typename Elem<NARROW_DT>::T;
    for (size_t i = body + tid; i < (size_t)count; i += gstride) {
        if constexpr (TO_F32)
            reinterpret_cast<float *>(dst)[i] = Elem<NARROW_DT>::load(reinterpret_cast<const N *>(src)[i]);
        else
            reinterpret_cast<N *>(dst)[i] = Elem<NARROW_DT>::store(reinterpret_cast<const float *>(src)[i]);
    }
}

// ---- any float pair in one pass ------------------------------------------
// shape.cast (execution/shape_cast_intrinsic.go:56-115) widens every source
// element to float64 and then writes float32(value) narrowed to the target
// (NewBfloat16FromFloat32(float32(v)), Fromfloat32(float32(v)), ...; float64
// targets take the float64 as is).  Widening a bf16 / f16 / fp8 / f32 value is
// exact, so for those sources the f64 step is the f32 value itself; an f64
// source is rounded to f32 first (RNE), then narrowed: two roundings, as the
// reference does.  cast_pair_kernel moves units of 8 elements (16 B of a 16-bit side,
// 8 B of fp8, 32 B of f32, 64 B of f64) so every wave-wide access is contiguous.
template <int DT> struct Unit8;
template <> struct Unit8<PUTER_BF16> {
    static __device__ __forceinline__ void load(const void *p, size_t u, float (&f)[8]) {
        unpack(ld_stream(reinterpret_cast<const uint4 *>(p) + u), f, 1);
    }
    static __device__ __forceinline__ void store(void *p, size_t u, const float (&f)[8]) {
        st_stream(pack_vec<PUTER_BF16>(f), reinterpret_cast<uint4 *>(p) + u);
    }
};
template <> struct Unit8<PUTER_F16> {
    static __device__ __forceinline__ void load(const void *p, size_t u, float (&f)[8]) {
        unpack(ld_stream(reinterpret_cast<const uint4 *>(p) + u), f, 0);
    }
    static __device__ __forceinline__ void store(void *p, size_t u, const float (&f)[8]) {
        st_stream(pack_vec<PUTER_F16>(f), reinterpret_cast<uint4 *>(p) + u);
    }
};
template <int DT> struct Unit8Fp8 {
    static __device__ __forceinline__ void load(const void *p, size_t u, float (&f)[8]) {
        const uint2 w = Narrow<2>::load(p, u);
        float a[4], b[4];
        widen4<DT>(w.x, a);
        widen4<DT>(w.y, b);
#pragma unroll
        for (int i = 0; i < 4; ++i) { f[i] = a[i]; f[4 + i] = b[i]; }
    }
    static __device__ __forceinline__ void store(void *p, size_t u, const float (&f)[8]) {
        const float a[4] = {f[0], f[1], f[2], f[3]}, b[4] = {f[4], f[5], f[6], f[7]};
        uint2 w;
        narrow4<DT>(a, w.x);
        narrow4<DT>(b, w.y);
        Narrow<2>::store(p, u, w);
    }
};
template <> struct Unit8<PUTER_F8E4M3> : Unit8Fp8<PUTER_F8E4M3> {};
template <> struct Unit8<PUTER_F8E5M2> : Unit8Fp8<PUTER_F8E5M2> {};
template <> struct Unit8<PUTER_F64> {
    static __device__ __forceinline__ void load(const void *p, size_t u, float (&f)[8]) {
        const uint4 *q = reinterpret_cast<const uint4 *>(p) + 4 * u;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint4 v = ld_stream(q + i);
            f[2 * i] = __uint_as_float(f64_to_f32_bits(((uint64_t)v.y << 32) | v.x));
            f[2 * i + 1] = __uint_as_float(f64_to_f32_bits(((uint64_t)v.w << 32) | v.z));
        }
    }
    static __device__ __forceinline__ void store(void *p, size_t u, const float (&f)[8]) {
        uint4 *q = reinterpret_cast<uint4 *>(p) + 4 * u;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint64_t a = f32_to_f64_bits(__float_as_uint(f[2 * i]));
            const uint64_t b = f32_to_f64_bits(__float_as_uint(f[2 * i + 1]));
            st_stream(make_uint4((uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b, (uint32_t)(b >> 32)), q + i);
        }
    }
};

// one element of DT as f32 (f64: RNE to f32) / f32 written as DT
template <int DT> __device__ __forceinline__ float load_one(const void *p, size_t i) {
    if constexpr (DT == PUTER_F64) return __uint_as_float(f64_to_f32_bits(reinterpret_cast<const uint64_t *>(p)[i]));
    else return Elem<DT>::load(reinterpret_cast<const typename Elem<DT>::T *>(p)[i]);
}
template <int DT> __device__ __forceinline__ void store_one(void *p, size_t i, float v) {
    if constexpr (DT == PUTER_F64) reinterpret_cast<uint64_t *>(p)[i] = f32_to_f64_bits(__float_as_uint(v));
    else reinterpret_cast<typename Elem<DT>::T *>(p)[i] = Elem<DT>::store(v);
}

template <int SRC, int DST>
__global__ __launch_bounds__(256) void cast_pair_kernel(void *__restrict__ dst, const void *__restrict__ src,
                                                        int64_t count, int vectorised) {
    const size_t tid = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t gstride = (size_t)gridDim.x * 256;
    size_t body = 0;
    if (vectorised) {
        const size_t units = (size_t)count / 8;
        for (size_t base = (size_t)blockIdx.x * 256 * 2 + threadIdx.x; base < units; base += gstride * 2) {
            float f[2][8];
#pragma unroll
            for (int k = 0; k < 2; ++k)
                if (base + k * 256 < units) Unit8<SRC>::load(src, base + k * 256, f[k]);
#pragma unroll
            for (int k = 0; k < 2; ++k)
                if (base + k * 256 < units) Unit8<DST>::store(dst, base + k * 256, f[k]);
        }
        body = units * 8;
    }
    for (size_t i = body + tid; i < (size_t)count; i += gstride) store_one<DST>(dst, i, load_one<SRC>(src, i));
}

template <int SRC, int DST>
static int launch_pair(void *dst, const void *src, int64_t count, hipStream_t s) {
    const int vectorised = aligned16(dst) && aligned16(src);
    int64_t blocks = vectorised ? (count / 8 + 511) / 512 : (count + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    if (blocks < 1) blocks = 1;
    cast_pair_kernel<SRC, DST><<<(unsigned)blocks, 256, 0, s>>>(dst, src, count, vectorised);
    return check_launch("cast");
}

template <int SRC>
static int launch_pair_to(void *dst, int dst_dtype, const void *src, int64_t count, hipStream_t s) {
    switch (dst_dtype) {
    case PUTER_BF16: return launch_pair<SRC, PUTER_BF16>(dst, src, count, s);
    case PUTER_F16: return launch_pair<SRC, PUTER_F16>(dst, src, count, s);
    case PUTER_F8E4M3: return launch_pair<SRC, PUTER_F8E4M3>(dst, src, count, s);
    case PUTER_F8E5M2: return launch_pair<SRC, PUTER_F8E5M2>(dst, src, count, s);
    case PUTER_F64: return launch_pair<SRC, PUTER_F64>(dst, src, count, s);
    }
    return fail(PUTER_ERR_INVALID, "cast: unsupported pair %d -> %d", SRC, dst_dtype);
}

static int launch_float_pair(void *dst, int dst_dtype, const void *src, int src_dtype, int64_t count,
                             hipStream_t s) {
    switch (src_dtype) {
    case PUTER_BF16: return launch_pair_to<PUTER_BF16>(dst, dst_dtype, src, count, s);
    case PUTER_F16: return launch_pair_to<PUTER_F16>(dst, dst_dtype, src, count, s);
    case PUTER_F8E4M3: return launch_pair_to<PUTER_F8E4M3>(dst, dst_dtype, src, count, s);
    case PUTER_F8E5M2: return launch_pair_to<PUTER_F8E5M2>(dst, dst_dtype, src, count, s);
    case PUTER_F64: return launch_pair_to<PUTER_F64>(dst, dst_dtype, src, count, s);
    }
    return fail(PUTER_ERR_INVALID, "cast: unsupported pair %d -> %d", src_dtype, dst_dtype);
}

// f32 -> f32 is a plain copy (the reference converts element-wise; bit-identical)
__global__ __launch_bounds__(256) void copy_f32_kernel(float *__restrict__ dst,
                                                       const float *__restrict__ src, int64_t count) {
    const size_t stride = (size_t)gridDim.x * 256;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < (size_t)count; i += stride) dst[i] = src[i];
}

static unsigned cast_grid(int64_t count, int vectorised) {
    const int64_t per_block = vectorised ? 256 * 4 * kUnroll : 256;
    int64_t blocks = (count + per_block - 1) / per_block;
    if (blocks > 8192) blocks = 8192;  // grid-stride beyond 32 blocks per CU
    if (blocks < 1) blocks = 1;
    return (unsigned)blocks;
}

template <int NARROW_DT, bool TO_F32>
static int launch_cast(void *dst, const void *src, int64_t count, hipStream_t stream) {
    const int vectorised = aligned16(dst) && aligned16(src);
    cast_kernel<NARROW_DT, TO_F32><<<cast_grid(count, vectorised), 256, 0, stream>>>(dst, src, count, vectorised);
    return check_launch("cast");
}

// int8 / int4 / f64 legs (quant.hip)
int cast_ext(void *dst, int dst_dtype, const void *src, int src_dtype, int64_t count, hipStream_t s);

}  // namespace puter

using namespace puter;

extern "C" int puter_hip_cast(void *dst, int dst_dtype, const void *src, int src_dtype,
                              int64_t count, void *stream) {
    if (count < 0) return fail(PUTER_ERR_INVALID, "cast: negative count");
    if (count == 0) return PUTER_OK;
    if (!dst || !src) return fail(PUTER_ERR_NIL, "cast: nil buffer");
    hipStream_t s = as_stream(stream);
    const auto flt = [](int dt) { return is_float_dtype(dt) || dt == PUTER_F64; };
    if (src_dtype == dst_dtype && src_dtype != PUTER_F32 && flt(src_dtype)) {
        // shape.cast returns a same-dtype input unchanged (shape_cast_intrinsic.go:35-41): a byte copy
        const size_t bytes = (size_t)count * (src_dtype == PUTER_F64 ? 8 : dtype_bytes(src_dtype));
        const hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, s);
        if (e != hipSuccess) return fail(PUTER_ERR_LAUNCH, "cast: copy: %s", hipGetErrorString(e));
        return PUTER_OK;
    }
    // float <-> float without an f32 side (f64 included): one pass through f32
    if (flt(src_dtype) && flt(dst_dtype) && src_dtype != PUTER_F32 && dst_dtype != PUTER_F32)
        return launch_float_pair(dst, dst_dtype, src, src_dtype, count, s);
    const auto ext = [](int dt) { return dt == PUTER_I8 || dt == PUTER_I4 || dt == PUTER_F64; };
    if (ext(dst_dtype) || ext(src_dtype)) return cast_ext(dst, dst_dtype, src, src_dtype, count, s);
    if (!is_float_dtype(dst_dtype) || !is_float_dtype(src_dtype))
        return fail(PUTER_ERR_INVALID, "cast: unsupported pair %d -> %d", src_dtype, dst_dtype);
    if (src_dtype == PUTER_F32) {
        switch (dst_dtype) {
        case PUTER_F32:
            copy_f32_kernel<<<cast_grid(count, 0), 256, 0, s>>>(static_cast<float *>(dst),
                                                               static_cast<const float *>(src), count);
            return check_launch("cast");
        case PUTER_BF16: return launch_cast<PUTER_BF16, false>(dst, src, count, s);
        case PUTER_F16: return launch_cast<PUTER_F16, false>(dst, src, count, s);
        case PUTER_F8E4M3: return launch_cast<PUTER_F8E4M3, false>(dst, src, count, s);
        case PUTER_F8E5M2: return launch_cast<PUTER_F8E5M2, false>(dst, src, count, s);
        }
    }
    switch (src_dtype) {
    case PUTER_BF16: return launch_cast<PUTER_BF16, true>(dst, src, count, s);
    case PUTER_F16: return launch_cast<PUTER_F16, true>(dst, src, count, s);
    case PUTER_F8E4M3: return launch_cast<PUTER_F8E4M3, true>(dst, src, count, s);
    case PUTER_F8E5M2: return launch_cast<PUTER_F8E5M2, true>(dst, src, count, s);
    }
    return fail(PUTER_ERR_INVALID, "cast: unsupported pair");
}
