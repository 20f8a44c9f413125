// dtype casts between f32 and bf16 / f16 / fp8-E4M3FN / fp8-E5M2 (the int8,
// int4 and f64 pairs are in quant.hip).
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
    const auto ext = [](int dt) { return dt == PUTER_I8 || dt == PUTER_I4 || dt == PUTER_F64; };
    if (ext(dst_dtype) || ext(src_dtype)) return cast_ext(dst, dst_dtype, src, src_dtype, count, as_stream(stream));
    if (!is_float_dtype(dst_dtype) || !is_float_dtype(src_dtype) ||
        (dst_dtype != PUTER_F32 && src_dtype != PUTER_F32))
        return fail(PUTER_ERR_INVALID, "cast: unsupported pair %d -> %d", src_dtype, dst_dtype);
    hipStream_t s = as_stream(stream);
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
