// dtype casts between f32 and bf16 / f16 / fp8-E4M3FN / fp8-E5M2.
// Reference: convert/bf16_f32.go:11-38, convert/f16_f32.go:10-42,
// convert/fp8_f32.go:8-65 (slice-to-slice, len(dst) == len(src)).
//
// HBM-bound streaming kernel: each thread moves one 16-element chunk per
// iteration with 16-byte loads/stores (f32 side: 4 x 16 B, 16-bit side:
// 2 x 16 B, fp8 side: 1 x 16 B), grid-stride over the chunks; the ragged tail
// (< 16 elements or unaligned pointers) goes element by element.
#include "common.hpp"

namespace puter {

template <int DT>
__device__ __forceinline__ void load16(const void *src, size_t chunk, float (&f)[16]) {
    constexpr int N = Vec<DT>::N;  // elements per 16 bytes
#pragma unroll
    for (int v = 0; v < 16 / N; ++v) {
        float t[N];
        load_vec<DT>(src, chunk * (16 / N) + v, t);
#pragma unroll
        for (int i = 0; i < N; ++i) f[v * N + i] = t[i];
    }
}

template <int DT>
__device__ __forceinline__ void store16(void *dst, size_t chunk, const float (&f)[16]) {
    constexpr int N = Vec<DT>::N;
#pragma unroll
    for (int v = 0; v < 16 / N; ++v) {
        float t[N];
#pragma unroll
        for (int i = 0; i < N; ++i) t[i] = f[v * N + i];
        reinterpret_cast<uint4 *>(dst)[chunk * (16 / N) + v] = pack_vec<DT>(t);
    }
}

template <int SRC, int DST>
__global__ __launch_bounds__(256) void cast_kernel(void *__restrict__ dst,
                                                   const void *__restrict__ src, int64_t count,
                                                   int vectorised) {
    using S = typename Elem<SRC>::T;
    using D = typename Elem<DST>::T;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t tid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t body = 0;
    if (vectorised) {
        const size_t chunks = (size_t)count / 16;
        for (size_t c = tid; c < chunks; c += stride) {
            float f[16];
            load16<SRC>(src, c, f);
            store16<DST>(dst, c, f);
        }
        body = chunks * 16;
    }
    for (size_t i = body + tid; i < (size_t)count; i += stride) {
        const float v = Elem<SRC>::load(reinterpret_cast<const S *>(src)[i]);
        reinterpret_cast<D *>(dst)[i] = Elem<DST>::store(v);
    }
}

template <int SRC, int DST>
static int launch_cast(void *dst, const void *src, int64_t count, hipStream_t stream) {
    const int vectorised = aligned16(dst) && aligned16(src);
    const int64_t units = vectorised ? (count / 16 + 1) : count;
    int64_t blocks = (units + 255) / 256;
    if (blocks > 16384) blocks = 16384;
    if (blocks < 1) blocks = 1;
    cast_kernel<SRC, DST><<<(unsigned)blocks, 256, 0, stream>>>(dst, src, count, vectorised);
    return check_launch("cast");
}

}  // namespace puter

using namespace puter;

extern "C" int puter_hip_cast(void *dst, int dst_dtype, const void *src, int src_dtype,
                              int64_t count, void *stream) {
    if (count < 0) return fail(PUTER_ERR_INVALID, "cast: negative count");
    if (count == 0) return PUTER_OK;
    if (!dst || !src) return fail(PUTER_ERR_NIL, "cast: nil buffer");
    if (!is_float_dtype(dst_dtype) || !is_float_dtype(src_dtype) ||
        (dst_dtype != PUTER_F32 && src_dtype != PUTER_F32))
        return fail(PUTER_ERR_INVALID, "cast: unsupported pair %d -> %d", src_dtype, dst_dtype);
    hipStream_t s = as_stream(stream);
    if (src_dtype == PUTER_F32) {
        switch (dst_dtype) {
        case PUTER_F32: return launch_cast<PUTER_F32, PUTER_F32>(dst, src, count, s);
        case PUTER_BF16: return launch_cast<PUTER_F32, PUTER_BF16>(dst, src, count, s);
        case PUTER_F16: return launch_cast<PUTER_F32, PUTER_F16>(dst, src, count, s);
        case PUTER_F8E4M3: return launch_cast<PUTER_F32, PUTER_F8E4M3>(dst, src, count, s);
        case PUTER_F8E5M2: return launch_cast<PUTER_F32, PUTER_F8E5M2>(dst, src, count, s);
        }
    }
    switch (src_dtype) {
    case PUTER_BF16: return launch_cast<PUTER_BF16, PUTER_F32>(dst, src, count, s);
    case PUTER_F16: return launch_cast<PUTER_F16, PUTER_F32>(dst, src, count, s);
    case PUTER_F8E4M3: return launch_cast<PUTER_F8E4M3, PUTER_F32>(dst, src, count, s);
    case PUTER_F8E5M2: return launch_cast<PUTER_F8E5M2, PUTER_F32>(dst, src, count, s);
    }
    return fail(PUTER_ERR_INVALID, "cast: unsupported pair");
}
