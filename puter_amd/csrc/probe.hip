// HBM stream probe (diagnostic; no counterpart in the reference): the
// 2-read / 2-write traffic of the fused GatedResidual+norm without its
// arithmetic, in the launch shapes the norm kernels use, so a measured stream
// rate sits beside the norm kernels' rates as their practical ceiling.
//   shape 0: flat, one 16-byte vector of each input per thread;
//   shape 1: a block of 1024 threads per 1024-vector row, a block-wide sum
//            (wave butterfly + one LDS round) between the two stores, as the
//            block-per-row norm kernel does;
//   shape 2: a wave per 1024-vector row, 16 vectors per lane, a wave-wide sum
//            between the two stores, as the wave-per-row norm kernel does.
// c = a + b (as u32 lanes) is stored before the sum, d = (a ^ b) + (sum & 1)
// after it, so neither store can be dropped.
#include "common.hpp"

namespace puter {

typedef unsigned int pu32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ pu32x4 pld(const pu32x4 *p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ void pst(pu32x4 v, pu32x4 *p) { __builtin_nontemporal_store(v, p); }
__device__ __forceinline__ float lanesum(pu32x4 v) {
    return __uint_as_float(v.x & 0x3FFFFFFFu) + __uint_as_float(v.y & 0x3FFFFFFFu);
}

__global__ __launch_bounds__(256) void probe_flat(const pu32x4 *a, const pu32x4 *b, pu32x4 *c, pu32x4 *d, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const pu32x4 x = pld(a + i), y = pld(b + i);
    pst(x + y, c + i);
    pst(x ^ y, d + i);
}

__global__ __launch_bounds__(1024) void probe_block_row(const pu32x4 *a, const pu32x4 *b, pu32x4 *c, pu32x4 *d) {
    __shared__ float red[16];
    const int64_t i = (int64_t)blockIdx.x * 1024 + threadIdx.x;
    const pu32x4 x = pld(a + i), y = pld(b + i);
    const pu32x4 h = x + y;
    pst(h, c + i);
    float s = wave_sum(lanesum(h));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    float t = 0.0f;
    for (int w = 0; w < 16; ++w) t += red[w];
    pst((x ^ y) + (__float_as_uint(t) & 1u), d + i);
}

__global__ __launch_bounds__(256) void probe_wave_row(const pu32x4 *a, const pu32x4 *b, pu32x4 *c, pu32x4 *d,
                                                      int64_t rows) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int64_t off = row * 1024;
    pu32x4 x[16], y[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        x[j] = pld(a + off + j * 64 + lane);
        y[j] = pld(b + off + j * 64 + lane);
    }
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const pu32x4 h = x[j] + y[j];
        pst(h, c + off + j * 64 + lane);
        s += lanesum(h);
    }
    s = wave_sum(s);
#pragma unroll
    for (int j = 0; j < 16; ++j) pst((x[j] ^ y[j]) + (__float_as_uint(s) & 1u), d + off + j * 64 + lane);
}

}  // namespace puter

using namespace puter;

extern "C" int puter_hip_stream_probe(const void *a, const void *b, void *c, void *d, int64_t vectors, int shape,
                                      void *stream) {
    if (vectors < 0 || shape < 0 || shape > 2) return fail(PUTER_ERR_INVALID, "stream probe: invalid arguments");
    if (vectors == 0) return PUTER_OK;
    if (!a || !b || !c || !d) return fail(PUTER_ERR_NIL, "stream probe: nil buffer");
    if (!aligned16(a) || !aligned16(b) || !aligned16(c) || !aligned16(d))
        return fail(PUTER_ERR_INVALID, "stream probe: buffers must be 16-byte aligned");
    if (shape != 0 && vectors % 1024 != 0) return fail(PUTER_ERR_INVALID, "stream probe: rows are 1024 vectors");
    if (vectors / 256 > 0x7FFFFFFF) return fail(PUTER_ERR_INVALID, "stream probe: too large");
    hipStream_t s = as_stream(stream);
    const pu32x4 *pa = static_cast<const pu32x4 *>(a), *pb = static_cast<const pu32x4 *>(b);
    pu32x4 *pc = static_cast<pu32x4 *>(c), *pd = static_cast<pu32x4 *>(d);
    if (shape == 0) probe_flat<<<(unsigned)((vectors + 255) / 256), 256, 0, s>>>(pa, pb, pc, pd, vectors);
    else if (shape == 1) probe_block_row<<<(unsigned)(vectors / 1024), 1024, 0, s>>>(pa, pb, pc, pd);
    else probe_wave_row<<<(unsigned)((vectors / 1024 + 3) / 4), 256, 0, s>>>(pa, pb, pc, pd, vectors / 1024);
    return check_launch("stream probe");
}
