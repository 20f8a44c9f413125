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
// The MFMA rate probe further down measures the matrix cores' rate on random
// operands, alone and in the prefill kernel's dataflow without memory traffic.
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

// MFMA rate probe (diagnostic): 256-thread blocks held at two per CU (2 waves per
// SIMD, as the prefill kernel runs) by 64 KiB of dynamic LDS that is never touched.
// Operands come from a 16 KiB buffer of random bf16 read once into registers (the
// matrix cores draw more power, and the part clocks lower, on random data than on
// constants); each lane's 8 Q^T and 8 K fragments are 16 bytes at (i * 64 + lane).
//   mode 0: 32 v_mfma_f32_32x32x16_bf16 per iteration on 4 accumulator chains;
//   mode 1: the prefill's per-tile dataflow for 32 queries x 64 keys x 128 dims with
//           no memory traffic: S^T = K . Q^T (16 MFMAs into two chunks), p =
//           exp2(s c - m) with the row sum and the narrowing to bf16, O^T += V^T .
//           P^T (16 MFMAs; V^T fragments reuse the K registers).
// Each wave stores one float per lane so that nothing is dropped.
typedef __bf16 pbf16x8 __attribute__((ext_vector_type(8)));
typedef float pf32x16 __attribute__((ext_vector_type(16)));

template <int MODE>
__global__ __launch_bounds__(256, 2) void probe_mfma(const pbf16x8 *ops, float *out, int iters) {
    const int lane = threadIdx.x & 63;
    pbf16x8 qf[8], kf[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        qf[i] = ops[i * 64 + lane];
        kf[i] = ops[512 + i * 64 + lane];
    }
    float res = 0.0f;
    if constexpr (MODE == 0) {
        pf32x16 acc[4] = {};
        for (int it = 0; it < iters; ++it) {
#pragma unroll
            for (int t = 0; t < 8; ++t)
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[t], qf[(t + c) & 7], acc[c], 0, 0, 0);
        }
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int r = 0; r < 16; ++r) res += acc[c][r];
    } else {
        pf32x16 o[4] = {};
        float l = 0.0f;
        const float sc = 0.1275f;   // 1/sqrt(128) * log2(e)
        for (int it = 0; it < iters; ++it) {
            pf32x16 s[2] = {};
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int t = 0; t < 8; ++t)
                    s[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[(t + c) & 7], qf[t], s[c], 0, 0, 0);
            pbf16x8 pf[2][2];
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int h = 0; h < 2; ++h)
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[c][8 * h + j], sc, -1.0f));
                        l += p;
                        pf[c][h][j] = (__bf16)p;
                    }
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int h = 0; h < 2; ++h)
#pragma unroll
                    for (int d = 0; d < 4; ++d)
                        o[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[(4 * c + 2 * h + d) & 7], pf[c][h], o[d], 0, 0, 0);
        }
#pragma unroll
        for (int d = 0; d < 4; ++d)
#pragma unroll
            for (int r = 0; r < 16; ++r) res += o[d][r];
        res += l;
    }
    out[(int64_t)blockIdx.x * 256 + threadIdx.x] = res;
}

}  // namespace puter

using namespace puter;

extern "C" int puter_hip_mfma_probe(const void *operands, void *out, int64_t blocks, int iters, int mode,
                                    void *stream) {
    if (blocks < 0 || blocks > 0x7FFFFFFF || iters < 0 || mode < 0 || mode > 1)
        return fail(PUTER_ERR_INVALID, "mfma probe: invalid arguments");
    if (blocks == 0) return PUTER_OK;
    if (!operands || !out) return fail(PUTER_ERR_NIL, "mfma probe: nil buffer");
    if (!aligned16(operands) || !aligned16(out)) return fail(PUTER_ERR_INVALID, "mfma probe: buffers must be 16-byte aligned");
    hipStream_t s = as_stream(stream);
    const pbf16x8 *ops = static_cast<const pbf16x8 *>(operands);
    float *o = static_cast<float *>(out);
    constexpr size_t pin = 64 * 1024;   // two blocks per CU
    if (mode == 0) {
        if (hipFuncSetAttribute((const void *)probe_mfma<0>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)pin) != hipSuccess)
            return fail(PUTER_ERR_LAUNCH, "mfma probe: cannot set the LDS size");
        probe_mfma<0><<<(unsigned)blocks, 256, pin, s>>>(ops, o, iters);
    } else {
        if (hipFuncSetAttribute((const void *)probe_mfma<1>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)pin) != hipSuccess)
            return fail(PUTER_ERR_LAUNCH, "mfma probe: cannot set the LDS size");
        probe_mfma<1><<<(unsigned)blocks, 256, pin, s>>>(ops, o, iters);
    }
    return check_launch("mfma probe");
}

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
