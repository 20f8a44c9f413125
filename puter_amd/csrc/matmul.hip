// f32 Matmul: out[rows, cols] = left[rows, inner] . right[inner, cols], row-major.
// Reference: device/interface.go:409-415, device/cpu/matmul/compute.go:46-62.
// Support kernel for the f32 pre-norm attention block (Q/K/V/O projections):
// 64x64 output tile per 256-thread block, 16-deep K slices staged in LDS, a
// 4x4 register micro-tile per thread, f32 FMA accumulation.
#include "common.hpp"

namespace puter {

constexpr int kTile = 64, kDepth = 16;

__global__ __launch_bounds__(256) void matmul_f32_kernel(float *__restrict__ out,
                                                         const float *__restrict__ A,
                                                         const float *__restrict__ B,
                                                         int64_t M, int64_t K, int64_t N) {
    __shared__ float As[kDepth][kTile + 4];
    __shared__ float Bs[kDepth][kTile + 4];
    const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
    const int64_t row0 = (int64_t)blockIdx.y * kTile, col0 = (int64_t)blockIdx.x * kTile;
    float acc[4][4] = {};
    for (int64_t k0 = 0; k0 < K; k0 += kDepth) {
        for (int i = threadIdx.x; i < kTile * kDepth; i += 256) {
            const int r = i / kDepth, c = i % kDepth;          // A tile: 64 rows x 16
            const int64_t gr = row0 + r, gc = k0 + c;
            As[c][r] = (gr < M && gc < K) ? A[gr * K + gc] : 0.0f;
            const int br = i / kTile, bc = i % kTile;          // B tile: 16 rows x 64
            const int64_t gbr = k0 + br, gbc = col0 + bc;
            Bs[br][bc] = (gbr < K && gbc < N) ? B[gbr * N + gbc] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < kDepth; ++k) {
            float a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = As[k][ty * 4 + i];
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = Bs[k][tx * 4 + j];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t r = row0 + ty * 4 + i, c = col0 + tx * 4 + j;
            if (r < M && c < N) out[r * N + c] = acc[i][j];
        }
}

}  // namespace puter

using namespace puter;

extern "C" int puter_hip_matmul(void *out, const void *left, const void *right, int64_t rows,
                                int64_t inner, int64_t cols, int dtype, void *stream) {
    if (rows < 0 || inner < 0 || cols < 0) return fail(PUTER_ERR_INVALID, "matmul: negative shape");
    if (dtype != PUTER_F32) return fail(PUTER_ERR_INVALID, "matmul: unsupported dtype %d (F32 only)", dtype);
    if (rows == 0 || cols == 0) return PUTER_OK;
    if (!out || !left || !right) return fail(PUTER_ERR_NIL, "matmul: nil buffer");
    if (inner == 0) {
        hipError_t e = hipMemsetAsync(out, 0, (size_t)(rows * cols) * sizeof(float), as_stream(stream));
        return e == hipSuccess ? PUTER_OK : fail(PUTER_ERR_LAUNCH, "matmul: %s", hipGetErrorString(e));
    }
    const dim3 grid((unsigned)((cols + kTile - 1) / kTile), (unsigned)((rows + kTile - 1) / kTile));
    if (grid.y > 65535) return fail(PUTER_ERR_INVALID, "matmul: too many rows");
    matmul_f32_kernel<<<grid, 256, 0, as_stream(stream)>>>(static_cast<float *>(out), static_cast<const float *>(left),
                                                          static_cast<const float *>(right), rows, inner, cols);
    return check_launch("matmul");
}
