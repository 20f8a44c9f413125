/*
 * f32 Matmul for the CPU oracle (test infrastructure only; see oracle.h).
 * Restates device/cpu/matmul/compute.go:46-62 and f32_apply.go:5-15:
 * out[rows, cols] = left[rows, inner] . right[inner, cols], row-major, each
 * output accumulated in f32 over `inner` in index order.
 */
#include "oracle.h"

int or_matmul_f32(float *out, const float *left, const float *right,
                  int64_t rows, int64_t inner, int64_t cols) {
    if (rows < 0 || inner < 0 || cols < 0) return -6;
#pragma omp parallel for schedule(static) num_threads(oracle_get_threads())
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t c = 0; c < cols; ++c) {
            float s = 0.0f;
            for (int64_t i = 0; i < inner; ++i) s += left[r * inner + i] * right[i * cols + c];
            out[r * cols + c] = s;
        }
    }
    return 0;
}
