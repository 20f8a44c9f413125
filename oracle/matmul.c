/*
 * Matmul for the CPU oracle (test infrastructure only; see oracle.h).
 * out[rows, cols] = left[rows, inner] . right[inner, cols], row-major, following
 * device/cpu/matmul/compute.go:46-62 (dispatchMatmul):
 *   F32   f32_apply.go:5-15 -> matmulFloat32Scalar select_generic.go:25-37: each
 *         output accumulated in f32 over `inner` in index order;
 *   F64   f32_apply.go:17-27 -> matmulFloat64Scalar select_generic.go:39-...: the
 *         same in f64;
 *   BF16 / F16  runMatmulReducedCols compute.go:74-92: operands widened to f32
 *         (loadBF16 / loadF16 :9-22), summed in f32 in index order, the sum stored
 *         with the format's round-to-nearest-even (storeBF16 / storeF16 :14-28).
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

int or_matmul(void *out, const void *left, const void *right, int64_t rows, int64_t inner,
              int64_t cols, int dtype) {
    if (rows < 0 || inner < 0 || cols < 0) return -6;
    if (dtype == OR_F32) return or_matmul_f32(out, left, right, rows, inner, cols);
    if (dtype == OR_F64) {
        const double *l = left, *rt = right;
        double *o = out;
#pragma omp parallel for schedule(static) num_threads(oracle_get_threads())
        for (int64_t r = 0; r < rows; ++r)
            for (int64_t c = 0; c < cols; ++c) {
                double s = 0.0;
                for (int64_t i = 0; i < inner; ++i) s += l[r * inner + i] * rt[i * cols + c];
                o[r * cols + c] = s;
            }
        return 0;
    }
    if (dtype != OR_BF16 && dtype != OR_F16) return -6;
#pragma omp parallel for schedule(static) num_threads(oracle_get_threads())
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < cols; ++c) {
            float s = 0.0f;
            for (int64_t i = 0; i < inner; ++i)
                s += or_load(left, (size_t)(r * inner + i), dtype) * or_load(right, (size_t)(i * cols + c), dtype);
            or_store(out, (size_t)(r * cols + c), s, dtype);
        }
    return 0;
}
