/*
 * Paged KV write / gather for the CPU oracle (test infrastructure only; see
 * oracle.h).  Restates device/cpu/shape/page_generic.go:5-95 (byte copies of
 * `inner` elements per row) with the bounds checks of device/cpu/shape/page.go:139-146
 * (write) and :191-203 (gather), and the layer offset of
 * execution/page_intrinsic.go:361-438 (`storageOffset` elements into a rank-5
 * [layers, pages, pageSize, ...] storage).
 */
#include "oracle.h"

#include <string.h>

int or_page_write(const void *storage, const void *values, const int32_t *page_ids,
                  const int32_t *offsets, void *output, int64_t page_count, int64_t page_size,
                  int64_t inner, int64_t value_rows, int64_t storage_offset, int elem_size) {
    if (page_count < 0 || page_size <= 0 || inner < 0 || value_rows < 0) return -6;
    if (value_rows == 0 || inner == 0) return 0;
    for (int64_t r = 0; r < value_rows; ++r) {
        if (page_ids[r] < 0 || page_ids[r] >= page_count) return -6;
        if (offsets[r] < 0 || offsets[r] >= page_size) return -6;
    }
    size_t row_bytes = (size_t)inner * (size_t)elem_size;
    const char *src = (const char *)storage + (size_t)storage_offset * (size_t)elem_size;
    char *dst = (char *)output + (size_t)storage_offset * (size_t)elem_size;
    if (dst != src) memcpy(dst, src, (size_t)(page_count * page_size) * row_bytes);
    for (int64_t r = 0; r < value_rows; ++r) {
        size_t slot = (size_t)((int64_t)page_ids[r] * page_size + offsets[r]);
        memcpy(dst + slot * row_bytes, (const char *)values + (size_t)r * row_bytes, row_bytes);
    }
    return 0;
}

int or_page_gather(const void *storage, const int32_t *page_table, void *output,
                   int64_t page_count, int64_t page_size, int64_t inner, int64_t out_rows,
                   int64_t storage_offset, int64_t table_len, int elem_size) {
    if (page_count < 0 || page_size <= 0 || inner < 0 || out_rows < 0) return -6;
    if (out_rows > table_len * page_size) out_rows = table_len * page_size;
    for (int64_t r = 0; r < out_rows; r += page_size) {
        int32_t id = page_table[r / page_size];
        if (id < 0 || id >= page_count) return -6;
    }
    size_t row_bytes = (size_t)inner * (size_t)elem_size;
    const char *src = (const char *)storage + (size_t)storage_offset * (size_t)elem_size;
#pragma omp parallel for schedule(static) num_threads(oracle_get_threads())
    for (int64_t r = 0; r < out_rows; ++r) {
        size_t slot = (size_t)((int64_t)page_table[r / page_size] * page_size + r % page_size);
        memcpy((char *)output + (size_t)r * row_bytes, src + slot * row_bytes, row_bytes);
    }
    return 0;
}
