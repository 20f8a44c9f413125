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

/* fp8 quantising page write (the library's extension hook
 * puter_hip_kv_page_write_fp8; no reference method): byte = E4M3(x / scale[h])
 * with IEEE f32 division and the saturating RNE narrowing of or_f32_to_e4m3,
 * h = element / head_dim.  Row placement and bounds as or_page_write
 * (page_generic.go:5-43, page.go:139-146).  In place. */
int or_page_write_fp8(uint8_t *storage, const void *values, const int32_t *page_ids,
                      const int32_t *offsets, int64_t page_count, int64_t page_size,
                      int64_t kv_heads, int64_t head_dim, int64_t value_rows,
                      int64_t storage_offset, const float *scales, int value_dtype) {
    if (page_count < 0 || page_size <= 0 || kv_heads <= 0 || head_dim <= 0 || value_rows < 0) return -6;
    for (int64_t r = 0; r < value_rows; ++r) {
        if (page_ids[r] < 0 || page_ids[r] >= page_count) return -6;
        if (offsets[r] < 0 || offsets[r] >= page_size) return -6;
    }
    const int64_t inner = kv_heads * head_dim;
    uint8_t *dst = storage + storage_offset;
    for (int64_t r = 0; r < value_rows; ++r) {
        uint8_t *row = dst + ((int64_t)page_ids[r] * page_size + offsets[r]) * inner;
        for (int64_t e = 0; e < inner; ++e) {
            const float x = or_load(values, (size_t)(r * inner + e), value_dtype);
            row[e] = or_f32_to_e4m3(x / scales[e / head_dim]);
        }
    }
    return 0;
}
