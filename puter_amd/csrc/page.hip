// Paged KV cache: KVPageWrite / KVPageGather device hooks.
// Reference: execution/page_intrinsic.go:13-24 (hook signatures), :135-352
// (callers), CPU semantics device/cpu/shape/page_generic.go:5-95 (row copies of
// `inner` elements) and the bounds rules of device/cpu/shape/page.go:139-146,191-203.
//
// Pure byte movement: rows are copied with 16-byte vectors when the row size and
// the pointers allow it, one 64-lane wave per row (a 2 KiB bf16 row of 8 heads x
// 128 is two wave-wide loads).
//
// Page ids live on the device, and the host cannot read them without a
// synchronisation the reference's zero-host-sync contract forbids, so they are
// checked on the device.  The reference's CPU path rejects the whole call with
// ErrShapeMismatch when any id or slot is out of range
// (device/cpu/shape/page.go:139-146,191-203); here such a row is skipped (write)
// or zero-filled (gather), so no access ever leaves the storage, and the lane
// that finds it stores PUTER_ERR_INVALID into the caller's status word, which
// the caller reads at its next synchronisation (the Metal backend's device path
// does the same with an error flag, device/metal/internal/runtime/shape.metal:97-176).
//
// Write order: the reference copies the value rows in order, so when several
// rows target one (page, slot) the last one wins (page_generic.go:23-27).  The
// rows are copied in parallel here, and a row skips its copy when a later row
// targets the same slot: each wave scans the later rows' (id, slot) pairs, 64
// per step, O(value_rows - row) reads that hit the cache.
#include "common.hpp"

namespace puter {

__device__ __forceinline__ void flag_invalid(int32_t *status) {
    if (status) *status = PUTER_ERR_INVALID;
}

// true when a row after `row` targets the same (id, slot); wave-uniform
__device__ __forceinline__ bool overwritten_later(const int32_t *__restrict__ ids, const int32_t *__restrict__ offsets,
                                                  int64_t row, int64_t value_rows, int32_t id, int32_t off, int lane) {
    for (int64_t j0 = row + 1; j0 < value_rows; j0 += 64) {
        const int64_t j = j0 + lane;
        const bool hit = j < value_rows && ids[j] == id && offsets[j] == off;
        if (__any(hit)) return true;
    }
    return false;
}

template <typename V>
__global__ __launch_bounds__(256) void page_gather_kernel(const char *__restrict__ storage,
                                                          const int32_t *__restrict__ table,
                                                          char *__restrict__ out, int64_t page_count,
                                                          int64_t page_size, int64_t row_units,
                                                          int64_t out_rows, int32_t *status) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= out_rows) return;
    const int32_t id = table[row / page_size];
    V *dst = reinterpret_cast<V *>(out) + row * row_units;
    if (id < 0 || id >= page_count) {
        if (lane == 0) flag_invalid(status);
        for (int64_t u = lane; u < row_units; u += 64) dst[u] = V{};
        return;
    }
    const V *src = reinterpret_cast<const V *>(storage) + ((int64_t)id * page_size + row % page_size) * row_units;
    for (int64_t u = lane; u < row_units; u += 64) dst[u] = src[u];
}

template <typename V>
__global__ __launch_bounds__(256) void page_write_kernel(char *__restrict__ storage,
                                                         const char *__restrict__ values,
                                                         const int32_t *__restrict__ ids,
                                                         const int32_t *__restrict__ offsets,
                                                         int64_t page_count, int64_t page_size,
                                                         int64_t row_units, int64_t value_rows,
                                                         int32_t *status) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= value_rows) return;
    const int32_t id = ids[row], off = offsets[row];
    if (id < 0 || id >= page_count || off < 0 || off >= page_size) {
        if (lane == 0) flag_invalid(status);
        return;
    }
    if (overwritten_later(ids, offsets, row, value_rows, id, off, lane)) return;
    V *dst = reinterpret_cast<V *>(storage) + ((int64_t)id * page_size + off) * row_units;
    const V *src = reinterpret_cast<const V *>(values) + row * row_units;
    for (int64_t u = lane; u < row_units; u += 64) dst[u] = src[u];
}

// fp8 quantising write: one wave per value row; lane handles 16 consecutive
// elements at a time (one 16-byte fp8 store; head = element / head_dim).
template <int DT>
__global__ __launch_bounds__(256) void page_write_fp8_kernel(uint8_t *__restrict__ storage,
                                                             const void *__restrict__ values,
                                                             const int32_t *__restrict__ ids,
                                                             const int32_t *__restrict__ offsets,
                                                             const float *__restrict__ scales,
                                                             int64_t page_count, int64_t page_size,
                                                             int64_t head_dim, int64_t inner, int64_t value_rows,
                                                             int32_t *status) {
    using T = typename Elem<DT>::T;
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= value_rows) return;
    const int32_t id = ids[row], off = offsets[row];
    if (id < 0 || id >= page_count || off < 0 || off >= page_size) {
        if (lane == 0) flag_invalid(status);
        return;
    }
    if (overwritten_later(ids, offsets, row, value_rows, id, off, lane)) return;
    uint8_t *dst = storage + ((int64_t)id * page_size + off) * inner;
    const T *src = reinterpret_cast<const T *>(values) + row * inner;
    for (int64_t e0 = (int64_t)lane * 16; e0 < inner; e0 += 64 * 16) {
        uint32_t w[4] = {0, 0, 0, 0};
        const int n = (int)min((int64_t)16, inner - e0);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            if (i < n) {
                const int64_t e = e0 + i;
                const float q = __fdiv_rn(Elem<DT>::load(src[e]), scales[e / head_dim]);
                w[i >> 2] |= f32_to_e4m3(q) << (8 * (i & 3));
            }
        }
        if (n == 16) {
            *reinterpret_cast<uint4 *>(dst + e0) = make_uint4(w[0], w[1], w[2], w[3]);
        } else {
            for (int i = 0; i < n; ++i) dst[e0 + i] = (uint8_t)(w[i >> 2] >> (8 * (i & 3)));
        }
    }
}

static bool all_aligned(const void *const *p, int n, uintptr_t mask) {
    for (int i = 0; i < n; ++i)
        if (reinterpret_cast<uintptr_t>(p[i]) & mask) return false;
    return true;
}

}  // namespace puter

using namespace puter;

extern "C" {

int puter_hip_kv_page_write(const void *storage, const void *values, const int32_t *page_ids,
                            const int32_t *offsets, void *output, int64_t page_count,
                            int64_t page_size, int64_t inner, int64_t value_rows,
                            int64_t storage_offset, int dtype, int32_t *status, void *stream) {
    const int es = dtype_bytes(dtype);
    if (es == 0) return fail(PUTER_ERR_INVALID, "kv page write: unsupported dtype %d", dtype);
    if (page_count < 0 || page_size <= 0 || inner < 0 || value_rows < 0 || storage_offset < 0)
        return fail(PUTER_ERR_INVALID, "kv page write: invalid shape");
    if (value_rows == 0 || inner == 0) return PUTER_OK;
    if (!storage || !values || !page_ids || !offsets || !output) return fail(PUTER_ERR_NIL, "kv page write: nil buffer");
    if (reinterpret_cast<uintptr_t>(status) & 3) return fail(PUTER_ERR_INVALID, "kv page write: misaligned status word");
    hipStream_t s = as_stream(stream);
    const size_t row_bytes = (size_t)inner * es;
    const char *src_base = static_cast<const char *>(storage) + (size_t)storage_offset * es;
    char *dst_base = static_cast<char *>(output) + (size_t)storage_offset * es;
    // pageWrite*Generic copies storage to output first (page_generic.go:23); the
    // device caller passes output == storage (page_intrinsic.go:199-205), a no-op
    if (dst_base != src_base) {
        hipError_t e = hipMemcpyAsync(dst_base, src_base, (size_t)(page_count * page_size) * row_bytes,
                                      hipMemcpyDeviceToDevice, s);
        if (e != hipSuccess) return fail(PUTER_ERR_LAUNCH, "kv page write: copy: %s", hipGetErrorString(e));
    }
    const unsigned blocks = (unsigned)((value_rows + 3) / 4);
    const void *ptrs[2] = {dst_base, values};
    if (row_bytes % 16 == 0 && all_aligned(ptrs, 2, 15))
        page_write_kernel<uint4><<<blocks, 256, 0, s>>>(dst_base, (const char *)values, page_ids, offsets,
                                                        page_count, page_size, (int64_t)(row_bytes / 16), value_rows, status);
    else if (row_bytes % 4 == 0 && all_aligned(ptrs, 2, 3))
        page_write_kernel<uint32_t><<<blocks, 256, 0, s>>>(dst_base, (const char *)values, page_ids, offsets,
                                                           page_count, page_size, (int64_t)(row_bytes / 4), value_rows, status);
    else
        page_write_kernel<uint8_t><<<blocks, 256, 0, s>>>(dst_base, (const char *)values, page_ids, offsets,
                                                          page_count, page_size, (int64_t)row_bytes, value_rows, status);
    return check_launch("kv page write");
}

int puter_hip_kv_page_write_fp8(void *storage, const void *values, const int32_t *page_ids,
                                const int32_t *offsets, int64_t page_count, int64_t page_size,
                                int64_t kv_heads, int64_t head_dim, int64_t value_rows,
                                int64_t storage_offset, const float *scales, int value_dtype,
                                int32_t *status, void *stream) {
    if (!is_norm_dtype(value_dtype)) return fail(PUTER_ERR_INVALID, "kv page write fp8: unsupported value dtype %d", value_dtype);
    if (page_count < 0 || page_size <= 0 || kv_heads <= 0 || head_dim <= 0 || value_rows < 0 || storage_offset < 0)
        return fail(PUTER_ERR_INVALID, "kv page write fp8: invalid shape");
    if (value_rows == 0) return PUTER_OK;
    if (!storage || !values || !page_ids || !offsets || !scales) return fail(PUTER_ERR_NIL, "kv page write fp8: nil buffer");
    if (reinterpret_cast<uintptr_t>(status) & 3) return fail(PUTER_ERR_INVALID, "kv page write fp8: misaligned status word");
    const int64_t inner = kv_heads * head_dim;
    uint8_t *dst = static_cast<uint8_t *>(storage) + storage_offset;
    // the 16-byte fp8 stores need 16-byte aligned rows
    if (((reinterpret_cast<uintptr_t>(dst) | (uintptr_t)inner) & 15) != 0)
        return fail(PUTER_ERR_INVALID, "kv page write fp8: pool rows must be 16-byte aligned");
    hipStream_t s = as_stream(stream);
    const unsigned blocks = (unsigned)((value_rows + 3) / 4);
    switch (value_dtype) {
    case PUTER_F32: page_write_fp8_kernel<PUTER_F32><<<blocks, 256, 0, s>>>(dst, values, page_ids, offsets, scales, page_count, page_size, head_dim, inner, value_rows, status); break;
    case PUTER_BF16: page_write_fp8_kernel<PUTER_BF16><<<blocks, 256, 0, s>>>(dst, values, page_ids, offsets, scales, page_count, page_size, head_dim, inner, value_rows, status); break;
    case PUTER_F16: page_write_fp8_kernel<PUTER_F16><<<blocks, 256, 0, s>>>(dst, values, page_ids, offsets, scales, page_count, page_size, head_dim, inner, value_rows, status); break;
    }
    return check_launch("kv page write fp8");
}

int puter_hip_kv_page_gather(const void *storage, const int32_t *page_table, void *output,
                             int64_t page_count, int64_t page_size, int64_t inner,
                             int64_t out_rows, int64_t storage_offset, int dtype, int32_t *status,
                             void *stream) {
    const int es = dtype_bytes(dtype);
    if (es == 0) return fail(PUTER_ERR_INVALID, "kv page gather: unsupported dtype %d", dtype);
    if (page_count < 0 || page_size <= 0 || inner < 0 || out_rows < 0 || storage_offset < 0)
        return fail(PUTER_ERR_INVALID, "kv page gather: invalid shape");
    if (out_rows == 0 || inner == 0) return PUTER_OK;
    if (!storage || !page_table || !output) return fail(PUTER_ERR_NIL, "kv page gather: nil buffer");
    if (reinterpret_cast<uintptr_t>(status) & 3) return fail(PUTER_ERR_INVALID, "kv page gather: misaligned status word");
    hipStream_t s = as_stream(stream);
    const size_t row_bytes = (size_t)inner * es;
    const char *src = static_cast<const char *>(storage) + (size_t)storage_offset * es;
    const unsigned blocks = (unsigned)((out_rows + 3) / 4);
    const void *ptrs[2] = {src, output};
    if (row_bytes % 16 == 0 && all_aligned(ptrs, 2, 15))
        page_gather_kernel<uint4><<<blocks, 256, 0, s>>>(src, page_table, (char *)output, page_count,
                                                         page_size, (int64_t)(row_bytes / 16), out_rows, status);
    else if (row_bytes % 4 == 0 && all_aligned(ptrs, 2, 3))
        page_gather_kernel<uint32_t><<<blocks, 256, 0, s>>>(src, page_table, (char *)output, page_count,
                                                            page_size, (int64_t)(row_bytes / 4), out_rows, status);
    else
        page_gather_kernel<uint8_t><<<blocks, 256, 0, s>>>(src, page_table, (char *)output, page_count,
                                                           page_size, (int64_t)row_bytes, out_rows, status);
    return check_launch("kv page gather");
}

}  // extern "C"
