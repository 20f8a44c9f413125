// Paged KV cache: KVPageWrite / KVPageGather device hooks.
// Reference: execution/page_intrinsic.go:13-24 (hook signatures), :135-352
// (callers), CPU semantics device/cpu/shape/page_generic.go:5-95 (row copies of
// `inner` elements) and the bounds rules of device/cpu/shape/page.go:139-146,191-203.
//
// Pure byte movement: rows are copied with 16-byte vectors when the row size and
// the pointers allow it (a 2 KiB bf16 row of 8 heads x 128 is two wave-wide
// loads); the gather takes one 64-lane wave per row.
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
// rows are copied in parallel here, and a row skips its store when a later row
// targets the same slot.  Each block (1024 threads; 256 for calls of at most
// 8192 rows) takes R consecutive rows (R a power of two, 8 to 1024, about
// value_rows / 512 so that a large call has about 512 blocks, two per CU,
// resident at once), puts their (page id, slot) keys in an
// LDS hash table (a key's entry keeps the highest
// local row, so duplicates inside the block resolve there), then all threads
// stream the keys of every row after the block with coalesced loads, 8 per
// thread in flight, and mark the entries those rows hit.  A row stores iff it is
// its entry's highest row and no later row hit the entry.  The stream reads
// 8 B per later row per block: about value_rows^2 * 4 / R bytes per call, which
// the L2 serves (the id / slot arrays are 8 B per row); a 16K-row write streams
// 32 MB of keys beside its 64 MB of rows, and its first block (the longest
// stream) covers its 16K later rows in two round trips.
#include "common.hpp"

namespace puter {

__device__ __forceinline__ void flag_invalid(int32_t *status) {
    if (status) *status = PUTER_ERR_INVALID;
}

constexpr int kWriteMaxRows = 1024;  // rows per write block, at most
// threads per write block: 256 up to kSmallWriteRows rows, else 1024
constexpr int kSmallWriteRows = 8192;
constexpr int kScanKeys = 16;        // later-row keys per thread per scan step
constexpr uint64_t kNoKey = ~(uint64_t)0;
constexpr int kBufWord3 = 0x00020000;  // buffer resource word 3: raw buffer, dword access

// The block's share of LDS for the last-row-wins table (dynamic shared memory,
// write_lds_bytes(R)): a 65536-bit filter with one bit set per block key (a
// later row whose bit is clear cannot match: one LDS read per streamed key, no
// probe chain), T = 2R entries of (key, highest local row, hit flag), and per
// local row its entry (-1: the row is out of range and stores nothing).
constexpr int kFilterWords = 2048;  // 65536 bits
struct WriteTable {
    uint32_t *filter;
    uint64_t *key;
    int *last;
    int *hit;
    int *entry;
    int bits;  // log2 T
};
static inline size_t write_lds_bytes(int64_t r) {
    return (size_t)kFilterWords * 4 + (size_t)r * 2 * (8 + 4 + 4) + (size_t)r * 4;
}

__device__ __forceinline__ WriteTable write_table(char *lds, int64_t r, int bits) {
    WriteTable t;
    t.filter = reinterpret_cast<uint32_t *>(lds);
    t.key = reinterpret_cast<uint64_t *>(t.filter + kFilterWords);
    t.last = reinterpret_cast<int *>(t.key + 2 * r);
    t.hit = t.last + 2 * r;
    t.entry = t.hit + 2 * r;
    t.bits = bits;
    return t;
}

// key of a (page id, slot) pair and its table position, in 32-bit arithmetic
__device__ __forceinline__ uint64_t write_key(int32_t id, int32_t off) {
    return ((uint64_t)(uint32_t)id << 32) | (uint32_t)off;
}
__device__ __forceinline__ uint32_t write_mix(int32_t id, int32_t off) {
    return (uint32_t)id * 0x9E3779B1u + (uint32_t)off * 0x85EBCA77u;
}
__device__ __forceinline__ uint32_t write_hash(int32_t id, int32_t off, int bits) {
    return write_mix(id, off) >> (32 - bits);
}
// id in [0, page_count) and off in [0, page_size), both bounds clamped to int32
// (ids and slots are int32)
__device__ __forceinline__ bool write_valid(int32_t id, int32_t off, int32_t pc, int32_t ps) {
    return id >= 0 && id < pc && off >= 0 && off < ps;
}

// Keys of the later rows [jb, jb + kScanKeys * THREADS): unconditional
// buffer loads that share one VGPR offset (the thread's) and step by an SGPR
// offset, so they hold no addresses of their own; the resources end at the last
// row and lanes past it read zeros (skipped by index in scan_probe).
struct ScanChunk {
    int32_t id[kScanKeys], off[kScanKeys];
};
template <int THREADS>
__device__ __forceinline__ void scan_load(ScanChunk &c, const int32_t *__restrict__ ids,
                                          const int32_t *__restrict__ offsets, int64_t jb, int64_t value_rows) {
    const int tid = threadIdx.x;
    const int64_t stride = (int64_t)THREADS * kScanKeys;
    const int bytes = (int)(max((int64_t)0, min(value_rows - jb, stride)) * 4);
    const __amdgpu_buffer_rsrc_t ir = __builtin_amdgcn_make_buffer_rsrc((void *)(ids + jb), (short)0, bytes, kBufWord3);
    const __amdgpu_buffer_rsrc_t orc =
        __builtin_amdgcn_make_buffer_rsrc((void *)(offsets + jb), (short)0, bytes, kBufWord3);
#pragma unroll
    for (int u = 0; u < kScanKeys; ++u) {
        c.id[u] = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(ir, tid * 4, u * THREADS * 4, 0);
        c.off[u] = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(orc, tid * 4, u * THREADS * 4, 0);
    }
}
// Marks the table entries that the chunk's keys hit (`left` = rows from the
// chunk's first row to the last row): a key whose filter bit is clear matches
// no block key; the few that pass take the exact lookup.
template <int THREADS>
__device__ __forceinline__ void scan_probe(const WriteTable &t, const ScanChunk &c, int64_t left, int32_t pc,
                                           int32_t ps) {
    const int tid = threadIdx.x, T = 1 << t.bits;
    uint32_t maybe = 0;  // bit u: key u's filter bit is set
#pragma unroll
    for (int u = 0; u < kScanKeys; ++u) {
        const uint32_t f = write_mix(c.id[u], c.off[u]) & 0xFFFFu;
        maybe |= ((t.filter[f >> 5] >> (f & 31)) & 1u) << u;
    }
    while (maybe) {
        const int u = __builtin_ctz(maybe);
        maybe &= maybe - 1;
        int32_t kid = c.id[0], koff = c.off[0];
#pragma unroll
        for (int w = 1; w < kScanKeys; ++w)
            if (w == u) kid = c.id[w], koff = c.off[w];
        if (tid + u * THREADS >= left || !write_valid(kid, koff, pc, ps)) continue;
        const uint64_t k = write_key(kid, koff);
        uint32_t h = write_hash(kid, koff, t.bits);
        // the table holds at most T / 2 keys: an empty entry ends every probe
        for (uint64_t cur = t.key[h]; cur != kNoKey; cur = t.key[h]) {
            if (cur == k) {
                t.hit[h] = 1;
                break;
            }
            h = (h + 1) & (uint32_t)(T - 1);
        }
    }
}

// (The write kernels take their block size as the template constant THREADS,
// not blockDim.x, which is read from the dispatch packet by a load whose wait
// would drain every load issued before it.)
//
// Which of the block's rows [row0, row0 + nrows) store (after the call, every
// thread of the block sees t.entry / t.last / t.hit): out-of-range ids or slots
// flag the status word and store nothing; among the rows of one slot only the
// highest stores.  Thread i < nrows brings local row i's (id, slot), and every
// thread the keys of its share of the first chunk of later rows (c0, from row
// row0 + nrows), both loaded by the caller at the kernel's start so that they
// and its other loads share one round trip (nrows <= the block's threads).
// Later chunks (16 x THREADS rows each: 16K for a 1024-thread block) are loaded
// here.  Ends with a barrier.
template <int THREADS>
__device__ void write_winners(const WriteTable &t, int32_t my_id, int32_t my_off, const ScanChunk &c0,
                              const int32_t *__restrict__ ids, const int32_t *__restrict__ offsets,
                              int64_t row0, int nrows, int64_t value_rows, int64_t page_count,
                              int64_t page_size, int32_t *status) {
    const int tid = threadIdx.x, T = 1 << t.bits;
    const int32_t pc = (int32_t)min(page_count, (int64_t)0x7FFFFFFF);
    const int32_t ps = (int32_t)min(page_size, (int64_t)0x7FFFFFFF);
    for (int e = tid; e < T; e += THREADS) {
        t.key[e] = kNoKey;
        t.last[e] = -1;
        t.hit[e] = 0;
    }
    for (int w = tid; w < kFilterWords; w += THREADS) t.filter[w] = 0;
    __syncthreads();
    if (tid < nrows) {
        if (!write_valid(my_id, my_off, pc, ps)) {
            flag_invalid(status);
            t.entry[tid] = -1;
        } else {
            const uint64_t k = write_key(my_id, my_off);
            uint32_t h = write_hash(my_id, my_off, t.bits);
            // at most nrows <= T / 2 keys: an empty entry is always reached
            for (;;) {
                const uint64_t prev = atomicCAS(reinterpret_cast<unsigned long long *>(&t.key[h]),
                                                (unsigned long long)kNoKey, (unsigned long long)k);
                if (prev == kNoKey || prev == k) break;
                h = (h + 1) & (uint32_t)(T - 1);
            }
            atomicMax(&t.last[h], tid);
            t.entry[tid] = (int)h;
            const uint32_t f = write_mix(my_id, my_off) & 0xFFFFu;
            atomicOr(&t.filter[f >> 5], 1u << (f & 31));
        }
    }
    __syncthreads();
    const int64_t first = row0 + nrows;
    const int64_t stride = (int64_t)THREADS * kScanKeys;
    if (first < value_rows) scan_probe<THREADS>(t, c0, value_rows - first, pc, ps);
    for (int64_t jb = first + stride; jb < value_rows; jb += stride) {
        ScanChunk c;
        scan_load<THREADS>(c, ids, offsets, jb, value_rows);
        scan_probe<THREADS>(t, c, value_rows - jb, pc, ps);
    }
    __syncthreads();
}

__device__ __forceinline__ bool write_wins(const WriteTable &t, int i) {
    const int e = t.entry[i];
    return e >= 0 && t.last[e] == i && t.hit[e] == 0;
}
// Unconditional loads of one V unit through a buffer resource (a unit past the
// resource's range reads as zero): with no branch around them the compiler's
// wait counts stay exact, so later waits need not drain these loads.
template <typename V> __device__ __forceinline__ V buf_load(__amdgpu_buffer_rsrc_t r, int vo, int so);
template <> __device__ __forceinline__ uint4 buf_load<uint4>(__amdgpu_buffer_rsrc_t r, int vo, int so) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, vo, so, 0);
    return make_uint4(v[0], v[1], v[2], v[3]);
}
template <> __device__ __forceinline__ uint32_t buf_load<uint32_t>(__amdgpu_buffer_rsrc_t r, int vo, int so) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, vo, so, 0);
}
template <> __device__ __forceinline__ uint8_t buf_load<uint8_t>(__amdgpu_buffer_rsrc_t r, int vo, int so) {
    return __builtin_amdgcn_raw_buffer_load_b8(r, vo, so, 0);
}

// the pool row (page id * page_size + slot) of a local row that passed write_wins
__device__ __forceinline__ int64_t write_slot(const WriteTable &t, int i, int64_t page_size) {
    const uint64_t k = t.key[t.entry[i]];
    return (int64_t)(k >> 32) * page_size + (int64_t)(uint32_t)k;
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
    // the gathered rows are read and written once here: non-temporal 16-byte
    // accesses (configs[4]'s pool, 290,592 rows of 2 KiB: 224.9 -> 193.5 us, 5.29 ->
    // 6.15 TB/s; issuing a lane's loads of the row before its stores gained nothing)
    for (int64_t u = lane; u < row_units; u += 64) {
        if constexpr (sizeof(V) == 16) st_stream(ld_stream(src + u), dst + u);
        else dst[u] = src[u];
    }
}

// One block per R rows (rows_per_block, a power of two; dynamic LDS of
// write_lds_bytes(R)).  The winning rows are copied as one flat run of V units
// over the block's rows, four units per thread in flight; rows of a power-of-two
// unit count (2 KiB rows of 8 x 128 bf16 are 128 uint4) locate a unit's row by
// a shift, others by a division.  The first four units of every thread are
// loaded before the table work (after the thread's own id and slot), so their
// HBM round trip runs under the table's; only the stores wait for it.
template <typename V, int THREADS>
__global__ __launch_bounds__(THREADS) __attribute__((amdgpu_waves_per_eu(8))) void page_write_kernel(char *__restrict__ storage,
                                                         const char *__restrict__ values,
                                                         const int32_t *__restrict__ ids,
                                                         const int32_t *__restrict__ offsets,
                                                         int64_t page_count, int64_t page_size,
                                                         int64_t row_units, int64_t value_rows,
                                                         int64_t rows_per_block, int table_bits,
                                                         int unit_shift, int32_t *status) {
    extern __shared__ __align__(16) char lds[];
    const int tid = threadIdx.x;
    const int64_t row0 = (int64_t)blockIdx.x * rows_per_block;
    const int nrows = (int)min(rows_per_block, value_rows - row0);
    const WriteTable t = write_table(lds, rows_per_block, table_bits);
    // this thread's (id, slot), then its first four units, all unconditional
    // (buffer ranges end at the block's rows; lanes past them read zeros)
    const __amdgpu_buffer_rsrc_t idr =
        __builtin_amdgcn_make_buffer_rsrc((void *)(ids + row0), (short)0, nrows * 4, kBufWord3);
    const __amdgpu_buffer_rsrc_t offr =
        __builtin_amdgcn_make_buffer_rsrc((void *)(offsets + row0), (short)0, nrows * 4, kBufWord3);
    const int32_t my_id = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(idr, tid * 4, 0, 0);
    const int32_t my_off = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(offr, tid * 4, 0, 0);
    const V *src = reinterpret_cast<const V *>(values) + row0 * row_units;
    V *dst = reinterpret_cast<V *>(storage);
    const int64_t total = (int64_t)nrows * row_units;
    const int64_t B = THREADS;
    const int first_bytes = (int)(min(total, 4 * B) * (int64_t)sizeof(V));
    const __amdgpu_buffer_rsrc_t vr =
        __builtin_amdgcn_make_buffer_rsrc((void *)src, (short)0, first_bytes, kBufWord3);
    const int vo = tid * (int)sizeof(V), vs = (int)(B * sizeof(V));
    V v0 = buf_load<V>(vr, vo, 0);
    V v1 = buf_load<V>(vr, vo, vs);
    V v2 = buf_load<V>(vr, vo, 2 * vs);
    V v3 = buf_load<V>(vr, vo, 3 * vs);
    ScanChunk c0;
    scan_load<THREADS>(c0, ids, offsets, row0 + nrows, value_rows);
    write_winners<THREADS>(t, my_id, my_off, c0, ids, offsets, row0, nrows, value_rows, page_count, page_size, status);
    auto put = [&](int64_t q, const V &v) __attribute__((always_inline)) {
        if (q >= total) return;
        const int64_t i = unit_shift >= 0 ? q >> unit_shift : q / row_units;
        if (!write_wins(t, (int)i)) return;
        V *const p = &dst[write_slot(t, (int)i, page_size) * row_units + (q - i * row_units)];
        // non-temporal 16-byte stores (the pool rows are not re-read here): 16384 / 65536
        // rows of 2 KiB 13.0 -> 12.3 / 54.0 -> 47.4 us; non-temporal value loads lost
        if constexpr (sizeof(V) == 16) st_stream(v, p);
        else *p = v;
    };
    put(tid, v0);
    put(tid + B, v1);
    put(tid + 2 * B, v2);
    put(tid + 3 * B, v3);
    for (int64_t q0 = tid + 4 * B; q0 < total; q0 += 4 * B) {
        if (q0 < total) v0 = src[q0];
        if (q0 + B < total) v1 = src[q0 + B];
        if (q0 + 2 * B < total) v2 = src[q0 + 2 * B];
        if (q0 + 3 * B < total) v3 = src[q0 + 3 * B];
        put(q0, v0);
        put(q0 + B, v1);
        put(q0 + 2 * B, v2);
        put(q0 + 3 * B, v3);
    }
}

// fp8 quantising write: R rows per block as for the plain write, each winning
// row taken by one wave; a lane handles 16 consecutive elements at a time (one
// 16-byte fp8 store; head = element / head_dim).
template <int DT, int THREADS>
__global__ __launch_bounds__(THREADS) __attribute__((amdgpu_waves_per_eu(8))) void page_write_fp8_kernel(uint8_t *__restrict__ storage,
                                                             const void *__restrict__ values,
                                                             const int32_t *__restrict__ ids,
                                                             const int32_t *__restrict__ offsets,
                                                             const float *__restrict__ scales,
                                                             int64_t page_count, int64_t page_size,
                                                             int64_t head_dim, int64_t inner, int64_t value_rows,
                                                             int64_t rows_per_block, int table_bits,
                                                             int32_t *status) {
    using T = typename Elem<DT>::T;
    extern __shared__ __align__(16) char lds[];
    const int tid = threadIdx.x;
    const int64_t row0 = (int64_t)blockIdx.x * rows_per_block;
    const int nrows = (int)min(rows_per_block, value_rows - row0);
    const WriteTable t = write_table(lds, rows_per_block, table_bits);
    int32_t my_id = -1, my_off = -1;
    if (tid < nrows) {
        my_id = ids[row0 + tid];
        my_off = offsets[row0 + tid];
    }
    ScanChunk c0;
    scan_load<THREADS>(c0, ids, offsets, row0 + nrows, value_rows);
    write_winners<THREADS>(t, my_id, my_off, c0, ids, offsets, row0, nrows, value_rows, page_count, page_size, status);
    const int lane = threadIdx.x & 63;
    for (int i = threadIdx.x >> 6; i < nrows; i += THREADS / 64) {
        if (!write_wins(t, i)) continue;
        const int64_t row = row0 + i;
        uint8_t *dst = storage + write_slot(t, i, page_size) * inner;
        const T *src = reinterpret_cast<const T *>(values) + row * inner;
        for (int64_t e0 = (int64_t)lane * 16; e0 < inner; e0 += 64 * 16) {
            uint32_t w[4] = {0, 0, 0, 0};
            const int n = (int)min((int64_t)16, inner - e0);
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                if (k < n) {
                    const int64_t e = e0 + k;
                    const float q = __fdiv_rn(Elem<DT>::load(src[e]), scales[e / head_dim]);
                    w[k >> 2] |= f32_to_e4m3(q) << (8 * (k & 3));
                }
            }
            if (n == 16) {
                *reinterpret_cast<uint4 *>(dst + e0) = make_uint4(w[0], w[1], w[2], w[3]);
            } else {
                for (int k = 0; k < n; ++k) dst[e0 + k] = (uint8_t)(w[k >> 2] >> (8 * (k & 3)));
            }
        }
    }
}

// Rows per write block (a power of two, 8..1024, about rows / 512; at most 16
// for the 256-thread blocks of calls up to kSmallWriteRows rows, so R never
// exceeds the block's threads) and log2 of its table size (2R entries).
static int64_t write_rows_per_block(int64_t rows, int *table_bits) {
    int64_t r = 8;
    while (r < kWriteMaxRows && r * 512 < rows) r <<= 1;
    int bits = 0;
    while (((int64_t)1 << bits) < 2 * r) ++bits;
    *table_bits = bits;
    return r;
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
    int bits = 0;
    const int64_t per = write_rows_per_block(value_rows, &bits);
    const int64_t nblocks = (value_rows + per - 1) / per;
    if (nblocks > 0x7FFFFFFF) return fail(PUTER_ERR_INVALID, "kv page write: too many rows");
    const unsigned blocks = (unsigned)nblocks;
    const size_t lds = write_lds_bytes(per);
    const void *ptrs[2] = {dst_base, values};
    auto shift_of = [](int64_t units) {
        int sh = 0;
        while (((int64_t)1 << sh) < units) ++sh;
        return ((int64_t)1 << sh) == units ? sh : -1;
    };
    const bool small = value_rows <= kSmallWriteRows;
    auto launch = [&](auto unit, int64_t units) {
        using V = decltype(unit);
        const int sh = shift_of(units);
        if (small)
            page_write_kernel<V, 256><<<blocks, 256, lds, s>>>(dst_base, (const char *)values, page_ids, offsets,
                                                               page_count, page_size, units, value_rows, per, bits, sh,
                                                               status);
        else
            page_write_kernel<V, 1024><<<blocks, 1024, lds, s>>>(dst_base, (const char *)values, page_ids, offsets,
                                                                 page_count, page_size, units, value_rows, per, bits,
                                                                 sh, status);
    };
    if (row_bytes % 16 == 0 && all_aligned(ptrs, 2, 15)) launch(uint4{}, (int64_t)(row_bytes / 16));
    else if (row_bytes % 4 == 0 && all_aligned(ptrs, 2, 3)) launch(uint32_t{}, (int64_t)(row_bytes / 4));
    else launch(uint8_t{}, (int64_t)row_bytes);
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
    int bits = 0;
    const int64_t per = write_rows_per_block(value_rows, &bits);
    const int64_t nblocks = (value_rows + per - 1) / per;
    if (nblocks > 0x7FFFFFFF) return fail(PUTER_ERR_INVALID, "kv page write fp8: too many rows");
    const unsigned blocks = (unsigned)nblocks;
    const size_t lds = write_lds_bytes(per);
    const bool small = value_rows <= kSmallWriteRows;
#define PUTER_FP8_WRITE(DT)                                                                                    \
    if (small)                                                                                                 \
        page_write_fp8_kernel<DT, 256><<<blocks, 256, lds, s>>>(dst, values, page_ids, offsets, scales, page_count, \
                                                                page_size, head_dim, inner, value_rows, per, bits,   \
                                                                status);                                             \
    else                                                                                                       \
        page_write_fp8_kernel<DT, 1024><<<blocks, 1024, lds, s>>>(dst, values, page_ids, offsets, scales,          \
                                                                  page_count, page_size, head_dim, inner, value_rows, \
                                                                  per, bits, status);
    switch (value_dtype) {
    case PUTER_F32: PUTER_FP8_WRITE(PUTER_F32) break;
    case PUTER_BF16: PUTER_FP8_WRITE(PUTER_BF16) break;
    case PUTER_F16: PUTER_FP8_WRITE(PUTER_F16) break;
    }
#undef PUTER_FP8_WRITE
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
