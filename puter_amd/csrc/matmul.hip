// Matmul: out[rows, cols] = left[rows, inner] . right[inner, cols], row-major.
// Reference: device/interface.go:409-415, device/cpu/matmul/compute.go:46-92
// (dispatchMatmul: F32, F64, F16, BF16; the 16-bit formats widen to f32, sum in
// f32 and store the sum rounded to nearest even, compute.go:74-92).
//
// bf16 / f16: MFMA GEMM, two tile shapes from one template (NW = waves along N,
// MT = 32-row accumulator blocks per wave), K advancing 64 at a time:
//   NW = 4, MT = 4: a 512-thread block (8 waves, 2 x 4) computes a 256 x 256
//     output tile, one block per CU;
//   NW = 2, MT = 2: a 256-thread block (4 waves, 2 x 2) computes a 128 x 128
//     tile, two blocks per CU; taken where its rounds of blocks over the CUs
//     cost less (mfma_small_tiles).
// Wave (wm, wn) owns rows 32 MT wm .. +32 MT - 1 and columns 64 wn .. +63 as MT x 2
// v_mfma_f32_32x32x16 accumulators.  The A (64 MT x 64) and B (64 x 64 NW)
// slices are copied HBM -> LDS by buffer_load ... lds, double buffered, each
// slice's copies issued before the slice ahead of it is computed.  The block computes
// C^T = B^T . A^T so that a lane's accumulator column is one output row and its
// registers hold runs of 4 consecutive output columns (the epilogue regroups them
// in LDS into whole 128-byte row pieces before storing):
//   A operand (B^T[n, k]): 8 consecutive k of one column n of the row-major B
//     slice, read with ds_read_b64_tr_b16 (within a 16-lane group, result lane i
//     takes element i%4 of the 8 bytes addressed by lane 4j + i/4 as its element
//     j, so lanes 4j..4j+3 pointing at row k0 + j, columns 4m.. deliver columns
//     0..15 of rows k0..k0+3 transposed);
//   B operand (A^T[k, m]): 8 consecutive k of row m of the A slice, one 16-byte
//     LDS read.
// LDS layouts: the A slice keeps rows of 128 bytes (two per 256 bytes) with
// 16-byte chunk c of row r at c ^ ((r / 2) % 8); the B slice keeps
// rows of 128 NW bytes with chunk c of row r at c ^ 4 (r % 4); both make the
// operand reads bank-conflict free.  Buffer descriptors end with the matrices,
// so rows past M (A) or K (B) arrive as zeros; in the last K slice, A chunks past
// K are given an out-of-range offset and arrive as zeros too (so the garbage of
// the next row never meets a zero of B: 0 * Inf would be NaN).  Output tiles go
// to XCDs in 4 x 8 groups (consecutive block ids run round-robin over the 8
// XCDs), so the blocks an XCD runs at once share their A and B panels in its L2.
// Requirements of the MFMA path: N % 8 == 0, K % 8 == 0, 16-byte aligned
// buffers, 256 * K * 2 and BK * N * 2 below 2^31; other shapes take the generic
// kernel (one thread per output, f32 accumulation in index order).
//
// f32: small outputs of moderate depth take the small kernel (32 x 32 or 16 x 16
// tiles, K split over the 8 waves of each block on the f32 MFMA); other shapes with K
// and N multiples of 4 and 16-byte aligned buffers the f32 MFMA kernel (128 x 128
// tiles, v_mfma_f32_32x32x2_f32, K split across blocks for grids of fewer tiles than
// CUs); the rest a VALU kernel (64 x 64 tile per 256-thread block, 16-deep K slices in
// LDS, 4 x 4 register micro-tile, f32 FMA; K split across blocks for small grids).
// Split K always sums the f32 partials in chunk order.  f64: one thread per output,
// f64 sum in index order (matmulFloat64Scalar, device/cpu/matmul/select_generic.go:39-...).
#include "common.hpp"
#include <algorithm>
#include <atomic>
#include <cstdint>
#include <mutex>
#include <type_traits>
#include <vector>

namespace puter {

// ------------------------------------------------------------------- f32 --
constexpr int kTile = 64, kDepth = 16;

// Block (x, y, z) computes output tile (y, x) over K range [z kc, (z + 1) kc) (kc a
// multiple of kDepth); with ws set it stores its partial tile to ws[z] instead of
// the result (split K for grids too small to fill the GPU).
__global__ __launch_bounds__(256) void matmul_f32_kernel(float *__restrict__ out,
                                                         const float *__restrict__ A,
                                                         const float *__restrict__ B,
                                                         int64_t M, int64_t K, int64_t N,
                                                         float *__restrict__ ws, int64_t kc) {
    __shared__ float As[kDepth][kTile + 4];
    __shared__ float Bs[kDepth][kTile + 4];
    const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
    const int64_t row0 = (int64_t)blockIdx.y * kTile, col0 = (int64_t)blockIdx.x * kTile;
    const int64_t kbeg = (int64_t)blockIdx.z * kc, kend = std::min(K, kbeg + kc);
    float acc[4][4] = {};
    for (int64_t k0 = kbeg; k0 < kend; k0 += kDepth) {
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
            if (r < M && c < N) {
                if (ws) ws[((int64_t)blockIdx.z * M + r) * N + c] = acc[i][j];
                else out[r * N + c] = acc[i][j];
            }
        }
}

// f32, small outputs: one 512-thread block (8 waves) per TM x TM output tile
// (TM = 32 or 16), the 8 waves splitting K into 8 runs of kw (a multiple of 64)
// and summing theirs on the f32 MFMA: TM = 32 on v_mfma_f32_32x32x2_f32 (lane l:
// row / column l % 32; in step i of a 64-deep chunk k0, half h = l / 32 takes
// k = k0 + 32h + i), TM = 16 on v_mfma_f32_16x16x4_f32 (row / column l % 16;
// quarter q = l / 16 takes k = k0 + 16q + i).  A lane's A values are thus
// consecutive floats of its row and each B row is read by TM lanes at once.  The
// 8 partial tiles meet in LDS and are added in wave order.  One launch, no
// partials in global memory: the cross-block split below spends as long on
// writing and summing partials as on the products at these sizes.  16 x 16 tiles
// spread a small output over four times the CUs (128x512x512: 7.4 -> 4.1 us with
// them) but re-read the operands more (256x1024x1024: 13.2 against 16.0 us), so
// they serve outputs of fewer than 256 32 x 32 tiles.
// VEC: A is 16-byte aligned and K % 4 == 0 (A rows read as float4).
typedef float sm_f32x16 __attribute__((ext_vector_type(16)));
typedef float sm_f32x4 __attribute__((ext_vector_type(4)));
constexpr int kSmallWaves = 8;

template <int TM, bool VEC>
__global__ __launch_bounds__(512) void matmul_f32_small_kernel(float *__restrict__ out, const float *__restrict__ A,
                                                               const float *__restrict__ B, int64_t M, int64_t K,
                                                               int64_t N, int64_t kw) {
    constexpr int KL = 64 / (64 / TM);   // k's per lane per 64-deep chunk: 32 (TM 32), 16 (TM 16)
    using Acc = typename std::conditional<TM == 32, sm_f32x16, sm_f32x4>::type;
    __shared__ float part[kSmallWaves][TM][TM + 1];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane % TM, h = lane / TM;
    const int64_t row = (int64_t)blockIdx.y * TM + r, col = (int64_t)blockIdx.x * TM + r;
    const bool rok = row < M, cok = col < N;
    const int64_t kb = (int64_t)wave * kw, ke = std::min(K, kb + kw);
    const float *arow = A + (rok ? row : 0) * K;
    Acc acc = {};
    for (int64_t k0 = kb; k0 < ke; k0 += 64) {
        const int64_t kh = k0 + KL * h;  // this lane's k's: kh .. kh + KL - 1
        float a[KL], b[KL];
        if constexpr (VEC) {
#pragma unroll
            for (int q = 0; q < KL / 4; ++q) {
                const int64_t k = kh + 4 * q;  // K % 4 == 0: a group is all in or all out
                const float4 v = (rok && k < ke) ? *reinterpret_cast<const float4 *>(arow + k) : make_float4(0, 0, 0, 0);
                a[4 * q] = v.x;
                a[4 * q + 1] = v.y;
                a[4 * q + 2] = v.z;
                a[4 * q + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < KL; ++i) a[i] = (rok && kh + i < ke) ? arow[kh + i] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < KL; ++i) b[i] = (cok && kh + i < ke) ? B[(kh + i) * N + col] : 0.0f;
#pragma unroll
        for (int i = 0; i < KL; ++i) {
            if constexpr (TM == 32) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[i], acc, 0, 0, 0);
            else acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[i], acc, 0, 0, 0);
        }
    }
    // accumulator register j of lane l holds column l % TM and row 8(j/4) + 4h + j%4
    // (TM 32) or 4h + j (TM 16)
#pragma unroll
    for (int j = 0; j < (TM == 32 ? 16 : 4); ++j)
        part[wave][TM == 32 ? 8 * (j >> 2) + 4 * h + (j & 3) : 4 * h + j][r] = acc[j];
    __syncthreads();
    for (int o = threadIdx.x; o < TM * TM; o += 512) {
        const int i = o / TM, c = o % TM;
        const int64_t gr = (int64_t)blockIdx.y * TM + i, gc = (int64_t)blockIdx.x * TM + c;
        float t = part[0][i][c];
#pragma unroll
        for (int w = 1; w < kSmallWaves; ++w) t += part[w][i][c];
        if (gr < M && gc < N) out[gr * N + gc] = t;
    }
}

// ------------------------------------------------------- generic / f64 --
template <int DT>
__global__ __launch_bounds__(256) void matmul_generic_kernel(void *__restrict__ out, const void *__restrict__ A,
                                                             const void *__restrict__ B, int64_t M, int64_t K,
                                                             int64_t N) {
    for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < M * N; idx += (int64_t)gridDim.x * 256) {
        const int64_t r = idx / N, c = idx - r * N;
        if constexpr (DT == PUTER_F64) {
            const double *a = static_cast<const double *>(A) + r * K;
            const double *b = static_cast<const double *>(B) + c;
            double s = 0.0;
            for (int64_t i = 0; i < K; ++i) s += a[i] * b[i * N];
            static_cast<double *>(out)[idx] = s;
        } else {
            using T = typename Elem<DT>::T;
            const T *a = static_cast<const T *>(A) + r * K;
            const T *b = static_cast<const T *>(B) + c;
            float s = 0.0f;
            for (int64_t i = 0; i < K; ++i) s += Elem<DT>::load(a[i]) * Elem<DT>::load(b[i * N]);
            static_cast<T *>(out)[idx] = Elem<DT>::store(s);
        }
    }
}

__global__ __launch_bounds__(256) void matmul_zero_kernel(uint16_t *out, int64_t halves) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < halves; i += (int64_t)gridDim.x * 256) out[i] = 0;
}

static unsigned generic_blocks(int64_t n) { return (unsigned)std::min<int64_t>((n + 255) / 256, 65536); }

// ------------------------------------------------------------------ MFMA --
namespace mm {
constexpr int BUF_WORD3 = 0x00020000; // raw buffer, dword access
constexpr int OOB = 0x7FFFFFF0;       // an offset past every descriptor's range
}  // namespace mm

typedef __bf16 mm_bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 mm_f16x8 __attribute__((ext_vector_type(8)));
typedef short mm_i16x4 __attribute__((ext_vector_type(4)));
typedef float mm_f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int mm_u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void mm_lds_void;
typedef __attribute__((address_space(3))) mm_i16x4 mm_lds_i16x4;

struct MmArgs {
    const uint16_t *a, *b;
    uint16_t *c;
    int M, N, K;
    int tiles_m, tiles_n, groups_m;  // groups_m: 4-tile groups along M
};

template <int DT>
__device__ __forceinline__ mm_f32x16 mm_mfma(const mm_i16x4 (&a)[2], const uint4 &b, mm_f32x16 acc) {
    const uint4 av = __builtin_bit_cast(uint4, __builtin_shufflevector(a[0], a[1], 0, 1, 2, 3, 4, 5, 6, 7));
    if constexpr (DT == PUTER_BF16)
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(mm_bf16x8, av),
                                                       __builtin_bit_cast(mm_bf16x8, b), acc, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(mm_f16x8, av),
                                                      __builtin_bit_cast(mm_f16x8, b), acc, 0, 0, 0);
}

template <int DT, int NW, int MT, int BK, int S>
__global__ __launch_bounds__(128 * NW, NW == 4 ? 1 : 2) void matmul_mfma_kernel(MmArgs p) {
    using namespace mm;
    constexpr int BM = 64 * MT, BN = 64 * NW;   // 2 waves along M of 32 MT rows, NW along N of 64 columns
    constexpr int WR = 32 * MT;                 // rows per wave
    constexpr int RA = 2 * BK, RB = 2 * BN;            // LDS row bytes of the A and B slices
    constexpr int A_BYTES = BM * RA, B_BYTES = BK * RB;
    constexpr int AC = RA / 16;                         // 16-byte chunks per A row
    constexpr int APW = BM * RA / 1024 / (2 * NW);      // A copies per wave per slice
    constexpr int BPW = BK / 16;                        // B copies per wave per slice
    constexpr int KS = BK / 16;                         // k-steps per slice
    // a ring of S slices in separate arrays, so the compiler can tell the slice being
    // read from the ones being copied (unused ring positions shrink to 16 bytes)
    __shared__ __attribute__((aligned(1024))) char as0[A_BYTES];
    __shared__ __attribute__((aligned(1024))) char as1[A_BYTES];
    __shared__ __attribute__((aligned(1024))) char as2[S > 2 ? A_BYTES : 16];
    __shared__ __attribute__((aligned(1024))) char as3[S > 3 ? A_BYTES : 16];
    __shared__ __attribute__((aligned(1024))) char bs0[B_BYTES];
    __shared__ __attribute__((aligned(1024))) char bs1[B_BYTES];
    __shared__ __attribute__((aligned(1024))) char bs2[S > 2 ? B_BYTES : 16];
    __shared__ __attribute__((aligned(1024))) char bs3[S > 3 ? B_BYTES : 16];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, g = lane >> 5;
    const int wm = wave / NW, wn = wave % NW;

    // block -> output tile: XCD x runs the 4 x 8 tile groups x, x + 8, ...
    const int id = blockIdx.x;
    const int local = id >> 3, grp = (local >> 5) * 8 + (id & 7), w = local & 31;
    const int tm = (grp % p.groups_m) * 4 + (w & 3);
    const int tn = (grp / p.groups_m) * 8 + (w >> 2);
    if (tm >= p.tiles_m || tn >= p.tiles_n) return;
    const int m0 = tm * BM, n0 = tn * BN;
    const int M = p.M, N = p.N, K = p.K;

    // copy offsets (bytes, relative to the slice's descriptor base).  A: each copy
    // moves 1 KB = 1024 / RA rows of AC chunks; B: 1024 / RB rows of RB / 16 chunks
    int aoff[4], achunk[4];
#pragma unroll
    for (int i = 0; i < APW; ++i) {
        const int row = (BM / (2 * NW)) * wave + (1024 / RA) * i + lane / AC;
        achunk[i] = (lane % AC) ^ ((row / (256 / RA)) % AC);
        aoff[i] = row * K * 2 + achunk[i] * 16;
    }
    int boff[4];
#pragma unroll
    for (int i = 0; i < BPW; ++i) {
        const int row = (BK / (2 * NW)) * wave + (1024 / RB) * i + lane / (RB / 16);
        boff[i] = row * N * 2 + (((lane % (RB / 16)) ^ ((row & 3) << 2)) << 4);
    }
    // operand reads: A row 128 wm + 32 mt + l32 at k-step s is chunk 2 s + g (the
    // swizzle depends on l32 only); B rows 16 s + 8 (q / 2) + j (+4 for the second half)
    int ard[4];
    {
        const int sw = (l32 / (256 / RA)) % AC;
#pragma unroll
        for (int s = 0; s < KS; ++s) ard[s] = (WR * wm + l32) * RA + (((2 * s + g) ^ sw) << 4);
    }
    int brd[2];
    {
        const int q = lane >> 4, i = lane & 15, j = i >> 2, m = i & 3;
        const int row = 8 * (q >> 1) + j;
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            const int chunk = (4 * (2 * wn + nt) + 2 * (q & 1) + (m >> 1)) ^ ((row & 3) << 2);
            brd[nt] = row * RB + (chunk << 4) + 8 * (m & 1);
        }
    }

    const int64_t a_rows_bytes = (int64_t)(M - m0) * K * 2;
    auto copy_slice = [&](int k0, char *as, char *bs) __attribute__((always_inline)) {
        const int64_t abase = (int64_t)m0 * K + k0;
        const int64_t arange = std::min<int64_t>(a_rows_bytes - (int64_t)k0 * 2, OOB);
        const __amdgpu_buffer_rsrc_t ad = __builtin_amdgcn_make_buffer_rsrc(
            (void *)(p.a + abase), (short)0, (int)arange, BUF_WORD3);
        const int64_t bbase = (int64_t)k0 * N + n0;
        const int64_t brange = std::min<int64_t>(((int64_t)K * N - bbase) * 2, OOB);
        const __amdgpu_buffer_rsrc_t bd = __builtin_amdgcn_make_buffer_rsrc(
            (void *)(p.b + bbase), (short)0, (int)brange, BUF_WORD3);
        const bool tail = k0 + BK > K;
        // (constant trip counts: a loop bound that depends on the template arguments
        // loses the kernel's host stub)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (i < APW) {
                const int off = (tail && k0 + 8 * achunk[i] >= K) ? OOB : aoff[i];
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    ad, (mm_lds_void *)(as + ((BM / (2 * NW)) * wave + (1024 / RA) * i) * RA), 16, off, 0, 0, 0);
            }
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (i < BPW)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    bd, (mm_lds_void *)(bs + ((BK / (2 * NW)) * wave + (1024 / RB) * i) * RB), 16, boff[i], 0, 0, 0);
    };

    mm_f32x16 acc[MT][2];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) acc[mt][nt] = (mm_f32x16){};

    auto compute = [&](const char *as, const char *bs) __attribute__((always_inline)) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            if (s >= KS) break;
            mm_i16x4 bt[2][2];
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                const char *bp = bs + brd[nt] + s * 16 * RB;
                bt[nt][0] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((mm_lds_i16x4 *)bp);
                bt[nt][1] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((mm_lds_i16x4 *)(bp + 4 * RB));
            }
            uint4 af[MT];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) af[mt] = *reinterpret_cast<const uint4 *>(as + ard[s] + mt * 32 * RA);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) acc[mt][nt] = mm_mfma<DT>(bt[nt], af[mt], acc[mt][nt]);
        }
    };

    const int nk = (K + BK - 1) / BK;
    char *const abuf[4] = {as0, as1, as2, as3};
    char *const bbuf[4] = {bs0, bs1, bs2, bs3};
    // prologue: slices 0 .. S-2 in flight, slice 0 landed
#pragma unroll
    for (int i = 0; i < S - 1; ++i)
        if (i < nk) copy_slice(i * BK, abuf[i], bbuf[i]);
    if (S == 2 || nk < 2) __builtin_amdgcn_s_waitcnt(0x0F70);
    else if (S == 3) __builtin_amdgcn_s_waitcnt(0x0F70 | (APW + BPW));            // vmcnt(one slice)
    else if (nk < 3) __builtin_amdgcn_s_waitcnt(0x0F70 | (APW + BPW));
    else __builtin_amdgcn_s_waitcnt(0x0F70 | (2 * (APW + BPW)));
    __syncthreads();
    // slice kt: issue slice kt + S - 1 into the buffer slice kt - 1 used, compute kt,
    // wait for slice kt + 1
    auto slice = [&](int kt, int pos) __attribute__((always_inline)) {
        const int nxt = kt + S - 1;
        if (nxt < nk) copy_slice(nxt * BK, abuf[(pos + S - 1) % S], bbuf[(pos + S - 1) % S]);
        // keep the copies ahead of the compute: left alone, the scheduler sinks them
        // to the end of the slice, right before the wait, exposing their latency
        __builtin_amdgcn_sched_barrier(0);
        compute(abuf[pos], bbuf[pos]);
        const int pending = std::min(nk - 1, nxt) - (kt + 1);   // slices after kt + 1 in flight
        if (S == 2 || pending <= 0) __builtin_amdgcn_s_waitcnt(0x0F70);
        else if (pending == 1) __builtin_amdgcn_s_waitcnt(0x0F70 | (APW + BPW));
        else __builtin_amdgcn_s_waitcnt(0x0F70 | (2 * (APW + BPW)));
        __syncthreads();
    };
    int kt = 0;
    for (; kt + S <= nk; kt += S) {
#pragma unroll
        for (int i = 0; i < S; ++i) slice(kt + i, i);
    }
#pragma unroll
    for (int i = 0; i < S; ++i)
        if (kt + i < nk) slice(kt + i, i);

    // Epilogue.  Lane holds C[m0 + WR wm + 32 mt + l32][n0 + 64 wn + 32 nt + 8 (r/4) +
    // 4 g + r%4]: stored straight from the accumulators, each store instruction would
    // write 16 bytes into each of 32 rows.  Instead the wave parks its WR x 64 block,
    // narrowed, in LDS (the slice buffers are free after the last slice's barrier) and
    // stores it back as 8 whole 128-byte row pieces per instruction, non-temporal (C is
    // not re-read by this kernel): +2 to +7% on 8192^3, 8192 x 4096 x 14336 and 4096^3.
    // The wave owns HW 8 KB halves of the ring (64 rows of 128 bytes each: halves
    // HW w .. HW w + HW - 1, counted through the A buffers, then the B buffers); row r
    // keeps its 16-byte chunk c (8 columns) at c ^ (r / 2 % 8), so 16 consecutive rows
    // (r % 2 picking the half of the 256-byte bank line) and each row's 8 chunks fall
    // on distinct banks.  Measured: 128 bank-conflict cycles per wave and tile (0 in
    // the main loop), the same under c ^ (r % 8) and with the 8-byte halves also
    // swizzled, so not this layout's; about 0.03% of a tile's time.
    {
        constexpr int HW = MT / 2, HA = A_BYTES / 8192, HB = B_BYTES / 8192;
        static_assert(S * (HA + HB) >= 2 * NW * HW, "the ring holds every wave's block");
        char *const bufs[8] = {as0, as1, as2, as3, bs0, bs1, bs2, bs3};
        auto half_region = [&](int j) __attribute__((always_inline)) -> char * {
            char *r = as0;
            int base = 0;
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                if ((q & 3) >= S) continue;
                const int h = q < 4 ? HA : HB;
                if (j >= base && j < base + h) r = bufs[q] + (j - base) * 8192;
                base += h;
            }
            return r;
        };
        char *hs[HW];
#pragma unroll
        for (int hf = 0; hf < HW; ++hf) hs[hf] = half_region(HW * wave + hf);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            char *const hb = hs[mt >> 1] + (32 * (mt & 1) + l32) * 128;
#pragma unroll
            for (int nt = 0; nt < 2; ++nt)
#pragma unroll
                for (int rb = 0; rb < 4; ++rb) {
                    uint32_t h[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) h[i] = Elem<DT>::store(acc[mt][nt][4 * rb + i]);
                    const int chunk = (4 * nt + rb) ^ ((l32 >> 1) & 7);
                    *reinterpret_cast<uint2 *>(hb + chunk * 16 + 8 * g) =
                        make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
                }
        }
        __builtin_amdgcn_wave_barrier();   // the wave's rows are in LDS before other lanes read them
        // lane: row 8 i + lane / 8 of the block, columns 8 (lane % 8) .. +7
        const int r8 = lane >> 3, c8 = lane & 7;
        const int col = n0 + 64 * wn + 8 * c8;
#pragma unroll
        for (int i = 0; i < WR / 8; ++i) {
            const int rr = 8 * (i & 7) + r8;   // row inside the half
            const mm_u32x4 v = *reinterpret_cast<const mm_u32x4 *>(hs[i >> 3] + rr * 128 + ((c8 ^ ((rr >> 1) & 7)) << 4));
            const int row = m0 + WR * wm + 8 * i + r8;
            if (row < M && col < N)   // N % 8 == 0: a chunk is wholly inside or outside
                __builtin_nontemporal_store(v, reinterpret_cast<mm_u32x4 *>(p.c + (int64_t)row * N + col));
        }
    }
}

// Launches the MFMA kernel with NW waves along N and MT accumulator blocks of 32
// rows per wave (256 x 256 tiles: NW = 4, MT = 4; 128 x 128: NW = 2, MT = 2), 64-deep
// slices double buffered; returns 1 when the shape does not fit it.
template <int DT, int NW, int MT>
static int launch_mfma(void *out, const void *left, const void *right, int64_t M, int64_t K, int64_t N,
                       hipStream_t s) {
    constexpr int BK = 64, S = 2;
    constexpr int BM = 64 * MT;
    if (256 * K * 2 >= mm::OOB || BK * N * 2 >= mm::OOB || M > 0x3FFFFFFF || N > 0x3FFFFFFF) return 1;
    MmArgs p;
    p.a = static_cast<const uint16_t *>(left);
    p.b = static_cast<const uint16_t *>(right);
    p.c = static_cast<uint16_t *>(out);
    p.M = (int)M; p.N = (int)N; p.K = (int)K;
    p.tiles_m = (int)((M + BM - 1) / BM);
    p.tiles_n = (int)((N + 64 * NW - 1) / (64 * NW));
    p.groups_m = (p.tiles_m + 3) / 4;
    const int64_t groups = (int64_t)p.groups_m * ((p.tiles_n + 7) / 8);
    const int64_t blocks = (groups + 7) / 8 * 8 * 32;
    if (blocks > 0x7FFFFFFF) return 1;
    matmul_mfma_kernel<DT, NW, MT, BK, S><<<(unsigned)blocks, 128 * NW, 0, s>>>(p);
    return 0;
}

// ---------------------------------------------------------- f32 MFMA --
// Large f32 outputs on v_mfma_f32_32x32x2_f32 (exact f32 products, f32 sums).  A
// 256-thread block (4 waves, 2 x 2) computes a 128 x 128 tile, K advancing 32 at a
// time through LDS (double buffered; slices copied HBM -> LDS by buffer_load ... lds),
// two blocks per CU.  Wave (wm, wn) owns rows 64 wm .. +63 and columns 64 wn .. +63
// as 2 x 2 accumulators; a lane's accumulator holds C[8 (r/4) + 4 h + r%4][lane % 32]
// of its 32 x 32 block (h = lane / 32).  k order: MFMA step s (0..15) of a slice
// gives half h of the wave k = 8 (s / 4) + 4 h + s % 4 (an MFMA may pair its two k's
// in any order, as long as A and B agree), so a lane's A operands for four steps are
// one 16-byte run of its row.  LDS layouts: the A slice keeps rows of 32 floats (128
// bytes) with 16-byte chunk c of row r at c ^ (r / 2 % 8), so the 16 rows an LDS
// cycle serves fall on distinct banks; the B slice keeps rows of 128 floats (512
// bytes) with chunk c of row k at c ^ 8 (k / 4 % 2), so the two half-waves (rows k
// and k + 4, one float per lane) read opposite halves of the bank line.  Rows past
// M or K arrive as zeros through the buffer ranges, and in the last slice A chunks
// past K as well (the next row's values must not meet B's zero rows: 0 * Inf would
// be NaN); columns past N are computed from whatever follows and never stored.
// Requirements: K % 4 == 0, N % 4 == 0, 16-byte aligned buffers.
namespace mf {
constexpr int BM = 128, BN = 128, BK = 32;
constexpr int RA = BK * 4, RB = BN * 4;              // LDS row bytes: 128, 512
constexpr int A_BYTES = BM * RA, B_BYTES = BK * RB;  // 16 KB each
}  // namespace mf

struct MfArgs {
    const float *a, *b;
    float *c;
    float *ws;  // split K: [chunks][M][N] partials (chunk = blockIdx.y), or null
    int M, N, K;
    int kc;     // K per chunk (a multiple of 32; K when unsplit)
    int tiles_m, tiles_n, groups_m;
    int grouped;  // XCD-grouped tile order (else block x = tile, row-major)
};

typedef float mf_f32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256, 2) void matmul_f32_mfma_kernel(MfArgs p) {
    using namespace mf;
    using mm::OOB;
    using mm::BUF_WORD3;
    __shared__ __attribute__((aligned(1024))) char as0[A_BYTES];
    __shared__ __attribute__((aligned(1024))) char as1[A_BYTES];
    __shared__ __attribute__((aligned(1024))) char bs0[B_BYTES];
    __shared__ __attribute__((aligned(1024))) char bs1[B_BYTES];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, h = lane >> 5;
    const int wm = wave >> 1, wn = wave & 1;

    // block -> output tile.  Grouped: XCD x runs the 4 x 8 tile groups x, x + 8, ...
    // (as the 16-bit kernel), so the blocks an XCD runs at once share A and B panels in
    // its L2.  Grids of fewer tiles than CUs (split K) number the tiles plainly: the
    // grouped order would put a grid of one group on a single XCD (32 x 8192 x 1024,
    // 8 tiles in 16 chunks: 497 us)
    const int id = blockIdx.x;
    int tm, tn;
    if (p.grouped) {
        const int local = id >> 3, grp = (local >> 5) * 8 + (id & 7), w = local & 31;
        tm = (grp % p.groups_m) * 4 + (w & 3);
        tn = (grp / p.groups_m) * 8 + (w >> 2);
        if (tm >= p.tiles_m || tn >= p.tiles_n) return;
    } else {
        tm = id / p.tiles_n;
        tn = id - tm * p.tiles_n;
    }
    const int m0 = tm * BM, n0 = tn * BN;
    const int M = p.M, N = p.N, K = p.K;
    const int kb = blockIdx.y * p.kc, ke = min(K, kb + p.kc);   // this block's K range

    // copy offsets (bytes from the slice's descriptor base).  A: copy i of wave w
    // fills rows 32 w + 8 i .. +7 (lane: row + lane / 8, LDS chunk lane % 8, holding
    // the row's chunk (lane % 8) ^ swizzle); B: rows 8 w + 2 i, +1 (lane: row + lane
    // / 32, LDS chunk lane % 32)
    int aoff[4], achunk[4], boff[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int ra = 32 * wave + 8 * i + (lane >> 3);
        achunk[i] = (lane & 7) ^ ((ra >> 1) & 7);
        aoff[i] = ra * K * 4 + achunk[i] * 16;
        const int rb = 8 * wave + 2 * i + (lane >> 5);
        boff[i] = rb * N * 4 + (((lane & 31) ^ (8 * ((rb >> 2) & 1))) << 4);
    }
    // operand reads: A row 64 wm + 32 mt + l32, 4-step group g at chunk (2 g + h) ^
    // swizzle; B column 64 wn + 32 nt + l32 of row k, stored at column ^ 32 h (k / 4 % 2
    // = h for every k a half-wave reads)
    const int asw = (l32 >> 1) & 7;
    int ard[2], brd[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) ard[mt] = (64 * wm + 32 * mt + l32) * RA;
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) brd[nt] = (((64 * wn + 32 * nt + l32) ^ (32 * h)) << 2) + 4 * h * RB;

    const int64_t a_rows_bytes = (int64_t)(M - m0) * K * 4;
    auto copy_slice = [&](int k0, char *as, char *bs) __attribute__((always_inline)) {
        const int64_t abase = (int64_t)m0 * K + k0;
        const int64_t arange = std::min<int64_t>(a_rows_bytes - (int64_t)k0 * 4, OOB);
        const __amdgpu_buffer_rsrc_t ad =
            __builtin_amdgcn_make_buffer_rsrc((void *)(p.a + abase), (short)0, (int)arange, BUF_WORD3);
        const int64_t bbase = (int64_t)k0 * N + n0;
        const int64_t brange = std::min<int64_t>(((int64_t)K * N - bbase) * 4, OOB);
        const __amdgpu_buffer_rsrc_t bd =
            __builtin_amdgcn_make_buffer_rsrc((void *)(p.b + bbase), (short)0, (int)brange, BUF_WORD3);
        const bool tail = k0 + BK > K;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int off = (tail && k0 + 4 * achunk[i] >= K) ? OOB : aoff[i];
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ad, (mm_lds_void *)(as + (32 * wave + 8 * i) * RA), 16, off, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(bd, (mm_lds_void *)(bs + (8 * wave + 2 * i) * RB), 16, boff[i], 0, 0, 0);
    };

    mm_f32x16 acc[2][2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) acc[mt][nt] = (mm_f32x16){};

    auto compute = [&](const char *as, const char *bs) __attribute__((always_inline)) {
#pragma unroll
        for (int g = 0; g < BK / 8; ++g) {
            mf_f32x4 av[2];
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
                av[mt] = *reinterpret_cast<const mf_f32x4 *>(as + ard[mt] + (((2 * g + h) ^ asw) << 4));
            float bv[2][4];
#pragma unroll
            for (int nt = 0; nt < 2; ++nt)
#pragma unroll
                for (int s = 0; s < 4; ++s)
                    bv[nt][s] = *reinterpret_cast<const float *>(bs + brd[nt] + (8 * g + s) * RB);
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                    for (int nt = 0; nt < 2; ++nt)
                        acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[mt][s], bv[nt][s], acc[mt][nt], 0, 0, 0);
        }
    };

    const int nk = (ke - kb + BK - 1) / BK;
    copy_slice(kb, as0, bs0);
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
    __syncthreads();
    auto slice = [&](int kt, char *ac, char *bc, char *an, char *bn) __attribute__((always_inline)) {
        if (kt + 1 < nk) copy_slice(kb + (kt + 1) * BK, an, bn);
        __builtin_amdgcn_sched_barrier(0);   // keep the copies ahead of the compute
        compute(ac, bc);
        __builtin_amdgcn_s_waitcnt(0x0F70);
        __syncthreads();
    };
    int kt = 0;
    for (; kt + 1 < nk; kt += 2) {
        slice(kt, as0, bs0, as1, bs1);
        slice(kt + 1, as1, bs1, as0, bs0);
    }
    if (kt < nk) slice(kt, as0, bs0, as1, bs1);

    // lane writes C[row][n0 + 64 wn + 32 nt + l32]: 32 consecutive floats of a row
    // per half-wave and register (non-temporal for the result; the partials of a
    // split stay cacheable for the reduce that follows)
    const int col0 = n0 + 64 * wn + l32;
    float *const cbase = p.ws ? p.ws + (int64_t)blockIdx.y * M * N : p.c;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = m0 + 64 * wm + 32 * mt + 8 * (r >> 2) + 4 * h + (r & 3);
            if (row >= M) continue;
            float *crow = cbase + (int64_t)row * N;
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                if (col0 + 32 * nt >= N) continue;
                if (p.ws) crow[col0 + 32 * nt] = acc[mt][nt][r];
                else __builtin_nontemporal_store(acc[mt][nt][r], crow + col0 + 32 * nt);
            }
        }
}

// ------------------------------------------------ small outputs, 16-bit --
// The 16-bit counterpart of matmul_f32_small_kernel: one 512-thread block per
// TM x TM output tile, its 8 waves splitting K into runs of kw (a multiple of
// 64) on v_mfma_f32_32x32x16 (TM 32: in a 64-deep chunk k0, half h = lane / 32
// takes k0 + 32h .. +31, MFMA q of the chunk k0 + 32h + 8q .. +7) or
// v_mfma_f32_16x16x32 (TM 16: quarter h = lane / 16 takes k0 + 16h .. +15, MFMA q
// k0 + 16h + 8q .. +7), so a lane's A values are 16-byte runs of its row and each
// B row is read by TM lanes at once; the 8 partial tiles meet in LDS, are added
// in wave order and rounded once.  Requires K % 8 == 0 and A 16-byte aligned.
template <int DT, int TM>
__global__ __launch_bounds__(512) void matmul16_small_kernel(uint16_t *__restrict__ out, const uint16_t *__restrict__ A,
                                                             const uint16_t *__restrict__ B, int64_t M, int64_t K,
                                                             int64_t N, int64_t kw) {
    constexpr int KL = 64 / (64 / TM), NQ = KL / 8;   // k's per lane per chunk, MFMAs per chunk
    using Acc = typename std::conditional<TM == 32, mm_f32x16, sm_f32x4>::type;
    __shared__ float part[kSmallWaves][TM][TM + 1];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane % TM, h = lane / TM;
    const int64_t row = (int64_t)blockIdx.y * TM + r, col = (int64_t)blockIdx.x * TM + r;
    const bool rok = row < M, cok = col < N;
    const int64_t kb = (int64_t)wave * kw, ke = std::min(K, kb + kw);
    const uint16_t *arow = A + (rok ? row : 0) * K;
    Acc acc = {};
    for (int64_t k0 = kb; k0 < ke; k0 += 64) {
        const int64_t kh = k0 + KL * h;
        uint4 a[NQ];
#pragma unroll
        for (int q = 0; q < NQ; ++q) {  // K % 8 == 0: an 8-run is all in or all out
            const int64_t k = kh + 8 * q;
            a[q] = (rok && k < ke) ? *reinterpret_cast<const uint4 *>(arow + k) : make_uint4(0, 0, 0, 0);
        }
        uint32_t bv[KL];
#pragma unroll
        for (int i = 0; i < KL; ++i) bv[i] = (cok && kh + i < ke) ? B[(kh + i) * N + col] : 0u;
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            const uint4 b = make_uint4(bv[8 * q] | (bv[8 * q + 1] << 16), bv[8 * q + 2] | (bv[8 * q + 3] << 16),
                                       bv[8 * q + 4] | (bv[8 * q + 5] << 16), bv[8 * q + 6] | (bv[8 * q + 7] << 16));
            if constexpr (TM == 32) {
                if constexpr (DT == PUTER_BF16)
                    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(mm_bf16x8, a[q]),
                                                                  __builtin_bit_cast(mm_bf16x8, b), acc, 0, 0, 0);
                else
                    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(mm_f16x8, a[q]),
                                                                 __builtin_bit_cast(mm_f16x8, b), acc, 0, 0, 0);
            } else {
                if constexpr (DT == PUTER_BF16)
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(mm_bf16x8, a[q]),
                                                                  __builtin_bit_cast(mm_bf16x8, b), acc, 0, 0, 0);
                else
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(mm_f16x8, a[q]),
                                                                 __builtin_bit_cast(mm_f16x8, b), acc, 0, 0, 0);
            }
        }
    }
    // accumulator register j of lane l holds column l % TM and row 8(j/4) + 4h + j%4
    // (TM 32) or 4h + j (TM 16)
#pragma unroll
    for (int j = 0; j < (TM == 32 ? 16 : 4); ++j)
        part[wave][TM == 32 ? 8 * (j >> 2) + 4 * h + (j & 3) : 4 * h + j][r] = acc[j];
    __syncthreads();
    for (int o = threadIdx.x; o < TM * TM; o += 512) {
        const int i = o / TM, c = o % TM;
        const int64_t gr = (int64_t)blockIdx.y * TM + i, gc = (int64_t)blockIdx.x * TM + c;
        float t = part[0][i][c];
#pragma unroll
        for (int w = 1; w < kSmallWaves; ++w) t += part[w][i][c];
        if (gr < M && gc < N) out[gr * N + gc] = Elem<DT>::store(t);
    }
}

// ------------------------------------ skinny (M <= 512) and small outputs --
// Decode-time projections (a few rows against a large weight matrix) are bound by
// streaming `right` once; the kernel also serves outputs too small to fill the
// CUs with 128 x 128 tiles (see launch_matmul16).  A 256-thread block computes a 64 x 128 tile over one
// chunk of K (split K, at most one wave of 512 blocks when split), copying 64-deep slices HBM -> LDS on a
// 3-stage ring (two slices in flight per block, two blocks per CU); wave w owns
// columns 32 w .. +31 as 2 accumulators (rows 0..31, 32..63).  LDS layouts: A rows
// of 128 bytes, chunk c of row r at c ^ (r/2 % 8); B rows of 256 bytes, chunk c at
// c ^ 4 (r % 4).  With more than one chunk, each block writes its f32 partial tile to
// a scratch buffer (the library's, one per device) and matmul_splitk_reduce_kernel
// sums the chunks in order (so the result does not depend on scheduling) and
// rounds once.
namespace sk {
constexpr int BM = 64, BN = 128, BK = 64;
constexpr int RA = 2 * BK, RB = 2 * BN;
constexpr int A_BYTES = BM * RA, B_BYTES = BK * RB;  // 8 KB, 16 KB
constexpr int CPW = 6;                               // copies per wave per slice (2 A + 4 B)
}  // namespace sk

struct SkArgs {
    const uint16_t *a, *b;
    uint16_t *c;
    float *ws;  // [chunks][M][N] partials, or null: store the result
    int M, N, K, kc;
};

template <int DT>
__global__ __launch_bounds__(256, 2) void matmul_skinny_kernel(SkArgs p) {
    using namespace sk;
    using mm::OOB;
    using mm::BUF_WORD3;
    __shared__ __attribute__((aligned(1024))) char a0s[A_BYTES];
    __shared__ __attribute__((aligned(1024))) char a1s[A_BYTES];
    __shared__ __attribute__((aligned(1024))) char a2s[A_BYTES];
    __shared__ __attribute__((aligned(1024))) char b0s[B_BYTES];
    __shared__ __attribute__((aligned(1024))) char b1s[B_BYTES];
    __shared__ __attribute__((aligned(1024))) char b2s[B_BYTES];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, g = lane >> 5;
    const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM, kb = blockIdx.z * p.kc;
    const int M = p.M, N = p.N, K = p.K;
    const int nk = (min(K, kb + p.kc) - kb + BK - 1) / BK;

    int aoff[2], achunk[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {  // A: wave copies rows 16 w .. +15, 8 rows per copy
        const int row = 16 * wave + 8 * i + (lane >> 3);
        achunk[i] = (lane & 7) ^ ((row >> 1) & 7);
        aoff[i] = row * K * 2 + achunk[i] * 16;
    }
    int boff[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // B: wave copies rows 16 w .. +15, 4 rows per copy
        const int row = 16 * wave + 4 * i + (lane >> 4);
        boff[i] = row * N * 2 + (((lane & 15) ^ ((row & 3) << 2)) << 4);
    }
    int ard[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) ard[s] = l32 * RA + (((2 * s + g) ^ ((l32 >> 1) & 7)) << 4);
    int brd;
    {
        const int q = lane >> 4, i = lane & 15, j = i >> 2, m = i & 3;
        const int row = 8 * (q >> 1) + j;
        brd = row * RB + (((4 * wave + 2 * (q & 1) + (m >> 1)) ^ ((row & 3) << 2)) << 4) + 8 * (m & 1);
    }

    const int64_t a_rows_bytes = (int64_t)(M - m0) * K * 2;
    auto copy_slice = [&](int k0, char *as, char *bs) __attribute__((always_inline)) {
        const int64_t abase = (int64_t)m0 * K + k0;
        const int64_t arange = std::min<int64_t>(a_rows_bytes - (int64_t)k0 * 2, OOB);
        const __amdgpu_buffer_rsrc_t ad = __builtin_amdgcn_make_buffer_rsrc(
            (void *)(p.a + abase), (short)0, (int)arange, BUF_WORD3);
        const int64_t bbase = (int64_t)k0 * N + n0;
        const int64_t brange = std::min<int64_t>(((int64_t)K * N - bbase) * 2, OOB);
        const __amdgpu_buffer_rsrc_t bd = __builtin_amdgcn_make_buffer_rsrc(
            (void *)(p.b + bbase), (short)0, (int)brange, BUF_WORD3);
        const bool tail = k0 + BK > K;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int off = (tail && k0 + 8 * achunk[i] >= K) ? OOB : aoff[i];
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ad, (mm_lds_void *)(as + (16 * wave + 8 * i) * RA), 16, off, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(bd, (mm_lds_void *)(bs + (16 * wave + 4 * i) * RB), 16, boff[i], 0, 0, 0);
    };

    mm_f32x16 acc[2] = {(mm_f32x16){}, (mm_f32x16){}};
    auto compute = [&](const char *as, const char *bs) __attribute__((always_inline)) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            mm_i16x4 bt[2];
            bt[0] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((mm_lds_i16x4 *)(bs + brd + s * 16 * RB));
            bt[1] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((mm_lds_i16x4 *)(bs + brd + s * 16 * RB + 4 * RB));
            uint4 af[2];
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) af[mt] = *reinterpret_cast<const uint4 *>(as + ard[s] + mt * 32 * RA);
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) acc[mt] = mm_mfma<DT>(bt, af[mt], acc[mt]);
        }
    };

    // ring of 3: slice kt lives in buffer kt % 3; slices kt + 1 and kt + 2 are in flight
    // while kt is computed, and the copy of kt + 2 reuses the buffer kt - 1 finished with
    copy_slice(kb, a0s, b0s);
    if (nk > 1) copy_slice(kb + BK, a1s, b1s);
    if (nk > 1) __builtin_amdgcn_s_waitcnt(0x0F70 | CPW);  // vmcnt(6): slice 0 landed
    else __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
    auto slice = [&](int kt, const char *ac, const char *bc, char *an, char *bn) __attribute__((always_inline)) {
        if (kt + 2 < nk) copy_slice(kb + (kt + 2) * BK, an, bn);
        __builtin_amdgcn_sched_barrier(0);
        compute(ac, bc);
        if (kt + 2 < nk) __builtin_amdgcn_s_waitcnt(0x0F70 | CPW);  // slice kt + 1 landed
        else __builtin_amdgcn_s_waitcnt(0x0F70);
        __syncthreads();
    };
    int kt = 0;
    for (; kt + 3 <= nk; kt += 3) {
        slice(kt, a0s, b0s, a2s, b2s);
        slice(kt + 1, a1s, b1s, a0s, b0s);
        slice(kt + 2, a2s, b2s, a1s, b1s);
    }
    if (kt < nk) slice(kt, a0s, b0s, a2s, b2s);
    if (kt + 1 < nk) slice(kt + 1, a1s, b1s, a0s, b0s);

    // lane holds C[m0 + 32 mt + l32][n0 + 32 wave + 8 (r/4) + 4 g + r%4]
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
        const int row = m0 + 32 * mt + l32;
        if (row >= M) continue;
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
            const int col = n0 + 32 * wave + 8 * rb + 4 * g;
            if (col >= N) continue;
            const mm_f32x16 &v = acc[mt];
            if (p.ws) {
                float *dst = p.ws + ((int64_t)blockIdx.z * M + row) * N + col;
                *reinterpret_cast<float4 *>(dst) = make_float4(v[4 * rb], v[4 * rb + 1], v[4 * rb + 2], v[4 * rb + 3]);
            } else {
                uint32_t h[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) h[i] = Elem<DT>::store(v[4 * rb + i]);
                *reinterpret_cast<uint2 *>(p.c + (int64_t)row * N + col) =
                    make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
            }
        }
    }
}

// out = round(sum over chunks z = 0, 1, ... of ws[z]), 4 outputs per thread
template <int DT>
__global__ __launch_bounds__(256) void matmul_splitk_reduce_kernel(uint16_t *c, const float *ws, int64_t quads,
                                                                   int chunks) {
    const float4 *w4 = reinterpret_cast<const float4 *>(ws);
    for (int64_t v = (int64_t)blockIdx.x * 256 + threadIdx.x; v < quads; v += (int64_t)gridDim.x * 256) {
        float4 t = w4[v];
        for (int z = 1; z < chunks; ++z) {
            const float4 u = w4[(int64_t)z * quads + v];
            t.x += u.x; t.y += u.y; t.z += u.z; t.w += u.w;
        }
        const uint32_t h0 = Elem<DT>::store(t.x), h1 = Elem<DT>::store(t.y);
        const uint32_t h2 = Elem<DT>::store(t.z), h3 = Elem<DT>::store(t.w);
        reinterpret_cast<uint2 *>(c)[v] = make_uint2(h0 | (h1 << 16), h2 | (h3 << 16));
    }
}

// Split-K partials: one scratch buffer per device, kept for the life of the
// process and grown on demand.  A call on another stream than the buffer's last
// user first waits (on the device, hipStreamWaitEvent) for that user's
// completion event, so calls on different streams never overlap on the buffer.
// Nothing waits on the host: a growth frees the old buffer and allocates the new
// one in stream order on the calling stream (hipFreeAsync / hipMallocAsync),
// after the last user's work.  The mutex is held from acquisition until the
// call's launches and event are enqueued.
//
// Under stream capture (a HIP graph being recorded) a call allocates, frees,
// waits on and records nothing: it uses the buffer it finds when that is large
// enough and otherwise fails with PUTER_ERR_INVALID before any launch.  The
// graph keeps the buffer's address, so a buffer a capture has used is never
// freed: a later growth retires it (kept until the process ends) and allocates
// the new one beside it.  Replays of such a graph share the buffer with eager
// calls until that growth; the caller orders them (one stream, or its own
// events), as it orders any two uses of one buffer.
struct SplitScratch {
    std::mutex mu;
    void *ptr = nullptr;
    size_t bytes = 0;
    hipEvent_t done = nullptr;  // recorded after the last call that used ptr
    hipStream_t last = nullptr;
    bool used = false;
    bool pinned = false;        // a captured graph holds ptr
    std::vector<void *> retired;  // pinned buffers replaced by a growth
};
static SplitScratch g_split_scratch[64];

// Whether s is recording a graph (an invalidated capture counts: it must not
// allocate either).
static int stream_capturing(hipStream_t s, bool *capturing) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &st) != hipSuccess)
        return fail(PUTER_ERR_LAUNCH, "scratch: cannot query the stream's capture status");
    *capturing = st != hipStreamCaptureStatusNone;
    return PUTER_OK;
}

static int scratch_acquire(SplitScratch &sc, size_t need, hipStream_t s) {
    if (!sc.done && hipEventCreateWithFlags(&sc.done, hipEventDisableTiming) != hipSuccess)
        return fail(PUTER_ERR_UNAVAILABLE, "matmul: cannot create the split-K event");
    if (sc.used && sc.last != s && hipStreamWaitEvent(s, sc.done, 0) != hipSuccess)
        return fail(PUTER_ERR_LAUNCH, "matmul: cannot order the split-K scratch");
    if (sc.bytes < need) {
        if (sc.ptr && sc.pinned) {
            sc.retired.push_back(sc.ptr);  // a graph may still replay into it
            sc.ptr = nullptr;
            sc.bytes = 0;
            sc.pinned = false;
        } else if (sc.ptr) {
            // s is ordered after the last user (above, or it is that user)
            if (hipFreeAsync(sc.ptr, s) != hipSuccess)
                return fail(PUTER_ERR_LAUNCH, "matmul: cannot release the split-K scratch");
            sc.ptr = nullptr;
            sc.bytes = 0;
        }
        const size_t grown = (need + ((size_t)1 << 20) - 1) & ~(((size_t)1 << 20) - 1);
        if (hipMallocAsync(&sc.ptr, grown, s) != hipSuccess) {
            sc.ptr = nullptr;
            return fail(PUTER_ERR_UNAVAILABLE, "matmul: split-K scratch of %zu bytes unavailable", grown);
        }
        sc.bytes = grown;
    }
    return PUTER_OK;
}

ScratchLease::ScratchLease(size_t bytes, hipStream_t s) : s_(s) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
        status_ = fail(PUTER_ERR_UNAVAILABLE, "scratch: no device");
        return;
    }
    sc_ = &g_split_scratch[dev];
    lock_ = std::unique_lock<std::mutex>(sc_->mu);
    bool capturing = false;
    if ((status_ = stream_capturing(s, &capturing)) != PUTER_OK) return;
    if (capturing) {
        if (sc_->bytes < bytes) {
            status_ = fail(PUTER_ERR_INVALID,
                           "scratch: %zu bytes needed under stream capture, %zu held; the library's scratch "
                           "cannot grow while a graph is captured (make the same call, or a larger one, "
                           "outside the capture first)",
                           bytes, sc_->bytes);
            return;
        }
        sc_->pinned = true;
        captured_ = true;
        ptr_ = sc_->ptr;
        return;
    }
    status_ = scratch_acquire(*sc_, bytes, s);
    if (status_ == PUTER_OK) ptr_ = sc_->ptr;
}

int ScratchLease::finish() {
    if (status_ != PUTER_OK) return status_;
    if (captured_) return PUTER_OK;
    if (hipEventRecord(sc_->done, s_) != hipSuccess) return fail(PUTER_ERR_LAUNCH, "scratch: cannot record the event");
    sc_->last = s_;
    sc_->used = true;
    return PUTER_OK;
}

// Returns 1 when the shape does not fit the skinny kernel.
// ---- the allocation-free Matmul (puter_hip_matmul_noalloc) -----------------
// Its split-K partials live in a file-scope device array (one copy per GPU,
// held until the process ends) instead of the growable scratch.  The array
// holds 16 MiB, the most any split-K launch here can need: at most 512 blocks
// (chunks x tiles) of 64 x 128 f32 partials for the 16-bit formats and for the
// f32 VALU kernel's 64 x 64 tiles; the f32 MFMA kernel's chunk count is capped so
// that its partials (chunks x rows x cols floats) fit it.  Host code never passes the array's name to a kernel (in host code it
// is a stand-in, not a device address): it passes the address
// hipGetSymbolAddress returns, looked up once per device on that device's first
// call.  Every no-alloc call on a GPU shares that GPU's array, so such calls
// must not overlap on one GPU; each call writes every partial it reads, so
// nothing needs clearing between calls.
namespace noalloc {
constexpr size_t kScratchBytes = (size_t)512 * 64 * 128 * sizeof(float);
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];
static std::mutex mu;
static float *ptr[64];  // per device: scratch's device address

static int address(float **out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
        return fail(PUTER_ERR_UNAVAILABLE, "matmul (no-alloc): no device");
    std::lock_guard<std::mutex> g(mu);
    if (!ptr[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(PUTER_ERR_UNAVAILABLE, "matmul (no-alloc): scratch address: %s", hipGetErrorString(e));
        ptr[dev] = static_cast<float *>(p);
    }
    *out = ptr[dev];
    return PUTER_OK;
}
}  // namespace noalloc

// Where a call's split-K partials go: `fixed` (the no-alloc scratch) when set,
// else a lease of the library's growable scratch.
struct PartialsTarget {
    float *fixed = nullptr;
};

// min_depth > 0: chunks of K at least min_depth deep (fewer chunks otherwise).
template <int DT>
static int launch_skinny(void *out, const void *left, const void *right, int64_t M, int64_t K, int64_t N,
                         hipStream_t s, PartialsTarget tgt, int64_t min_depth) {
    if (64 * K * 2 >= mm::OOB || sk::BK * N * 2 >= mm::OOB || N > 0x3FFFFFFF) return 1;
    const int64_t tiles_n = (N + sk::BN - 1) / sk::BN, tiles_m = (M + sk::BM - 1) / sk::BM;
    if (tiles_n > 0x7FFFFFFF) return 1;
    const int64_t slices = (K + sk::BK - 1) / sk::BK;
    // as many chunks as keep the grid within one wave of 512 blocks (2 per CU): a
    // partial second wave would run at a fraction of the bandwidth; at most 8, as
    // the partials written and summed grow with the chunk count (against at most
    // 64: 64x4096x4096 18.1 -> 14.7 us, 32x2048x2048 17.2 -> 8.2, 1x4096x4096
    // 11.0 -> 10.1; 4 lost on 64x14336x4096, 41.4 against 29.0)
    int64_t chunks = std::min<int64_t>(std::max<int64_t>(512 / (tiles_m * tiles_n), 1), slices);
    chunks = std::min<int64_t>(chunks, 8);
    if (min_depth > 0) chunks = std::max<int64_t>(1, std::min<int64_t>(chunks, K / min_depth));
    const int64_t per = (slices + chunks - 1) / chunks;  // slices per chunk
    chunks = (slices + per - 1) / per;
    SkArgs p{static_cast<const uint16_t *>(left), static_cast<const uint16_t *>(right), static_cast<uint16_t *>(out),
             nullptr, (int)M, (int)N, (int)K, (int)(per * sk::BK)};
    const dim3 grid((unsigned)tiles_n, (unsigned)tiles_m, (unsigned)chunks);
    if (chunks == 1) {
        matmul_skinny_kernel<DT><<<grid, 256, 0, s>>>(p);
        return check_launch("matmul skinny");
    }
    const size_t need = (size_t)(chunks * M * N) * sizeof(float);
    const int64_t quads = M * N / 4;
    if (tgt.fixed) {
        if (need > noalloc::kScratchBytes)
            return fail(PUTER_ERR_INVALID, "matmul (no-alloc): split-K partials of %zu bytes exceed the %zu-byte scratch",
                        need, noalloc::kScratchBytes);
        p.ws = tgt.fixed;
        matmul_skinny_kernel<DT><<<grid, 256, 0, s>>>(p);
        matmul_splitk_reduce_kernel<DT><<<(unsigned)std::min<int64_t>((quads + 255) / 256, 4096), 256, 0, s>>>(
            static_cast<uint16_t *>(out), p.ws, quads, (int)chunks);
        return check_launch("matmul split-k");
    }
    ScratchLease lease(need, s);
    if (lease.status()) return lease.status();
    p.ws = static_cast<float *>(lease.ptr());
    matmul_skinny_kernel<DT><<<grid, 256, 0, s>>>(p);
    matmul_splitk_reduce_kernel<DT><<<(unsigned)std::min<int64_t>((quads + 255) / 256, 4096), 256, 0, s>>>(
        static_cast<uint16_t *>(out), p.ws, quads, (int)chunks);
    const int rc = check_launch("matmul split-k");
    const int fin = lease.finish();
    return rc ? rc : fin;
}

// Compute units of the current device, cached per device (256 on MI355X).
int device_cus() {
    static std::atomic<int> cus[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cus[dev].load(std::memory_order_relaxed);
    if (n <= 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

// Tile shape of the MFMA GEMM by wave quantisation: 256 x 256 tiles run one block
// per CU, 128 x 128 tiles two; a full round of the small tiles does half the work
// of a round of the large ones in 0.59 of its time (measured 1100 against 1300
// TFLOP/s on large shapes), so the shape with the smaller rounds x cost wins.  Small
// tiles: 2048^3 351 -> 623 TFLOP/s, 1024 x 4096 x 4096 385 -> 697, 6144 x 4096 x 4096
// 956 -> 1081 (1.5 rounds of large tiles); large: 4096^3 1257 against 1070.
static bool mfma_small_tiles(int64_t M, int64_t N) {
    const int64_t cus = device_cus();
    const int64_t large = ((M + 255) / 256) * ((N + 255) / 256), small = ((M + 127) / 128) * ((N + 127) / 128);
    const int64_t r_large = (large + cus - 1) / cus, r_small = (small + 2 * cus - 1) / (2 * cus);
    return 59 * r_small < 100 * r_large;
}

template <int DT>
static int launch_matmul16(void *out, const void *left, const void *right, int64_t M, int64_t K, int64_t N,
                           hipStream_t s, PartialsTarget tgt) {
    if (N % 8 == 0 && K % 8 == 0 && aligned16(out) && aligned16(left) && aligned16(right)) {
        // small outputs of moderate depth with a small right operand: K split inside
        // each block (as for f32; 128x512x512 7.5 -> 6.3 us, 256x1024x1024 17.5 ->
        // 10.0).  Its B reads are 2-byte gathers, so a few rows against a large
        // weight stay on the skinny kernel (64x4096x4096: 52.7 against 17.5 us), as
        // do shapes under 128 rows (level or slower) and over 256 (512x1024x1024:
        // 18.4 against 16.2)
        const int64_t tiles32 = ((N + 31) / 32) * ((M + 31) / 32);
        const int64_t kw = ((K + kSmallWaves - 1) / kSmallWaves + 63) / 64 * 64;
        const int64_t sk_tiles = ((M + sk::BM - 1) / sk::BM) * ((N + sk::BN - 1) / sk::BN);
        if (M >= 128 && M <= 256 && K * N <= ((int64_t)1 << 22) && sk_tiles < 256 && tiles32 >= 32 && K >= 128 &&
            kw / 64 <= std::max<int64_t>(2, tiles32 / 32)) {
            uint16_t *o = static_cast<uint16_t *>(out);
            const uint16_t *l = static_cast<const uint16_t *>(left), *r = static_cast<const uint16_t *>(right);
            if (tiles32 < 256) {   // 16 x 16 tiles: four times the blocks
                const dim3 g16((unsigned)((N + 15) / 16), (unsigned)((M + 15) / 16));
                matmul16_small_kernel<DT, 16><<<g16, 512, 0, s>>>(o, l, r, M, K, N, kw);
            } else {
                const dim3 g32((unsigned)((N + 31) / 32), (unsigned)((M + 31) / 32));
                matmul16_small_kernel<DT, 32><<<g32, 512, 0, s>>>(o, l, r, M, K, N, kw);
            }
            return check_launch("matmul");
        }
        // Rows <= 512 (decode-step projections) take the split-K kernel; so do more rows
        // when 128 x 128 tiles would not fill one round of two blocks per CU, its 64 x
        // 128 tiles and K chunks (each at least 1024 deep) spreading the work further
        // (same process: 1024 x 8192 x 1024 198 -> 470 TFLOP/s, 768 x 16384 x 1024 148 ->
        // 543, 2048^3 612 -> 651 unsplit; 1024^3 split four ways fell 165 -> 105, hence
        // the depth floor; from one full round up the MFMA kernels win: 4096 x 1024 x
        // 2048 845 against 601)
        const bool few_tiles = ((M + 127) / 128) * ((N + 127) / 128) < 2 * (int64_t)device_cus();
        if (M <= 512 || few_tiles) {
            const int rc = launch_skinny<DT>(out, left, right, M, K, N, s, tgt, M <= 512 ? 0 : 1024);
            if (rc != 1) return rc;
        }
        const int rc = mfma_small_tiles(M, N) ? launch_mfma<DT, 2, 2>(out, left, right, M, K, N, s)
                                              : launch_mfma<DT, 4, 4>(out, left, right, M, K, N, s);
        if (rc == 0) return check_launch("matmul mfma");
    }
    matmul_generic_kernel<DT><<<generic_blocks(M * N), 256, 0, s>>>(out, left, right, M, K, N);
    return check_launch("matmul");
}

}  // namespace puter

using namespace puter;

// out = sum over chunks z = 0, 1, ... of ws[z] (f32)
__global__ __launch_bounds__(256) void matmul_splitk_reduce_f32_kernel(float *c, const float *ws, int64_t n,
                                                                       int chunks) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
        float t = ws[i];
        for (int z = 1; z < chunks; ++z) t += ws[(int64_t)z * n + i];
        c[i] = t;
    }
}

// Launches the f32 MFMA kernel over `chunks` K chunks (f32 partials in the scratch,
// summed in chunk order, when more than one); returns 1 when the shape does not fit it.
static int launch_f32_mfma(float *out, const float *left, const float *right, int64_t M, int64_t K, int64_t N,
                           int64_t chunks, hipStream_t s, PartialsTarget tgt) {
    if (K % 4 || N % 4 || !aligned16(out) || !aligned16(left) || !aligned16(right)) return 1;
    if (128 * K * 4 >= mm::OOB || mf::BK * N * 4 >= mm::OOB || M > 0x3FFFFFFF || N > 0x3FFFFFFF) return 1;
    MfArgs p;
    p.a = left;
    p.b = right;
    p.c = out;
    p.ws = nullptr;
    p.M = (int)M; p.N = (int)N; p.K = (int)K;
    const int64_t slices = (K + mf::BK - 1) / mf::BK;
    const int64_t per = (slices + chunks - 1) / chunks;   // slices per chunk
    chunks = (slices + per - 1) / per;
    p.kc = (int)(per * mf::BK);
    p.tiles_m = (int)((M + mf::BM - 1) / mf::BM);
    p.tiles_n = (int)((N + mf::BN - 1) / mf::BN);
    p.groups_m = (p.tiles_m + 3) / 4;
    const int64_t tiles = (int64_t)p.tiles_m * p.tiles_n;
    const int64_t groups = (int64_t)p.groups_m * ((p.tiles_n + 7) / 8);
    p.grouped = tiles >= device_cus();
    const int64_t blocks = p.grouped ? (groups + 7) / 8 * 8 * 32 : tiles;
    if (blocks > 0x7FFFFFFF) return 1;
    const dim3 grid((unsigned)blocks, (unsigned)chunks);
    if (chunks == 1) {
        matmul_f32_mfma_kernel<<<grid, 256, 0, s>>>(p);
        return check_launch("matmul f32 mfma");
    }
    const size_t need = (size_t)(chunks * M * N) * sizeof(float);
    auto launch = [&](float *ws) {
        p.ws = ws;
        matmul_f32_mfma_kernel<<<grid, 256, 0, s>>>(p);
        matmul_splitk_reduce_f32_kernel<<<(unsigned)std::min<int64_t>((M * N + 255) / 256, 4096), 256, 0, s>>>(
            out, ws, M * N, (int)chunks);
        return check_launch("matmul f32 mfma split-k");
    };
    if (tgt.fixed) {
        if (need > noalloc::kScratchBytes)
            return fail(PUTER_ERR_INVALID, "matmul (no-alloc): split-K partials of %zu bytes exceed the %zu-byte scratch",
                        need, noalloc::kScratchBytes);
        return launch(tgt.fixed);
    }
    ScratchLease lease(need, s);
    if (lease.status()) return lease.status();
    const int rc = launch(static_cast<float *>(lease.ptr()));
    const int fin = lease.finish();
    return rc ? rc : fin;
}

// f32: small outputs of moderate depth take the small kernel; other shapes with K and
// N multiples of 4 and 16-byte aligned buffers the f32 MFMA kernel; the rest the VALU
// kernel (64 x 64 tiles), whose grids of fewer than 256 tiles split K (16-deep steps)
// into as many chunks as keep the grid within 512 blocks, each chunk at least two
// steps deep (one-step chunks spent more time writing and summing partials than
// computing: 128x512x512 18.3 -> 12.9 us), partials in the split-K scratch.
static int launch_matmul_f32(float *out, const float *left, const float *right, int64_t M, int64_t K, int64_t N,
                             hipStream_t s, PartialsTarget tgt) {
    const dim3 grid((unsigned)((N + kTile - 1) / kTile), (unsigned)((M + kTile - 1) / kTile));
    if (grid.y > 65535) return fail(PUTER_ERR_INVALID, "matmul: too many rows");
    const int64_t tiles = (int64_t)grid.x * grid.y, steps = (K + kDepth - 1) / kDepth;
    const int64_t tiles32 = ((N + 31) / 32) * ((M + 31) / 32);
    // small output, moderate depth: one launch splitting K inside each block, used
    // while each wave's 64-deep steps (run one after another) number at most
    // max(2, tiles32 / 32): a longer K over few tiles is faster split across blocks
    // (32x8192x1024: 92 against 54 us)
    const int64_t kw = ((K + kSmallWaves - 1) / kSmallWaves + 63) / 64 * 64;
    if (tiles < 256 && tiles32 >= 32 && K >= 128 && kw / 64 <= std::max<int64_t>(2, tiles32 / 32)) {
        const bool vec = aligned16(left) && K % 4 == 0;
        if (tiles32 < 256) {   // 16 x 16 tiles: four times the blocks
            const dim3 g16((unsigned)((N + 15) / 16), (unsigned)((M + 15) / 16));
            if (vec) matmul_f32_small_kernel<16, true><<<g16, 512, 0, s>>>(out, left, right, M, K, N, kw);
            else matmul_f32_small_kernel<16, false><<<g16, 512, 0, s>>>(out, left, right, M, K, N, kw);
        } else {
            const dim3 g32((unsigned)((N + 31) / 32), (unsigned)((M + 31) / 32));
            if (vec) matmul_f32_small_kernel<32, true><<<g32, 512, 0, s>>>(out, left, right, M, K, N, kw);
            else matmul_f32_small_kernel<32, false><<<g32, 512, 0, s>>>(out, left, right, M, K, N, kw);
        }
        return check_launch("matmul");
    }
    // the f32 MFMA kernel (128 x 128 tiles, two blocks per CU).  Grids of fewer tiles
    // than CUs split K into chunks (at least 256 deep, at most 16) toward two blocks
    // per CU, f32 partials summed in order (1024 x 8192 x 1024: 13.5 -> 107 TFLOP/s
    // against the VALU kernel, 1024^3 12 -> 56, 512 x 4096 x 4096 28 -> 105);
    // splitting grids of a half round or more lost (2048^3 117 unsplit, 109 in two
    // chunks), and aiming at one block per CU lost where few chunks remain (1536^3 63
    // against 72-82, 128 x 8192 x 8192 101 against 111)
    if (K >= 64) {
        const int64_t cus = device_cus(), t128 = ((M + 127) / 128) * ((N + 127) / 128);
        int64_t mchunks = 1;
        if (t128 < cus)
            mchunks = std::max<int64_t>(1, std::min<int64_t>(std::min<int64_t>((2 * cus + t128 - 1) / t128, 16), K / 256));
        // the partials of every split fit the allocation-free entry point's 16 MiB
        // array, for both entry points alike (the same chunks: bit-identical results)
        mchunks = std::min<int64_t>(mchunks, std::max<int64_t>(1, (int64_t)(noalloc::kScratchBytes / ((size_t)(M * N) * sizeof(float)))));
        const int rc = launch_f32_mfma(out, left, right, M, K, N, mchunks, s, tgt);
        if (rc != 1) return rc;
    }
    int64_t chunks = tiles < 256 ? std::max<int64_t>(std::min<int64_t>(std::min<int64_t>(std::max<int64_t>(512 / tiles, 1), steps / 2), 64), 1) : 1;
    const int64_t per = (steps + chunks - 1) / chunks;
    chunks = (steps + per - 1) / per;
    if (chunks == 1) {
        matmul_f32_kernel<<<grid, 256, 0, s>>>(out, left, right, M, K, N, nullptr, K);
        return check_launch("matmul");
    }
    const size_t need = (size_t)(chunks * M * N) * sizeof(float);
    auto launch = [&](float *ws) {
        matmul_f32_kernel<<<dim3(grid.x, grid.y, (unsigned)chunks), 256, 0, s>>>(out, left, right, M, K, N, ws,
                                                                                   per * kDepth);
        matmul_splitk_reduce_f32_kernel<<<(unsigned)std::min<int64_t>((M * N + 255) / 256, 4096), 256, 0, s>>>(
            out, ws, M * N, (int)chunks);
        return check_launch("matmul split-k");
    };
    if (tgt.fixed) {
        if (need > noalloc::kScratchBytes)
            return fail(PUTER_ERR_INVALID, "matmul (no-alloc): split-K partials of %zu bytes exceed the %zu-byte scratch",
                        need, noalloc::kScratchBytes);
        return launch(tgt.fixed);
    }
    ScratchLease lease(need, s);
    if (lease.status()) return lease.status();
    const int rc = launch(static_cast<float *>(lease.ptr()));
    const int fin = lease.finish();
    return rc ? rc : fin;
}

static int matmul_entry(void *out, const void *left, const void *right, int64_t rows, int64_t inner,
                        int64_t cols, int dtype, void *stream, bool no_alloc) {
    if (rows < 0 || inner < 0 || cols < 0) return fail(PUTER_ERR_INVALID, "matmul: negative shape");
    if (dtype != PUTER_F32 && dtype != PUTER_F64 && dtype != PUTER_BF16 && dtype != PUTER_F16)
        return fail(PUTER_ERR_INVALID, "matmul: unsupported dtype %d", dtype);
    if (rows == 0 || cols == 0) return PUTER_OK;
    if (!out || !left || !right) return fail(PUTER_ERR_NIL, "matmul: nil buffer");
    if (rows * cols > ((int64_t)1 << 40)) return fail(PUTER_ERR_INVALID, "matmul: output too large");
    hipStream_t s = as_stream(stream);
    if (inner == 0) {  // empty sums: zeros (a fill kernel, safe under graph capture)
        const int64_t halves = rows * cols * (dtype == PUTER_F64 ? 4 : dtype == PUTER_F32 ? 2 : 1);
        matmul_zero_kernel<<<generic_blocks(halves), 256, 0, s>>>(static_cast<uint16_t *>(out), halves);
        return check_launch("matmul");
    }
    PartialsTarget tgt;
    if (no_alloc) {
        const int rc = noalloc::address(&tgt.fixed);
        if (rc) return rc;
    }
    switch (dtype) {
    case PUTER_BF16: return launch_matmul16<PUTER_BF16>(out, left, right, rows, inner, cols, s, tgt);
    case PUTER_F16: return launch_matmul16<PUTER_F16>(out, left, right, rows, inner, cols, s, tgt);
    case PUTER_F64:
        matmul_generic_kernel<PUTER_F64><<<generic_blocks(rows * cols), 256, 0, s>>>(out, left, right, rows, inner, cols);
        return check_launch("matmul");
    default: break;
    }
    return launch_matmul_f32(static_cast<float *>(out), static_cast<const float *>(left),
                             static_cast<const float *>(right), rows, inner, cols, s, tgt);
}

extern "C" int puter_hip_matmul(void *out, const void *left, const void *right, int64_t rows,
                                int64_t inner, int64_t cols, int dtype, void *stream) {
    return matmul_entry(out, left, right, rows, inner, cols, dtype, stream, false);
}

extern "C" int puter_hip_matmul_noalloc(void *out, const void *left, const void *right, int64_t rows,
                                        int64_t inner, int64_t cols, int dtype, void *stream) {
    return matmul_entry(out, left, right, rows, inner, cols, dtype, stream, true);
}
