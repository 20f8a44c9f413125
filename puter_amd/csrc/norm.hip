// LayerNorm family (RMSNorm, LayerNorm, AdaptiveRMSNorm, ModulatedLayerNorm),
// GatedResidual, and the fused GatedResidual -> RMSNorm / LayerNorm.
//
// Reference semantics: device/cpu/layernorm/compute.go (rows :350-570,
// validation :604-644), gated residual execution/math_gated_residual_intrinsic.go:206-223.
// The per-row scalar steps (rounding of 16-bit sums, float64 rsqrt, the order
// of the products) follow those functions; only the summation order inside a
// row differs (lane-sequential then a wave64 butterfly), which the reference's
// own SIMD kernels also change.
//
// Fast paths keep the row in registers, so every tensor is read once and
// written once (for the fused op, 8 B/elem of HBM traffic in bf16):
//   - norm_row_kernel: a block per row, 1-8 16-byte vectors per thread per
//     tensor (long rows, many rows);
//   - norm_wave_kernel: one wave64 per row, 4 rows per 256-thread block, the row
//     as VPL 16-byte vectors per lane (lane l owns vectors j*64 + l, so each
//     wave-wide load is one contiguous 1 KiB burst); register-only butterflies.
// Any other shape or alignment uses the generic block-per-row kernel, which
// re-reads the row from memory for each pass.
#include "common.hpp"

namespace puter {

enum NormOp { OP_RMS = 0, OP_LN = 1, OP_ADAPTIVE = 2, OP_MODULATED = 3 };

struct NormArgs {
    const void *x;       // input, or the residual when fused with the gated residual
    const void *branch;  // gated residual branch
    const void *mod;     // modulation (gate row / adaptive scale,shift / modulated shift,scale)
    const void *scale;
    const void *bias;
    void *hidden;        // gated residual output
    void *out;           // normalised output
    int64_t rows, H, rows_per_batch, mod_cols;
    int64_t gate_off;    // (3*set + 2) * H
    int64_t mod_off;     // 3*set*H for ModulatedLayerNorm, 0 otherwise
    double eps;
};

// RMS-type inverse (RMSNorm / AdaptiveRMSNorm) from the raw sum of squares.
template <int DT, int OP>
__device__ __forceinline__ float rms_inverse(float ss, int64_t H, double eps) {
    if constexpr (OP == OP_RMS) {
        if constexpr (DT == PUTER_F32) {
            // applyRMSRowF32 compute.go:350-363
            return (float)(1.0 / sqrt((double)ss / (double)H + eps));
        } else {
            // applyRMSRowBF16/F16 compute.go:365-385: dot rounded to 16 bit
            const float ms = round_reduction<DT>(ss) / (float)H;
            return (float)(1.0 / sqrt((double)ms + eps));
        }
    } else {
        // adaptiveRMSNormMeanSquare* compute.go:435-482 then :387-433
        const float ms = ss / (float)H;
        return (float)(1.0 / sqrt((double)ms + eps));
    }
}

// LayerNorm-type mean from the raw row sum.
template <int DT, int OP>
__device__ __forceinline__ float ln_mean(float s, int64_t H) {
    if constexpr (DT == PUTER_F32) return (float)((double)s / (double)H);  // computeRowMean :335-337
    else if constexpr (DT == PUTER_BF16) return round_reduction<DT>(s) / (float)H;  // :484-487
    else return s / (float)H;                                   // layerNormMeanF16 :572-580
}

template <int DT, int OP>
__device__ __forceinline__ float ln_inverse(float sq, int64_t H, double eps) {
    if constexpr (OP == OP_LN) {
        if constexpr (DT == PUTER_F32) return (float)(1.0 / sqrt((double)sq / (double)H + 1e-5));
        else return (float)(1.0 / sqrt((double)(sq / (float)H + 1e-5f)));  // :488-489
    } else {  // OP_MODULATED :522-559
        if constexpr (DT == PUTER_F32) return (float)(1.0 / sqrt((double)sq / (double)H + eps));
        else return (float)(1.0 / sqrt((double)(sq / (float)H) + eps));
    }
}

// Apply for one element.  c = column; gamma/beta/modulation already loaded.
template <int DT, int OP>
__device__ __forceinline__ float apply_one(float h, float mean, float inv, float g, float b) {
    if constexpr (OP == OP_RMS) {
        if constexpr (DT == PUTER_F32) { const float combined = inv * g; return h * combined; }
        else return h * inv * g;
    } else if constexpr (OP == OP_LN) {
        float d = h - mean;
        d = d * inv;
        d = d * g;
        return d + b;
    } else if constexpr (OP == OP_ADAPTIVE) {  // g = scale, b = shift
        const float normalized = h * inv;
        return normalized * (1 + g) + b;
    } else {                                   // OP_MODULATED: g = scale, b = shift
        const float normalized = (h - mean) * inv;
        return normalized * (1 + g) + b;
    }
}

// ------------------------------------------------------------ fast path --
// SHARE (fused gated residual + RMSNorm/LayerNorm, the block's 4 rows in one
// modulation batch): the gate row, gamma (and beta) are staged once per block
// in LDS instead of being re-read from L2 by every wave.
template <int DT, int OP, bool GR, int VPL, bool SHARE = false>
__global__ __launch_bounds__(256) void norm_wave_kernel(NormArgs a) {
#pragma clang fp contract(off)
    constexpr int N = Vec<DT>::N;
    constexpr int ROWV = VPL * 64;  // 16-byte vectors per row
    extern __shared__ uint4 tbl[];  // SHARE: [gate | gamma | beta] rows
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (!SHARE && row >= a.rows) return;
    const bool live = row < a.rows;
    const int64_t H = a.H;
    const size_t row_vec = (size_t)(live ? row : 0) * (size_t)(H / N);
    const int64_t batch = (live ? row : 0) / a.rows_per_batch;

    uint4 hv[VPL];
    if constexpr (GR) {
        const uint4 *res = reinterpret_cast<const uint4 *>(a.x) + row_vec;
        const uint4 *br = reinterpret_cast<const uint4 *>(a.branch) + row_vec;
        const uint4 *gate = reinterpret_cast<const uint4 *>(a.mod) +
                            (size_t)(batch * a.mod_cols + a.gate_off) / N;
        uint4 rv[VPL], bv[VPL], gv[VPL];
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
            rv[j] = ld_stream(res + j * 64 + lane);
            bv[j] = ld_stream(br + j * 64 + lane);
            if constexpr (!SHARE) gv[j] = gate[j * 64 + lane];
        }
        if constexpr (SHARE) {
            // the row loads above are in flight while the block fills the table
            const int64_t b0 = ((int64_t)blockIdx.x * 4) / a.rows_per_batch;
            const uint4 *g0 = reinterpret_cast<const uint4 *>(a.mod) + (size_t)(b0 * a.mod_cols + a.gate_off) / N;
            const uint4 *gm = reinterpret_cast<const uint4 *>(a.scale);
            const uint4 *bt = reinterpret_cast<const uint4 *>(a.bias);
            for (int i = threadIdx.x; i < ROWV; i += 256) {
                tbl[i] = g0[i];
                tbl[ROWV + i] = gm[i];
                if constexpr (OP == OP_LN) tbl[2 * ROWV + i] = bt[i];
            }
            __syncthreads();
            if (!live) return;
#pragma unroll
            for (int j = 0; j < VPL; ++j) gv[j] = tbl[j * 64 + lane];
        }
        uint4 *hid = reinterpret_cast<uint4 *>(a.hidden) + row_vec;
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
            float r[N], b[N], g[N], o[N];
            unpack_vec<DT>(rv[j], r);
            unpack_vec<DT>(bv[j], b);
            unpack_vec<DT>(gv[j], g);
#pragma unroll
            for (int i = 0; i < N; ++i) o[i] = r[i] + g[i] * b[i];
            hv[j] = pack_vec<DT>(o);
            st_stream(hv[j], hid + j * 64 + lane);
        }
    } else {
        const uint4 *x = reinterpret_cast<const uint4 *>(a.x) + row_vec;
#pragma unroll
        for (int j = 0; j < VPL; ++j) hv[j] = ld_stream(x + j * 64 + lane);
    }

    float mean = 0.0f, inv;
    if constexpr (OP == OP_RMS || OP == OP_ADAPTIVE) {
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
            float h[N];
            unpack_vec<DT>(hv[j], h);
#pragma unroll
            for (int i = 0; i < N; ++i) ss += h[i] * h[i];
        }
        inv = rms_inverse<DT, OP>(wave_sum(ss), H, a.eps);
    } else {
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
            float h[N];
            unpack_vec<DT>(hv[j], h);
#pragma unroll
            for (int i = 0; i < N; ++i) s += h[i];
        }
        mean = ln_mean<DT, OP>(wave_sum(s), H);
        float sq = 0.0f;
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
            float h[N];
            unpack_vec<DT>(hv[j], h);
#pragma unroll
            for (int i = 0; i < N; ++i) {
                const float d = h[i] - mean;
                sq += d * d;
            }
        }
        inv = ln_inverse<DT, OP>(wave_sum(sq), H, a.eps);
    }

    const uint4 *gp;
    const uint4 *bp = nullptr;
    if constexpr (SHARE) {
        gp = tbl + ROWV;
        if constexpr (OP == OP_LN) bp = tbl + 2 * ROWV;
    } else if constexpr (OP == OP_RMS || OP == OP_LN) {
        gp = reinterpret_cast<const uint4 *>(a.scale);
        if constexpr (OP == OP_LN) bp = reinterpret_cast<const uint4 *>(a.bias);
    } else {
        const uint4 *m = reinterpret_cast<const uint4 *>(a.mod) +
                         (size_t)(batch * a.mod_cols + a.mod_off) / N;
        if constexpr (OP == OP_ADAPTIVE) { gp = m; bp = m + H / N; }      // scale, shift
        else { bp = m; gp = m + H / N; }                                  // shift, scale
    }
    uint4 *out = reinterpret_cast<uint4 *>(a.out) + row_vec;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
        float h[N], g[N], b[N], o[N];
        unpack_vec<DT>(hv[j], h);
        unpack_vec<DT>(gp[j * 64 + lane], g);
        if (bp) unpack_vec<DT>(bp[j * 64 + lane], b);
        else {
#pragma unroll
            for (int i = 0; i < N; ++i) b[i] = 0.0f;
        }
#pragma unroll
        for (int i = 0; i < N; ++i) o[i] = apply_one<DT, OP>(h[i], mean, inv, g[i], b[i]);
        st_stream(pack_vec<DT>(o), out + j * 64 + lane);
    }
}

// ------------------------------------------------------- row-block path --
// A block per R rows, each row spread over the whole block: thread t owns the V
// 16-byte vectors j*T + t of every row (T = blockDim.x, T*V*N = H), so every tensor is
// read once and written once, with V loads of each input per row in flight per
// thread (launch_norm picks V per op).  The sums go through a wave butterfly and one
// LDS round (T/64 partials, one barrier per reduction, the R rows' sums side by
// side), so a row's sum is taken in the same order whatever R is.  Every launch uses
// R = 1: two rows per block (all their loads issued before the first barrier) gained
// 7-9% on the unfused norms at one vector per thread, but fewer threads per row with
// more vectors each gained more (see launch_norm), and R = 2 lost 1-3% elsewhere.
template <int DT, int OP, bool GR, int V, int R>
__global__ __launch_bounds__(1024) void norm_row_kernel(NormArgs a) {
#pragma clang fp contract(off)
    constexpr int N = Vec<DT>::N;
    __shared__ float red[2][R][16];
    const int T = blockDim.x, t = threadIdx.x, lane = t & 63, wave = t >> 6, nw = T >> 6;
    const int64_t H = a.H;
    const int64_t row0 = (int64_t)blockIdx.x * R;
    auto block_totals = [&](float (&v)[R], int slot) __attribute__((always_inline)) {
#pragma unroll
        for (int r = 0; r < R; ++r) v[r] = wave_sum(v[r]);
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r) red[slot][r][wave] = v[r];
        }
        __syncthreads();
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float s = 0.0f;
            for (int w = 0; w < nw; ++w) s += red[slot][r][w];
            v[r] = s;
        }
    };
    uint4 hv[R][V];
    if constexpr (GR) {
        uint4 rv[R][V], bv[R][V];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const size_t row_vec = (size_t)(row0 + r) * (size_t)(H / N);
            const uint4 *res = reinterpret_cast<const uint4 *>(a.x) + row_vec;
            const uint4 *br = reinterpret_cast<const uint4 *>(a.branch) + row_vec;
#pragma unroll
            for (int j = 0; j < V; ++j) {
                rv[r][j] = ld_stream(res + j * T + t);
                bv[r][j] = ld_stream(br + j * T + t);
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int64_t batch = (row0 + r) / a.rows_per_batch;
            const size_t row_vec = (size_t)(row0 + r) * (size_t)(H / N);
            const uint4 *gate = reinterpret_cast<const uint4 *>(a.mod) + (size_t)(batch * a.mod_cols + a.gate_off) / N;
            uint4 *hid = reinterpret_cast<uint4 *>(a.hidden) + row_vec;
#pragma unroll
            for (int j = 0; j < V; ++j) {
                float rr[N], b[N], g[N], o[N];
                unpack_vec<DT>(rv[r][j], rr);
                unpack_vec<DT>(bv[r][j], b);
                unpack_vec<DT>(gate[j * T + t], g);
#pragma unroll
                for (int i = 0; i < N; ++i) o[i] = rr[i] + g[i] * b[i];
                hv[r][j] = pack_vec<DT>(o);
                st_stream(hv[r][j], hid + j * T + t);
            }
        }
    } else {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint4 *x = reinterpret_cast<const uint4 *>(a.x) + (size_t)(row0 + r) * (size_t)(H / N);
#pragma unroll
            for (int j = 0; j < V; ++j) hv[r][j] = ld_stream(x + j * T + t);
        }
    }
    float mean[R], inv[R];
    if constexpr (OP == OP_RMS || OP == OP_ADAPTIVE) {
        float ss[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            ss[r] = 0.0f;
#pragma unroll
            for (int j = 0; j < V; ++j) {
                float h[N];
                unpack_vec<DT>(hv[r][j], h);
#pragma unroll
                for (int i = 0; i < N; ++i) ss[r] += h[i] * h[i];
            }
        }
        block_totals(ss, 0);
#pragma unroll
        for (int r = 0; r < R; ++r) { mean[r] = 0.0f; inv[r] = rms_inverse<DT, OP>(ss[r], H, a.eps); }
    } else {
        float s[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            s[r] = 0.0f;
#pragma unroll
            for (int j = 0; j < V; ++j) {
                float h[N];
                unpack_vec<DT>(hv[r][j], h);
#pragma unroll
                for (int i = 0; i < N; ++i) s[r] += h[i];
            }
        }
        block_totals(s, 0);
        float sq[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            mean[r] = ln_mean<DT, OP>(s[r], H);
            sq[r] = 0.0f;
#pragma unroll
            for (int j = 0; j < V; ++j) {
                float h[N];
                unpack_vec<DT>(hv[r][j], h);
#pragma unroll
                for (int i = 0; i < N; ++i) {
                    const float d = h[i] - mean[r];
                    sq[r] += d * d;
                }
            }
        }
        block_totals(sq, 1);
#pragma unroll
        for (int r = 0; r < R; ++r) inv[r] = ln_inverse<DT, OP>(sq[r], H, a.eps);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int64_t batch = (row0 + r) / a.rows_per_batch;
        const uint4 *gp;
        const uint4 *bp = nullptr;
        if constexpr (OP == OP_RMS || OP == OP_LN) {
            gp = reinterpret_cast<const uint4 *>(a.scale);
            if constexpr (OP == OP_LN) bp = reinterpret_cast<const uint4 *>(a.bias);
        } else {
            const uint4 *m = reinterpret_cast<const uint4 *>(a.mod) + (size_t)(batch * a.mod_cols + a.mod_off) / N;
            if constexpr (OP == OP_ADAPTIVE) { gp = m; bp = m + H / N; }
            else { bp = m; gp = m + H / N; }
        }
        uint4 *out = reinterpret_cast<uint4 *>(a.out) + (size_t)(row0 + r) * (size_t)(H / N);
#pragma unroll
        for (int j = 0; j < V; ++j) {
            float h[N], g[N], b[N], o[N];
            unpack_vec<DT>(hv[r][j], h);
            unpack_vec<DT>(gp[j * T + t], g);
            if (bp) unpack_vec<DT>(bp[j * T + t], b);
            else {
#pragma unroll
                for (int i = 0; i < N; ++i) b[i] = 0.0f;
            }
#pragma unroll
            for (int i = 0; i < N; ++i) o[i] = apply_one<DT, OP>(h[i], mean[r], inv[r], g[i], b[i]);
            st_stream(pack_vec<DT>(o), out + j * T + t);
        }
    }
}

// ---------------------------------------------------------- generic path --
__device__ __forceinline__ float block_sum(float v, float *smem) {
    v = wave_sum(v);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    __syncthreads();
    if (lane == 0) smem[wave] = v;
    __syncthreads();
    float t = 0.0f;
    const int waves = blockDim.x >> 6;
    for (int w = 0; w < waves; ++w) t += smem[w];
    return t;
}

// One block per row; `has_norm` = false runs the gated residual alone.
template <int DT, int OP, bool GR>
__global__ __launch_bounds__(256) void norm_block_kernel(NormArgs a, int has_norm) {
#pragma clang fp contract(off)
    using T = typename Elem<DT>::T;
    __shared__ float smem[4];
    const int64_t row = blockIdx.x;
    const int64_t H = a.H;
    const size_t off = (size_t)row * (size_t)H;
    const int64_t batch = row / a.rows_per_batch;
    const T *src = reinterpret_cast<const T *>(a.x) + off;
    if constexpr (GR) {
        const T *br = reinterpret_cast<const T *>(a.branch) + off;
        const T *gate = reinterpret_cast<const T *>(a.mod) + batch * a.mod_cols + a.gate_off;
        T *hid = reinterpret_cast<T *>(a.hidden) + off;
        for (int64_t c = threadIdx.x; c < H; c += blockDim.x) {
            const float o = Elem<DT>::load(src[c]) + Elem<DT>::load(gate[c]) * Elem<DT>::load(br[c]);
            hid[c] = Elem<DT>::store(o);
        }
        src = hid;  // each thread re-reads only the elements it wrote
    }
    if (!has_norm) return;
    float mean = 0.0f, inv;
    if constexpr (OP == OP_RMS || OP == OP_ADAPTIVE) {
        float ss = 0.0f;
        for (int64_t c = threadIdx.x; c < H; c += blockDim.x) {
            const float h = Elem<DT>::load(src[c]);
            ss += h * h;
        }
        inv = rms_inverse<DT, OP>(block_sum(ss, smem), H, a.eps);
    } else {
        float s = 0.0f;
        for (int64_t c = threadIdx.x; c < H; c += blockDim.x) s += Elem<DT>::load(src[c]);
        mean = ln_mean<DT, OP>(block_sum(s, smem), H);
        float sq = 0.0f;
        for (int64_t c = threadIdx.x; c < H; c += blockDim.x) {
            const float d = Elem<DT>::load(src[c]) - mean;
            sq += d * d;
        }
        inv = ln_inverse<DT, OP>(block_sum(sq, smem), H, a.eps);
    }
    const T *gp;
    const T *bp = nullptr;
    if constexpr (OP == OP_RMS || OP == OP_LN) {
        gp = reinterpret_cast<const T *>(a.scale);
        if constexpr (OP == OP_LN) bp = reinterpret_cast<const T *>(a.bias);
    } else {
        const T *m = reinterpret_cast<const T *>(a.mod) + batch * a.mod_cols + a.mod_off;
        if constexpr (OP == OP_ADAPTIVE) { gp = m; bp = m + H; }
        else { bp = m; gp = m + H; }
    }
    T *out = reinterpret_cast<T *>(a.out) + off;
    for (int64_t c = threadIdx.x; c < H; c += blockDim.x) {
        const float b = bp ? Elem<DT>::load(bp[c]) : 0.0f;
        out[c] = Elem<DT>::store(apply_one<DT, OP>(Elem<DT>::load(src[c]), mean, inv,
                                                    Elem<DT>::load(gp[c]), b));
    }
}

// Element-wise gated residual alone, 16-byte vectors: block (row, 256-vector
// chunk of the row), one vector of each input per thread, so no index division
// and the launch shape that streams HBM best (one vector per thread).
template <int DT>
__global__ __launch_bounds__(256) void gated_residual_vec_kernel(NormArgs a) {
#pragma clang fp contract(off)
    constexpr int N = Vec<DT>::N;
    const int64_t vec_per_row = a.H / N;
    const int64_t col = (int64_t)blockIdx.y * 256 + threadIdx.x;
    if (col >= vec_per_row) return;
    const int64_t row = blockIdx.x;
    const int64_t batch = row / a.rows_per_batch;
    const size_t v = (size_t)row * (size_t)vec_per_row + (size_t)col;
    float r[N], b[N], g[N], o[N];
    unpack_vec<DT>(ld_stream(reinterpret_cast<const uint4 *>(a.x) + v), r);
    unpack_vec<DT>(ld_stream(reinterpret_cast<const uint4 *>(a.branch) + v), b);
    load_vec<DT>(a.mod, (size_t)((batch * a.mod_cols + a.gate_off) / N + col), g);
#pragma unroll
    for (int i = 0; i < N; ++i) o[i] = r[i] + g[i] * b[i];
    st_stream(pack_vec<DT>(o), reinterpret_cast<uint4 *>(a.hidden) + v);
}

// --------------------------------------------------------------- launch --
template <int DT, int OP, bool GR>
static int launch_norm(const NormArgs &a, hipStream_t s, bool vec_ok) {
    constexpr int N = Vec<DT>::N;
    // Launch shape, chosen by same-process measurements on MI355X (bf16 sweep of
    // 1024 / 16384 / 65536 rows x 2048 / 4096 / 8192): with thousands of rows and
    // rows of at least 512 16-byte vectors, a block per row streams 3-12% faster
    // than the wave-per-row kernel.  The fused GatedResidual+RMSNorm does best at
    // one vector per thread (up to 1024 threads), the fused LayerNorm at up to 512
    // threads; the unfused norms with fewer threads and more vectors each: V = 2
    // for RMSNorm (4096 columns: 5725 -> 5908 / 6015 -> 6201 GB/s at 16384 / 65536
    // rows against V = 1), V = 8 for the two-reduction LayerNorm, whose barriers
    // cost less over fewer waves (4096 columns, 64 threads: 4667 -> 5638 / 5014 ->
    // 5999; 8192, 128 threads: 5352 -> 5659 / 5641 -> 5799 against 512 threads).
    // Fewer rows (latency-bound) and shorter rows keep the wave per row.
    const int64_t U = a.H / N;
    constexpr bool two_pass = OP == OP_LN || OP == OP_MODULATED;
    if (vec_ok && a.H % (64 * N) == 0 && a.rows >= 4096 && U >= 512) {
        int64_t V = 1, max_t = 1024;
        if constexpr (GR) max_t = two_pass ? 512 : 1024;
        else V = two_pass ? 8 : 2;
        while (U / V > max_t) V *= 2;
        if (V <= 8 && U % V == 0 && (U / V) % 64 == 0) {
            const unsigned T = (unsigned)(U / V), blocks = (unsigned)a.rows;
            switch (V) {
            case 1: norm_row_kernel<DT, OP, GR, 1, 1><<<blocks, T, 0, s>>>(a); break;
            case 2: norm_row_kernel<DT, OP, GR, 2, 1><<<blocks, T, 0, s>>>(a); break;
            case 4: norm_row_kernel<DT, OP, GR, 4, 1><<<blocks, T, 0, s>>>(a); break;
            default: norm_row_kernel<DT, OP, GR, 8, 1><<<blocks, T, 0, s>>>(a); break;
            }
            return check_launch("norm");
        }
    }
    if (vec_ok && a.H % (64 * N) == 0) {
        const int64_t vpl = a.H / (64 * N);
        const unsigned blocks = (unsigned)((a.rows + 3) / 4);
        if constexpr (GR && (OP == OP_RMS || OP == OP_LN)) {
            if (a.rows_per_batch % 4 == 0) {   // a block's 4 rows share one gate row
                const size_t lds = (size_t)a.H * sizeof(typename Elem<DT>::T) * (OP == OP_LN ? 3 : 2);
                switch (vpl) {
                case 2: norm_wave_kernel<DT, OP, GR, 2, true><<<blocks, 256, lds, s>>>(a); return check_launch("norm");
                case 4: norm_wave_kernel<DT, OP, GR, 4, true><<<blocks, 256, lds, s>>>(a); return check_launch("norm");
                case 8: norm_wave_kernel<DT, OP, GR, 8, true><<<blocks, 256, lds, s>>>(a); return check_launch("norm");
                case 16: norm_wave_kernel<DT, OP, GR, 16, true><<<blocks, 256, lds, s>>>(a); return check_launch("norm");
                default: break;
                }
            }
        }
        switch (vpl) {
        case 2: norm_wave_kernel<DT, OP, GR, 2><<<blocks, 256, 0, s>>>(a); return check_launch("norm");
        case 4: norm_wave_kernel<DT, OP, GR, 4><<<blocks, 256, 0, s>>>(a); return check_launch("norm");
        case 8: norm_wave_kernel<DT, OP, GR, 8><<<blocks, 256, 0, s>>>(a); return check_launch("norm");
        case 16: norm_wave_kernel<DT, OP, GR, 16><<<blocks, 256, 0, s>>>(a); return check_launch("norm");
        default: break;
        }
    }
    norm_block_kernel<DT, OP, GR><<<(unsigned)a.rows, 256, 0, s>>>(a, 1);
    return check_launch("norm(generic)");
}

template <int OP, bool GR>
static int dispatch_norm(const NormArgs &a, int dtype, hipStream_t s) {
    const int n = 16 / dtype_bytes(dtype);
    bool vec_ok = aligned16(a.x) && aligned16(a.out) && aligned16(a.scale ? a.scale : a.x) &&
                  aligned16(a.bias ? a.bias : a.x) && aligned16(a.mod ? a.mod : a.x) &&
                  aligned16(a.branch ? a.branch : a.x) && aligned16(a.hidden ? a.hidden : a.x);
    if (a.mod) vec_ok = vec_ok && (a.mod_cols % n == 0) && (a.gate_off % n == 0) && (a.mod_off % n == 0);
    switch (dtype) {
    case PUTER_F32: return launch_norm<PUTER_F32, OP, GR>(a, s, vec_ok);
    case PUTER_BF16: return launch_norm<PUTER_BF16, OP, GR>(a, s, vec_ok);
    case PUTER_F16: return launch_norm<PUTER_F16, OP, GR>(a, s, vec_ok);
    }
    return fail(PUTER_ERR_INVALID, "norm: unsupported dtype %d", dtype);
}

static int check_common(int64_t rows, int64_t H, int dtype, const char *what) {
    if (rows < 0 || H < 0) return fail(PUTER_ERR_INVALID, "%s: negative shape", what);
    if (!is_norm_dtype(dtype)) return fail(PUTER_ERR_INVALID, "%s: unsupported dtype %d", what, dtype);
    if (rows > 0x7FFFFFFF) return fail(PUTER_ERR_INVALID, "%s: rows exceed the grid limit", what);
    return PUTER_OK;
}

static int check_gated(int64_t rows, int64_t H, int64_t rpb, int64_t mod_cols, int set,
                       const char *what) {
    // resolveGatedResidualLayout math_gated_residual_intrinsic.go:131-139
    if (rpb <= 0 || rows % rpb != 0) return fail(PUTER_ERR_INVALID, "%s: invalid rows_per_batch", what);
    if (set < 0 || mod_cols < ((int64_t)set * 3 + 3) * H)
        return fail(PUTER_ERR_INVALID, "%s: modulation width too small", what);
    return PUTER_OK;
}

}  // namespace puter

using namespace puter;

extern "C" {

int puter_hip_rmsnorm(const void *input, const void *scale, void *output, int64_t rows,
                      int64_t last_dim, double epsilon, int dtype, void *stream) {
    int rc = check_common(rows, last_dim, dtype, "rmsnorm");
    if (rc) return rc;
    if (rows == 0 || last_dim == 0) return PUTER_OK;
    if (!(epsilon > 0)) return fail(PUTER_ERR_INVALID, "rmsnorm: epsilon must be positive, got %g", epsilon);
    if (!input || !scale || !output) return fail(PUTER_ERR_NIL, "rmsnorm: nil buffer");
    NormArgs a{input, nullptr, nullptr, scale, nullptr, nullptr, output, rows, last_dim, 1, 0, 0, 0, epsilon};
    return dispatch_norm<OP_RMS, false>(a, dtype, as_stream(stream));
}

int puter_hip_layernorm(const void *input, const void *scale, const void *bias, void *output,
                        int64_t rows, int64_t last_dim, int dtype, void *stream) {
    int rc = check_common(rows, last_dim, dtype, "layernorm");
    if (rc) return rc;
    if (rows == 0 || last_dim == 0) return PUTER_OK;
    if (!input || !scale || !bias || !output) return fail(PUTER_ERR_NIL, "layernorm: nil buffer");
    NormArgs a{input, nullptr, nullptr, scale, bias, nullptr, output, rows, last_dim, 1, 0, 0, 0, 1e-5};
    return dispatch_norm<OP_LN, false>(a, dtype, as_stream(stream));
}

int puter_hip_adaptive_rmsnorm(const void *input, const void *modulation, void *output,
                               int64_t rows, int64_t last_dim, int64_t rows_per_batch,
                               int64_t modulation_cols, double epsilon, int dtype, void *stream) {
    int rc = check_common(rows, last_dim, dtype, "adaptive rmsnorm");
    if (rc) return rc;
    if (rows == 0 || last_dim == 0) return PUTER_OK;
    // validateAdaptiveRMSNorm compute.go:624-644
    if (!(epsilon > 0)) return fail(PUTER_ERR_INVALID, "adaptive rmsnorm: epsilon must be positive");
    if (rows_per_batch <= 0 || rows % rows_per_batch != 0)
        return fail(PUTER_ERR_INVALID, "adaptive rmsnorm: rows must be divisible by rowsPerBatch");
    if (modulation_cols < 2 * last_dim) return fail(PUTER_ERR_INVALID, "adaptive rmsnorm: modulation width too small");
    if (!input || !modulation || !output) return fail(PUTER_ERR_NIL, "adaptive rmsnorm: nil buffer");
    NormArgs a{input, nullptr, modulation, nullptr, nullptr, nullptr, output, rows, last_dim,
               rows_per_batch, modulation_cols, 0, 0, epsilon};
    return dispatch_norm<OP_ADAPTIVE, false>(a, dtype, as_stream(stream));
}

int puter_hip_modulated_layernorm(const void *input, const void *modulation, void *output,
                                  int64_t rows, int64_t last_dim, int64_t rows_per_batch,
                                  int64_t modulation_cols, double epsilon, int set, int dtype,
                                  void *stream) {
    int rc = check_common(rows, last_dim, dtype, "modulated layernorm");
    if (rc) return rc;
    if (rows == 0 || last_dim == 0) return PUTER_OK;
    // validateModulatedLayerNorm compute.go:604-622
    if (!(epsilon > 0) || set < 0) return fail(PUTER_ERR_INVALID, "modulated layernorm: invalid config");
    if (rows_per_batch <= 0 || rows % rows_per_batch != 0)
        return fail(PUTER_ERR_INVALID, "modulated layernorm: rows must be divisible by rowsPerBatch");
    if (modulation_cols < ((int64_t)set * 3 + 2) * last_dim)
        return fail(PUTER_ERR_INVALID, "modulated layernorm: modulation width too small");
    if (!input || !modulation || !output) return fail(PUTER_ERR_NIL, "modulated layernorm: nil buffer");
    NormArgs a{input, nullptr, modulation, nullptr, nullptr, nullptr, output, rows, last_dim,
               rows_per_batch, modulation_cols, 0, (int64_t)set * 3 * last_dim, epsilon};
    return dispatch_norm<OP_MODULATED, false>(a, dtype, as_stream(stream));
}

int puter_hip_gated_residual(const void *residual, const void *branch, const void *modulation,
                             void *output, int64_t rows, int64_t last_dim,
                             int64_t rows_per_batch, int64_t modulation_cols, int set,
                             int dtype, void *stream) {
    int rc = check_common(rows, last_dim, dtype, "gated residual");
    if (rc) return rc;
    if (rows == 0 || last_dim == 0) return PUTER_OK;
    rc = check_gated(rows, last_dim, rows_per_batch, modulation_cols, set, "gated residual");
    if (rc) return rc;
    if (!residual || !branch || !modulation || !output) return fail(PUTER_ERR_NIL, "gated residual: nil buffer");
    NormArgs a{residual, branch, modulation, nullptr, nullptr, output, nullptr, rows, last_dim,
               rows_per_batch, modulation_cols, ((int64_t)set * 3 + 2) * last_dim, 0, 0.0};
    hipStream_t s = as_stream(stream);
    const int n = 16 / dtype_bytes(dtype);
    const bool vec_ok = aligned16(residual) && aligned16(branch) && aligned16(modulation) &&
                        aligned16(output) && last_dim % n == 0 && modulation_cols % n == 0;
    const int64_t chunks = (last_dim / n + 255) / 256;
    if (vec_ok && chunks <= 65535) {
        const dim3 grid((unsigned)rows, (unsigned)chunks);
        switch (dtype) {
        case PUTER_F32: gated_residual_vec_kernel<PUTER_F32><<<grid, 256, 0, s>>>(a); break;
        case PUTER_BF16: gated_residual_vec_kernel<PUTER_BF16><<<grid, 256, 0, s>>>(a); break;
        case PUTER_F16: gated_residual_vec_kernel<PUTER_F16><<<grid, 256, 0, s>>>(a); break;
        }
        return check_launch("gated residual");
    }
    switch (dtype) {
    case PUTER_F32: norm_block_kernel<PUTER_F32, OP_RMS, true><<<(unsigned)rows, 256, 0, s>>>(a, 0); break;
    case PUTER_BF16: norm_block_kernel<PUTER_BF16, OP_RMS, true><<<(unsigned)rows, 256, 0, s>>>(a, 0); break;
    case PUTER_F16: norm_block_kernel<PUTER_F16, OP_RMS, true><<<(unsigned)rows, 256, 0, s>>>(a, 0); break;
    }
    return check_launch("gated residual(generic)");
}

int puter_hip_gated_residual_rmsnorm(const void *residual, const void *branch,
                                     const void *modulation, const void *scale, void *hidden,
                                     void *normed, int64_t rows, int64_t last_dim,
                                     int64_t rows_per_batch, int64_t modulation_cols, int set,
                                     double epsilon, int dtype, void *stream) {
    int rc = check_common(rows, last_dim, dtype, "gated residual rmsnorm");
    if (rc) return rc;
    if (rows == 0 || last_dim == 0) return PUTER_OK;
    rc = check_gated(rows, last_dim, rows_per_batch, modulation_cols, set, "gated residual rmsnorm");
    if (rc) return rc;
    if (!(epsilon > 0)) return fail(PUTER_ERR_INVALID, "gated residual rmsnorm: epsilon must be positive");
    if (!residual || !branch || !modulation || !scale || !hidden || !normed)
        return fail(PUTER_ERR_NIL, "gated residual rmsnorm: nil buffer");
    NormArgs a{residual, branch, modulation, scale, nullptr, hidden, normed, rows, last_dim,
               rows_per_batch, modulation_cols, ((int64_t)set * 3 + 2) * last_dim, 0, epsilon};
    return dispatch_norm<OP_RMS, true>(a, dtype, as_stream(stream));
}

int puter_hip_gated_residual_layernorm(const void *residual, const void *branch,
                                       const void *modulation, const void *scale,
                                       const void *bias, void *hidden, void *normed,
                                       int64_t rows, int64_t last_dim, int64_t rows_per_batch,
                                       int64_t modulation_cols, int set, int dtype,
                                       void *stream) {
    int rc = check_common(rows, last_dim, dtype, "gated residual layernorm");
    if (rc) return rc;
    if (rows == 0 || last_dim == 0) return PUTER_OK;
    rc = check_gated(rows, last_dim, rows_per_batch, modulation_cols, set, "gated residual layernorm");
    if (rc) return rc;
    if (!residual || !branch || !modulation || !scale || !bias || !hidden || !normed)
        return fail(PUTER_ERR_NIL, "gated residual layernorm: nil buffer");
    NormArgs a{residual, branch, modulation, scale, bias, hidden, normed, rows, last_dim,
               rows_per_batch, modulation_cols, ((int64_t)set * 3 + 2) * last_dim, 0, 1e-5};
    return dispatch_norm<OP_LN, true>(a, dtype, as_stream(stream));
}

}  // extern "C"
