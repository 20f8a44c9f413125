// RoPE and MultiAxisRoPE.
// Reference: device/cpu/rope/compute.go:11-330 (angles in float64: theta =
// pos * base^(-2i/D) (+ Llama-3 wavelength smoothing), cos/sin rounded to f32,
// rotation e' = e*c - o*s, o' = e*s + o*c in f32, 16-bit RNE store).
//
// Layout [seq, heads, D].  One block owns PPB consecutive positions: it first
// fills an LDS table of (cos, sin) for its positions x D/2 pairs in float64
// (the angle depends on (position, pair) only, so every head reuses it), then
// streams the positions' [heads * D] slabs through 16-byte vectors.  Each
// element is read and written once (4 B/elem in bf16); the float64 work is
// D/2 sincos per position, not per element.  input may alias output.
#include "common.hpp"

namespace puter {

struct RopeArgs {
    const void *in;
    void *out;
    int64_t seq, heads, dim;
    int64_t start;
    double base, factor, low, high;
    int64_t orig_ctx;
    int mode, scaling;
    int ppb;  // positions per block
};

__device__ __forceinline__ double rope_inv_freq(const RopeArgs &a, int64_t pair) {
    // ropeInverseFrequency compute.go:98-107
    const double exponent = -(double)(2 * pair) / (double)a.dim;
    const double inv = pow(a.base, exponent);
    if (a.scaling != 1) return inv;
    // llama3ScaledInverseFrequency compute.go:109-126
    const double wavelength = (2.0 * M_PI) / inv;
    const double lowW = (double)a.orig_ctx / a.low;
    const double highW = (double)a.orig_ctx / a.high;
    if (wavelength > lowW) return inv / a.factor;
    if (wavelength < highW) return inv;
    const double smooth = ((double)a.orig_ctx / wavelength - a.low) / (a.high - a.low);
    return (1.0 - smooth) * (inv / a.factor) + smooth * inv;
}

constexpr int kRopeLds = 8192;  // max (cos, sin) entries per block (64 KiB of LDS)
constexpr int kRopeVpt = 4;     // 16-byte vectors per thread in the register-resident kernel
                                // (4 measured faster than 2 or 8 on the Q/K config)
constexpr int kRopeGroupLds = 2048;  // (cos, sin) entries per group table in the pipelined kernel
constexpr int kRopeMaxBlocks = 2048; // 8 blocks per CU on MI355X's 256 CUs

// Register-resident, pipelined variant (a group of a.ppb positions is at most
// 256 * kRopeVpt vectors).  Blocks stride over the position groups; each block
// computes the float64 inverse frequencies once, then for every group it
// owns: issue the next group's loads and fill the next group's (cos, sin)
// table (float64) while the current group's data is rotated and stored.  The
// table is double buffered in LDS, the data in registers.  MODE 0
// interleaved, 1 half.  FAST: every group is full and its items fill all
// 256 * ITEMS slots, so the loop has no per-item branch and the group barrier
// waits for LDS only; with no branch around any load or store the compiler
// waits for exactly the current group's loads instead of draining every
// outstanding access (which would also wait for the stores just issued).
template <int DT, int MODE, bool FAST>
__global__ __launch_bounds__(256) void rope_reg_kernel(RopeArgs a) {
#pragma clang fp contract(off)
    extern __shared__ float2 cs[];  // [2][ppb * half] tables, then half doubles
    constexpr int N = Vec<DT>::N;
    constexpr int ITEMS = MODE == 0 ? kRopeVpt : kRopeVpt / 2;
    // group-local sizes fit 32 bits: a group holds <= 256 * kRopeVpt vectors
    const int half = (int)(a.dim / 2);
    const int dim = (int)a.dim;
    const int slab = (int)(a.heads * a.dim);
    const int vhalf = half / N;
    const int ppb = a.ppb;
    const int tsize = ppb * half;
    const int64_t ngroups = (a.seq + ppb - 1) / ppb;
    const int tid = threadIdx.x;
    double *invf = reinterpret_cast<double *>(cs + 2 * tsize);

    // Every group has the same layout, so each item's vector offset inside the
    // group, its table index and its position are computed once and packed
    // into one register: offset < 1024 (10 bits), table index < 2048 (11
    // bits), position < 1024 (10 bits).  Item k covers group vector tid + 256k
    // (MODE 0) or the (lo, hi) pair of the k-th half-row vector (MODE 1).
    // Quotients of operands below 2^12 come from a float reciprocal:
    // (x + 0.5) / d is at least 0.5 / d from an integer, far more than the
    // float rounding, so truncation gives floor(x / d) exactly.
    auto quot = [](int x, float rcp) -> int { return (int)(((float)x + 0.5f) * rcp); };
    const float r_slab = 1.0f / (float)slab, r_dim = 1.0f / (float)dim;
    const float r_vhalf = 1.0f / (float)vhalf, r_heads = 1.0f / (float)a.heads;
    uint32_t info[ITEMS];
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
        const int w = tid + 256 * k;
        int voff, tix, p;
        if constexpr (MODE == 0) {
            const int e0 = w * N;
            p = quot(e0, r_slab);
            const int in_slab = e0 - p * slab;
            voff = w;
            tix = p * half + (in_slab - quot(in_slab, r_dim) * dim) / 2;
        } else {
            const int row = quot(w, r_vhalf), j = w - row * vhalf;
            p = quot(row, r_heads);
            voff = row * (dim / N) + j;
            tix = p * half + j * N;
        }
        if (p >= ppb) voff = tix = 0;  // inactive in every group
        info[k] = (uint32_t)voff | ((uint32_t)tix << 10) | ((uint32_t)min(p, 1023) << 21);
    }
    const uint4 *inv = reinterpret_cast<const uint4 *>(a.in);
    uint4 *outv = reinterpret_cast<uint4 *>(a.out);
    // exact: the group's items fill all 256 * ITEMS slots, so every item of a
    // full group is live and the loads / stores need no per-item guard
    auto live = [&](int k, int np) -> bool { return FAST || (int)(info[k] >> 21) < np; };
    auto load = [&](int64_t g, uint4 (&lo)[ITEMS], uint4 (&hi)[ITEMS]) __attribute__((always_inline)) {
        const int np = (int)min((int64_t)ppb, a.seq - g * ppb);
        const uint4 *gb = inv + g * ppb * (int64_t)(slab / N);  // first vector of the group
#pragma unroll
        for (int k = 0; k < ITEMS; ++k) {
            if (live(k, np)) {
                const int voff = info[k] & 1023;
                lo[k] = ld_stream(gb + voff);
                if constexpr (MODE == 1) hi[k] = ld_stream(gb + voff + vhalf);
            }
        }
    };
    auto table = [&](int64_t g, float2 *t) __attribute__((always_inline)) {
        const int64_t p0 = g * ppb;
        const int n = (int)min((int64_t)ppb, a.seq - p0) * half;
        for (int e = tid; e < n; e += 256) {
            const int p = e / half, pair = e - p * half;
            const double theta = (double)(p0 + p + a.start) * invf[pair];
            double sn, cn;
            sincos(theta, &sn, &cn);
            t[e] = make_float2((float)cn, (float)sn);
        }
    };

    // rotate and store group g from registers with table c0
    auto rotate = [&](int64_t g, const float2 *c0, const uint4 (&lo)[ITEMS], const uint4 (&hi)[ITEMS])
                      __attribute__((always_inline)) {
        const int np = (int)min((int64_t)ppb, a.seq - g * ppb);
        uint4 *gb = outv + g * ppb * (int64_t)(slab / N);
#pragma unroll
        for (int k = 0; k < ITEMS; ++k) {
            if (!live(k, np)) continue;
            const int voff = info[k] & 1023, tix = (info[k] >> 10) & 2047;
            if constexpr (MODE == 0) {
                float f[N], o[N];
                unpack_vec<DT>(lo[k], f);
#pragma unroll
                for (int i = 0; i < N / 2; ++i) {
                    const float2 c = c0[tix + i];
                    o[2 * i] = f[2 * i] * c.x - f[2 * i + 1] * c.y;
                    o[2 * i + 1] = f[2 * i] * c.y + f[2 * i + 1] * c.x;
                }
                st_stream(pack_vec<DT>(o), gb + voff);
            } else {
                float e[N], od[N], oe[N], oo[N];
                unpack_vec<DT>(lo[k], e);
                unpack_vec<DT>(hi[k], od);
#pragma unroll
                for (int i = 0; i < N; ++i) {
                    const float2 c = c0[tix + i];
                    oe[i] = e[i] * c.x - od[i] * c.y;
                    oo[i] = e[i] * c.y + od[i] * c.x;
                }
                st_stream(pack_vec<DT>(oe), gb + voff);
                st_stream(pack_vec<DT>(oo), gb + voff + vhalf);
            }
        }
    };

    // first group: loads go out before the float64 inverse frequencies
    int64_t g = blockIdx.x;
    if (g >= ngroups) return;  // block-uniform: the whole block leaves together
    uint4 lo[ITEMS], hi[ITEMS];
    load(g, lo, hi);
    for (int pair = tid; pair < half; pair += 256) invf[pair] = rope_inv_freq(a, pair);
    __syncthreads();
    table(g, cs);
    __syncthreads();
    int buf = 0;
    // every iteration of this loop has a next group, so its loads and table are
    // issued unconditionally (no branch around them: the compiler then waits
    // for exactly the current group's loads); the block's last group is
    // rotated after the loop with nothing left to prefetch
    for (; g + gridDim.x < ngroups; g += gridDim.x) {
        const int64_t nx = g + gridDim.x;
        uint4 nlo[ITEMS], nhi[ITEMS];
        load(nx, nlo, nhi);
        table(nx, cs + (buf ^ 1) * tsize);
        rotate(g, cs + buf * tsize, lo, hi);
#pragma unroll
        for (int k = 0; k < ITEMS; ++k) {
            lo[k] = nlo[k];
            hi[k] = nhi[k];
        }
        // next table complete; this table free for the group after next.
        // FAST waits for LDS only (loads / stores stay in flight).
        if (FAST) {
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
            __builtin_amdgcn_s_barrier();
        } else {
            __syncthreads();
        }
        buf ^= 1;
    }
    rotate(g, cs + buf * tsize, lo, hi);
}

template <int DT>
__global__ __launch_bounds__(256) void rope_kernel(RopeArgs a) {
#pragma clang fp contract(off)
    extern __shared__ float2 cs[];
    const int64_t half = a.dim / 2;
    const int64_t p0 = (int64_t)blockIdx.x * a.ppb;
    const int64_t np = min((int64_t)a.ppb, a.seq - p0);
    for (int64_t t = threadIdx.x; t < np * half; t += blockDim.x) {
        const int64_t p = t / half, pair = t - p * half;
        const double theta = (double)(p0 + p + a.start) * rope_inv_freq(a, pair);
        double sn, cn;
        sincos(theta, &sn, &cn);
        cs[t] = make_float2((float)cn, (float)sn);
    }
    __syncthreads();
    using T = typename Elem<DT>::T;
    constexpr int N = Vec<DT>::N;
    const int64_t slab = a.heads * a.dim;           // elements per position
    const T *in = reinterpret_cast<const T *>(a.in) + p0 * slab;
    T *out = reinterpret_cast<T *>(a.out) + p0 * slab;
    if (a.mode == 0) {
        // interleaved pairs (2i, 2i+1): a 16-byte vector holds N/2 whole pairs
        const int64_t nvec = np * slab / N;
        for (int64_t v = threadIdx.x; v < nvec; v += blockDim.x) {
            const int64_t e0 = v * N;
            const int64_t p = e0 / slab;
            const int64_t pair0 = (e0 - p * slab) % a.dim / 2;
            float f[N], o[N];
            load_vec<DT>(in, (size_t)v, f);
#pragma unroll
            for (int i = 0; i < N / 2; ++i) {
                const float2 c = cs[p * half + pair0 + i];
                const float e = f[2 * i], od = f[2 * i + 1];
                o[2 * i] = e * c.x - od * c.y;
                o[2 * i + 1] = e * c.y + od * c.x;
            }
            reinterpret_cast<uint4 *>(out)[v] = pack_vec<DT>(o);
        }
    } else {
        // half mode (i, i + D/2): a vector of the first half pairs with the
        // vector D/2 further on; each thread owns both
        const int64_t vhalf = half / N;            // vectors per half-row
        const int64_t nwork = np * a.heads * vhalf;
        for (int64_t w = threadIdx.x; w < nwork; w += blockDim.x) {
            const int64_t row = w / vhalf, j = w - row * vhalf;
            const int64_t p = row / a.heads;
            const size_t lo = (size_t)(row * a.dim / N + j);
            const size_t hi = lo + (size_t)vhalf;
            float e[N], od[N], oe[N], oo[N];
            load_vec<DT>(in, lo, e);
            load_vec<DT>(in, hi, od);
#pragma unroll
            for (int i = 0; i < N; ++i) {
                const float2 c = cs[p * half + j * N + i];
                oe[i] = e[i] * c.x - od[i] * c.y;
                oo[i] = e[i] * c.y + od[i] * c.x;
            }
            reinterpret_cast<uint4 *>(out)[lo] = pack_vec<DT>(oe);
            reinterpret_cast<uint4 *>(out)[hi] = pack_vec<DT>(oo);
        }
    }
}

// Element-wise fallback for shapes the vector path cannot take (odd sizes,
// unaligned pointers): same table, one pair per thread iteration.
template <int DT>
__global__ __launch_bounds__(256) void rope_scalar_kernel(RopeArgs a) {
#pragma clang fp contract(off)
    extern __shared__ float2 cs[];
    const int64_t half = a.dim / 2;
    const int64_t p0 = (int64_t)blockIdx.x * a.ppb;
    const int64_t np = min((int64_t)a.ppb, a.seq - p0);
    for (int64_t t = threadIdx.x; t < np * half; t += blockDim.x) {
        const int64_t p = t / half, pair = t - p * half;
        const double theta = (double)(p0 + p + a.start) * rope_inv_freq(a, pair);
        double sn, cn;
        sincos(theta, &sn, &cn);
        cs[t] = make_float2((float)cn, (float)sn);
    }
    __syncthreads();
    using T = typename Elem<DT>::T;
    const T *in = reinterpret_cast<const T *>(a.in);
    T *out = reinterpret_cast<T *>(a.out);
    const int64_t npairs = np * a.heads * half;
    for (int64_t w = threadIdx.x; w < npairs; w += blockDim.x) {
        const int64_t row = w / half, pair = w - row * half;
        const int64_t p = row / a.heads;
        const size_t base = (size_t)((p0 * a.heads + row) * a.dim);
        const size_t ei = a.mode == 1 ? base + pair : base + 2 * pair;
        const size_t oi = a.mode == 1 ? base + half + pair : ei + 1;
        const float2 c = cs[p * half + pair];
        const float e = Elem<DT>::load(in[ei]), od = Elem<DT>::load(in[oi]);
        out[ei] = Elem<DT>::store(e * c.x - od * c.y);
        out[oi] = Elem<DT>::store(e * c.y + od * c.x);
    }
}

// MultiAxisRoPE compute.go:195-330: one thread per pair, angle in float64.
struct MultiAxisArgs {
    const void *in;
    void *out;
    int64_t batch, seq, heads, dim;
    double base;
    int64_t latent_seq, latent_side;
    int axis_count;
    int64_t starts[5];
};

template <int DT>
__global__ __launch_bounds__(256) void multi_axis_rope_kernel(MultiAxisArgs a) {
#pragma clang fp contract(off)
    using T = typename Elem<DT>::T;
    const int64_t half = a.dim / 2;
    const int64_t total = a.batch * a.seq * a.heads * half;
    const int64_t text_len = max(a.seq - a.latent_seq, (int64_t)0);
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t po = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; po < total; po += stride) {
        const int64_t pair = po % half;
        const int64_t head = (po / half) % a.heads;
        const int64_t s = (po / (half * a.heads)) % a.seq;
        const int64_t b = po / (half * a.heads * a.seq);
        const size_t even = (size_t)(((b * a.seq + s) * a.heads + head) * a.dim + pair * 2);
        int axis = 0;
        int64_t local = pair, axis_pairs = 0;
        for (int k = 0; k < a.axis_count; ++k) {
            if (pair < a.starts[k + 1]) {
                axis = k;
                local = pair - a.starts[k];
                axis_pairs = a.starts[k + 1] - a.starts[k];
                break;
            }
        }
        int64_t position;
        if (s < text_len) {
            position = ((a.axis_count == 4 && axis == 3) || (a.axis_count < 4 && axis == 0)) ? s : 0;
        } else {
            const int64_t img = s - text_len;
            position = axis == 1 ? img / a.latent_side : axis == 2 ? img % a.latent_side : 0;
        }
        float c = 1.0f, sn = 0.0f;
        const double axis_dim = (double)(axis_pairs * 2);
        if (axis_dim != 0) {
            const double exponent = -2.0 * (double)local / axis_dim;
            const double angle = (double)position * pow(a.base, exponent);
            double s64, c64;
            sincos(angle, &s64, &c64);
            c = (float)c64;
            sn = (float)s64;
        }
        const T *in = reinterpret_cast<const T *>(a.in);
        T *out = reinterpret_cast<T *>(a.out);
        const float e = Elem<DT>::load(in[even]), o = Elem<DT>::load(in[even + 1]);
        out[even] = Elem<DT>::store(e * c - o * sn);
        out[even + 1] = Elem<DT>::store(e * sn + o * c);
    }
}

// RoPEPairs (device/interface.go:605-609, device/cpu/rope/ops.go:25-38,
// RopePairsGeneric f32_generic.go:3-11): f32 only; pair i of `input` rotated by
// (cos[i], sin[i]): out[2i] = e*c - o*s, out[2i+1] = e*s + o*c, each product and
// difference rounded on its own (no contraction).  Two pairs per thread as one
// 16-byte input vector and two 8-byte cos / sin reads when the buffers allow.
__global__ __launch_bounds__(256) void rope_pairs_kernel(float *__restrict__ out, const float *__restrict__ in,
                                                         const float *__restrict__ cosb,
                                                         const float *__restrict__ sinb, int64_t pairs,
                                                         int vectorised) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t first = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    auto rot = [](float e, float o, float c, float sn, float &re, float &ro) __attribute__((always_inline)) {
        re = __fsub_rn(__fmul_rn(e, c), __fmul_rn(o, sn));
        ro = __fadd_rn(__fmul_rn(e, sn), __fmul_rn(o, c));
    };
    if (vectorised) {
        const int64_t units = pairs / 2;
        for (int64_t u = first; u < units; u += stride) {
            const float4 x = reinterpret_cast<const float4 *>(in)[u];
            const float2 c = reinterpret_cast<const float2 *>(cosb)[u];
            const float2 sn = reinterpret_cast<const float2 *>(sinb)[u];
            float4 y;
            rot(x.x, x.y, c.x, sn.x, y.x, y.y);
            rot(x.z, x.w, c.y, sn.y, y.z, y.w);
            reinterpret_cast<float4 *>(out)[u] = y;
        }
        if (first == 0 && (pairs & 1)) {
            const int64_t p = pairs - 1;
            rot(in[2 * p], in[2 * p + 1], cosb[p], sinb[p], out[2 * p], out[2 * p + 1]);
        }
        return;
    }
    for (int64_t p = first; p < pairs; p += stride) {
        float re, ro;
        rot(in[2 * p], in[2 * p + 1], cosb[p], sinb[p], re, ro);
        out[2 * p] = re;
        out[2 * p + 1] = ro;
    }
}

template <int DT>
static int launch_rope(RopeArgs a, hipStream_t s) {
    constexpr int N = Vec<DT>::N;
    const int64_t half = a.dim / 2;
    const int64_t slab = a.heads * a.dim;
    const bool vec = aligned16(a.in) && aligned16(a.out) && slab % N == 0 &&
                     (a.mode == 0 ? (a.dim % N == 0) : (half % N == 0));
    const int64_t slab_vec = slab / N;
    if (vec && slab_vec <= 256 * kRopeVpt && half <= kRopeGroupLds) {
        // as many positions per group as fill the registers, bounded by the table
        int64_t ppb = (256 * kRopeVpt) / slab_vec;
        if (ppb * half > kRopeGroupLds) ppb = kRopeGroupLds / half;
        if (ppb < 1) ppb = 1;
        a.ppb = (int)ppb;
        const int64_t groups = (a.seq + ppb - 1) / ppb;
        const unsigned blocks = (unsigned)min(groups, (int64_t)kRopeMaxBlocks);
        const size_t lds = 2 * (size_t)(ppb * half) * sizeof(float2) + (size_t)half * sizeof(double);
        constexpr int items = 256 * kRopeVpt;  // vectors a group can hold
        const bool fast = a.seq % ppb == 0 && ppb * slab_vec == items;
        if (a.mode == 0) {
            if (fast) rope_reg_kernel<DT, 0, true><<<blocks, 256, lds, s>>>(a);
            else rope_reg_kernel<DT, 0, false><<<blocks, 256, lds, s>>>(a);
        } else {
            if (fast) rope_reg_kernel<DT, 1, true><<<blocks, 256, lds, s>>>(a);
            else rope_reg_kernel<DT, 1, false><<<blocks, 256, lds, s>>>(a);
        }
        return check_launch("rope");
    }
    // ~4096 elements of work per block, bounded by the LDS table
    int64_t ppb = slab >= 4096 ? 1 : 4096 / slab;
    if (ppb * half > kRopeLds) ppb = kRopeLds / half;
    if (ppb < 1) ppb = 1;
    a.ppb = (int)ppb;
    const unsigned blocks = (unsigned)((a.seq + ppb - 1) / ppb);
    const size_t lds = (size_t)(ppb * half) * sizeof(float2);
    if (vec) rope_kernel<DT><<<blocks, 256, lds, s>>>(a);
    else rope_scalar_kernel<DT><<<blocks, 256, lds, s>>>(a);
    return check_launch("rope");
}

}  // namespace puter

using namespace puter;

extern "C" {

int puter_hip_rope(const puter_rope_config *config, const void *input, void *output,
                   int64_t seq_len, int64_t num_heads, int64_t head_dim, int dtype, void *stream) {
    if (!config) return fail(PUTER_ERR_NIL, "rope: nil config");
    if (seq_len < 0 || num_heads < 0 || head_dim < 0) return fail(PUTER_ERR_INVALID, "rope: negative shape");
    // dispatchRoPE compute.go:17-19: silent no-op
    if (seq_len == 0 || num_heads == 0 || head_dim == 0 || head_dim % 2 != 0) return PUTER_OK;
    // RoPEConfig.Validate device/config.go:215-258
    const puter_rope_config &c = *config;
    if (!(c.base_freq > 0)) return fail(PUTER_ERR_INVALID, "rope: base frequency must be positive, got %g", c.base_freq);
    if (c.mode != 0 && c.mode != 1) return fail(PUTER_ERR_INVALID, "rope: unsupported mode %d", c.mode);
    if (c.scaling != 0 && c.scaling != 1) return fail(PUTER_ERR_INVALID, "rope: unsupported scaling %d", c.scaling);
    if (c.scaling == 1) {
        if (!(c.scaling_factor > 0)) return fail(PUTER_ERR_INVALID, "rope: scaling factor must be positive");
        if (!(c.low_freq_factor > 0)) return fail(PUTER_ERR_INVALID, "rope: low frequency factor must be positive");
        if (!(c.high_freq_factor > c.low_freq_factor))
            return fail(PUTER_ERR_INVALID, "rope: high frequency factor must exceed low frequency factor");
        if (c.original_context <= 0) return fail(PUTER_ERR_INVALID, "rope: original context must be positive");
    }
    if (!is_norm_dtype(dtype)) return fail(PUTER_ERR_INVALID, "rope: unsupported dtype %d", dtype);
    if (head_dim / 2 > kRopeLds) return fail(PUTER_ERR_INVALID, "rope: head_dim %lld too large", (long long)head_dim);
    if (!input || !output) return fail(PUTER_ERR_NIL, "rope: nil buffer");
    RopeArgs a{input, output, seq_len, num_heads, head_dim, c.start_position, c.base_freq,
               c.scaling_factor, c.low_freq_factor, c.high_freq_factor, c.original_context,
               c.mode, c.scaling, 1};
    hipStream_t s = as_stream(stream);
    switch (dtype) {
    case PUTER_F32: return launch_rope<PUTER_F32>(a, s);
    case PUTER_BF16: return launch_rope<PUTER_BF16>(a, s);
    case PUTER_F16: return launch_rope<PUTER_F16>(a, s);
    }
    return PUTER_ERR_INVALID;
}

int puter_hip_rope_pairs(void *output, const void *input, const void *cos_buffer, const void *sin_buffer,
                         int64_t half_dim, int dtype, void *stream) {
    if (half_dim < 0) return fail(PUTER_ERR_INVALID, "rope pairs: negative half_dim");
    // requireRoPEFloat32 device/cpu/rope/ops.go:10-14
    if (dtype != PUTER_F32) return fail(PUTER_ERR_INVALID, "rope pairs: unsupported dtype %d", dtype);
    if (half_dim == 0) return PUTER_OK;
    if (!output || !input || !cos_buffer || !sin_buffer) return fail(PUTER_ERR_NIL, "rope pairs: nil buffer");
    const int vec = aligned16(output) && aligned16(input) &&
                    ((reinterpret_cast<uintptr_t>(cos_buffer) | reinterpret_cast<uintptr_t>(sin_buffer)) & 7u) == 0;
    const int64_t units = vec ? (half_dim + 1) / 2 : half_dim;
    int64_t blocks = (units + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    rope_pairs_kernel<<<(unsigned)blocks, 256, 0, as_stream(stream)>>>(
        static_cast<float *>(output), static_cast<const float *>(input), static_cast<const float *>(cos_buffer),
        static_cast<const float *>(sin_buffer), half_dim, vec);
    return check_launch("rope pairs");
}

int puter_hip_multi_axis_rope(const puter_multi_axis_rope_config *config, const void *input,
                              void *output, int64_t batch, int64_t seq_len, int64_t num_heads,
                              int64_t head_dim, int dtype, void *stream) {
    if (!config) return fail(PUTER_ERR_NIL, "multi-axis rope: nil config");
    if (batch < 0 || seq_len < 0 || num_heads < 0 || head_dim < 0)
        return fail(PUTER_ERR_INVALID, "multi-axis rope: negative shape");
    if (batch == 0 || seq_len == 0 || num_heads == 0 || head_dim == 0 || head_dim % 2 != 0) return PUTER_OK;
    const puter_multi_axis_rope_config &c = *config;
    // MultiAxisRoPEConfig.Validate / ValidateHeadDim device/config.go:148-213
    if (!(c.base_freq > 0) || c.latent_seq_len <= 0 || c.latent_side <= 0 || c.axis_count <= 0 || c.axis_count > 4)
        return fail(PUTER_ERR_INVALID, "multi-axis rope: invalid config");
    int64_t total = 0;
    for (int k = 0; k < 4; ++k) {
        if (k >= c.axis_count) {
            if (c.axis_dims[k] != 0) return fail(PUTER_ERR_INVALID, "multi-axis rope: inactive axis %d has dimension", k);
            continue;
        }
        if (c.axis_dims[k] <= 0 || c.axis_dims[k] % 2 != 0)
            return fail(PUTER_ERR_INVALID, "multi-axis rope: axis %d dimension must be positive and even", k);
        total += c.axis_dims[k];
    }
    if (total != head_dim) return fail(PUTER_ERR_INVALID, "multi-axis rope: axis dimensions sum to %lld, head dimension is %lld",
                                       (long long)total, (long long)head_dim);
    if (!is_norm_dtype(dtype)) return fail(PUTER_ERR_INVALID, "multi-axis rope: unsupported dtype %d", dtype);
    if (!input || !output) return fail(PUTER_ERR_NIL, "multi-axis rope: nil buffer");
    MultiAxisArgs a{input, output, batch, seq_len, num_heads, head_dim, c.base_freq,
                    c.latent_seq_len, c.latent_side, c.axis_count, {0, 0, 0, 0, 0}};
    for (int k = 0; k < c.axis_count; ++k) a.starts[k + 1] = a.starts[k] + c.axis_dims[k] / 2;
    const int64_t pairs = batch * seq_len * num_heads * (head_dim / 2);
    int64_t blocks = (pairs + 255) / 256;
    if (blocks > 16384) blocks = 16384;
    hipStream_t s = as_stream(stream);
    switch (dtype) {
    case PUTER_F32: multi_axis_rope_kernel<PUTER_F32><<<(unsigned)blocks, 256, 0, s>>>(a); break;
    case PUTER_BF16: multi_axis_rope_kernel<PUTER_BF16><<<(unsigned)blocks, 256, 0, s>>>(a); break;
    case PUTER_F16: multi_axis_rope_kernel<PUTER_F16><<<(unsigned)blocks, 256, 0, s>>>(a); break;
    }
    return check_launch("multi-axis rope");
}

}  // extern "C"
