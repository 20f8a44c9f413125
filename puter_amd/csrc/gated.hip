// Gated activations (SwiGLU, GeGLU, GeGLUTanh, SiGLU, GLU, ReGLU, LinGLU, SeGLU) in
// tensor form and packed form, plus unary Silu / Gelu.
// Reference: device/cpu/activation/gated.go:10-136, compute.go:72-176 and the
// scalar math of device/cpu/math/f32.go:21-105, math/activation.go:26-57,286-308.
//
// The scalar functions are evaluated operation by operation as the reference
// does (FastExp32's polynomial rather than a hardware exp, no FMA contraction,
// IEEE division), so f32 results match the reference's generic Go code bit for
// bit; GeLU's erf runs in float64 as math.Erf does.
// Streaming: 16-byte loads of gate and up, one 16-byte store (bf16: 6 B/elem).
#include "common.hpp"

namespace puter {

__device__ __forceinline__ float sigmoid32(float v) {  // f32.go:88-95
    if (v >= 0) return __fdiv_rn(1.0f, __fadd_rn(1.0f, fast_exp32(-v)));
    const float e = fast_exp32(v);
    return __fdiv_rn(e, __fadd_rn(1.0f, e));
}
__device__ __forceinline__ float silu32(float v) {  // f32.go:97-99
    return __fdiv_rn(v, __fadd_rn(1.0f, fast_exp32(-v)));
}
// FastExp64 (device/cpu/math/f64.go:10-32): FastExp32's 2^f polynomial in
// float64, scaled by an exact ldexp.  The reference's 16-bit Silu is not
// FastSilu32: it looks the input up in a 65536-entry table filled with
// narrow(float32(FastSilu64(x))) (device/cpu/activation/lut.go:14-62,
// math/f64.go:90-92), so the 16-bit unary Silu runs in float64 here.
__device__ __forceinline__ double fast_exp64(double x) {
    if (x < -708.3964185322641) return 0.0;
    if (x > 709.782712893384) return 1.7976931348623157e308;
    const double z = __dmul_rn(x, 1.4426950408889634);
    int64_t k = (int64_t)z;
    if (z < 0) k--;
    const double f = __dsub_rn(z, (double)k);
    double p = __dmul_rn(f, 0.001333899727232439);
    p = __dmul_rn(f, __dadd_rn(0.009618127167766223, p));
    p = __dmul_rn(f, __dadd_rn(0.05550410706910451, p));
    p = __dmul_rn(f, __dadd_rn(0.2402265069591007, p));
    p = __dmul_rn(f, __dadd_rn(0.6931471805599453, p));
    return ldexp(__dadd_rn(1.0, p), (int)k);
}
__device__ __forceinline__ float silu64(float v) {  // float32(FastSilu64(float64(v)))
    const double x = (double)v;
    return (float)__ddiv_rn(x, __dadd_rn(1.0, fast_exp64(-x)));
}
__device__ __forceinline__ float gelu32(float v) {  // activation.go:54-57
    const double x = (double)v;
    return (float)(0.5 * x * (1.0 + erf(x * 0.7071067811865475)));
}
__device__ __forceinline__ float tanh_pade32(float x) {  // f32.go:73-86
    if (x > 4.92f) return 1.0f;
    if (x < -4.92f) return -1.0f;
    const float x2 = __fmul_rn(x, x);
    const float num = __fmul_rn(x, __fadd_rn(135135.0f, __fmul_rn(x2, __fadd_rn(17325.0f,
                                __fmul_rn(x2, __fadd_rn(378.0f, x2))))));
    const float den = __fadd_rn(135135.0f, __fmul_rn(x2, __fadd_rn(62370.0f,
                                __fmul_rn(x2, __fadd_rn(3150.0f, __fmul_rn(x2, 28.0f))))));
    return __fdiv_rn(num, den);
}
__device__ __forceinline__ float gelu_tanh32(float v) {  // f32.go:101-105
    const double x = (double)v;
    const double inner = 0.7978845608028654 * (x + 0.044715 * x * x * x);
    return (float)(0.5 * x * (1.0 + (double)tanh_pade32((float)inner)));
}

template <int KIND>
__device__ __forceinline__ float combine(float g, float u) {
    if constexpr (KIND == PUTER_GATE_SWIGLU) return __fmul_rn(silu32(g), u);
    else if constexpr (KIND == PUTER_GATE_GEGLU) return __fmul_rn(g, gelu32(u));
    else if constexpr (KIND == PUTER_GATE_GEGLU_TANH) return __fmul_rn(g, gelu_tanh32(u));
    else if constexpr (KIND == PUTER_GATE_SIGLU) return __fmul_rn(sigmoid32(g), u);
    else if constexpr (KIND == PUTER_GATE_GLU) return __fmul_rn(g, sigmoid32(u));
    else if constexpr (KIND == PUTER_GATE_REGLU) return __fmul_rn(g, u > 0 ? u : 0.0f);
    else if constexpr (KIND == PUTER_GATE_SEGLU) return __fmul_rn(u, sigmoid32(g));
    else return __fmul_rn(g, u);
}

// Tensor form: dst[i] = combine(gate[i], up[i]) over `count` elements.
template <int DT, int KIND>
__global__ __launch_bounds__(256) void gated_tensors_kernel(void *__restrict__ dst,
                                                            const void *__restrict__ gate,
                                                            const void *__restrict__ up,
                                                            int64_t count, int vectorised) {
    using T = typename Elem<DT>::T;
    constexpr int N = Vec<DT>::N;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t body = 0;
    if (vectorised) {
        const int64_t nvec = count / N;
        for (int64_t v = tid; v < nvec; v += stride) {
            float g[N], u[N], o[N];
            unpack_vec<DT>(ld_stream(reinterpret_cast<const uint4 *>(gate) + v), g);
            unpack_vec<DT>(ld_stream(reinterpret_cast<const uint4 *>(up) + v), u);
#pragma unroll
            for (int i = 0; i < N; ++i) o[i] = combine<KIND>(g[i], u[i]);
            st_stream(pack_vec<DT>(o), reinterpret_cast<uint4 *>(dst) + v);
        }
        body = nvec * N;
    }
    for (int64_t i = body + tid; i < count; i += stride) {
        const float g = Elem<DT>::load(reinterpret_cast<const T *>(gate)[i]);
        const float u = Elem<DT>::load(reinterpret_cast<const T *>(up)[i]);
        reinterpret_cast<T *>(dst)[i] = Elem<DT>::store(combine<KIND>(g, u));
    }
}

// Packed form: row b of `packed` is [gate(half) | up(half)] -> dst row b (half).
template <int DT, int KIND>
__global__ __launch_bounds__(256) void gated_packed_kernel(void *__restrict__ dst,
                                                           const void *__restrict__ packed,
                                                           int64_t batch, int64_t half,
                                                           int vectorised) {
    using T = typename Elem<DT>::T;
    constexpr int N = Vec<DT>::N;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (vectorised) {
        const int64_t vrow = half / N;
        const int64_t nvec = batch * vrow;
        for (int64_t v = tid; v < nvec; v += stride) {
            const int64_t b = v / vrow, j = v - b * vrow;
            const uint4 *row = reinterpret_cast<const uint4 *>(packed) + b * 2 * vrow;
            float g[N], u[N], o[N];
            unpack_vec<DT>(ld_stream(row + j), g);
            unpack_vec<DT>(ld_stream(row + vrow + j), u);
#pragma unroll
            for (int i = 0; i < N; ++i) o[i] = combine<KIND>(g[i], u[i]);
            st_stream(pack_vec<DT>(o), reinterpret_cast<uint4 *>(dst) + v);
        }
        return;
    }
    const int64_t total = batch * half;
    for (int64_t i = tid; i < total; i += stride) {
        const int64_t b = i / half, c = i - b * half;
        const T *row = reinterpret_cast<const T *>(packed) + b * 2 * half;
        const float g = Elem<DT>::load(row[c]), u = Elem<DT>::load(row[half + c]);
        reinterpret_cast<T *>(dst)[i] = Elem<DT>::store(combine<KIND>(g, u));
    }
}

template <int DT, int KIND>
__global__ __launch_bounds__(256) void unary_kernel(void *__restrict__ dst,
                                                    const void *__restrict__ src, int64_t count) {
    using T = typename Elem<DT>::T;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += stride) {
        const float v = Elem<DT>::load(reinterpret_cast<const T *>(src)[i]);
        // f32: FastSilu32 / FastGelu32 (activation/f32_generic.go:72-97); 16-bit: the
        // reference's table entries, float32(FastSilu64 / FastGelu64) narrowed
        // (FastGelu64 in float64 then float32 is gelu32's own arithmetic)
        float y;
        if constexpr (KIND == PUTER_UNARY_SILU) y = DT == PUTER_F32 ? silu32(v) : silu64(v);
        else y = gelu32(v);
        reinterpret_cast<T *>(dst)[i] = Elem<DT>::store(y);
    }
}

static unsigned grid_for(int64_t units) {
    int64_t b = (units + 255) / 256;
    if (b > (1 << 20)) b = 1 << 20;
    if (b < 1) b = 1;
    return (unsigned)b;
}

template <int DT, int KIND>
static void launch_tensors(void *dst, const void *g, const void *u, int64_t count, hipStream_t s) {
    const int vec = aligned16(dst) && aligned16(g) && aligned16(u);
    gated_tensors_kernel<DT, KIND><<<grid_for(vec ? count / Vec<DT>::N + 1 : count), 256, 0, s>>>(
        dst, g, u, count, vec);
}

template <int DT, int KIND>
static void launch_packed(void *dst, const void *p, int64_t batch, int64_t half, hipStream_t s) {
    const int vec = aligned16(dst) && aligned16(p) && half % Vec<DT>::N == 0;
    gated_packed_kernel<DT, KIND><<<grid_for(vec ? batch * half / Vec<DT>::N : batch * half), 256, 0, s>>>(
        dst, p, batch, half, vec);
}

template <int DT>
static int gated_by_kind(int kind, bool packed, void *dst, const void *a, const void *b,
                         int64_t n0, int64_t n1, hipStream_t s) {
#define PUTER_GATE_CASE(K)                                                   \
    case K:                                                                  \
        if (packed) launch_packed<DT, K>(dst, a, n0, n1, s);                 \
        else launch_tensors<DT, K>(dst, a, b, n0, s);                        \
        break;
    switch (kind) {
        PUTER_GATE_CASE(PUTER_GATE_SWIGLU)
        PUTER_GATE_CASE(PUTER_GATE_GEGLU)
        PUTER_GATE_CASE(PUTER_GATE_GEGLU_TANH)
        PUTER_GATE_CASE(PUTER_GATE_SIGLU)
        PUTER_GATE_CASE(PUTER_GATE_GLU)
        PUTER_GATE_CASE(PUTER_GATE_REGLU)
        PUTER_GATE_CASE(PUTER_GATE_LINGLU)
        PUTER_GATE_CASE(PUTER_GATE_SEGLU)
    default: return fail(PUTER_ERR_INVALID, "gated: unknown kind %d", kind);
    }
#undef PUTER_GATE_CASE
    return check_launch("gated");
}

static int gated_dispatch(int kind, bool packed, void *dst, const void *a, const void *b,
                          int64_t n0, int64_t n1, int dtype, hipStream_t s) {
    switch (dtype) {
    case PUTER_F32: return gated_by_kind<PUTER_F32>(kind, packed, dst, a, b, n0, n1, s);
    case PUTER_BF16: return gated_by_kind<PUTER_BF16>(kind, packed, dst, a, b, n0, n1, s);
    case PUTER_F16: return gated_by_kind<PUTER_F16>(kind, packed, dst, a, b, n0, n1, s);
    }
    return fail(PUTER_ERR_INVALID, "gated: unsupported dtype %d", dtype);
}

}  // namespace puter

using namespace puter;

extern "C" {

int puter_hip_gated_tensors(int kind, void *dst, const void *gate, const void *up, int64_t count,
                            int dtype, void *stream) {
    if (count < 0) return fail(PUTER_ERR_INVALID, "gated: negative count");
    if (count == 0) return PUTER_OK;
    if (!is_norm_dtype(dtype)) return fail(PUTER_ERR_INVALID, "gated: unsupported dtype %d", dtype);
    if (!dst || !gate || !up) return fail(PUTER_ERR_NIL, "gated: nil buffer");
    return gated_dispatch(kind, false, dst, gate, up, count, 0, dtype, as_stream(stream));
}

int puter_hip_gated_packed(int kind, void *dst, const void *packed, int64_t batch,
                           int64_t half_count, int dtype, void *stream) {
    if (batch < 0 || half_count < 0) return fail(PUTER_ERR_INVALID, "gated packed: negative shape");
    if (batch == 0 || half_count == 0) return PUTER_OK;
    if (!is_norm_dtype(dtype)) return fail(PUTER_ERR_INVALID, "gated packed: unsupported dtype %d", dtype);
    if (!dst || !packed) return fail(PUTER_ERR_NIL, "gated packed: nil buffer");
    return gated_dispatch(kind, true, dst, packed, nullptr, batch, half_count, dtype, as_stream(stream));
}

int puter_hip_unary(int kind, void *dst, const void *src, int64_t count, int dtype, void *stream) {
    if (count < 0) return fail(PUTER_ERR_INVALID, "unary: negative count");
    if (count == 0) return PUTER_OK;
    if (!is_norm_dtype(dtype)) return fail(PUTER_ERR_INVALID, "unary: unsupported dtype %d", dtype);
    if (kind != PUTER_UNARY_SILU && kind != PUTER_UNARY_GELU) return fail(PUTER_ERR_INVALID, "unary: unknown kind %d", kind);
    if (!dst || !src) return fail(PUTER_ERR_NIL, "unary: nil buffer");
    hipStream_t s = as_stream(stream);
    const unsigned g = grid_for(count);
#define PUTER_UNARY(DT)                                                                   \
    if (kind == PUTER_UNARY_SILU) unary_kernel<DT, PUTER_UNARY_SILU><<<g, 256, 0, s>>>(dst, src, count); \
    else unary_kernel<DT, PUTER_UNARY_GELU><<<g, 256, 0, s>>>(dst, src, count);
    switch (dtype) {
    case PUTER_F32: PUTER_UNARY(PUTER_F32) break;
    case PUTER_BF16: PUTER_UNARY(PUTER_BF16) break;
    case PUTER_F16: PUTER_UNARY(PUTER_F16) break;
    }
#undef PUTER_UNARY
    return check_launch("unary");
}

}  // extern "C"
