// ScaledDotProductAttention / FlashAttention: one head, Q/K [seq, depth],
// V/O [seq, valueDim].
// Reference: device/cpu/attention/ops.go:9-31 (FlashAttention calls
// ScaledDotProductAttention), compute.go:10-29,54-68 (zero seqQ or seqK is a
// no-op; scale = float32(1/sqrt(float64(depth)))), typed_compute.go:31-97 and
// select_flash_amd64.go:133-177 (per row: online softmax over the visible keys
// in order, causal hides key > row, i.e. top-left aligned; exponentials through
// flashExpFloat32, flash_attention.go:171-189, which is FastExp32 with -inf and
// anything below -88 mapped to 0; output acc * (1/normalizer), zeros when the
// normalizer is 0).  16-bit dots are rounded to the 16-bit format.
//
// General kernel: one wave64 per query row.  Each lane scores one key of a
// 64-key chunk; the chunk's keys are then folded into the running (max,
// normalizer, acc) one at a time, in key order, with the reference's exact
// sequence of exponentials (FastExp32's error is ~1e-5 relative, so regrouping
// the rescales would move f32 results by more than their tolerance); lanes own
// the output dims.  bf16 / f16 with depth = valueDim = 128 or 64 runs on the
// MFMA prefill kernel with one head and shift 0 (hardware exp2 in place of
// FastExp32; the difference is far below bf16 / f16 resolution).
#include "attention.hpp"

namespace puter {

struct FlashArgs {
    const void *q, *k, *v;
    void *o;
    int64_t seq_q, seq_k, depth, value_dim;
    int causal;
    float scale;
};

constexpr int64_t kFlashMaxDepth = 8192;     // Q row staged in LDS as f32 (32 KB)
constexpr int64_t kFlashMaxValueDim = 1024;  // 16 output dims per lane

__device__ __forceinline__ float flash_exp(float v) {
    if (v != v) return v;
    if (v < -88.0f) return 0.0f;  // includes -inf
    if (isinf(v)) return INFINITY;
    return fast_exp32(v);
}

template <int DT>
__global__ __launch_bounds__(64) void flash_generic_kernel(FlashArgs a) {
    using T = typename Elem<DT>::T;
    constexpr int NV = kFlashMaxValueDim / kWave;
    extern __shared__ float qrow[];
    const int64_t r = blockIdx.x;
    const int lane = threadIdx.x;
    const T *Q = reinterpret_cast<const T *>(a.q) + r * a.depth;
    const T *K = reinterpret_cast<const T *>(a.k);
    const T *V = reinterpret_cast<const T *>(a.v);
    T *O = reinterpret_cast<T *>(a.o) + r * a.value_dim;
    for (int64_t d = lane; d < a.depth; d += kWave) qrow[d] = Elem<DT>::load(Q[d]);
    __syncthreads();
    const int64_t k_hi = a.causal ? min(a.seq_k, r + 1) : a.seq_k;
    float m = -INFINITY, l = 0.0f;
    float acc[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) acc[j] = 0.0f;
    for (int64_t c0 = 0; c0 < k_hi; c0 += kWave) {
        // lane t scores key c0 + t (sequential f32 dot over depth)
        float s = -INFINITY;
        if (c0 + lane < k_hi) {
            const T *kr = K + (c0 + lane) * a.depth;
            float dot = 0.0f;
            for (int64_t d = 0; d < a.depth; ++d) dot += qrow[d] * Elem<DT>::load(kr[d]);
            s = round_reduction<DT>(dot) * a.scale;
        }
        // the keys of the chunk, in order, exactly as the reference's per-key loop
        const int n = (int)min((int64_t)kWave, k_hi - c0);
        for (int t = 0; t < n; ++t) {
            const float score = __shfl(s, t, kWave);
            const float old = m;
            if (score > m) m = score;
            const float alpha = flash_exp(old - m);
            const float shifted = flash_exp(score - m);
            l = l * alpha + shifted;
            const T *vr = V + (c0 + t) * a.value_dim;
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                const int64_t d = lane + kWave * j;
                if (d < a.value_dim) acc[j] = acc[j] * alpha + Elem<DT>::load(vr[d]) * shifted;
            }
        }
    }
    const float inv = l != 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int64_t d = lane + kWave * j;
        if (d < a.value_dim) O[d] = Elem<DT>::store(l != 0.0f ? acc[j] * inv : 0.0f);
    }
}

static int run_flash(const puter_flash_config *config, const void *q, const void *k,
                     const void *v, void *o, int64_t seq_q, int64_t seq_k, int64_t depth,
                     int64_t value_dim, int dtype, hipStream_t s) {
    if (!config) return fail(PUTER_ERR_NIL, "flash attention: nil config");
    if (!is_norm_dtype(dtype)) return fail(PUTER_ERR_INVALID, "flash attention: unsupported dtype %d", dtype);
    if (seq_q < 0 || seq_k < 0 || depth < 0 || value_dim < 0)
        return fail(PUTER_ERR_INVALID, "flash attention: negative shape");
    if (seq_q == 0 || seq_k == 0 || value_dim == 0) return PUTER_OK;
    if (depth == 0) return fail(PUTER_ERR_INVALID, "flash attention: depth must be positive");
    if (depth > kFlashMaxDepth || value_dim > kFlashMaxValueDim)
        return fail(PUTER_ERR_INVALID, "flash attention: depth %lld / value dim %lld above %lld / %lld",
                    (long long)depth, (long long)value_dim, (long long)kFlashMaxDepth,
                    (long long)kFlashMaxValueDim);
    if (seq_q > 0x7FFFFFFF) return fail(PUTER_ERR_INVALID, "flash attention: grid too large");
    if (!q || !k || !v || !o) return fail(PUTER_ERR_NIL, "flash attention: nil buffer");
    const float scale = (float)(1.0 / sqrt((double)depth));
    if ((dtype == PUTER_BF16 || dtype == PUTER_F16) && (depth == 128 || depth == 64) && value_dim == depth) {
        MhaArgs m{q, k, v, o, 1, seq_q, seq_k, 1, 1, depth, config->causal ? 1 : 0, 0, 0.0f, scale, 0};
        int status = PUTER_OK;
        if (launch_prefill_mfma(m, dtype, s, &status)) return status;
    }
    FlashArgs a{q, k, v, o, seq_q, seq_k, depth, value_dim, config->causal ? 1 : 0, scale};
    const size_t lds = sizeof(float) * (size_t)depth;
    switch (dtype) {
    case PUTER_F32: flash_generic_kernel<PUTER_F32><<<(unsigned)seq_q, kWave, lds, s>>>(a); break;
    case PUTER_BF16: flash_generic_kernel<PUTER_BF16><<<(unsigned)seq_q, kWave, lds, s>>>(a); break;
    case PUTER_F16: flash_generic_kernel<PUTER_F16><<<(unsigned)seq_q, kWave, lds, s>>>(a); break;
    }
    return check_launch("flash attention");
}

}  // namespace puter

using namespace puter;

extern "C" {

int puter_hip_scaled_dot_product_attention(const puter_flash_config *config, const void *query,
                                           const void *key, const void *value, void *output,
                                           int64_t seq_q, int64_t seq_k, int64_t depth,
                                           int64_t value_dim, int dtype, void *stream) {
    return run_flash(config, query, key, value, output, seq_q, seq_k, depth, value_dim, dtype,
                     as_stream(stream));
}

int puter_hip_flash_attention(const puter_flash_config *config, const void *query,
                              const void *key, const void *value, void *output, int64_t seq_q,
                              int64_t seq_k, int64_t depth, int64_t value_dim, int dtype,
                              void *stream) {
    return run_flash(config, query, key, value, output, seq_q, seq_k, depth, value_dim, dtype,
                     as_stream(stream));
}

}  // extern "C"
