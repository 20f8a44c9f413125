// MultiHeadAttention (GQA, causal, sliding window, ALiBi) for any dtype.
// Reference: device/cpu/attention/compute.go:31-90 and typed_compute.go:10-237:
// kv head = h / (H / Hkv); scale = float32(1/sqrt(float64(D))); score = dot * scale
// (16-bit dots rounded to the 16-bit format); causal mask k > q + seqK - seqQ;
// window mask q - k >= WindowSize; ALiBi score += slope * (k - q); softmax;
// out[d] = sum_k p_k v[k, d]; an all-masked row yields zeros (softmax.go:33-75).
//
// This file holds the general kernel (one block per (batch, head, query row),
// online softmax over 256-key chunks, one key's score per thread, P.V split over
// all 256 threads for head dims up to 128, f32 accumulation) and the
// dispatch: one query row in bf16 / f16 at head dim 128 without ALiBi goes to the
// split-K decode kernels (decode.hip), any other row alone over more than 768
// keys (few rows and heads) to this kernel split over 256-key chunks (partials
// merged by mha_split_combine_kernel); bf16 / f16 causal or non-causal prefill at head
// dim 128 or 64, with or without a sliding window or ALiBi, to the MFMA flash
// kernel (prefill.hip).
#include "attention.hpp"

namespace puter {

// SPLIT (one query row, seq_q == 1): block (split, head, batch) takes the
// 256-key chunk `split` of the row's visible keys and writes its (max, sum) and
// unnormalised output to a.part_ml / a.part_o; mha_split_combine_kernel merges
// the chunks in order.
template <int DT, bool SPLIT>
__global__ __launch_bounds__(256) void mha_generic_kernel(MhaArgs a) {
    using T = typename Elem<DT>::T;
    __shared__ float qrow[256];
    __shared__ float pk[256];
    __shared__ float red[4];
    __shared__ float accs[256];
    const int64_t qi = SPLIT ? 0 : blockIdx.x;
    const int64_t h = blockIdx.y;
    const int64_t b = blockIdx.z;
    const int tid = threadIdx.x;
    const int64_t D = a.dim;
    const int64_t group = a.heads / a.kv_heads;
    const int64_t kvh = h / group;
    const int64_t qs = a.heads * D, ks = a.kv_heads * D;
    const T *Q = reinterpret_cast<const T *>(a.q) + (b * a.seq_q + qi) * qs + h * D;
    const T *K = reinterpret_cast<const T *>(a.k) + b * a.seq_k * ks + kvh * D;
    const T *V = reinterpret_cast<const T *>(a.v) + b * a.seq_k * ks + kvh * D;
    T *O = reinterpret_cast<T *>(a.o) + (b * a.seq_q + qi) * qs + h * D;
    for (int64_t d = tid; d < D; d += 256) qrow[d] = Elem<DT>::load(Q[d]);
    __syncthreads();
    // P.V: thread tid sums output dim tid % DR over the keys j of each chunk with
    // j % parts == tid / DR (parts = 256 / DR independent partial sums for D <= 128,
    // added in part order at the end)
    const int DR = D <= 64 ? 64 : D <= 128 ? 128 : 256;
    const int parts = 256 / DR, dd = tid % DR, part = tid / DR;
    // keys visible to this row form [k_lo, k_hi)
    int64_t k_hi = a.seq_k;
    if (a.causal) k_hi = min(k_hi, qi + a.shift + 1);
    int64_t k_lo = 0;
    if (a.window > 0) k_lo = max(k_lo, qi - a.window + 1);
    if (SPLIT) {   // this block's chunk
        k_lo += 256 * (int64_t)blockIdx.x;
        k_hi = min(k_hi, k_lo + 256);
    }
    float m = -INFINITY, l = 0.0f, acc = 0.0f;
    const int wave = tid >> 6, lane = tid & 63;
    for (int64_t c0 = k_lo; c0 < k_hi; c0 += 256) {
        const int64_t k = c0 + tid;
        float s = -INFINITY;
        if (k < k_hi) {
            const T *kr = K + k * ks;
            float dot = 0.0f;
            // sixteen loads in flight per step, products added in index order
            int64_t d = 0;
            for (; d + 16 <= D; d += 16) {
                float kv[16];
#pragma unroll
                for (int u = 0; u < 16; ++u) kv[u] = Elem<DT>::load(kr[d + u]);
#pragma unroll
                for (int u = 0; u < 16; ++u) dot += qrow[d + u] * kv[u];
            }
            for (; d < D; ++d) dot += qrow[d] * Elem<DT>::load(kr[d]);
            s = round_reduction<DT>(dot) * a.scale;
            if (a.alibi != 0.0f) s += a.alibi * (float)(k - qi);
        }
        float cm = wave_max(s);
        __syncthreads();
        if (lane == 0) red[wave] = cm;
        __syncthreads();
        cm = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        const float m_new = fmaxf(m, cm);
        const float p = (s == -INFINITY) ? 0.0f : expf(s - m_new);
        pk[tid] = p;
        float ps = wave_sum(p);
        __syncthreads();
        if (lane == 0) red[wave] = ps;
        __syncthreads();
        ps = red[0] + red[1] + red[2] + red[3];
        const float alpha = (m == -INFINITY) ? 0.0f : expf(m - m_new);
        l = l * alpha + ps;
        if (dd < D) {
            float pp = 0.0f;
            const int64_t n = min((int64_t)256, k_hi - c0);
            // eight loads in flight per step (a loop with a run-time stride is not
            // unrolled by the compiler), products added in key order
            int64_t j = part;
            for (; j + 7 * parts < n; j += 8 * parts) {
                float vv[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) vv[u] = Elem<DT>::load(V[(c0 + j + u * parts) * ks + dd]);
#pragma unroll
                for (int u = 0; u < 8; ++u) pp += pk[j + u * parts] * vv[u];
            }
            for (; j < n; j += parts) pp += pk[j] * Elem<DT>::load(V[(c0 + j) * ks + dd]);
            acc = acc * alpha + pp;
        }
        m = m_new;
        __syncthreads();
    }
    accs[tid] = acc;
    __syncthreads();
    if (tid < D) {
        float t = accs[tid];
        for (int p = 1; p < parts; ++p) t += accs[p * DR + tid];
        if constexpr (SPLIT) {
            const int64_t slot = (b * a.heads + h) * gridDim.x + blockIdx.x;
            a.part_o[slot * D + tid] = t;
            if (tid == 0) a.part_ml[slot] = make_float2(m, l);
        } else {
            O[tid] = Elem<DT>::store(l > 0.0f ? t / l : 0.0f);
        }
    }
}

// Merges the splits of one-row general attention: block (head, batch), thread d:
// O[d] = sum_s o_s[d] e^(m_s - M) / sum_s l_s e^(m_s - M), M the largest m_s,
// the splits added in order; a row with no visible key is zero.
template <int DT>
__global__ __launch_bounds__(256) void mha_split_combine_kernel(MhaArgs a, int splits) {
    using T = typename Elem<DT>::T;
    const int64_t h = blockIdx.x, b = blockIdx.y;
    const int d = threadIdx.x;
    if (d >= a.dim) return;
    const int64_t base = (b * a.heads + h) * splits;
    float M = -INFINITY;
    for (int s = 0; s < splits; ++s) M = fmaxf(M, a.part_ml[base + s].x);
    float L = 0.0f, O = 0.0f;
    if (M != -INFINITY) {
        for (int s = 0; s < splits; ++s) {
            const float2 ml = a.part_ml[base + s];
            const float f = ml.x == -INFINITY ? 0.0f : expf(ml.x - M);
            L += ml.y * f;
            O += a.part_o[(base + s) * a.dim + d] * f;
        }
    }
    reinterpret_cast<T *>(a.o)[(b * a.seq_q) * a.heads * a.dim + h * a.dim + d] =
        Elem<DT>::store(L > 0.0f ? O / L : 0.0f);
}

// One query row over more than 256 keys (what the decode kernels do not take):
// the general kernel split over 256-key chunks, partials in the library's scratch.
template <int DT>
static int run_mha_split(MhaArgs a, hipStream_t s) {
    const int64_t splits = (a.seq_k + 255) / 256;
    const size_t need = (size_t)(a.batch * a.heads * splits) * (sizeof(float2) + (size_t)a.dim * sizeof(float));
    ScratchLease lease(need, s);
    if (lease.status()) return lease.status();
    a.part_ml = static_cast<float2 *>(lease.ptr());
    a.part_o = reinterpret_cast<float *>(a.part_ml + a.batch * a.heads * splits);
    mha_generic_kernel<DT, true><<<dim3((unsigned)splits, (unsigned)a.heads, (unsigned)a.batch), 256, 0, s>>>(a);
    mha_split_combine_kernel<DT><<<dim3((unsigned)a.heads, (unsigned)a.batch), 256, 0, s>>>(a, (int)splits);
    const int rc = check_launch("mha split");
    const int fin = lease.finish();
    return rc ? rc : fin;
}

static int run_mha(const puter_mha_config *config, const void *q, const void *k, const void *v,
                   void *o, int64_t batch, int64_t seq_q, int64_t seq_k, int dtype, hipStream_t s) {
    if (!config) return fail(PUTER_ERR_NIL, "mha: nil config");
    if (!is_norm_dtype(dtype)) return fail(PUTER_ERR_INVALID, "mha: unsupported dtype %d", dtype);
    if (batch < 0 || seq_q < 0 || seq_k < 0) return fail(PUTER_ERR_INVALID, "mha: negative shape");
    const int64_t H = config->num_heads, D = config->head_dim;
    const int64_t kvh = config->kv_head_count > 0 ? config->kv_head_count : H;
    if (H <= 0 || D <= 0) return fail(PUTER_ERR_INVALID, "mha: heads and head_dim must be positive");
    if (H % kvh != 0) return fail(PUTER_ERR_INVALID, "mha: %lld heads not divisible by %lld kv heads",
                                  (long long)H, (long long)kvh);
    if (D > 256) return fail(PUTER_ERR_INVALID, "mha: head_dim %lld > 256 unsupported", (long long)D);
    if (batch == 0 || seq_q == 0 || seq_k == 0) return PUTER_OK;
    if (!q || !k || !v || !o) return fail(PUTER_ERR_NIL, "mha: nil buffer");
    if (seq_q > 0x7FFFFFFF || H > 65535 || batch > 65535) return fail(PUTER_ERR_INVALID, "mha: grid too large");
    MhaArgs a{q, k, v, o, batch, seq_q, seq_k, H, kvh, D, config->causal ? 1 : 0,
              config->window_size, config->alibi_slope, (float)(1.0 / sqrt((double)D)), seq_k - seq_q};
    int status = PUTER_OK;
    if (launch_decode_contiguous(a, dtype, s, &status)) return status;
    // any other query row alone over at least four 256-key chunks, when the rows
    // and heads alone do not fill the GPU: its visible keys are all seq_k (a causal
    // row 0 sees k <= seq_k - 1, and a window compares keys with row index 0), split
    // over the chunks (bf16 8 x 64 heads over 4096 keys: 61 -> 21.5 us; two chunks
    // lost to the extra launch: 10.1 against 17.1 us over 512 keys)
    if (seq_q == 1 && seq_k > 768 && batch * H < 2048 && (seq_k + 255) / 256 <= 0x7FFFFFFF) {
        switch (dtype) {
        case PUTER_F32: return run_mha_split<PUTER_F32>(a, s);
        case PUTER_BF16: return run_mha_split<PUTER_BF16>(a, s);
        case PUTER_F16: return run_mha_split<PUTER_F16>(a, s);
        }
    }
    if (launch_prefill_mfma(a, dtype, s, &status)) return status;
    const dim3 grid((unsigned)seq_q, (unsigned)H, (unsigned)batch);
    switch (dtype) {
    case PUTER_F32: mha_generic_kernel<PUTER_F32, false><<<grid, 256, 0, s>>>(a); break;
    case PUTER_BF16: mha_generic_kernel<PUTER_BF16, false><<<grid, 256, 0, s>>>(a); break;
    case PUTER_F16: mha_generic_kernel<PUTER_F16, false><<<grid, 256, 0, s>>>(a); break;
    }
    return check_launch("mha");
}

}  // namespace puter

using namespace puter;

extern "C" {

int puter_hip_multi_head_attention(const puter_mha_config *config, const void *query,
                                   const void *key, const void *value, void *output,
                                   int64_t seq_q, int64_t seq_k, int dtype, void *stream) {
    return run_mha(config, query, key, value, output, 1, seq_q, seq_k, dtype, as_stream(stream));
}

int puter_hip_multi_head_attention_batched(const puter_mha_config *config, const void *query,
                                           const void *key, const void *value, void *output,
                                           int64_t batch, int64_t seq_q, int64_t seq_k,
                                           int dtype, void *stream) {
    return run_mha(config, query, key, value, output, batch, seq_q, seq_k, dtype, as_stream(stream));
}

}  // extern "C"
