/*
 * Multi-head attention for the CPU oracle (test infrastructure only; see
 * oracle.h).  Restates device/cpu/attention/compute.go:31-90
 * (dispatchMultiHeadAttention, multiHeadAttentionSlices) and
 * typed_compute.go:10-29,142-237 (typedRowDot, computeHeadScoresTyped,
 * writeHeadOutputTyped, runSingleHeadTyped) with softmax.go:5-84
 * (stableSoftmaxRow: f32 max, exp in float64, sequential f32 sum, divide).
 *
 * Layout (no batch dimension, as in the reference): Q/O [seqQ, H*D],
 * K/V [seqK, Hkv*D]; query head h reads kv head h / (H/Hkv).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static float row_dot(const void *a, size_t ao, const void *b, size_t bo, int64_t n, int dtype) {
    float s = 0.0f;
    for (int64_t i = 0; i < n; ++i) s += or_load(a, ao + (size_t)i, dtype) * or_load(b, bo + (size_t)i, dtype);
    if (dtype == OR_BF16) return or_bf16_to_f32(or_f32_to_bf16(s));
    if (dtype == OR_F16) return or_f16_to_f32(or_f32_to_f16(s));
    return s;
}

/* stableSoftmaxRow softmax.go:5-18 with normalizeInfiniteSoftmaxRow :33-75 */
static void stable_softmax(float *s, int64_t n) {
    if (n == 0) return;
    float m = s[0];
    for (int64_t i = 1; i < n; ++i)
        if (s[i] > m) m = s[i];
    if (isinf(m)) {
        int64_t pos = 0;
        if (m > 0)
            for (int64_t i = 0; i < n; ++i) pos += (isinf(s[i]) && s[i] > 0);
        if (m < 0 || pos == 0) {
            for (int64_t i = 0; i < n; ++i) s[i] = 0;
            return;
        }
        float w = 1 / (float)pos;
        for (int64_t i = 0; i < n; ++i) s[i] = (isinf(s[i]) && s[i] > 0) ? w : 0;
        return;
    }
    float sum = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
        float e = (float)exp((double)(s[i] - m));
        s[i] = e;
        sum += e;
    }
    if (sum == 0) return;
    for (int64_t i = 0; i < n; ++i) s[i] /= sum;
}

int or_mha_rows(const or_mha_config *c, const void *query, const void *key,
                const void *value, void *output, int64_t seq_q, int64_t seq_k,
                int64_t head_begin, int64_t head_end, int64_t q_begin, int64_t q_end,
                int dtype) {
    if (dtype != OR_F32 && dtype != OR_BF16 && dtype != OR_F16) return -6;
    if (c->num_heads <= 0 || c->head_dim <= 0) return -6;
    int64_t kv_heads = c->kv_head_count > 0 ? c->kv_head_count : c->num_heads;
    if (c->num_heads % kv_heads != 0) return -6;
    if (seq_q == 0 || seq_k == 0) return 0;
    int64_t D = c->head_dim, H = c->num_heads;
    int64_t group = H / kv_heads;
    float scale = (float)(1.0 / sqrt((double)D));
    int64_t q_stride = H * D, kv_stride = kv_heads * D;
    int64_t nq = q_end - q_begin, nh = head_end - head_begin;
    if (nq <= 0 || nh <= 0) return 0;
#pragma omp parallel num_threads(oracle_get_threads())
    {
        float *scores = (float *)malloc(sizeof(float) * (size_t)seq_k);
#pragma omp for schedule(dynamic, 4)
        for (int64_t w = 0; w < nq * nh; ++w) {
            int64_t h = head_begin + w / nq;
            int64_t q = q_begin + w % nq;
            int64_t kvh = h / group;
            size_t qo = (size_t)(q * q_stride + h * D);
            for (int64_t k = 0; k < seq_k; ++k) {
                float sc = row_dot(query, qo, key, (size_t)(k * kv_stride + kvh * D), D, dtype) * scale;
                if (c->causal && k > q + seq_k - seq_q) sc = -INFINITY;
                if (c->window_size > 0 && q - k >= c->window_size) sc = -INFINITY;
                if (c->alibi_slope != 0) sc += c->alibi_slope * (float)(k - q);
                scores[k] = sc;
            }
            stable_softmax(scores, seq_k);
            for (int64_t d = 0; d < D; ++d) {
                float sum = 0.0f;
                for (int64_t k = 0; k < seq_k; ++k)
                    sum += scores[k] * or_load(value, (size_t)(k * kv_stride + kvh * D + d), dtype);
                or_store(output, qo + (size_t)d, sum, dtype);
            }
        }
        free(scores);
    }
    return 0;
}

int or_mha(const or_mha_config *config, const void *query, const void *key, const void *value,
           void *output, int64_t seq_q, int64_t seq_k, int dtype) {
    return or_mha_rows(config, query, key, value, output, seq_q, seq_k, 0, config->num_heads, 0,
                       seq_q, dtype);
}

/* Paged decode as the reference runs it (execution/page_intrinsic.go:217-352 then
 * bind_router.go:640-684): gather the sequence's rows of the K and V page pools
 * through its page table, then MultiHeadAttention with seqQ = 1 (causal mask is
 * bottom-right aligned, so the one query sees every key).
 * Pools: [pages, page_size, kv_heads, head_dim]; table [batch, max_pages_per_seq].
 * bf16 and f16 caches follow the MHA path of their dtype (query and output in
 * the same dtype).  fp8-E4M3 caches have no reference
 * counterpart (device/cpu/shape/page.go:213-378 stops at f32/f16/bf16): they are
 * dequantised to f32 as decode(byte) * scale[kv head] and run through the f32
 * MHA path with the bf16 query widened; the output is stored as bf16. */
int or_paged_decode(const void *query, const void *key_pages, const void *value_pages,
                    const int32_t *page_table, const int32_t *context_lens,
                    int64_t batch, int64_t max_pages_per_seq, int64_t page_size,
                    int64_t num_heads, int64_t kv_heads, int64_t head_dim,
                    const float *k_scale, const float *v_scale, int kv_dtype,
                    void *output) {
    if (kv_dtype != OR_BF16 && kv_dtype != OR_F16 && kv_dtype != OR_F8E4M3) return -6;
    int64_t inner = kv_heads * head_dim;
    or_mha_config c = {num_heads, head_dim, 1, 0, 0.0f, kv_heads};
    for (int64_t b = 0; b < batch; ++b) {
        int64_t ctx = context_lens[b];
        if (ctx <= 0 || ctx > max_pages_per_seq * page_size) return -6;
        const int32_t *table = page_table + b * max_pages_per_seq;
        const uint16_t *q16 = (const uint16_t *)query + b * num_heads * head_dim;
        uint16_t *o16 = (uint16_t *)output + b * num_heads * head_dim;
        if (kv_dtype == OR_BF16 || kv_dtype == OR_F16) {
            uint16_t *kb = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)(ctx * inner));
            uint16_t *vb = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)(ctx * inner));
            for (int64_t r = 0; r < ctx; ++r) {
                size_t slot = (size_t)((int64_t)table[r / page_size] * page_size + r % page_size);
                memcpy(kb + r * inner, (const uint16_t *)key_pages + slot * inner, sizeof(uint16_t) * inner);
                memcpy(vb + r * inner, (const uint16_t *)value_pages + slot * inner, sizeof(uint16_t) * inner);
            }
            or_mha(&c, q16, kb, vb, o16, 1, ctx, kv_dtype);
            free(kb);
            free(vb);
        } else {
            float *kf = (float *)malloc(sizeof(float) * (size_t)(ctx * inner));
            float *vf = (float *)malloc(sizeof(float) * (size_t)(ctx * inner));
            float *qf = (float *)malloc(sizeof(float) * (size_t)(num_heads * head_dim));
            float *of = (float *)malloc(sizeof(float) * (size_t)(num_heads * head_dim));
            for (int64_t r = 0; r < ctx; ++r) {
                size_t slot = (size_t)((int64_t)table[r / page_size] * page_size + r % page_size);
                const uint8_t *ks = (const uint8_t *)key_pages + slot * inner;
                const uint8_t *vs = (const uint8_t *)value_pages + slot * inner;
                for (int64_t i = 0; i < inner; ++i) {
                    kf[r * inner + i] = or_e4m3_to_f32(ks[i]) * k_scale[i / head_dim];
                    vf[r * inner + i] = or_e4m3_to_f32(vs[i]) * v_scale[i / head_dim];
                }
            }
            for (int64_t i = 0; i < num_heads * head_dim; ++i) qf[i] = or_bf16_to_f32(q16[i]);
            or_mha(&c, qf, kf, vf, of, 1, ctx, OR_F32);
            for (int64_t i = 0; i < num_heads * head_dim; ++i) o16[i] = or_f32_to_bf16(of[i]);
            free(kf);
            free(vf);
            free(qf);
            free(of);
        }
    }
    return 0;
}

/* flashExpFloat32, device/cpu/attention/flash_attention.go:171-189: -inf or
 * anything below -88 is 0, +inf stays +inf, otherwise Activation.Exp, whose
 * generic f32 kernel is math.FastExp32 (activation/f32_generic.go:9-16). */
static float flash_exp(float v) {
    if (isinf(v) && v < 0) return 0.0f;
    if (v < -88.0f) return 0.0f;
    if (isinf(v)) return INFINITY;
    return or_fast_exp32(v);
}

/* ScaledDotProductAttention / FlashAttention (single head), restating
 * device/cpu/attention/compute.go:10-29,54-68 (dispatch: zero seqQ or seqK is a
 * no-op; scale = float32(1/sqrt(float64(depth)))) and the per-row online
 * softmax of typed_compute.go:31-97 (16-bit dtypes) and
 * select_flash_amd64.go:133-177 (f32): for every visible key in order
 * (causal hides key > row, top-left aligned), score = dot * scale (16-bit
 * dots rounded to the 16-bit format), running max, alpha =
 * flashExp(oldMax - max), shifted = flashExp(score - max), normalizer =
 * normalizer * alpha + shifted, acc[d] = acc[d] * alpha + v[d] * shifted;
 * output acc[d] * (1 / normalizer), or zeros when the normalizer is 0.
 * Layout: Q [seqQ, depth], K [seqK, depth], V [seqK, valueDim],
 * O [seqQ, valueDim]. */
int or_flash_attention(int causal, const void *query, const void *key, const void *value,
                       void *output, int64_t seq_q, int64_t seq_k, int64_t depth,
                       int64_t value_dim, int dtype) {
    if (dtype != OR_F32 && dtype != OR_BF16 && dtype != OR_F16) return -6;
    if (seq_q == 0 || seq_k == 0) return 0;
    if (seq_q < 0 || seq_k < 0 || depth <= 0 || value_dim < 0) return -6;
    const float scale = (float)(1.0 / sqrt((double)depth));
    float *acc = (float *)malloc(sizeof(float) * (size_t)(value_dim > 0 ? value_dim : 1));
    for (int64_t r = 0; r < seq_q; ++r) {
        float mx = -INFINITY, norm = 0.0f;
        for (int64_t d = 0; d < value_dim; ++d) acc[d] = 0.0f;
        for (int64_t k = 0; k < seq_k; ++k) {
            if (causal && k > r) continue;
            float score = row_dot(query, (size_t)(r * depth), key, (size_t)(k * depth), depth, dtype) * scale;
            float old = mx;
            if (score > mx) mx = score;
            float alpha = flash_exp(old - mx);
            float shifted = flash_exp(score - mx);
            norm = norm * alpha + shifted;
            for (int64_t d = 0; d < value_dim; ++d)
                acc[d] = acc[d] * alpha + or_load(value, (size_t)(k * value_dim + d), dtype) * shifted;
        }
        if (norm == 0) {
            for (int64_t d = 0; d < value_dim; ++d) or_store(output, (size_t)(r * value_dim + d), 0.0f, dtype);
            continue;
        }
        float inv = 1.0f / norm;
        for (int64_t d = 0; d < value_dim; ++d)
            or_store(output, (size_t)(r * value_dim + d), acc[d] * inv, dtype);
    }
    free(acc);
    return 0;
}
