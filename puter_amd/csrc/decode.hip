// Paged-KV decode attention (one query token per sequence, GQA), bf16 or
// fp8-E4M3 KV with a per-kv-head fp32 scale.
//
// Reference path: KVPageGather of K and V through the sequence's page table
// (execution/page_intrinsic.go:217-352, device/cpu/shape/page_generic.go:45-63)
// followed by MultiHeadAttention with seqQ = 1 (bind_router.go:640-684,
// device/cpu/attention/typed_compute.go:142-237).  Here the gather is fused:
// the kernel reads K/V rows straight from the page pools (no materialised
// [ctx, Hkv*D] copies), so HBM traffic is the KV bytes read once.
//
// Split-K ("flash decoding"): grid = (splits of kSplit tokens, kv head, batch).
// In a block, a group of LPT lanes owns one token (LPT x 16 B = the token's
// D-element K row of this kv head), so every group load is one contiguous
// 256 B (bf16) / 128 B (fp8) burst.  Each group keeps an online softmax for
// the G = Hq/Hkv query heads that share the kv head; groups merge through
// shuffles and LDS, and the block writes (m, l, o[D]) per query head.  A
// second kernel merges the splits by log-sum-exp and writes bf16.
#include "common.hpp"

namespace puter {

constexpr int kSplit = 256;   // tokens per split

struct DecodeArgs {
    const uint16_t *q;
    const void *kp, *vp;
    const int32_t *table, *ctx;
    const float *ks, *vs;
    uint16_t *out;
    float *part_o, *part_ml;
    int64_t batch, max_pages, page_size, num_pages, heads, kv_heads, max_splits, max_context;
    float scale;
};

template <int DT, int G>
__global__ __launch_bounds__(256) void decode_split_kernel(DecodeArgs a) {
#pragma clang fp contract(off)
    constexpr int D = 128;
    constexpr int ES = DT == PUTER_BF16 ? 2 : 1;
    constexpr int EPL = 16 / ES;              // elements per lane
    constexpr int LPT = D / EPL;              // lanes per token: 16 (bf16) / 8 (fp8)
    constexpr int TPW = 64 / LPT;             // tokens per wave step
    constexpr int TPB = TPW * 4;              // tokens per block step
    constexpr int STEPS = kSplit / TPB;
    __shared__ float red_m[4][G], red_l[4][G];
    __shared__ float red_o[4][G][D];

    const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    const int ctx = (int)min((int64_t)a.ctx[b], a.max_context);
    const int t0 = split * kSplit;
    if (t0 >= ctx) return;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int grp = lane / LPT, sub = lane % LPT;
    const int64_t inner = a.kv_heads * D;

    // query slice: G heads x EPL dims (this lane's dims sub*EPL ..)
    float q[G][EPL];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const uint16_t *qh = a.q + ((int64_t)b * a.heads + (int64_t)kvh * G + g) * D + sub * EPL;
#pragma unroll
        for (int i = 0; i < EPL; ++i) q[g][i] = bf16_to_f32(qh[i]);
    }
    const float kscale = DT == PUTER_BF16 ? 1.0f : a.ks[kvh];
    const int32_t *table = a.table + (int64_t)b * a.max_pages;

    float m[G], l[G], acc[G][EPL];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.0f;
#pragma unroll
        for (int i = 0; i < EPL; ++i) acc[g][i] = 0.0f;
    }

#pragma unroll 2
    for (int step = 0; step < STEPS; ++step) {
        const int t = t0 + step * TPB + wave * TPW + grp;
        if (t0 + step * TPB >= ctx) break;
        const bool valid = t < ctx;
        uint4 kv = make_uint4(0, 0, 0, 0), vv = make_uint4(0, 0, 0, 0);
        const int32_t page = valid ? table[t / a.page_size] : -1;
        const bool live = valid && page >= 0 && page < a.num_pages;  // bad ids read nothing
        if (live) {
            const int64_t row = (int64_t)page * a.page_size + t % a.page_size;
            const size_t off = (size_t)(row * inner + (int64_t)kvh * D) * ES + sub * 16;
            kv = ld_stream(reinterpret_cast<const uint4 *>(static_cast<const char *>(a.kp) + off));
            vv = ld_stream(reinterpret_cast<const uint4 *>(static_cast<const char *>(a.vp) + off));
        }
        float kf[EPL], vf[EPL];
        unpack_vec<DT>(kv, kf);
        unpack_vec<DT>(vv, vf);
        float s[G];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float d = 0.0f;
#pragma unroll
            for (int i = 0; i < EPL; ++i) d += q[g][i] * kf[i];
#pragma unroll
            for (int off = LPT / 2; off >= 1; off >>= 1) d += __shfl_xor(d, off, 64);
            if constexpr (DT == PUTER_BF16) s[g] = round_reduction<PUTER_BF16>(d) * a.scale;
            else s[g] = d * kscale * a.scale;
            if (!live) s[g] = -INFINITY;
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float mn = fmaxf(m[g], s[g]);
            const float alpha = m[g] == -INFINITY ? 0.0f : __expf(m[g] - mn);
            const float p = s[g] == -INFINITY ? 0.0f : __expf(s[g] - mn);
            l[g] = l[g] * alpha + p;
#pragma unroll
            for (int i = 0; i < EPL; ++i) acc[g][i] = acc[g][i] * alpha + p * vf[i];
            m[g] = mn;
        }
    }

    // merge the TPW token groups of the wave (lanes differing in the group bits)
#pragma unroll
    for (int off = LPT; off < 64; off <<= 1) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float mo = __shfl_xor(m[g], off, 64);
            const float lo = __shfl_xor(l[g], off, 64);
            const float mn = fmaxf(m[g], mo);
            const float fa = m[g] == -INFINITY ? 0.0f : __expf(m[g] - mn);
            const float fb = mo == -INFINITY ? 0.0f : __expf(mo - mn);
            l[g] = l[g] * fa + lo * fb;
#pragma unroll
            for (int i = 0; i < EPL; ++i) {
                const float ao = __shfl_xor(acc[g][i], off, 64);
                acc[g][i] = acc[g][i] * fa + ao * fb;
            }
            m[g] = mn;
        }
    }
    if (grp == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            if (sub == 0) { red_m[wave][g] = m[g]; red_l[wave][g] = l[g]; }
#pragma unroll
            for (int i = 0; i < EPL; ++i) red_o[wave][g][sub * EPL + i] = acc[g][i];
        }
    }
    __syncthreads();
    // 4 waves -> one partial per query head; thread layout: g = tid / D, d = tid % D
    for (int idx = threadIdx.x; idx < G * D; idx += 256) {
        const int g = idx / D, d = idx % D;
        float M = -INFINITY;
        for (int w = 0; w < 4; ++w) M = fmaxf(M, red_m[w][g]);
        float L = 0.0f, O = 0.0f;
        for (int w = 0; w < 4; ++w) {
            const float f = red_m[w][g] == -INFINITY ? 0.0f : __expf(red_m[w][g] - M);
            L += red_l[w][g] * f;
            O += red_o[w][g][d] * f;
        }
        const int64_t h = (int64_t)kvh * G + g;
        const int64_t slot = ((int64_t)b * a.heads + h) * a.max_splits + split;
        a.part_o[slot * D + d] = O;
        if (d == 0) {
            a.part_ml[slot * 2] = M;
            a.part_ml[slot * 2 + 1] = L;
        }
    }
}

template <int DT>
__global__ __launch_bounds__(128) void decode_combine_kernel(DecodeArgs a) {
    constexpr int D = 128;
    const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
    const int ctx = (int)min((int64_t)a.ctx[b], a.max_context);
    const int nsplit = (ctx + kSplit - 1) / kSplit;
    const int64_t base = ((int64_t)b * a.heads + h) * a.max_splits;
    float M = -INFINITY;
    for (int s = 0; s < nsplit; ++s) M = fmaxf(M, a.part_ml[(base + s) * 2]);
    float L = 0.0f, O = 0.0f;
    for (int s = 0; s < nsplit; ++s) {
        const float ms = a.part_ml[(base + s) * 2];
        const float f = ms == -INFINITY ? 0.0f : __expf(ms - M);
        L += a.part_ml[(base + s) * 2 + 1] * f;
        O += a.part_o[(base + s) * D + d] * f;
    }
    float r = L > 0.0f ? O / L : 0.0f;
    if constexpr (DT != PUTER_BF16) r *= a.vs[h / (a.heads / a.kv_heads)];
    a.out[((int64_t)b * a.heads + h) * D + d] = (uint16_t)f32_to_bf16(r);
}

static int64_t splits_for(int64_t max_context) { return (max_context + kSplit - 1) / kSplit; }

}  // namespace puter

using namespace puter;

extern "C" {

size_t puter_hip_paged_decode_workspace_bytes(int64_t batch, int64_t num_heads, int64_t head_dim,
                                              int64_t max_context) {
    if (batch <= 0 || num_heads <= 0 || head_dim <= 0 || max_context <= 0) return 0;
    const int64_t slots = batch * num_heads * splits_for(max_context);
    return (size_t)(slots * (head_dim + 2)) * sizeof(float);
}

int puter_hip_paged_decode_attention(const void *query, const void *key_pages,
                                     const void *value_pages, const int32_t *page_table,
                                     const int32_t *context_lens, int64_t batch,
                                     int64_t max_pages_per_seq, int64_t page_size,
                                     int64_t num_pages, int64_t num_heads, int64_t kv_heads, int64_t head_dim,
                                     int64_t max_context, const float *k_scale,
                                     const float *v_scale, int kv_dtype, void *output,
                                     void *workspace, size_t workspace_bytes, void *stream) {
    if (batch < 0 || max_pages_per_seq < 0 || page_size <= 0 || num_pages < 0 || num_heads <= 0 || kv_heads <= 0)
        return fail(PUTER_ERR_INVALID, "paged decode: invalid shape");
    if (batch == 0) return PUTER_OK;
    if (head_dim != 128) return fail(PUTER_ERR_INVALID, "paged decode: head_dim %lld unsupported (128)", (long long)head_dim);
    if (num_heads % kv_heads != 0) return fail(PUTER_ERR_INVALID, "paged decode: heads not divisible by kv heads");
    const int64_t G = num_heads / kv_heads;
    if (G != 1 && G != 2 && G != 4 && G != 8) return fail(PUTER_ERR_INVALID, "paged decode: group size %lld unsupported", (long long)G);
    if (kv_dtype != PUTER_BF16 && kv_dtype != PUTER_F8E4M3) return fail(PUTER_ERR_INVALID, "paged decode: kv dtype %d unsupported", kv_dtype);
    if (max_context <= 0 || max_context > max_pages_per_seq * page_size)
        return fail(PUTER_ERR_INVALID, "paged decode: max_context must be in [1, max_pages_per_seq*page_size]");
    if (!query || !key_pages || !value_pages || !page_table || !context_lens || !output || !workspace)
        return fail(PUTER_ERR_NIL, "paged decode: nil buffer");
    if (kv_dtype == PUTER_F8E4M3 && (!k_scale || !v_scale)) return fail(PUTER_ERR_NIL, "paged decode: fp8 needs scales");
    const size_t need = puter_hip_paged_decode_workspace_bytes(batch, num_heads, head_dim, max_context);
    if (workspace_bytes < need) return fail(PUTER_ERR_INVALID, "paged decode: workspace %zu < %zu bytes", workspace_bytes, need);
    const int64_t splits = splits_for(max_context);
    if (splits > 0x7FFFFFFF || batch > 65535 || kv_heads > 65535) return fail(PUTER_ERR_INVALID, "paged decode: grid too large");
    float *ws = static_cast<float *>(workspace);
    const int64_t slots = batch * num_heads * splits;
    DecodeArgs a{static_cast<const uint16_t *>(query), key_pages, value_pages, page_table, context_lens,
                 k_scale, v_scale, static_cast<uint16_t *>(output), ws, ws + slots * head_dim,
                 batch, max_pages_per_seq, page_size, num_pages, num_heads, kv_heads, splits,
                 max_context, (float)(1.0 / sqrt((double)head_dim))};
    hipStream_t s = as_stream(stream);
    const dim3 grid((unsigned)splits, (unsigned)kv_heads, (unsigned)batch);
#define PUTER_DECODE(DT)                                                              \
    switch (G) {                                                                      \
    case 1: decode_split_kernel<DT, 1><<<grid, 256, 0, s>>>(a); break;                \
    case 2: decode_split_kernel<DT, 2><<<grid, 256, 0, s>>>(a); break;                \
    case 4: decode_split_kernel<DT, 4><<<grid, 256, 0, s>>>(a); break;                \
    case 8: decode_split_kernel<DT, 8><<<grid, 256, 0, s>>>(a); break;                \
    }                                                                                 \
    decode_combine_kernel<DT><<<dim3((unsigned)num_heads, (unsigned)batch), 128, 0, s>>>(a);
    if (kv_dtype == PUTER_BF16) { PUTER_DECODE(PUTER_BF16) }
    else { PUTER_DECODE(PUTER_F8E4M3) }
#undef PUTER_DECODE
    return check_launch("paged decode");
}

}  // extern "C"
