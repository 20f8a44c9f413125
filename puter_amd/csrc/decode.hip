// Paged-KV decode attention (one query token per sequence, GQA), bf16 or
// fp8-E4M3 KV with a per-kv-head fp32 scale.
//
// Reference path: KVPageGather of K and V through the sequence's page table
// (execution/page_intrinsic.go:217-352, device/cpu/shape/page_generic.go:45-63)
// followed by MultiHeadAttention with seqQ = 1 (bind_router.go:640-684,
// device/cpu/attention/typed_compute.go:142-237).  The gather is fused: K/V
// rows are read straight from the page pools (no materialised [ctx, Hkv*D]
// copies), so HBM traffic is the KV bytes read once.
//
// Split-K ("flash decoding"): grid = (kv head, 256-token splits, batch), the kv
// head fastest so the blocks reading the 8 head slices of the same pages run
// together; each of a block's 4 waves owns 64 consecutive tokens.  (An MFMA
// version of the value product, V^T transposed through LDS, measured slower
// for bf16: its LDS tile halves the blocks per CU of this memory-bound kernel.)
//   scores: S^T[token, head] = K . Q^T with v_mfma_f32_16x16x32_bf16 (A = 16
//     tokens x 32 dims loaded straight from the page pool into registers, B =
//     the G query heads of the kv group, zero-padded to 16 columns); a lane then
//     holds 16 scores of one head, so the softmax over the wave's 64 tokens is
//     an in-lane reduction plus two shuffles - no per-token rescaling.
//   values: O[head, d] += p[head, token] * V[token, d] on the VALU: lane owns 8
//     dims of every 4th token (16-byte V loads), reads the token's G
//     probabilities from a per-wave LDS row, and accumulates G x 8 sums.
// A wave's 4 token-group partials are summed in registers (lane-row swaps),
// the 4 waves' partials merge through LDS into one (m, l, o[D]) per query
// head; decode_combine_kernel merges the splits by log-sum-exp.
#include "common.hpp"

namespace puter {

constexpr int kSplit = 256;  // tokens per split (4 waves x 64)

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

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

// 8 consecutive KV elements of one row as bf16.  fp8-E4M3 is widened with the
// hardware v_cvt_pk_f32_fp8 (OCP E4M3FN on gfx950: exact for every code; every
// E4M3 value is also a bf16 value, so the narrowing to bf16 is exact too).
template <int KV>
__device__ __forceinline__ uint4 load8_as_bf16(const void *pool, size_t elem_off) {
    if constexpr (KV == PUTER_BF16) {
        return ld_stream(reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(pool) + elem_off));
    } else {
        const uint2 raw = *reinterpret_cast<const uint2 *>(static_cast<const uint8_t *>(pool) + elem_off);
        const uint32_t w[2] = {raw.x, raw.y};
        uint32_t o[4];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const auto f0 = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[k], false);  // bytes 0, 1
            const auto f1 = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[k], true);   // bytes 2, 3
            const bf16x2_t h0 = {(__bf16)f0[0], (__bf16)f0[1]};
            const bf16x2_t h1 = {(__bf16)f1[0], (__bf16)f1[1]};
            o[2 * k] = __builtin_bit_cast(uint32_t, h0);
            o[2 * k + 1] = __builtin_bit_cast(uint32_t, h1);
        }
        return make_uint4(o[0], o[1], o[2], o[3]);
    }
}

template <int KV, int G>
__global__ __launch_bounds__(256) void decode_mfma_kernel(DecodeArgs a) {
    constexpr int D = 128;
    __shared__ float p_lds[4][64][G];          // per wave: probabilities [token][head]
    __shared__ float red_m[4][G], red_l[4][G];
    __shared__ float red_o[4][G][D];           // [wave][head][d], token groups already summed

    const int kvh = blockIdx.x, split = blockIdx.y, b = blockIdx.z;
    const int ctx = (int)min((int64_t)a.ctx[b], a.max_context);
    const int t0 = split * kSplit;
    if (t0 >= ctx) return;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int l16 = lane & 15, grp = lane >> 4;
    const int64_t inner = a.kv_heads * D;
    const int ps = (int)a.page_size;
    const int32_t *table = a.table + (int64_t)b * a.max_pages;
    const int tw0 = t0 + wave * 64;

    // B operand (Q^T): lane holds Q[head l16][32t + 8grp .. +7]; heads >= G are zero
    bf16x8_t qb[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        uint4 u = make_uint4(0, 0, 0, 0);
        if (l16 < G)
            u = *reinterpret_cast<const uint4 *>(a.q + ((int64_t)b * a.heads + (int64_t)kvh * G + l16) * D + 32 * t + 8 * grp);
        qb[t] = __builtin_bit_cast(bf16x8_t, u);
    }

    // Token resolution, once per lane: lane L owns token tw0 + L and looks up
    // its page (one coalesced read of the page-table row); the pool row index
    // (page * page_size + slot, -1 for dead tokens and bad page ids, which are
    // masked and never read) is then passed to the lanes that load that token
    // by a cross-lane shuffle.
    int myrow = -1;
    {
        const int tok = tw0 + lane;
        if (tok < ctx) {
            const int pidx = tok / ps;
            const int32_t page = table[pidx];
            if (page >= 0 && page < a.num_pages) myrow = page * ps + (tok - pidx * ps);
        }
    }
    const int64_t head_off = (int64_t)kvh * D;
    auto row_off = [&](int row) -> int64_t { return (int64_t)row * inner + head_off; };

    // K rows for the wave's 4 tiles of 16 tokens (A operand: token l16, dims 32t + 8grp)
    f32x4_t s[4];
    bool klive[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = __shfl(myrow, 16 * i + l16, 64);
        klive[i] = row >= 0;
        const int64_t off = klive[i] ? row_off(row) : 0;
        s[i] = (f32x4_t){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint4 kv = load8_as_bf16<KV>(a.kp, (size_t)(off + 32 * t + 8 * grp));
            s[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kv), qb[t], s[i], 0, 0, 0);
        }
    }
    // V rows this lane accumulates: tokens tw0 + 4k + grp, dims 8*l16 .. +7
    uint4 vv[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const int row = __shfl(myrow, 4 * k + grp, 64);
        const int64_t off = row >= 0 ? row_off(row) : 0;
        const uint4 v = load8_as_bf16<KV>(a.vp, (size_t)(off + 8 * l16));
        vv[k] = row >= 0 ? v : make_uint4(0, 0, 0, 0);   // masked rows contribute exact zeros
    }

    // softmax over the wave's 64 tokens; lane's scores: head l16, tokens 16i + 4grp + r
    const float kscale = KV == PUTER_BF16 ? 1.0f : a.ks[kvh];
    const float c = a.scale * kscale * 1.4426950408889634f;
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int tok = tw0 + 16 * i + 4 * grp + r;
            float v = s[i][r];
            if constexpr (KV == PUTER_BF16) v = round_reduction<PUTER_BF16>(v);  // bf16 dot, typed_compute.go:16-20
            // liveness of this token: the tile's K row owner is lane (4grp + r) of the 16
            const bool live = __shfl(klive[i] ? 1 : 0, 4 * grp + r, 16) != 0;
            v = live ? v * c : -INFINITY;
            s[i][r] = v;
            mx = fmaxf(mx, v);
        }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float mref = mx == -INFINITY ? 0.0f : mx;
    float lsum = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float p = s[i][r] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(s[i][r] - mref);
            lsum += p;
            if (l16 < G) p_lds[wave][16 * i + 4 * grp + r][l16] = p;
        }
    lsum += __shfl_xor(lsum, 16, 64);
    lsum += __shfl_xor(lsum, 32, 64);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");

    // O partial for token group grp: acc[h][j] = sum_k p[h][4k+grp] * V[4k+grp][8 l16 + j]
    float acc[G][8];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[h][j] = 0.0f;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        float v[8];
        unpack_vec<PUTER_BF16>(vv[k], v);
        float p[G];
#pragma unroll
        for (int h = 0; h < G; ++h) p[h] = p_lds[wave][4 * k + grp][h];
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[h][j] = __builtin_fmaf(p[h], v[j], acc[h][j]);
    }
    // sum the 4 token groups (16-lane rows) in registers: permlane16_swap pairs
    // rows (0,1) and (2,3), permlane32_swap then pairs the two halves, leaving
    // the full sum in every row; row grp stores head grp % G's values
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            float v = acc[h][j];
            const auto p16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
            v = __uint_as_float(p16[0]) + __uint_as_float(p16[1]);
            const auto p32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
            acc[h][j] = __uint_as_float(p32[0]) + __uint_as_float(p32[1]);
        }
    if (lane < G) {  // lanes 0..G-1 hold head l16 = lane with grp 0
        red_m[wave][lane] = mx;
        red_l[wave][lane] = lsum;
    }
#pragma unroll
    for (int h = 0; h < G; ++h)
        if ((h & 3) == grp)
#pragma unroll
            for (int j = 0; j < 8; ++j) red_o[wave][h][8 * l16 + j] = acc[h][j];
    __syncthreads();

    // merge the 4 waves -> one partial per query head
    for (int idx = threadIdx.x; idx < G * D; idx += 256) {
        const int h = idx / D, d = idx % D;
        float M = -INFINITY;
        for (int w = 0; w < 4; ++w) M = fmaxf(M, red_m[w][h]);
        float L = 0.0f, O = 0.0f;
        for (int w = 0; w < 4; ++w) {
            const float f = red_m[w][h] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(red_m[w][h] - M);
            L += red_l[w][h] * f;
            O += red_o[w][h][d] * f;
        }
        const int64_t slot = ((int64_t)b * a.heads + (int64_t)kvh * G + h) * a.max_splits + split;
        a.part_o[slot * D + d] = O;
        if (d == 0) {
            a.part_ml[slot * 2] = M;   // log2-domain max of the scaled scores
            a.part_ml[slot * 2 + 1] = L;
        }
    }
}

// One (query head, sequence) per block, one output dim per thread: merge the
// sequence's split partials by log-sum-exp.  The (m, l) pairs are read by
// all threads (the same addresses: one transaction), the split loop is
// unrolled 4-wide so its loads are in flight together.
template <int KV>
__global__ __launch_bounds__(128) void decode_combine_kernel(DecodeArgs a) {
    constexpr int D = 128;
    const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
    const int ctx = (int)min((int64_t)a.ctx[b], a.max_context);
    const int nsplit = (ctx + kSplit - 1) / kSplit;
    const int64_t base = ((int64_t)b * a.heads + h) * a.max_splits;
    const float2 *ml = reinterpret_cast<const float2 *>(a.part_ml) + base;
    const float *po = a.part_o + base * D + d;
    float M = -INFINITY;
    for (int s = 0; s < nsplit; ++s) M = fmaxf(M, ml[s].x);
    float L = 0.0f, O = 0.0f;
    int s = 0;
    for (; s + 4 <= nsplit; s += 4) {
        float2 m4[4];
        float o4[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            m4[u] = ml[s + u];
            o4[u] = po[(int64_t)(s + u) * D];
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const float f = m4[u].x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m4[u].x - M);
            L += m4[u].y * f;
            O += o4[u] * f;
        }
    }
    for (; s < nsplit; ++s) {
        const float2 m1 = ml[s];
        const float f = m1.x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m1.x - M);
        L += m1.y * f;
        O += po[(int64_t)s * D] * f;
    }
    float r = L > 0.0f ? O / L : 0.0f;
    if constexpr (KV != PUTER_BF16) r *= a.vs[h / (a.heads / a.kv_heads)];
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
    if (num_pages > 0 && (num_pages > 0x7FFFFFFF / page_size || max_pages_per_seq > 0x7FFFFFFF / page_size))
        return fail(PUTER_ERR_INVALID, "paged decode: pool rows (num_pages * page_size) must stay below 2^31");
    if (max_context <= 0 || max_context > max_pages_per_seq * page_size)
        return fail(PUTER_ERR_INVALID, "paged decode: max_context must be in [1, max_pages_per_seq*page_size]");
    if (!query || !key_pages || !value_pages || !page_table || !context_lens || !output || !workspace)
        return fail(PUTER_ERR_NIL, "paged decode: nil buffer");
    if (kv_dtype == PUTER_F8E4M3 && (!k_scale || !v_scale)) return fail(PUTER_ERR_NIL, "paged decode: fp8 needs scales");
    if (!aligned16(query) || !aligned16(key_pages) || !aligned16(value_pages))
        return fail(PUTER_ERR_INVALID, "paged decode: query and pools must be 16-byte aligned");
    const size_t need = puter_hip_paged_decode_workspace_bytes(batch, num_heads, head_dim, max_context);
    if (workspace_bytes < need) return fail(PUTER_ERR_INVALID, "paged decode: workspace %zu < %zu bytes", workspace_bytes, need);
    const int64_t splits = splits_for(max_context);
    if (splits > 65535 || batch > 65535 || kv_heads > 0x7FFFFFFF) return fail(PUTER_ERR_INVALID, "paged decode: grid too large");
    float *ws = static_cast<float *>(workspace);
    const int64_t slots = batch * num_heads * splits;
    DecodeArgs a{static_cast<const uint16_t *>(query), key_pages, value_pages, page_table, context_lens,
                 k_scale, v_scale, static_cast<uint16_t *>(output), ws, ws + slots * head_dim,
                 batch, max_pages_per_seq, page_size, num_pages, num_heads, kv_heads, splits,
                 max_context, (float)(1.0 / sqrt((double)head_dim))};
    hipStream_t s = as_stream(stream);
    const dim3 grid((unsigned)kv_heads, (unsigned)splits, (unsigned)batch);
#define PUTER_DECODE(KV)                                                              \
    switch (G) {                                                                      \
    case 1: decode_mfma_kernel<KV, 1><<<grid, 256, 0, s>>>(a); break;                 \
    case 2: decode_mfma_kernel<KV, 2><<<grid, 256, 0, s>>>(a); break;                 \
    case 4: decode_mfma_kernel<KV, 4><<<grid, 256, 0, s>>>(a); break;                 \
    case 8: decode_mfma_kernel<KV, 8><<<grid, 256, 0, s>>>(a); break;                 \
    }                                                                                 \
    decode_combine_kernel<KV><<<dim3((unsigned)num_heads, (unsigned)batch), 128, 0, s>>>(a);
    if (kv_dtype == PUTER_BF16) { PUTER_DECODE(PUTER_BF16) }
    else { PUTER_DECODE(PUTER_F8E4M3) }
#undef PUTER_DECODE
    return check_launch("paged decode");
}

}  // extern "C"
