// MFMA flash-attention prefill: bf16 Q/K/V, f32 accumulation, bf16 output,
// head_dim 128, GQA, optional causal mask: key k is visible to query q when
// k <= q + shift.  MultiHeadAttention passes shift = seqK - seqQ (bottom-right
// aligned, device/cpu/attention/typed_compute.go:166-168);
// ScaledDotProductAttention passes 0 (typed_compute.go:60-62).
//
// Work split: one 256-thread block (4 wave64s) per (128-query tile, head,
// batch); wave w owns 32 queries.  K/V stream through LDS in 64-key tiles,
// double buffered (the next tile's global loads are in flight while the
// current tile is computed; one barrier per tile).
//
// Everything is computed transposed so the softmax needs no cross-lane
// reductions beyond one swap between the two half-waves:
//   S^T[key, q] = K . Q^T        (v_mfma_f32_32x32x16_bf16, A = K from LDS,
//                                 B = Q^T held in registers for the whole loop)
// The 32x32 accumulator puts query q = lane%32 in every register of a lane,
// so a row max / row sum is an in-lane reduction over the lane's 16 keys plus
// one xor-32 shuffle.  exp2 runs on the scaled scores; P^T, narrowed to bf16
// in registers, is already in the B-operand layout of
//   O^T[d, q] += V^T . P^T       (A = V^T read from a transposed LDS tile)
// because the accumulator's key order (8*(r/4) + 4*(lane/32) + r%4) is used as
// the k-order of both operands.  The online-softmax rescale of O is one
// multiply per accumulator register (all of a lane's outputs share a query).
//
// Causal blocks visit only the key tiles at or below their diagonal and mask
// only the diagonal tiles.  Blocks are dispatched heaviest-first, and the
// block -> (batch, head) map puts the query heads that share a kv head on the
// same XCD (consecutive block ids go round-robin over the 8 XCDs), so the
// K/V tiles they re-read hit that XCD's L2.
#include "attention.hpp"

namespace puter {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

namespace fa {
constexpr int D = 128;        // head dim
constexpr int BM = 128;       // queries per block (4 waves x 32)
constexpr int BN = 64;        // keys per tile
constexpr int KS = D + 8;     // K tile row stride in LDS (elements): 272 B rows, conflict-free b128 reads
constexpr int VS = BN + 4;    // V^T tile row stride (elements): 136 B rows, conflict-free b64 reads
constexpr int KTILE = BN * KS;
constexpr int VTILE = D * VS;
}  // namespace fa

struct PrefillArgs {
    const uint16_t *q, *k, *v;
    uint16_t *o;
    int batch, seq_q, seq_k, heads, kv_heads, qtiles;
    int causal, xcd_map;
    int shift;         // causal: key k visible to query q iff k <= q + shift
    float scale_log2;  // softmax scale * log2(e)
};

__device__ __forceinline__ void prefill_load_tile(const PrefillArgs &a, const uint16_t *kbase,
                                                  const uint16_t *vbase, int kv0, int tid,
                                                  uint4 (&kr)[4], uint4 (&vr)[4]) {
    using namespace fa;
    const int64_t rs = (int64_t)a.kv_heads * D;  // row stride of K/V in elements
    // Keys past the end are clamped to the last row (branch-free loads): their
    // scores are masked to -inf, so they contribute p = 0 times finite data.
    const int last = a.seq_k - 1;
    // K: 64 rows x 16 chunks of 16 B; thread takes chunks tid + 256*i
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int c = tid + 256 * i;
        const int row = c >> 4, col = c & 15;
        const int key = min(kv0 + row, last);
        kr[i] = *reinterpret_cast<const uint4 *>(kbase + (int64_t)key * rs + col * 8);
    }
    // V: thread takes keys kb*4 .. +3 of the 8 dims db*8 .. +7.  Lanes of a
    // wave vary kb fastest so the transposed LDS writes below hit distinct banks.
    const int kb = tid & 15, db = tid >> 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int key = min(kv0 + kb * 4 + i, last);
        vr[i] = *reinterpret_cast<const uint4 *>(vbase + (int64_t)key * rs + db * 8);
    }
}

__device__ __forceinline__ void prefill_store_tile(uint16_t *ks, uint16_t *vt, int tid,
                                                   const uint4 (&kr)[4], const uint4 (&vr)[4]) {
    using namespace fa;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int c = tid + 256 * i;
        const int row = c >> 4, col = c & 15;
        *reinterpret_cast<uint4 *>(ks + row * KS + col * 8) = kr[i];
    }
    // transpose 4 keys x 8 dims into V^T rows: one 8-byte write per dim; the
    // 16 lanes of a write pass differ in kb -> consecutive 8-byte slots of one row
    const int kb = tid & 15, db = tid >> 4;
    const uint32_t w[4][4] = {{vr[0].x, vr[0].y, vr[0].z, vr[0].w}, {vr[1].x, vr[1].y, vr[1].z, vr[1].w},
                              {vr[2].x, vr[2].y, vr[2].z, vr[2].w}, {vr[3].x, vr[3].y, vr[3].z, vr[3].w}};
#pragma unroll
    for (int word = 0; word < 4; ++word) {
        // v_perm_b32: low halves of keys (0,1) / (2,3) -> dim 2*word, high halves -> dim 2*word+1
        const uint2 lo = make_uint2(__builtin_amdgcn_perm(w[1][word], w[0][word], 0x05040100u),
                                    __builtin_amdgcn_perm(w[3][word], w[2][word], 0x05040100u));
        const uint2 hi = make_uint2(__builtin_amdgcn_perm(w[1][word], w[0][word], 0x07060302u),
                                    __builtin_amdgcn_perm(w[3][word], w[2][word], 0x07060302u));
        *reinterpret_cast<uint2 *>(vt + (db * 8 + 2 * word) * VS + kb * 4) = lo;
        *reinterpret_cast<uint2 *>(vt + (db * 8 + 2 * word + 1) * VS + kb * 4) = hi;
    }
}

__global__ __launch_bounds__(256, 2) void prefill_bf16_d128_kernel(PrefillArgs a) {
    using namespace fa;
    __shared__ __attribute__((aligned(16))) uint16_t k_lds[2][KTILE];
    __shared__ __attribute__((aligned(16))) uint16_t v_lds[2][VTILE];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int l32 = lane & 31, g = lane >> 5;

    // block -> (query tile, batch, head)
    const int id = blockIdx.x;
    int qt, b, h;
    if (a.xcd_map) {
        // Query tiles go heaviest first over the whole grid.  Inside one tile
        // index, consecutive block ids (dispatched round-robin over the 8
        // XCDs) are mapped so the G query heads of a kv group (batch, kv head)
        // land on the same XCD and share its L2 for their K/V tiles.  (Walking
        // one group at a time per XCD measured slower: it loses the global
        // heaviest-first order.)
        const int bh = a.batch * a.heads;
        const int G = a.heads / a.kv_heads;
        qt = a.causal ? (a.qtiles - 1 - id / bh) : (id / bh);
        const int j = id % bh;
        const int xcd = j & 7, slot = j >> 3;
        const int grp = (slot / G) * 8 + xcd;
        b = grp / a.kv_heads;
        h = (grp % a.kv_heads) * G + slot % G;
    } else {
        const int bh = a.batch * a.heads;
        qt = a.causal ? (a.qtiles - 1 - id / bh) : (id / bh);
        b = (id % bh) / a.heads;
        h = id % a.heads;
    }
    const int kvh = h / (a.heads / a.kv_heads);
    const int q0 = qt * BM;
    const int off = a.shift;  // causal alignment
    const int64_t qrs = (int64_t)a.heads * D, krs = (int64_t)a.kv_heads * D;
    const uint16_t *qbase = a.q + (int64_t)b * a.seq_q * qrs + (int64_t)h * D;
    const uint16_t *kbase = a.k + (int64_t)b * a.seq_k * krs + (int64_t)kvh * D;
    const uint16_t *vbase = a.v + (int64_t)b * a.seq_k * krs + (int64_t)kvh * D;

    // this lane's query and its Q^T operand fragments (8 k-steps of 16 dims)
    const int qw0 = q0 + wave * 32;
    const int qi = qw0 + l32;
    bf16x8 qf[8];
    const int qload = min(qi, a.seq_q - 1);  // rows past the end compute garbage, never stored
#pragma unroll
    for (int t = 0; t < 8; ++t)
        qf[t] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4 *>(qbase + (int64_t)qload * qrs + 16 * t + 8 * g));

    // key range of the block
    int kend = a.seq_k;
    if (a.causal) kend = min(kend, min(q0 + BM, a.seq_q) - 1 + off + 1);
    const int ntiles = kend > 0 ? (kend + BN - 1) / BN : 0;

    f32x16 o[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) o[d] = (f32x16){};
    float m = -INFINITY, lsum = 0.0f;
    const int q_last_wave = min(qw0 + 31, a.seq_q - 1);

    if (ntiles > 0) {
        uint4 kr0[4], vr0[4];
        prefill_load_tile(a, kbase, vbase, 0, tid, kr0, vr0);
        prefill_store_tile(k_lds[0], v_lds[0], tid, kr0, vr0);
    }
    __syncthreads();

    for (int it = 0; it < ntiles; ++it) {
        const int kv0 = it * BN;
        const int buf = it & 1;
        // next tile's loads go out before the compute and land in registers
        // that live only inside this iteration (unconditional: the last
        // iteration re-reads its own tile, which is cheaper than a branch
        // around the loads)
        uint4 kr[4], vr[4];
        prefill_load_tile(a, kbase, vbase, min(kv0 + BN, (ntiles - 1) * BN), tid, kr, vr);

        // waves whose queries all precede this tile (causal) skip it
        const bool active = !a.causal || kv0 <= q_last_wave + off;
        if (active) {
            const uint16_t *ks = k_lds[buf];
            const uint16_t *vt = v_lds[buf];
            // S^T chunks: keys kv0 + 32c + (8*(r/4) + 4g + r%4), query qi
            f32x16 s[2] = {(f32x16){}, (f32x16){}};
#pragma unroll
            for (int t = 0; t < 8; ++t)     // two independent accumulation chains interleaved
#pragma unroll
                for (int c = 0; c < 2; ++c) {
                    const bf16x8 kf = *reinterpret_cast<const bf16x8 *>(ks + (32 * c + l32) * KS + 16 * t + 8 * g);
                    s[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[t], s[c], 0, 0, 0);
                }
            const bool need_mask = (kv0 + BN > a.seq_k) || (a.causal && kv0 + BN - 1 > qw0 + off);
            if (need_mask) {
#pragma unroll
                for (int c = 0; c < 2; ++c)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int key = kv0 + 32 * c + 8 * (r >> 2) + 4 * g + (r & 3);
                        const bool dead = key >= a.seq_k || (a.causal && key > qi + off);
                        if (dead) s[c][r] = -INFINITY;
                    }
            }
            float tmax = -INFINITY;
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int r = 0; r < 16; ++r) tmax = fmaxf(tmax, s[c][r]);
            tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
            const float mnew = fmaxf(m, tmax);
            const float mref = mnew == -INFINITY ? 0.0f : mnew * a.scale_log2;
            const float alpha = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m * a.scale_log2 - mref);
            m = mnew;
            float psum = 0.0f;
            bf16x8 pf[2][2];
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int t = 0; t < 2; ++t)
#pragma unroll
                    for (int jj = 0; jj < 8; ++jj) {
                        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[c][8 * t + jj], a.scale_log2, -mref));
                        psum += p;
                        pf[c][t][jj] = (__bf16)p;
                    }
            lsum = lsum * alpha + psum;
            // (a wave-uniform skip of this rescale measured slower: the branch
            // splits the block and stops MFMA/VALU interleaving)
#pragma unroll
            for (int d = 0; d < 4; ++d)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[d][r] *= alpha;
            // O^T[d, q] += V^T[d, keys] . P^T[keys, q]; four independent chains
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int t = 0; t < 2; ++t)
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        const uint16_t *row = vt + (32 * d + l32) * VS + 32 * c + 16 * t + 4 * g;
                        const bf16x4 lo = *reinterpret_cast<const bf16x4 *>(row);
                        const bf16x4 hi = *reinterpret_cast<const bf16x4 *>(row + 8);
                        const bf16x8 vf = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
                        o[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf[c][t], o[d], 0, 0, 0);
                    }
        }
        if (it + 1 < ntiles) prefill_store_tile(k_lds[buf ^ 1], v_lds[buf ^ 1], tid, kr, vr);
        __syncthreads();
    }

    // normalise and store: lane holds O[qi][32d + 8*(r/4) + 4g + r%4]
    const float ltot = lsum + __shfl_xor(lsum, 32, 64);
    const float inv = ltot > 0.0f ? 1.0f / ltot : 0.0f;
    if (qi < a.seq_q) {
        uint16_t *orow = a.o + (int64_t)b * a.seq_q * qrs + (int64_t)qi * qrs + (int64_t)h * D;
#pragma unroll
        for (int d = 0; d < 4; ++d)
#pragma unroll
            for (int rb = 0; rb < 4; ++rb) {
                // v_cvt_pk_bf16_f32: round-to-nearest-even, as the software rule
                bf16x4 v;
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = (__bf16)(o[d][4 * rb + i] * inv);
                *reinterpret_cast<bf16x4 *>(orow + 32 * d + 8 * rb + 4 * g) = v;
            }
    }
}

bool launch_prefill_mfma(const MhaArgs &m, int dtype, hipStream_t s, int *status) {
    if (dtype != PUTER_BF16 || m.dim != 128 || m.window > 0 || m.alibi != 0.0f) return false;
    if (m.seq_q > 0x3FFFFFFF || m.seq_k > 0x3FFFFFFF || m.shift > 0x3FFFFFFF || m.shift < -0x3FFFFFFF)
        return false;
    const uintptr_t mask = 15;
    if ((reinterpret_cast<uintptr_t>(m.q) | reinterpret_cast<uintptr_t>(m.k) |
         reinterpret_cast<uintptr_t>(m.v) | reinterpret_cast<uintptr_t>(m.o)) & mask)
        return false;
    PrefillArgs a;
    a.q = static_cast<const uint16_t *>(m.q);
    a.k = static_cast<const uint16_t *>(m.k);
    a.v = static_cast<const uint16_t *>(m.v);
    a.o = static_cast<uint16_t *>(m.o);
    a.batch = (int)m.batch;
    a.seq_q = (int)m.seq_q;
    a.seq_k = (int)m.seq_k;
    a.heads = (int)m.heads;
    a.kv_heads = (int)m.kv_heads;
    a.qtiles = (int)((m.seq_q + fa::BM - 1) / fa::BM);
    a.causal = m.causal;
    a.shift = (int)m.shift;
    const int G = a.heads / a.kv_heads;
    a.xcd_map = ((a.batch * a.kv_heads) % 8 == 0) ? 1 : 0;
    (void)G;
    a.scale_log2 = m.scale * 1.4426950408889634f;
    const int64_t blocks = (int64_t)a.qtiles * a.batch * a.heads;
    if (blocks > 0x7FFFFFFF) return false;
    prefill_bf16_d128_kernel<<<(unsigned)blocks, 256, 0, s>>>(a);
    *status = check_launch("prefill mfma");
    return true;
}

}  // namespace puter
