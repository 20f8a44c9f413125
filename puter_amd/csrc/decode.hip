// Paged-KV decode attention (one query token per sequence, GQA): bf16 or f16
// K/V, or fp8-E4M3 K/V with a per-kv-head fp32 scale.
//
// Reference path: KVPageGather of K and V through the sequence's page table
// (execution/page_intrinsic.go:217-352, device/cpu/shape/page_generic.go:45-63)
// followed by MultiHeadAttention with seqQ = 1 (bind_router.go:640-684,
// device/cpu/attention/typed_compute.go:142-237).  The gather is fused: K/V
// rows are read straight from the page pools (no materialised [ctx, Hkv*D]
// copies), so HBM traffic is the KV bytes read once.  MultiHeadAttention with
// one query row (the reference's own decode step, after its gather) runs the
// same kernels over the contiguous K/V rows.
//
// Split-K ("flash decoding"): grid = (kv head, 256-token split, sequence); each
// XCD runs a group of kv heads of one split back to back, so the blocks reading
// adjacent head slices of the same pages share an XCD; decode_block_kernel runs
// four waves of 64 tokens per split, every row load of a wave issued at once,
// the waves' partials merged in LDS.
//   loads: every load instruction reads whole KV rows (16 lanes x 16 bytes =
//     one 256-byte 16-bit row), which measured 17-25% faster than loading K in
//     the MFMA operand layout (16 rows x 64 bytes per instruction) or copying
//     it HBM -> LDS directly.
//   scores: S^T[token, head] = K . Q^T with v_mfma_f32_16x16x32; K rows reach
//     the operand layout through a wave-private LDS tile (swizzled, bank-
//     conflict free), B = the G query heads of the kv group, zero-padded to 16
//     columns; a lane then holds 8 scores of one head.
//   values: O^T[d, head] = V^T . P^T on the same MFMA, V rows (fp8 widened to
//     bf16) through the wave's LDS tile and read back transposed by
//     ds_read_b64_tr_b16, P as hi + lo halves; the VALU FMA form it replaced
//     left the fp8 kernel VALU-bound (78% VALU busy).
// Each split leaves one (m, l, o[D]) per query head; decode_combine_kernel
// merges the splits by log-sum-exp.
#include "attention.hpp"
#include "common.hpp"
#include <algorithm>
#include <type_traits>

namespace puter {

constexpr int kSplit = 256;  // tokens per split (one block: four waves of 64 tokens)

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

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

// 8 fp8-E4M3 codes (8 bytes) -> 8 bf16, two codes per v_cvt_scalef32_pk_bf16_fp8
// (OCP E4M3FN, scale 1).  Every E4M3 value is a bf16 value; on MI355X this
// instruction gives the same bf16 bits as the exact v_cvt_pk_f32_fp8 widening
// narrowed to bf16, for all 65536 code pairs (NaN for NaN), in half the
// instructions.
__device__ __forceinline__ uint4 fp8x8_to_bf16(uint2 raw) {
    const uint32_t w[2] = {raw.x, raw.y};
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        o[2 * k] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[k], 1.0f, false));     // bytes 0, 1
        o[2 * k + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[k], 1.0f, true));  // bytes 2, 3
    }
    return make_uint4(o[0], o[1], o[2], o[3]);
}

// Paged decode, block form: one 256-thread block per (kv head, 256-token split,
// sequence); wave w takes the split's tokens 64w .. 64w + 63 and issues every K
// and V row load of its 64 tokens at once (16-byte pieces: 32 KB of bf16 in
// flight per wave), then computes them: scores on MFMA through a wave-private
// LDS tile, the softmax of its 64 tokens against their own max, P.V on MFMA
// through the same tile.  The four waves' (m, l, o) merge through LDS into the
// split's partial (m, l, o[D]) per query head.  Measured in one process on the
// 64-sequence decode pool (contexts U[512, 8192], page 16, 32 query heads over 8)
// against a one-wave-per-split walk over 32-token sub-chunks:
// bf16 +1%, fp8 +4%; MFMA P.V with 16-byte fp8 row pieces then took fp8 from
// 144.6 to 138.0 us (bf16 unchanged).
// GT: the query heads per kv head (1, 2, 4 or 8), or 0 for any other count up to
// 16, read from the arguments (the score and P.V MFMAs are 16 heads wide either
// way; the heads past the group are zero).
template <int KV, int GT, bool O32>
__global__ __launch_bounds__(256, 2) void decode_block_kernel(DecodeArgs a) {
    constexpr int D = 128, TW = 64;
    const int G = GT ? GT : (int)(a.heads / a.kv_heads);
    constexpr bool BF = KV == PUTER_BF16;
    constexpr bool H16 = KV == PUTER_F16;   // f16 pools, query and output
    constexpr bool W16 = BF || H16;          // 16-bit K/V rows (else fp8)
    using P8 = typename std::conditional<H16, f16x8_t, bf16x8_t>::type;   // MFMA operand
    using PE = typename std::conditional<H16, _Float16, __bf16>::type;
    // per-wave 32-row tiles: K rows (256 bytes 16-bit, 128 fp8), then V rows (fp8
    // widened to bf16: 256 bytes), then the o merge (rows of kORow floats: the
    // 4 extra floats put the heads' rows on different banks)
    // With a compiled group size (at most 8 heads) the padded o rows and the
    // (m, l) pairs fit in the 32 KB of tiles, so a block takes exactly 32 KB and
    // five fit on a CU; the run-time group size (up to 16 heads) takes 33 KB.
    constexpr int kORow = D + 4;
    constexpr int kTile = GT ? 32 * 256 : 32 * 256 + 256;
    __shared__ __attribute__((aligned(1024))) char k_lds[4][kTile];
    __shared__ float ml_spill[GT ? 1 : 4 * 16 * 2];

    // Block order.  Consecutive dispatch ids go round-robin over the 8 XCDs; XCD x
    // runs a group of gk kv heads of chunk (split, sequence) 8n + x one after
    // another, so for each token it reads gk adjacent head slices (1 KB: four
    // heads of 16-bit rows, eight of fp8) instead of one slice per XCD.  Against
    // one kv head per XCD: bf16 225.5 -> 220.4 us, fp8 136.4 -> 132.6 us on the
    // 64-sequence decode pool (one process); eight bf16 heads (2 KB) gave 223.7 us.
    int kvh, split, b;
    int64_t chunk;
    {
        int gk = W16 ? 4 : 8;
        while (gk > 1 && a.kv_heads % gk) gk >>= 1;
        const int64_t KVn = gridDim.x, NG = KVn / gk, C = (int64_t)gridDim.y * gridDim.z * NG;
        const int64_t L = blockIdx.x + KVn * (blockIdx.y + (int64_t)gridDim.y * blockIdx.z);
        const int64_t full = (C / 8) * 8 * gk;   // ids in whole rounds of 8 groups
        int64_t kvl, cg;
        if (L < full) {
            kvl = (L >> 3) % gk;
            cg = ((L >> 3) / gk) * 8 + (L & 7);
        } else {
            kvl = (L - full) % gk;
            cg = (C / 8) * 8 + (L - full) / gk;
        }
        kvh = (int)((cg % NG) * gk + kvl);
        chunk = cg / NG;
    }
    const int tid = threadIdx.x, lane = tid & 63, l16 = lane & 15, grp = lane >> 4;
    int ctx;
    if (a.ctx && a.batch <= 256 && !W16) {
        // fp8 pools, live chunks first: chunk c is the c-th live (sequence, split) pair,
        // sequences in order, so the blocks past the last live pair, which exit at once,
        // are dispatched after all the work instead of among it (every wave of the block
        // finds the same pair: a prefix sum of the sequences' split counts, 64 at a
        // time).  On the 64-sequence decode pool, interleaved in one process, bit-
        // identical: fp8 133.9 -> 131.4 us; the 16-bit kernel lost 1.4% with it (212.4
        // -> 215.3 us) and keeps the plain order
        b = -1;
        split = 0;
        ctx = 0;
        int64_t base = 0;
        for (int j0 = 0; j0 < a.batch; j0 += 64) {   // wave-uniform
            const int j = j0 + lane;
            const int cx = j < a.batch ? (int)min((int64_t)a.ctx[j], a.max_context) : 0;
            const int ns = cx > 0 ? (cx + kSplit - 1) / kSplit : 0;
            int incl = ns;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int t = __shfl_up(incl, o, 64);
                if (lane >= o) incl += t;
            }
            const int total = __shfl(incl, 63, 64);
            if (chunk < base + total) {
                const int lj = __builtin_ctzll(__ballot(base + incl > chunk));
                b = j0 + lj;
                split = __builtin_amdgcn_readfirstlane((int)(chunk - base - (__shfl(incl, lj, 64) - __shfl(ns, lj, 64))));
                ctx = __builtin_amdgcn_readfirstlane(__shfl(cx, lj, 64));
                break;
            }
            base += total;
        }
        if (b < 0) return;   // the whole block: past the last live pair
    } else {
        split = (int)(chunk % gridDim.y);
        b = (int)(chunk / gridDim.y);
        ctx = a.ctx ? (int)min((int64_t)a.ctx[b], a.max_context) : (int)a.max_context;
    }
    const int t0 = split * kSplit;
    if (t0 >= ctx) return;   // the whole block
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tw0 = t0 + TW * wave;
    const int64_t inner = a.kv_heads * D;
    const int ps = (int)a.page_size;
    const int64_t head_off = (int64_t)kvh * D;
    constexpr int EB = W16 ? 2 : 1;
    const uint8_t *kpool = static_cast<const uint8_t *>(a.kp);
    const uint8_t *vpool = static_cast<const uint8_t *>(a.vp);
    float acc[8][4];   // lane (grp, l16 < G): O[head l16][16 mt + 4 grp + r] = acc[mt][r]
#pragma unroll
    for (int mt = 0; mt < 8; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[mt][r] = 0.0f;
    float m_w = -INFINITY, l_w = 0.0f;   // lane l16 < G: head l16's max (log2 domain) and sum

    if (tw0 < ctx) {   // wave-uniform
        int myrow = -1;   // pool row of token tw0 + lane (-1: past the context or a bad page id)
        {
            const int tok = tw0 + lane;
            if (tok < ctx) {
                const int pidx = tok / ps;
                const int32_t page = a.table ? a.table[(int64_t)b * a.max_pages + pidx] : b * (int)a.max_pages + pidx;
                if (page >= 0 && page < a.num_pages) myrow = page * ps + (tok - pidx * ps);
            }
        }
        // every K and V row of the wave's 64 tokens, 16 bytes per lane: 16-bit rows
        // (256 bytes) as token 4k + grp, piece l16; fp8 rows (128 bytes) as token
        // 8k + g8, piece l8 (dead rows read pool row 0: masked below)
        constexpr int NL = W16 ? 16 : 8;   // row loads per lane and tensor
        const int g8 = lane >> 3, l8 = lane & 7;
        uint4 kb[NL], vb[NL];
#pragma unroll
        for (int k = 0; k < NL; ++k) {
            const int row = max(__shfl(myrow, W16 ? 4 * k + grp : 8 * k + g8, 64), 0);
            if constexpr (O32) {   // pools under 4 GiB: 32-bit offsets from the pool base
                const uint32_t off = (uint32_t)row * (uint32_t)(inner * EB) + (uint32_t)(head_off * EB) + 16u * (W16 ? l16 : l8);
                kb[k] = ld_stream(reinterpret_cast<const uint4 *>(kpool + off));
                vb[k] = ld_stream(reinterpret_cast<const uint4 *>(vpool + off));
            } else {
                const int64_t off = ((int64_t)row * inner + head_off) * EB + 16 * (W16 ? l16 : l8);
                kb[k] = ld_stream(reinterpret_cast<const uint4 *>(kpool + off));
                vb[k] = ld_stream(reinterpret_cast<const uint4 *>(vpool + off));
            }
        }
        // B operand (Q^T): lane holds Q[head l16][32t + 8grp .. +7]; heads >= G are zero.
        // fp8 rows take the dims in another order, the same for K and Q (the dot is
        // a sum over all dims): MFMAs 2p and 2p + 1 give lane group grp dims
        // 64p + 16grp .. + 7 and + 8 .. + 15, 16 consecutive codes of a K row, read
        // as one 16-byte piece
        P8 qb[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            uint4 u = make_uint4(0, 0, 0, 0);
            const int dim0 = W16 ? 32 * t + 8 * grp : 64 * (t >> 1) + 16 * grp + 8 * (t & 1);
            if (l16 < G)
                u = *reinterpret_cast<const uint4 *>(a.q + ((int64_t)b * a.heads + (int64_t)kvh * G + l16) * D + dim0);
            qb[t] = __builtin_bit_cast(P8, u);
        }
        const uint64_t live = __ballot(myrow >= 0);   // token t live iff bit t
        char *tile = k_lds[wave];
        // every token live (the common case below a sequence's last 64 tokens):
        // the mask tests below are skipped (wave-uniform branches)
        const bool full = live == ~0ull;
        // scores S^T[token, head], 32 tokens at a time: K rows -> the wave's LDS
        // tile, then A = tile rows 16i + l16, B = Q^T; lane: head l16, tokens
        // 16i + 4grp + r.  bf16 rows keep 16-byte piece c at c ^ (r % 16); fp8 rows
        // (128 bytes, one 128-byte bank line each) keep it at c ^ (r % 8), so the
        // 8 rows of the 8 lanes an LDS cycle serves for a 16-byte read or write
        // fall on distinct banks
        f32x4_t s[4];
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            if (half) __builtin_amdgcn_wave_barrier();   // the first half's tile reads are done
            if constexpr (W16) {
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const int r = 4 * k + grp;
                    *reinterpret_cast<uint4 *>(tile + r * 256 + ((l16 ^ (r & 15)) << 4)) = kb[8 * half + k];
                }
            } else {
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int r = 8 * k + g8;
                    *reinterpret_cast<uint4 *>(tile + r * 128 + ((l8 ^ (r & 7)) << 4)) = kb[4 * half + k];
                }
            }
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                f32x4_t acc_s = (f32x4_t){0.0f, 0.0f, 0.0f, 0.0f};
                const int row = 16 * i + l16;
                uint4 k8[2];   // fp8: 16-byte pieces 4p + grp of the row (codes for MFMAs 2p, 2p + 1)
                if constexpr (!W16) {
#pragma unroll
                    for (int pp = 0; pp < 2; ++pp)
                        k8[pp] = *reinterpret_cast<const uint4 *>(tile + row * 128 + (((4 * pp + grp) ^ (row & 7)) << 4));
                }
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    uint4 kv;
                    if constexpr (W16) kv = *reinterpret_cast<const uint4 *>(tile + row * 256 + (((4 * t + grp) ^ l16) << 4));
                    else kv = (t & 1) ? fp8x8_to_bf16(make_uint2(k8[t >> 1].z, k8[t >> 1].w))
                                      : fp8x8_to_bf16(make_uint2(k8[t >> 1].x, k8[t >> 1].y));
                    if constexpr (H16) acc_s = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(P8, kv), qb[t], acc_s, 0, 0, 0);
                    else acc_s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(P8, kv), qb[t], acc_s, 0, 0, 0);
                }
                s[2 * half + i] = acc_s;
            }
        }
        const float c = a.scale * (W16 ? 1.0f : a.ks[kvh]) * 1.4426950408889634f;
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float v = s[i][r];
                if constexpr (BF) v = round_reduction<PUTER_BF16>(v);  // bf16 dot, typed_compute.go:16-20
                if constexpr (H16) v = (float)(_Float16)v;              // f16 dot, likewise (RNE)
                s[i][r] = v * c;
            }
        if (!full) {
            const uint64_t lg = live >> (4 * grp);   // bit 16i + r: token 16i + 4grp + r
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (!((lg >> (16 * i + r)) & 1)) s[i][r] = -INFINITY;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) mx = fmaxf(mx, s[i][r]);
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float mref = mx == -INFINITY ? 0.0f : mx;
        float lsum = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                // exp2(-inf - mref) is exactly 0 for a dead token (mref finite)
                const float p = __builtin_amdgcn_exp2f(s[i][r] - mref);
                lsum += p;
                s[i][r] = p;
            }
        lsum += __shfl_xor(lsum, 16, 64);
        lsum += __shfl_xor(lsum, 32, 64);
        m_w = mx;
        l_w = lsum;
        // O^T[d, head] = V^T[d, tokens] . P^T[tokens, head] on v_mfma_f32_16x16x32_bf16,
        // 32 tokens per step.  The k order of both operands: slot j of lane group
        // grp is token 16 (j / 4) + 4 grp + j % 4 of the step, which is where the
        // score accumulator left this lane's p (head l16), so P^T needs no shuffle.
        // P enters as hi + lo halves in the operand format (two MFMAs: a 16-bit
        // significand for bf16, 22 for f16): the products keep f32-grade
        // accuracy, as the reference's f32 weights do.
        P8 ph[2], pl[2];
#pragma unroll
        for (int st = 0; st < 2; ++st)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float p = s[2 * st + (j >> 2)][j & 3];
                const PE hi = (PE)p;
                ph[st][j] = hi;
                pl[st][j] = (PE)(p - (float)hi);
            }
        f32x4_t ot[8];
#pragma unroll
        for (int mt = 0; mt < 8; ++mt) ot[mt] = (f32x4_t){0.0f, 0.0f, 0.0f, 0.0f};
        // V^T from the wave's tile: row r (token of the step) keeps its 16-byte
        // chunk c at c ^ vsw(r), vsw(r) = 2 (r % 8) + r % 2: the transposing reads
        // below (4 rows x 32 bytes per 16 lanes) hit distinct banks, and so do the
        // fp8 writes (two rows' even chunks per 16 lanes land on opposite chunk
        // parities).  Lane l16 of group grp reads row 4 grp + l16 / 4 (and + 16),
        // dims 16 mt + 4 (l16 % 4) .. + 3; within the 16 lanes the read hands
        // lane i dims 16 mt + i of those 4 rows.
        auto vsw = [](int r) { return (2 * (r & 7)) | (r & 1); };
        const int vr = 4 * grp + (l16 >> 2);
        const int vq = l16 & 3;   // dims 4 vq .. + 3 of the 32-byte run: 8-byte unit vq
#pragma unroll
        for (int st = 0; st < 2; ++st) {
            __builtin_amdgcn_wave_barrier();   // the tile's previous reads are done
            if constexpr (W16) {
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const int kk = 8 * st + k, r = 4 * k + grp;
                    uint4 w = vb[kk];
                    if (!full) {   // dead rows: exact zeros
                        const uint32_t keep = ((live >> (4 * kk + grp)) & 1) ? 0xFFFFFFFFu : 0u;
                        w = make_uint4(w.x & keep, w.y & keep, w.z & keep, w.w & keep);
                    }
                    *reinterpret_cast<uint4 *>(tile + r * 256 + ((l16 ^ vsw(r)) << 4)) = w;
                }
            } else {   // 16 fp8 codes (dims 16 l8 .. + 15) -> two bf16 pieces 2 l8, 2 l8 + 1
                // lanes l8 >= 4 write their odd piece first, so each of the two writes
                // puts the 8 lanes of one LDS cycle (one row) on 8 distinct banks
                const int odd = (l8 >> 2) & 1;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int kk = 4 * st + k, r = 8 * k + g8;
                    uint4 raw = vb[kk];
                    if (!full) {
                        const uint32_t keep = ((live >> (8 * kk + g8)) & 1) ? 0xFFFFFFFFu : 0u;
                        raw = make_uint4(raw.x & keep, raw.y & keep, raw.z & keep, raw.w & keep);
                    }
                    const uint2 first = odd ? make_uint2(raw.z, raw.w) : make_uint2(raw.x, raw.y);
                    const uint2 second = odd ? make_uint2(raw.x, raw.y) : make_uint2(raw.z, raw.w);
                    *reinterpret_cast<uint4 *>(tile + r * 256 + (((2 * l8 + odd) ^ vsw(r)) << 4)) = fp8x8_to_bf16(first);
                    *reinterpret_cast<uint4 *>(tile + r * 256 + (((2 * l8 + 1 - odd) ^ vsw(r)) << 4)) = fp8x8_to_bf16(second);
                }
            }
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int mt = 0; mt < 8; ++mt) {
                const int unit = ((2 * mt + (vq >> 1)) ^ vsw(vr)) * 2 + (vq & 1);   // 8-byte unit in the row
                const char *p = tile + vr * 256 + unit * 8;
                const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)(p));
                const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)(p + 16 * 256));
                const P8 va = __builtin_bit_cast(P8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
                if constexpr (H16) {
                    ot[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, ph[st], ot[mt], 0, 0, 0);
                    ot[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pl[st], ot[mt], 0, 0, 0);
                } else {
                    ot[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, ph[st], ot[mt], 0, 0, 0);
                    ot[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pl[st], ot[mt], 0, 0, 0);
                }
            }
        }
        // lane (grp, l16): O[head l16][16 mt + 4 grp + r] = ot[mt][r]
#pragma unroll
        for (int mt = 0; mt < 8; ++mt)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[mt][r] = ot[mt][r];
    }
    // merge the four waves: (m, l) per head and o[head][128] through LDS (the o
    // rows reuse the tiles, so every wave must be done with its tile first)
    __syncthreads();
    float *o_lds = reinterpret_cast<float *>(&k_lds[0][0]);   // [4][G][kORow]
    // [4][G][2]: after the o rows inside the tiles, or beside them (run-time G)
    float(*ml_lds)[GT ? GT : 16][2] = reinterpret_cast<float(*)[GT ? GT : 16][2]>(
        GT ? o_lds + 4 * (GT ? GT : 16) * kORow : ml_spill);
    if (grp == 0 && l16 < G) {
        ml_lds[wave][l16][0] = m_w;
        ml_lds[wave][l16][1] = l_w;
    }
    if (l16 < G) {
#pragma unroll
        for (int mt = 0; mt < 8; ++mt)
            *reinterpret_cast<float4 *>(o_lds + (wave * G + l16) * kORow + 16 * mt + 4 * grp) =
                make_float4(acc[mt][0], acc[mt][1], acc[mt][2], acc[mt][3]);
    }
    __syncthreads();
    const int64_t slot0 = ((int64_t)b * a.heads + (int64_t)kvh * G) * a.max_splits + split;
    for (int idx = tid; idx < G * D; idx += 256) {
        const int h = idx / D, d = idx - h * D;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < 4; ++w) M = fmaxf(M, ml_lds[w][h][0]);
        float L = 0.0f, O = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const float mw = ml_lds[w][h][0];
            const float f = mw == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mw - M);
            L += ml_lds[w][h][1] * f;
            O += o_lds[(w * G + h) * kORow + d] * f;
        }
        const int64_t slot = slot0 + (int64_t)h * a.max_splits;
        a.part_o[slot * D + d] = O;
        if (d == 0) {
            a.part_ml[slot * 2] = M;
            a.part_ml[slot * 2 + 1] = L;
        }
    }
}

// One (query head, sequence) per block, one output dim per thread: merge the
// sequence's split partials by log-sum-exp in one pass over batches of 16
// splits.  Every (m, l) and o load of a batch is issued before any is used (the
// (m, l) pairs are the same addresses for all threads: one transaction), then the
// batch folds into the running (M, L, O), rescaled when its max exceeds M; a
// sequence of up to 16 splits is one round trip to memory.
template <int KV, int SPLIT = kSplit>
__global__ __launch_bounds__(128) void decode_combine_kernel(DecodeArgs a) {
    constexpr int D = 128, NB = 16;
    const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
    const int ctx = a.ctx ? (int)min((int64_t)a.ctx[b], a.max_context) : (int)a.max_context;
    const int nsplit = (ctx + SPLIT - 1) / SPLIT;
    const int64_t base = ((int64_t)b * a.heads + h) * a.max_splits;
    const float2 *ml = reinterpret_cast<const float2 *>(a.part_ml) + base;
    const float *po = a.part_o + base * D + d;
    float M = -INFINITY, L = 0.0f, O = 0.0f;
    for (int s0 = 0; s0 < nsplit; s0 += NB) {
        float2 mv[NB];
        float ov[NB];
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const bool in = s0 + u < nsplit;
            mv[u] = in ? ml[s0 + u] : make_float2(-INFINITY, 0.0f);
            ov[u] = in ? po[(int64_t)(s0 + u) * D] : 0.0f;
        }
        float mb = M;
#pragma unroll
        for (int u = 0; u < NB; ++u) mb = fmaxf(mb, mv[u].x);
        if (mb == -INFINITY) continue;   // every split so far saw no live token
        const float fo = M == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(M - mb);
        L *= fo;
        O *= fo;
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const float f = mv[u].x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mv[u].x - mb);
            L += mv[u].y * f;
            O += ov[u] * f;
        }
        M = mb;
    }
    float r = L > 0.0f ? O / L : 0.0f;
    if constexpr (KV == PUTER_F8E4M3) r *= a.vs[h / (a.heads / a.kv_heads)];
    if constexpr (KV == PUTER_F16) a.out[((int64_t)b * a.heads + h) * D + d] = Elem<PUTER_F16>::store(r);
    else a.out[((int64_t)b * a.heads + h) * D + d] = (uint16_t)f32_to_bf16(r);
}

// An empty pool masks every token: the output is zero.
__global__ __launch_bounds__(256) void decode_zero_kernel(uint16_t *out, int64_t n) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        out[i] = 0;
}

static int64_t splits_for(int64_t max_context) { return (max_context + kSplit - 1) / kSplit; }

}  // namespace puter

using namespace puter;

namespace puter {

// MultiHeadAttention with one query row per sequence (the reference's decode step:
// gathered K/V, seqQ 1, typed_compute.go:206-237), bf16 or f16, head_dim 128, no
// ALiBi: the paged decode kernels over the contiguous K/V (sequence b's keys are
// page b of seq_k rows), partials in the library's scratch.  A causal mask with
// one query row sees every key (bottom-right alignment), as does no mask, and so
// does a sliding window: it compares key indices with the query's row index
// (typed_compute.go:172), 0 here, so q - k >= window holds for no key.
bool launch_decode_contiguous(const MhaArgs &m, int dtype, hipStream_t s, int *status) {
    if ((dtype != PUTER_BF16 && dtype != PUTER_F16) || m.dim != 128 || m.seq_q != 1 || m.alibi != 0.0f)
        return false;
    const int64_t G = m.heads / m.kv_heads;
    if (G < 1 || G > 16) return false;
    if (!aligned16(m.q) || !aligned16(m.k) || !aligned16(m.v) || !aligned16(m.o)) return false;
    if (m.batch > 65535 || m.seq_k > 0x7FFFFFFF / std::max<int64_t>(m.batch, 1) || m.kv_heads > 0x7FFFFFFF)
        return false;
    const int64_t splits = splits_for(m.seq_k);
    if (splits > 65535) return false;
    const size_t need = (size_t)(m.batch * m.heads * splits) * (128 + 2) * sizeof(float);
    ScratchLease lease(need, s);
    if (lease.status()) {
        *status = lease.status();
        return true;
    }
    float *ws = static_cast<float *>(lease.ptr());
    const int64_t slots = m.batch * m.heads * splits;
    DecodeArgs a{static_cast<const uint16_t *>(m.q), m.k, m.v, nullptr, nullptr, nullptr, nullptr,
                 static_cast<uint16_t *>(m.o), ws, ws + slots * 128, m.batch, 1, m.seq_k, m.batch, m.heads,
                 m.kv_heads, splits, m.seq_k, m.scale};
    const dim3 grid((unsigned)m.kv_heads, (unsigned)splits, (unsigned)m.batch);
    const dim3 cgrid((unsigned)m.heads, (unsigned)m.batch);
    const bool o32 = (uint64_t)m.batch * (uint64_t)m.seq_k * (uint64_t)m.kv_heads * 128u * 2u < ((uint64_t)1 << 32);
#define PUTER_ONE_ROW_G(KVD, O)                                                        \
    switch (G) {                                                                       \
    case 1: decode_block_kernel<KVD, 1, O><<<grid, 256, 0, s>>>(a); break;             \
    case 2: decode_block_kernel<KVD, 2, O><<<grid, 256, 0, s>>>(a); break;             \
    case 4: decode_block_kernel<KVD, 4, O><<<grid, 256, 0, s>>>(a); break;             \
    case 8: decode_block_kernel<KVD, 8, O><<<grid, 256, 0, s>>>(a); break;             \
    default: decode_block_kernel<KVD, 0, O><<<grid, 256, 0, s>>>(a); break;            \
    }
#define PUTER_ONE_ROW(KVD)                                                             \
    if (o32) { PUTER_ONE_ROW_G(KVD, true) }                                            \
    else { PUTER_ONE_ROW_G(KVD, false) }                                               \
    decode_combine_kernel<KVD><<<cgrid, 128, 0, s>>>(a);
    if (dtype == PUTER_BF16) { PUTER_ONE_ROW(PUTER_BF16) }
    else { PUTER_ONE_ROW(PUTER_F16) }
#undef PUTER_ONE_ROW
#undef PUTER_ONE_ROW_G
    const int rc = check_launch("mha one-row decode");
    const int fin = lease.finish();
    *status = rc ? rc : fin;
    return true;
}

}  // namespace puter

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
    if (G < 1 || G > 16) return fail(PUTER_ERR_INVALID, "paged decode: group size %lld unsupported (at most 16 query heads per kv head)", (long long)G);
    if (kv_dtype != PUTER_BF16 && kv_dtype != PUTER_F16 && kv_dtype != PUTER_F8E4M3)
        return fail(PUTER_ERR_INVALID, "paged decode: kv dtype %d unsupported", kv_dtype);
    if (num_pages > 0 && (num_pages > 0x7FFFFFFF / page_size || max_pages_per_seq > 0x7FFFFFFF / page_size))
        return fail(PUTER_ERR_INVALID, "paged decode: pool rows (num_pages * page_size) must stay below 2^31");
    if (max_context <= 0 || max_context > max_pages_per_seq * page_size)
        return fail(PUTER_ERR_INVALID, "paged decode: max_context must be in [1, max_pages_per_seq*page_size]");
    if (!query || !key_pages || !value_pages || !page_table || !context_lens || !output || !workspace)
        return fail(PUTER_ERR_NIL, "paged decode: nil buffer");
    if (kv_dtype == PUTER_F8E4M3 && (!k_scale || !v_scale)) return fail(PUTER_ERR_NIL, "paged decode: fp8 needs scales");
    // the split kernel stores float4 partials into the workspace and the combine
    // kernel reads them back as float2
    if (!aligned16(query) || !aligned16(key_pages) || !aligned16(value_pages) || !aligned16(workspace))
        return fail(PUTER_ERR_INVALID, "paged decode: query, pools and workspace must be 16-byte aligned");
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
    if (num_pages == 0) {  // every page id is out of range: all tokens masked
        const int64_t n = batch * num_heads * head_dim;
        decode_zero_kernel<<<(unsigned)std::min<int64_t>((n + 255) / 256, 4096), 256, 0, s>>>(static_cast<uint16_t *>(output), n);
        return check_launch("paged decode");
    }
    const dim3 grid((unsigned)kv_heads, (unsigned)splits, (unsigned)batch);
    // pools under 4 GiB take 32-bit row offsets
    const bool o32 = (uint64_t)num_pages * (uint64_t)page_size * (uint64_t)kv_heads * (uint64_t)head_dim *
                         (kv_dtype == PUTER_F8E4M3 ? 1u : 2u) < ((uint64_t)1 << 32);
#define PUTER_DECODE_G(KV, O)                                                         \
    switch (G) {                                                                      \
    case 1: decode_block_kernel<KV, 1, O><<<grid, 256, 0, s>>>(a); break;             \
    case 2: decode_block_kernel<KV, 2, O><<<grid, 256, 0, s>>>(a); break;             \
    case 4: decode_block_kernel<KV, 4, O><<<grid, 256, 0, s>>>(a); break;             \
    case 8: decode_block_kernel<KV, 8, O><<<grid, 256, 0, s>>>(a); break;             \
    default: decode_block_kernel<KV, 0, O><<<grid, 256, 0, s>>>(a); break;            \
    }
#define PUTER_DECODE(KV)                                                              \
    if (o32) { PUTER_DECODE_G(KV, true) }                                             \
    else { PUTER_DECODE_G(KV, false) }                                                \
    decode_combine_kernel<KV><<<dim3((unsigned)num_heads, (unsigned)batch), 128, 0, s>>>(a);
    if (kv_dtype == PUTER_BF16) { PUTER_DECODE(PUTER_BF16) }
    else if (kv_dtype == PUTER_F16) { PUTER_DECODE(PUTER_F16) }
    else { PUTER_DECODE(PUTER_F8E4M3) }
#undef PUTER_DECODE
#undef PUTER_DECODE_G
    return check_launch("paged decode");
}

}  // extern "C"
