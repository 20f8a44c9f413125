// MFMA flash-attention prefill: bf16 or f16 Q/K/V (prefill_kernel<dtype, head
// dim, window>; f32 Q/K/V on prefill_f32_kernel, described where it is defined),
// f32 accumulation, output in the input format, head_dim 128 or 64, GQA,
// optional causal mask: key k is visible to query q when
// k <= q + shift.  MultiHeadAttention passes shift = seqK - seqQ (bottom-right
// aligned, device/cpu/attention/typed_compute.go:166-168);
// ScaledDotProductAttention passes 0 (typed_compute.go:60-62).  Optional
// sliding window: key k is visible to query q only when q - k < window
// (typed_compute.go:172); a block skips the key tiles below its first query's
// window and masks those below its last query's.  Optional ALiBi: the score
// gains slope * (k - q) (typed_compute.go:176-178); every tile then takes the
// masked step.
//
// Work split: one 256-thread block (4 wave64s) per (128-query tile, head,
// batch); wave w owns 32 queries; two blocks share a CU (2 waves per SIMD, so
// one wave's softmax VALU work overlaps the other's MFMAs).  K/V stream
// through LDS in 64-key tiles, double buffered.  The tiles are copied
// straight from HBM into LDS by buffer_load ... lds (no register staging, no
// LDS write instructions): the next tile's copy is issued while the current
// tile's first MFMAs run and waited for (vmcnt) only at the tile's closing barrier.
// The buffer descriptors' range ends with the last row of the sequence, so
// rows past the end arrive as zeros.  The wave index is read through
// readfirstlane so all per-wave control flow is scalar.
//
// LDS layouts (one tile of 64 key rows each, no padding; 256-byte rows at head
// dim 128, 128-byte rows at 64): K row r keeps its 16-byte chunk c at position
// c ^ kswz(r) and V row r at c ^ vswz(r) (PfDim below); both swizzles make the
// fragment reads below bank-conflict free.  The V^T
// operand is read from the row-major V tile with ds_read_b64_tr_b16: within a
// 16-lane group, result lane i gets element i%4 of the 8 bytes addressed by
// lane 4j + i/4 as its element j, so lanes 4j..4j+3 pointing at four 4-dim
// runs of key row j deliver dims 0..15 of keys 0..3 transposed.
//
// Everything is computed transposed so the softmax needs no cross-lane
// reductions beyond one permlane32 swap between the two half-waves:
//   S^T[key, q] = K . Q^T        (v_mfma_f32_32x32x16_bf16, A = K from LDS,
//                                 B = Q^T held in registers for the whole loop)
// The 32x32 accumulator puts query q = lane%32 in every register of a lane,
// so a row max / row sum is an in-lane reduction over the lane's 16 keys plus
// one swap.  exp2 runs on the scaled scores; P^T, narrowed to bf16 in
// registers, is already in the B-operand layout of
//   O^T[d, q] += V^T . P^T       (A = V^T read from a transposed LDS tile)
// because the accumulator's key order (8*(r/4) + 4*(lane/32) + r%4) is used as
// the k-order of both operands.
//
// Online softmax with a lazy rescale: each query keeps a reference maximum m
// (scaled log2 domain) and p = exp2(s*c - m).  O and l are rescaled only when
// some query of the wave sees a score more than 2^8 above its reference
// (wave-uniform branch, rare after the first tiles); otherwise p may exceed 1
// by at most 2^8, which f32 accumulation and bf16 P absorb exactly as well.
// The tile max is not even computed on the common path: p is evaluated against
// the current reference and, as every p is at most its lane's partial row sum,
// a sum <= 2^8 proves no score crossed the threshold; only otherwise is the max
// taken and p redone.  The final O / l is the same softmax.
//
// The mask-free tiles are software-pipelined inside each wave
// (prefill_step_pipelined): the softmax VALU work of one 32-key chunk is
// interleaved with the MFMAs of the next phase (S of the other chunk, or P.V),
// and the K / V^T fragment reads run ahead of the MFMAs that use them, so a
// wave keeps the matrix core busy through its own softmax instead of leaving
// that to the SIMD's other wave (+8-9% on B4 S4096 causal bf16 against the
// unpipelined step, both timed in one process).
//
// Causal blocks visit only the key tiles at or below their diagonal.  Tiles
// that no query of the block needs masked run a mask-free loop; the few tiles
// on the diagonal (and the sequence tail) run a masked loop.  Blocks are
// dispatched heaviest-first, and the block -> (batch, head) map puts the query
// heads that share a kv head on the same XCD (consecutive block ids go
// round-robin over the 8 XCDs), so the K/V tiles they re-read hit that XCD's L2.
#include "attention.hpp"

#include <climits>

namespace puter {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

// element, fragment types and MFMA of the two 16-bit formats
template <int DT> struct PfFormat;
template <> struct PfFormat<PUTER_BF16> {
    using E = __bf16;
    using V8 = bf16x8;
    using V4 = bf16x4;
};
template <> struct PfFormat<PUTER_F16> {
    using E = _Float16;
    using V8 = f16x8;
    using V4 = f16x4;
};
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

namespace fa {
constexpr int BM = 128;       // queries per block (4 waves x 32)
constexpr int BN = 64;        // keys per tile
constexpr float RESCALE_SLACK = 8.0f;   // log2 headroom before O and l are rescaled
constexpr float RESCALE_LIMIT = 256.0f; // 2^RESCALE_SLACK: the largest p allowed
// buffer descriptor word 3 for raw (untyped, stride 0) dword access on gfx9
constexpr int BUF_WORD3 = 0x00020000;
}  // namespace fa

// Per-head-dim layout of the K / V tiles (D = 128 or 64; 16-bit elements).
// Rows are D * 2 bytes (16 or 8 chunks of 16 bytes).  K row r keeps chunk c at
// c ^ kswz(r): with 256-byte rows kswz = r % 16, with 128-byte rows (two rows per
// 64-bank line) kswz = (r / 2) % 8, so the 16 rows a fragment read touches fall
// on distinct banks either way.  V row r keeps chunk c at c ^ vswz(r): 4 (r % 4)
// for 256-byte rows, 4 ((r / 2) % 2) for 128-byte rows, so the four rows x 32
// bytes of each transposing read (and the rows two apart that share a bank
// line) do not collide.  Both swizzles are unchanged by row offsets of 8, 16
// and 32, which the fragment reads add to a base row.
template <int D> struct PfDim {
    static_assert(D == 128 || D == 64, "head dim 128 or 64");
    static constexpr int RB = D * 2;           // row bytes
    static constexpr int NC = RB / 16;         // 16-byte chunks per row
    static constexpr int TILE = fa::BN * RB;   // one K or V tile: 16 or 8 KB
    static constexpr int KS = D / 16;          // S MFMA k-steps (16 dims each)
    static constexpr int DB = D / 32;          // O^T blocks of 32 dims
    static constexpr int RPI = 64 / NC;        // rows per copy instruction (64 lanes x 16 B)
    static constexpr int NI = 16 / RPI;        // copy instructions per wave and tensor
    static constexpr int kswz(int r) { return D == 128 ? (r & 15) : ((r >> 1) & 7); }
    static constexpr int vswz(int r) { return D == 128 ? ((r & 3) << 2) : (((r >> 1) & 1) << 2); }
};

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

struct PrefillArgs {
    const uint16_t *q, *k, *v;
    uint16_t *o;
    int batch, seq_q, seq_k, heads, kv_heads, qtiles;
    int causal, xcd_map;
    int shift;         // causal: key k visible to query q iff k <= q + shift
    int window;        // > 0: key k visible to query q only if k > q - window
    float alibi_s;     // ALiBi slope / scale: the dot gains alibi_s * (k - q) before scaling
    float scale_log2;  // softmax scale * log2(e)
    // f32 kernel, key range split over blockIdx.y (split_tiles key tiles each): per
    // split, query row and head the (max, sum) and the unnormalised output row, in
    // [split][batch][query][head] order; null when unsplit
    int split_tiles = 0;
    float2 *part_ml = nullptr;
    float *part_o = nullptr;
};

template <int D> struct PrefillState {
    f32x16 o[D / 32];  // O^T accumulators: lane's query, dims 32d + 8*(r/4) + 4*(lane/32) + r%4
    float m;      // reference max, scaled log2 domain (-inf: none yet)
    float l;      // this lane's half of the row sum
};

__device__ __forceinline__ float swap_halves_max(float t) {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(t), __float_as_uint(t), false, false);
    return fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
}
__device__ __forceinline__ float swap_halves_sum(float t) {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(t), __float_as_uint(t), false, false);
    return __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
}

__device__ __forceinline__ void wait_tile_copies() {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's HBM -> LDS copies landed
}

// Copy K/V rows [kv0, kv0 + 64) of this head into LDS.  Each copy instruction
// fills RPI consecutive rows (64 lanes x 16 bytes): wave w copies rows
// 4 RPI i + RPI w + lane / NC (i < NI), lane L filling chunk L % NC of its row
// with the row's chunk (L % NC) ^ swizzle(row) (kg / vg hold those byte offsets).
template <int D>
__device__ __forceinline__ void prefill_copy_tile(const PrefillArgs &a, const uint16_t *kbase,
                                                  const uint16_t *vbase, int kv0, const int *kg,
                                                  const int *vg, char *kdst, char *vdst, int wave) {
    using namespace fa;
    using T = PfDim<D>;
    const int rs2 = a.kv_heads * D * 2;  // K/V row stride in bytes
    const int rows = min(a.seq_k - kv0, BN);   // <= 0: an empty range, every lane reads zeros
    const int bytes = rows > 0 ? (rows - 1) * rs2 + D * 2 : 0;
    const int64_t base = rows > 0 ? (int64_t)kv0 * a.kv_heads * D : 0;
    const __amdgpu_buffer_rsrc_t kd =
        __builtin_amdgcn_make_buffer_rsrc((void *)(kbase + base), (short)0, bytes, BUF_WORD3);
    const __amdgpu_buffer_rsrc_t vd =
        __builtin_amdgcn_make_buffer_rsrc((void *)(vbase + base), (short)0, bytes, BUF_WORD3);
#pragma unroll
    for (int i = 0; i < T::NI; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(kd, (lds_void *)(kdst + (4 * T::RPI * i + T::RPI * wave) * T::RB), 16,
                                                 kg[i], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < T::NI; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(vd, (lds_void *)(vdst + (4 * T::RPI * i + T::RPI * wave) * T::RB), 16,
                                                 vg[i], 0, 0, 0);
}

// One 64-key tile for this wave's 32 queries.  masked applies the causal and
// sequence-end mask (diagonal and tail tiles only).  ka / va: this lane's byte
// offsets of its K fragments (per 16-dim step t) and V^T fragments (per
// 32-dim block d) inside a tile.
template <int DT>
__device__ __forceinline__ f32x16 pf_mfma(typename PfFormat<DT>::V8 a, typename PfFormat<DT>::V8 b, f32x16 c) {
    if constexpr (DT == PUTER_BF16) return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    else return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

template <int DT, int D, bool GEN>
__device__ __forceinline__ void prefill_step(const PrefillArgs &a, const char *ks, const char *vs,
                                             const typename PfFormat<DT>::V8 (&qf)[PfDim<D>::KS], PrefillState<D> &st,
                                             int qi, int kv0, const int (&ka)[PfDim<D>::KS],
                                             const int (&va)[PfDim<D>::DB], int g, bool masked) {
    using namespace fa;
    using T = PfDim<D>;
    using V8 = typename PfFormat<DT>::V8;
    using E = typename PfFormat<DT>::E;
    // S^T chunks: keys kv0 + 32c + (8*(r/4) + 4g + r%4), query qi; two
    // independent accumulation chains interleaved
    f32x16 s[2] = {(f32x16){}, (f32x16){}};
#pragma unroll
    for (int t = 0; t < T::KS; ++t)
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const V8 kf = *reinterpret_cast<const V8 *>(ks + c * 32 * T::RB + ka[t]);
            s[c] = pf_mfma<DT>(kf, qf[t], s[c]);
        }
    if constexpr (DT == PUTER_F16) {
        // f16 dots are rounded to f16 as the reference's typed row dot does
        // (attention/typed_compute.go:16-20); bf16 keeps the f32 dot
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int r = 0; r < 16; ++r) s[c][r] = (float)(_Float16)s[c][r];
    }
    if (masked) {
        // key kv0 + 32c + 8(r/4) + 4g + r%4 is visible iff its offset past
        // kv0 + 4g lies in [lo, lim] (the query's first and last visible keys,
        // relative; the first is the sliding window's lower edge, GEN only).  GEN
        // also adds the ALiBi bias slope * (k - q) (as alibi_s * (k - q) before the
        // scale), after the f16 rounding of the dot, as the reference adds it to
        // the scaled score (typed_compute.go:176-178)
        const int last = a.causal ? min(qi + a.shift, a.seq_k - 1) : a.seq_k - 1;
        const int lim = last - kv0 - 4 * g;
        const bool win = GEN && a.window > 0;
        const int lo = win ? qi - a.window + 1 - kv0 - 4 * g : 0;
        if (GEN && a.alibi_s != 0.0f) {
            const float base = (float)(kv0 + 4 * g - qi);
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    s[c][r] += a.alibi_s * (base + (float)(32 * c + 8 * (r >> 2) + (r & 3)));
        }
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int off = 32 * c + 8 * (r >> 2) + (r & 3);
                s[c][r] = (off > lim || (win && off < lo)) ? -INFINITY : s[c][r];
            }
    }
    // Fast path: every lane already has a reference and p = exp2(s*c - m) is
    // evaluated without the tile max; since every p <= the row sum, a sum <= 2^8
    // bounds every p as the max test would.  Otherwise (first tile, or a score
    // far above the reference) the max is taken, O and l rescaled, p redone.
    float psum = 0.0f;
    V8 pf[2][2];
    bool done = false;
    if (!__any(st.m == -INFINITY)) {
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[c][8 * h + j], a.scale_log2, -st.m));
                    psum += p;
                    pf[c][h][j] = (E)p;
                }
        done = !__any(psum > RESCALE_LIMIT);  // each p of this lane <= its partial sum
    }
    if (!done) {
        float tmax = -INFINITY;
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int r = 0; r < 16; ++r) tmax = fmaxf(tmax, s[c][r]);
        tmax = swap_halves_max(tmax) * a.scale_log2;
        if (__any(tmax > st.m + RESCALE_SLACK)) {
            const float mnew = fmaxf(st.m, tmax);
            const float alpha = st.m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(st.m - mnew);
            st.m = mnew;
            st.l *= alpha;
#pragma unroll
            for (int d = 0; d < D / 32; ++d)
#pragma unroll
                for (int r = 0; r < 16; ++r) st.o[d][r] *= alpha;
        }
        const float mref = st.m == -INFINITY ? 0.0f : st.m;
        psum = 0.0f;
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[c][8 * h + j], a.scale_log2, -mref));
                    psum += p;
                    pf[c][h][j] = (E)p;
                }
    }
    st.l += psum;
    // O^T[d, q] += V^T[d, keys] . P^T[keys, q]: the V^T fragment (dims 32d +
    // lane%32, keys 32c + 16h + 4g + 0..3 and + 8) is two transposing reads
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int d = 0; d < T::DB; ++d) {
                const char *p = vs + (32 * c + 16 * h) * T::RB + va[d];
                const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)(p));
                const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)(p + 8 * T::RB));
                const V8 vf = __builtin_bit_cast(V8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
                st.o[d] = pf_mfma<DT>(vf, pf[c][h], st.o[d]);
            }
}

// a score dot as the reference's typed row dot leaves it: f16 dots rounded to
// f16 (attention/typed_compute.go:16-20); bf16 keeps the f32 dot
template <int DT> __device__ __forceinline__ float pf_score(float x) {
    if constexpr (DT == PUTER_F16) return (float)(_Float16)x;
    else return x;
}

// Online-softmax update for one 32-key chunk that needs the slow path (first
// tile, or a score more than 2^8 above the reference): take the chunk max,
// rescale O and l if the reference moves, and redo p against it.
template <int DT, int D>
__device__ __forceinline__ float prefill_chunk_slow(const PrefillArgs &a, const f32x16 &s, PrefillState<D> &st,
                                                    typename PfFormat<DT>::V8 (&pf)[2]) {
    using namespace fa;
    using E = typename PfFormat<DT>::E;
    float tmax = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) tmax = fmaxf(tmax, pf_score<DT>(s[r]));
    tmax = swap_halves_max(tmax) * a.scale_log2;
    if (__any(tmax > st.m + RESCALE_SLACK)) {
        const float mnew = fmaxf(st.m, tmax);
        const float alpha = st.m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(st.m - mnew);
        st.m = mnew;
        st.l *= alpha;
#pragma unroll
        for (int d = 0; d < D / 32; ++d)
#pragma unroll
            for (int r = 0; r < 16; ++r) st.o[d][r] *= alpha;
    }
    const float mref = st.m == -INFINITY ? 0.0f : st.m;
    float psum = 0.0f;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(pf_score<DT>(s[8 * h + j]), a.scale_log2, -mref));
            psum += p;
            pf[h][j] = (E)p;
        }
    return psum;
}

// One mask-free 64-key tile, software-pipelined inside the wave so the softmax
// VALU work runs under MFMAs instead of between them:
//   phase 1: S chunk 0 (keys 0..31), 8 MFMAs;
//   phase 2: S chunk 1 MFMAs, each followed by a share of chunk 0's p = exp2(s c - m);
//   phase 3: O += V^T P^T for chunk 0 (8 MFMAs), each followed by a share of chunk 1's p;
//   phase 4: O += V^T P^T for chunk 1.
// The p of a chunk are evaluated against the current reference m; the chunk's
// row-sum check (every p <= its lane's partial sum, so a sum <= 2^8 bounds them
// all) sends it to prefill_chunk_slow otherwise.  Chunk 1's check comes after
// chunk 0's contribution is in O and l, so a rescale there covers it.
// sched_group_barrier fixes the interleave (the scheduler would otherwise
// cluster the MFMAs and the VALU work apart).  The next tile's HBM -> LDS copy
// (rows kvn.., into kn / vn; kvn = seq_k for none) is issued in phases 1 and 2,
// one copy instruction beside every other MFMA, instead of as one burst before
// them (bit-identical; +1-2.5% on B4 S4096 / S2048 causal and non-causal, timed
// interleaved in one process).
template <int DT, int D>
__device__ __forceinline__ void prefill_step_pipelined(const PrefillArgs &a, const char *ks, const char *vs,
                                                       const typename PfFormat<DT>::V8 (&qf)[PfDim<D>::KS],
                                                       PrefillState<D> &st, const int (&ka)[PfDim<D>::KS],
                                                       const int (&va)[PfDim<D>::DB], const uint16_t *kbase,
                                                       const uint16_t *vbase, int kvn, const int (&kg)[PfDim<D>::NI],
                                                       const int (&vg)[PfDim<D>::NI], char *kn, char *vn, int wave) {
    using namespace fa;
    prefill_copy_tile<D>(a, kbase, vbase, kvn, kg, vg, kn, vn, wave);
    using T = PfDim<D>;
    using V8 = typename PfFormat<DT>::V8;
    using E = typename PfFormat<DT>::E;
    constexpr int KS = T::KS, NM = 2 * T::DB;   // S MFMAs per chunk, P.V MFMAs per chunk
    constexpr int E2 = 16 / KS, E3 = 16 / NM;   // p values evaluated beside each MFMA (phases 2, 3)
    constexpr int RA = KS < 4 ? KS : 4;         // K reads issued ahead of the first S MFMA
    f32x16 s0 = (f32x16){}, s1 = (f32x16){};
    V8 p0[2], p1[2];
    const float m = st.m, c = a.scale_log2;
    // phase 1 + 2
#pragma unroll
    for (int t = 0; t < KS; ++t) {
        const V8 kf = *reinterpret_cast<const V8 *>(ks + ka[t]);
        s0 = pf_mfma<DT>(kf, qf[t], s0);
    }
    float ps0 = 0.0f;
#pragma unroll
    for (int t = 0; t < KS; ++t) {
        const V8 kf = *reinterpret_cast<const V8 *>(ks + 32 * T::RB + ka[t]);
        s1 = pf_mfma<DT>(kf, qf[t], s1);
#pragma unroll
        for (int r = E2 * t; r < E2 * t + E2; ++r) {
            const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(pf_score<DT>(s0[r]), c, -m));
            ps0 += p;
            p0[r >> 3][r & 7] = (E)p;
        }
    }
    // K fragment reads run RA ahead of the MFMAs that use them (LDS latency
    // hidden behind the MFMAs in flight)
    __builtin_amdgcn_sched_group_barrier(0x100, RA, 0);      // K reads c0 t0 ..
#pragma unroll
    for (int t = 0; t < KS; ++t) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // S chunk 0 MFMA t
        if ((t & 1) && t / 2 < T::NI) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);   // a K copy
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // next K read (c0, then c1)
    }
#pragma unroll
    for (int t = 0; t < KS; ++t) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // S chunk 1 MFMA t
        if ((t & 1) && t / 2 < T::NI) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);   // a V copy
        if (t < KS - RA) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // remaining K reads of c1
        __builtin_amdgcn_sched_group_barrier(0x002, 3 * E2, 0);  // chunk 0 softmax share
    }
    if (__any(ps0 > RESCALE_LIMIT)) ps0 = prefill_chunk_slow<DT, D>(a, s0, st, p0);
    st.l += ps0;
    // phase 3: chunk 0's P.V with chunk 1's softmax between the MFMAs
    const float m1 = st.m;
    float ps1 = 0.0f;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int d = 0; d < T::DB; ++d) {
            const char *p = vs + 16 * h * T::RB + va[d];
            const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)(p));
            const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)(p + 8 * T::RB));
            const V8 vf = __builtin_bit_cast(V8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
            st.o[d] = pf_mfma<DT>(vf, p0[h], st.o[d]);
            const int r0 = E3 * (T::DB * h + d);
#pragma unroll
            for (int r = r0; r < r0 + E3; ++r) {
                const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(pf_score<DT>(s1[r]), c, -m1));
                ps1 += pv;
                p1[r >> 3][r & 7] = (E)pv;
            }
        }
    // V^T fragment reads (two per MFMA) run two MFMAs ahead
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int t = 0; t < NM; ++t) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // P.V MFMA (chunk 0)
        if (t < NM - 2) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 3 * E3, 0);  // chunk 1 softmax share
    }
    if (__any(ps1 > RESCALE_LIMIT)) ps1 = prefill_chunk_slow<DT, D>(a, s1, st, p1);
    st.l += ps1;
    // phase 4: chunk 1's P.V
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int d = 0; d < T::DB; ++d) {
            const char *p = vs + (32 + 16 * h) * T::RB + va[d];
            const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)(p));
            const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)(p + 8 * T::RB));
            const V8 vf = __builtin_bit_cast(V8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
            st.o[d] = pf_mfma<DT>(vf, p1[h], st.o[d]);
        }
    __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);
#pragma unroll
    for (int t = 0; t < NM; ++t) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (t < NM - 3) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
}

// GEN: a sliding window (a.window > 0) or an ALiBi slope is set; without either
// that code compiles away.  With ALiBi every tile takes the masked step, which
// adds the bias.
template <int DT, int D, bool GEN>
__global__ __launch_bounds__(256, 2) void prefill_kernel(PrefillArgs a) {
    using namespace fa;
    using T = PfDim<D>;
    using V8 = typename PfFormat<DT>::V8;
    using V4 = typename PfFormat<DT>::V4;
    using E = typename PfFormat<DT>::E;
    // four separate arrays (not one indexed by parity) so the compiler can
    // tell the tile being copied from the tile being read and does not wait
    // for the copy before the reads
    __shared__ __attribute__((aligned(1024))) char k0s[T::TILE];
    __shared__ __attribute__((aligned(1024))) char k1s[T::TILE];
    __shared__ __attribute__((aligned(1024))) char v0s[T::TILE];
    __shared__ __attribute__((aligned(1024))) char v1s[T::TILE];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, g = lane >> 5;

    // block -> (query tile, batch, head)
    const int id = blockIdx.x;
    const int bh = a.batch * a.heads;
    const int qt = a.causal ? (a.qtiles - 1 - id / bh) : (id / bh);  // heaviest tiles first
    int b, h;
    if (a.xcd_map) {
        // Inside one tile index, consecutive block ids (dispatched round-robin
        // over the 8 XCDs) are mapped so the G query heads of a kv group
        // (batch, kv head) land on the same XCD and share its L2 for their K/V
        // tiles.  (Walking one group at a time per XCD measured slower: it
        // loses the global heaviest-first order.)
        const int G = a.heads / a.kv_heads;
        const int j = id % bh;
        const int xcd = j & 7, slot = j >> 3;
        const int grp = (slot / G) * 8 + xcd;
        b = grp / a.kv_heads;
        h = (grp % a.kv_heads) * G + slot % G;
    } else {
        b = (id % bh) / a.heads;
        h = id % a.heads;
    }
    const int kvh = h / (a.heads / a.kv_heads);
    const int q0 = qt * BM;
    const int64_t qrs = (int64_t)a.heads * D, krs = (int64_t)a.kv_heads * D;
    const uint16_t *qbase = a.q + (int64_t)b * a.seq_q * qrs + (int64_t)h * D;
    const uint16_t *kbase = a.k + (int64_t)b * a.seq_k * krs + (int64_t)kvh * D;
    const uint16_t *vbase = a.v + (int64_t)b * a.seq_k * krs + (int64_t)kvh * D;

    // this lane's query and its Q^T operand fragments (KS k-steps of 16 dims)
    const int qfirst = q0 + 32 * wave;
    const int qlast = min(qfirst + 31, a.seq_q - 1);
    const int qi = qfirst + l32;
    V8 qf[T::KS];
    {
        const int qload = min(qi, a.seq_q - 1);  // rows past the end compute garbage, never stored
#pragma unroll
        for (int t = 0; t < T::KS; ++t)
            qf[t] = __builtin_bit_cast(V8, *reinterpret_cast<const uint4 *>(qbase + (int64_t)qload * qrs + 16 * t + 8 * g));
    }

    // key tiles of the block: [tlo, ntiles); tiles [tfree, nfree) need no mask for
    // any query of it.  Without a window tlo = tfree = 0; with one, the tiles below
    // the first query's window are skipped and those below the last query's window
    // edge are masked.
    int kend = a.seq_k;
    if (a.causal) kend = min(kend, min(q0 + BM, a.seq_q) + a.shift);
    const int ntiles = kend > 0 ? (kend + BN - 1) / BN : 0;
    int nfree = a.seq_k / BN;
    if (a.causal) nfree = min(nfree, q0 + a.shift + 1 > 0 ? (q0 + a.shift + 1) / BN : 0);
    nfree = min(nfree, ntiles);
    if (GEN && a.alibi_s != 0.0f) nfree = 0;   // the bias is added by the masked step only
    int tlo = 0, tfree = 0;
    if (GEN && a.window > 0) {
        const int qmax = min(q0 + BM, a.seq_q) - 1;
        tlo = min(max(0, q0 - a.window + 1) / BN, ntiles);
        tfree = max(tlo, (max(0, qmax - a.window + 1) + BN - 1) / BN);
    }

    // byte offsets of this lane's tile copies (source side, swizzled) ...
    int kg[T::NI], vg[T::NI];
    {
        const int rs2 = a.kv_heads * D * 2;
        const int pos = lane % T::NC;
#pragma unroll
        for (int i = 0; i < T::NI; ++i) {
            const int row = 4 * T::RPI * i + T::RPI * wave + lane / T::NC;
            kg[i] = row * rs2 + ((pos ^ T::kswz(row)) << 4);
            vg[i] = row * rs2 + ((pos ^ T::vswz(row)) << 4);
        }
    }
    // ... and of its fragment reads: K row l32 (+32c), chunk (2t + g) ^ kswz(l32);
    // V: lane group q = lane/16, i = lane%16 = 4j + m reads key row 4(q/2) + j,
    // dims 16(q%2) + 4m .. +3 of dim block d: chunk (4d + 2(q%2) + m/2) ^ vswz(row), half m%2
    int ka[T::KS], va[T::DB];
#pragma unroll
    for (int t = 0; t < T::KS; ++t) ka[t] = l32 * T::RB + (((2 * t + g) ^ T::kswz(l32)) << 4);
    {
        const int q = lane >> 4, i = lane & 15, j = i >> 2, m = i & 3;
        const int row = 4 * (q >> 1) + j;
#pragma unroll
        for (int d = 0; d < T::DB; ++d) {
            const int chunk = (4 * d + 2 * (q & 1) + (m >> 1)) ^ T::vswz(row);
            va[d] = row * T::RB + (chunk << 4) + 8 * (m & 1);
        }
    }
    PrefillState<D> st;
#pragma unroll
    for (int d = 0; d < T::DB; ++d) st.o[d] = (f32x16){};
    st.m = -INFINITY;
    st.l = 0.0f;

    // tile t lives in buffer t % 2
    if (tlo < ntiles)
        prefill_copy_tile<D>(a, kbase, vbase, tlo * BN, kg, vg, (tlo & 1) ? k1s : k0s, (tlo & 1) ? v1s : v0s, wave);
    wait_tile_copies();
    __syncthreads();
    // One tile: copy the next tile into the other buffers, compute this one, then
    // wait for the copy and meet at the barrier.  The mask-free tiles [0, nfree)
    // come first and run in a loop of their own (two tiles per iteration so the
    // buffer roles are fixed at compile time); the masked tiles (diagonal, tail)
    // follow in a second loop, so the O accumulators never pass through a merge
    // of the two paths (which cost a register copy of O per tile).
    auto tile_free = [&](int it, const char *kc, const char *vc, char *kn, char *vn) __attribute__((always_inline)) {
        // the next tile's copy runs inside the step (past the last tile: an empty one
        // into the free buffers, so the step has no branch around it)
        const int kvn = it + 1 < ntiles ? (it + 1) * BN : a.seq_k;
        prefill_step_pipelined<DT, D>(a, kc, vc, qf, st, ka, va, kbase, vbase, kvn, kg, vg, kn, vn, wave);
        wait_tile_copies();
        __syncthreads();
    };
    auto tile_masked = [&](int it) __attribute__((always_inline)) {
        const int kv0 = it * BN;
        const bool odd = it & 1;
        if (it + 1 < ntiles)
            prefill_copy_tile<D>(a, kbase, vbase, kv0 + BN, kg, vg, odd ? k0s : k1s, odd ? v0s : v1s, wave);
        // waves whose queries all precede this tile, or whose windows all start
        // past it, skip it
        if ((!a.causal || kv0 <= qlast + a.shift) && (!GEN || a.window <= 0 || kv0 + BN - 1 >= qfirst - a.window + 1))
            prefill_step<DT, D, GEN>(a, odd ? k1s : k0s, odd ? v1s : v0s, qf, st, qi, kv0, ka, va, g, true);
        wait_tile_copies();
        __syncthreads();
    };
    int it = tlo;
    for (; it < tfree && it < ntiles; ++it) tile_masked(it);   // the window's lower edge
    if (it < nfree && (it & 1)) {   // the paired loop below starts on an even tile
        tile_free(it, k1s, v1s, k0s, v0s);
        ++it;
    }
    for (; it + 1 < nfree; it += 2) {
        tile_free(it, k0s, v0s, k1s, v1s);
        tile_free(it + 1, k1s, v1s, k0s, v0s);
    }
    if (it < nfree) {
        tile_free(it, k0s, v0s, k1s, v1s);
        ++it;
    }
    for (; it < ntiles; ++it) tile_masked(it);

    // normalise and store: lane holds O[qi][32d + 8*(r/4) + 4g + r%4]
    const float ltot = swap_halves_sum(st.l);
    const float inv = ltot > 0.0f ? 1.0f / ltot : 0.0f;
    if (qi < a.seq_q) {
        uint16_t *orow = a.o + (int64_t)b * a.seq_q * qrs + (int64_t)qi * qrs + (int64_t)h * D;
#pragma unroll
        for (int d = 0; d < T::DB; ++d)
#pragma unroll
            for (int rb = 0; rb < 4; ++rb) {
                V4 v;
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = (E)(st.o[d][4 * rb + i] * inv);
                *reinterpret_cast<V4 *>(orow + 32 * d + 8 * rb + 4 * g) = v;
            }
    }
}

// ------------------------------------------------------------ f32 prefill --
// f32 MultiHeadAttention (head dim 128 or 64, causal or not, sliding window, ALiBi) on
// v_mfma_f32_32x32x2_f32: exact f32 products, f32 sums, softmax in f32 against a
// running maximum (the reference's stableSoftmaxRow takes the row max, exp in
// float64 and a sequential f32 sum; the order of the sums differs, the f32 bar
// holds).  One 256-thread block per (128-query tile, head, batch), wave w owning 32
// queries; K/V stream through LDS in 32-key tiles (16 KB each at D = 128), double
// buffered, copied HBM -> LDS by buffer_load ... lds; two blocks per CU.
//   S^T[key, q] = K . Q^T: MFMA step s of 4-step group g gives half h = lane / 32 of
//     the wave d = 8 g + 4 h + s, so a lane's K operands for a group are one 16-byte
//     LDS read of its key row (chunk c of row r at c ^ (r % 16): the 16 rows an LDS
//     cycle serves on distinct banks) and Q^T sits in registers for the whole loop.
//   The accumulator's register r = 4 g + s of lane (q, h) holds key 8 g + 4 h + s, so
//     P^T is already the B operand of O^T[d, q] += V^T . P^T for the same k order;
//     V^T's operand is one float per lane and step from the row-major V tile (row k
//     keeps column d at d ^ 32 (k / 4 % 2), so the two half-waves, rows k and k + 4,
//     read opposite halves of the bank line).
template <int D> struct PfF32Dim {
    static_assert(D == 128 || D == 64, "head dim 128 or 64");
    static constexpr int BN = 32;               // keys per tile
    static constexpr int RB = D * 4;            // row bytes
    static constexpr int NC = RB / 16;          // 16-byte chunks per row
    static constexpr int TILE = BN * RB;        // 16 or 8 KB
    static constexpr int KG = D / 8;            // 4-step groups over d
    static constexpr int DB = D / 32;           // O^T blocks of 32 dims
    static constexpr int RPI = 64 / NC;         // rows per copy instruction
    static constexpr int NI = BN / RPI / 4;     // copy instructions per wave and tensor
    static constexpr int kswz(int r) { return r & 15; }
    static constexpr int vswz(int r) { return ((r >> 2) & 1) << 3; }   // in chunks (8 = 32 floats)
};

template <int D, bool GEN>
__global__ __launch_bounds__(256, 2) void prefill_f32_kernel(PrefillArgs a) {
    using T = PfF32Dim<D>;
    constexpr int BM = fa::BM, BN = T::BN;
    __shared__ __attribute__((aligned(1024))) char k0s[T::TILE];
    __shared__ __attribute__((aligned(1024))) char k1s[T::TILE];
    __shared__ __attribute__((aligned(1024))) char v0s[T::TILE];
    __shared__ __attribute__((aligned(1024))) char v1s[T::TILE];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, h = lane >> 5;

    // block -> (query tile, batch, head), heaviest tiles first, a kv group's query
    // heads on one XCD (as prefill_kernel)
    const int id = blockIdx.x;
    const int bh = a.batch * a.heads;
    const int qt = a.causal ? (a.qtiles - 1 - id / bh) : (id / bh);
    int b, hd;
    if (a.xcd_map) {
        const int G = a.heads / a.kv_heads;
        const int j = id % bh;
        const int xcd = j & 7, slot = j >> 3;
        const int grp = (slot / G) * 8 + xcd;
        b = grp / a.kv_heads;
        hd = (grp % a.kv_heads) * G + slot % G;
    } else {
        b = (id % bh) / a.heads;
        hd = id % a.heads;
    }
    const int kvh = hd / (a.heads / a.kv_heads);
    const int q0 = qt * BM;
    const float *const qp = reinterpret_cast<const float *>(a.q);
    const float *const kp = reinterpret_cast<const float *>(a.k);
    const float *const vp = reinterpret_cast<const float *>(a.v);
    const int64_t qrs = (int64_t)a.heads * D, krs = (int64_t)a.kv_heads * D;
    const float *qbase = qp + (int64_t)b * a.seq_q * qrs + (int64_t)hd * D;
    const float *kbase = kp + (int64_t)b * a.seq_k * krs + (int64_t)kvh * D;
    const float *vbase = vp + (int64_t)b * a.seq_k * krs + (int64_t)kvh * D;

    // this lane's query and its Q^T operands: qf[g] = Q[qi][8 g + 4 h .. + 3]
    const int qfirst = q0 + 32 * wave;
    const int qlast = min(qfirst + 31, a.seq_q - 1);
    const int qi = qfirst + l32;
    f32x4 qf[T::KG];
    {
        const int qload = min(qi, a.seq_q - 1);   // rows past the end compute garbage, never stored
#pragma unroll
        for (int g = 0; g < T::KG; ++g)
            qf[g] = *reinterpret_cast<const f32x4 *>(qbase + (int64_t)qload * qrs + 8 * g + 4 * h);
    }

    int kend = a.seq_k;
    if (a.causal) kend = min(kend, min(q0 + BM, a.seq_q) + a.shift);
    const int ntiles = kend > 0 ? (kend + BN - 1) / BN : 0;
    int nfree = a.seq_k / BN;
    if (a.causal) nfree = min(nfree, q0 + a.shift + 1 > 0 ? (q0 + a.shift + 1) / BN : 0);
    nfree = min(nfree, ntiles);
    if (GEN && a.alibi_s != 0.0f) nfree = 0;   // the bias is added by the masked step only
    // a sliding window: the tiles below the block's first query's window are skipped,
    // those below its last query's window edge masked ([wlo, wfree))
    int wlo = 0, wfree = 0;
    if (GEN && a.window > 0) {
        const int qmax = min(q0 + BM, a.seq_q) - 1;
        wlo = min(max(0, q0 - a.window + 1) / BN, ntiles);
        wfree = max(wlo, (max(0, qmax - a.window + 1) + BN - 1) / BN);
    }

    // copy offsets (source side, swizzled): wave w fills rows 4 RPI i + RPI w + lane / NC
    int kg[4], vg[4];
    {
        const int rs4 = a.kv_heads * D * 4;
        const int pos = lane % T::NC;
#pragma unroll
        for (int i = 0; i < T::NI; ++i) {
            const int row = 4 * T::RPI * i + T::RPI * wave + lane / T::NC;
            kg[i] = row * rs4 + ((pos ^ T::kswz(row)) << 4);
            vg[i] = row * rs4 + ((pos ^ T::vswz(row)) << 4);
        }
    }
    auto copy_tile = [&](int kv0, char *kdst, char *vdst) __attribute__((always_inline)) {
        const int rs4 = a.kv_heads * D * 4;
        const int rows = min(a.seq_k - kv0, BN);
        const int bytes = (rows - 1) * rs4 + D * 4;
        const int64_t base = (int64_t)kv0 * a.kv_heads * D;
        const __amdgpu_buffer_rsrc_t kd =
            __builtin_amdgcn_make_buffer_rsrc((void *)(kbase + base), (short)0, bytes, fa::BUF_WORD3);
        const __amdgpu_buffer_rsrc_t vd =
            __builtin_amdgcn_make_buffer_rsrc((void *)(vbase + base), (short)0, bytes, fa::BUF_WORD3);
        // (constant trip counts with a guard: a loop bound that depends on the template
        // arguments inside a lambda loses the kernel's host stub)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (i < T::NI)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(kd, (lds_void *)(kdst + (4 * T::RPI * i + T::RPI * wave) * T::RB),
                                                         16, kg[i], 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (i < T::NI)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(vd, (lds_void *)(vdst + (4 * T::RPI * i + T::RPI * wave) * T::RB),
                                                         16, vg[i], 0, 0, 0);
    };
    // fragment reads: K row l32, group g at chunk (2 g + h) ^ kswz(l32); V row
    // 8 g + 4 h + s, column (32 db + l32) ^ 32 h (vswz(row) = 8 chunks iff h = 1)
    const int kr = l32 * T::RB;
    int vr[4];
#pragma unroll
    for (int db = 0; db < 4; ++db) vr[db] = 4 * h * T::RB + (((32 * db + l32) ^ (32 * h)) << 2);

    f32x16 o[4];
#pragma unroll
    for (int db = 0; db < 4; ++db) o[db] = (f32x16){};
    float m = -INFINITY, l = 0.0f;
    const float c = a.scale_log2;

    auto step = [&](const char *ks, const char *vs, int kv0, bool masked) __attribute__((always_inline)) {
        f32x16 sacc = (f32x16){};
#pragma unroll
        for (int g = 0; g < 16; ++g) {
            if (g >= T::KG) break;
            const f32x4 kv = *reinterpret_cast<const f32x4 *>(ks + kr + (((2 * g + h) ^ T::kswz(l32)) << 4));
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4) sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[s4], qf[g][s4], sacc, 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);   // one group's K read live at a time
        }
        // register r: key kv0 + 8 (r / 4) + 4 h + r % 4, query qi.  The masked step
        // also adds ALiBi's alibi_s * (k - q) (before the scale: slope * (k - q) on the
        // scaled score, typed_compute.go:176-178) and hides keys below the window
        if (masked) {
            const int last = a.causal ? min(qi + a.shift, a.seq_k - 1) : a.seq_k - 1;
            const int lim = last - kv0 - 4 * h;
            const int lo = GEN && a.window > 0 ? qi - a.window + 1 - kv0 - 4 * h : INT_MIN;
            if (GEN && a.alibi_s != 0.0f) {
                const float base = (float)(kv0 + 4 * h - qi);
#pragma unroll
                for (int r = 0; r < 16; ++r) sacc[r] += a.alibi_s * (base + (float)(8 * (r >> 2) + (r & 3)));
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int off = 8 * (r >> 2) + (r & 3);
                if (off > lim || off < lo) sacc[r] = -INFINITY;
            }
        }
        float tmax = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) tmax = fmaxf(tmax, sacc[r]);
        tmax = swap_halves_max(tmax) * c;
        if (__any(tmax > m)) {   // a new maximum: rescale O and l (wave-uniform branch)
            const float mnew = fmaxf(m, tmax);
            const float alpha = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - mnew);
            m = mnew;
            l *= alpha;
#pragma unroll
            for (int db = 0; db < 4; ++db) {
                if (db >= T::DB) break;
#pragma unroll
                for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
            }
        }
        const float mref = m == -INFINITY ? 0.0f : m;
        float psum = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            sacc[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[r], c, -mref));
            psum += sacc[r];
        }
        l += psum;
        // O^T += V^T . P^T, step (g, s4): V row 8 g + 4 h + s4, P^T register 4 g + s4; a
        // scheduling barrier per group keeps one group's V reads live at a time
#pragma unroll
        for (int g = 0; g < BN / 8; ++g) {
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
                for (int db = 0; db < 4; ++db) {
                    if (db >= T::DB) break;
                    const float vv = *reinterpret_cast<const float *>(vs + (8 * g + s4) * T::RB + vr[db]);
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv, sacc[4 * g + s4], o[db], 0, 0, 0);
                }
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // this block's key tiles: from the window's lower edge on, all of them or split
    // blockIdx.y's run of split_tiles
    int tlo = wlo, thi = ntiles;
    if (a.split_tiles > 0) {
        const int ylo = min(ntiles, (int)blockIdx.y * a.split_tiles);
        tlo = max(tlo, ylo);
        thi = min(ntiles, ylo + a.split_tiles);
    }
    if (tlo < thi) copy_tile(tlo * BN, k0s, v0s);
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
    __syncthreads();
    auto tile = [&](int it, const char *kc, const char *vc, char *kn, char *vn) __attribute__((always_inline)) {
        const int kv0 = it * BN;
        if (it + 1 < thi) copy_tile(kv0 + BN, kn, vn);
        // waves whose queries all precede the tile, or whose windows all start past it,
        // skip it
        const bool seen = (!a.causal || kv0 <= qlast + a.shift) && (!GEN || a.window <= 0 || kv0 + BN - 1 >= qfirst - a.window + 1);
        if (it >= wfree && it < nfree) step(kc, vc, kv0, false);
        else if (seen) step(kc, vc, kv0, true);
        __builtin_amdgcn_s_waitcnt(0x0F70);
        __syncthreads();
    };
    int it = tlo;
    for (; it + 1 < thi; it += 2) {
        tile(it, k0s, v0s, k1s, v1s);
        tile(it + 1, k1s, v1s, k0s, v0s);
    }
    if (it < thi) tile(it, k0s, v0s, k1s, v1s);

    const float ltot = swap_halves_sum(l);
    if (a.part_ml) {
        // split: the row's (max, sum) and unnormalised output to the partials
        if (qi < a.seq_q) {
            const int64_t prow = (((int64_t)blockIdx.y * a.batch + b) * a.seq_q + qi) * a.heads + hd;
            if (h == 0) a.part_ml[prow] = make_float2(m, ltot);
            float *orow = a.part_o + prow * D;
#pragma unroll
            for (int db = 0; db < 4; ++db) {
                if (db >= T::DB) break;
#pragma unroll
                for (int rb = 0; rb < 4; ++rb) {
                    f32x4 v;
#pragma unroll
                    for (int i = 0; i < 4; ++i) v[i] = o[db][4 * rb + i];
                    *reinterpret_cast<f32x4 *>(orow + 32 * db + 8 * rb + 4 * h) = v;
                }
            }
        }
        return;
    }
    // normalise and store: lane holds O[qi][32 db + 8 (r/4) + 4 h + r%4]
    const float inv = ltot > 0.0f ? 1.0f / ltot : 0.0f;
    if (qi < a.seq_q) {
        float *orow = reinterpret_cast<float *>(a.o) + (int64_t)b * a.seq_q * qrs + (int64_t)qi * qrs + (int64_t)hd * D;
#pragma unroll
        for (int db = 0; db < 4; ++db) {
            if (db >= T::DB) break;
#pragma unroll
            for (int rb = 0; rb < 4; ++rb) {
                f32x4 v;
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = o[db][4 * rb + i] * inv;
                *reinterpret_cast<f32x4 *>(orow + 32 * db + 8 * rb + 4 * h) = v;
            }
        }
    }
}

// Merges the key splits of prefill_f32_kernel: one wave per (batch, query, head) row,
// lanes over the head dims; the splits are folded in order with weights
// exp2(m_s - M) (m in the scaled log2 domain), O = sum w_s O_s / sum w_s l_s; a row
// with no visible key (every m = -inf) is 0, as in the unsplit kernel.
template <int D>
__global__ __launch_bounds__(256) void prefill_f32_combine_kernel(PrefillArgs a, int splits, int64_t rows) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int lane = threadIdx.x & 63;
    float M = -INFINITY;
    for (int s = 0; s < splits; ++s) M = fmaxf(M, a.part_ml[s * rows + row].x);
    float acc[D / 64] = {}, lsum = 0.0f;
    if (M != -INFINITY) {
        for (int s = 0; s < splits; ++s) {
            const float2 ml = a.part_ml[s * rows + row];
            const float w = ml.x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ml.x - M);
            lsum += w * ml.y;
            const float *po = a.part_o + (s * rows + row) * D;
#pragma unroll
            for (int j = 0; j < D / 64; ++j) acc[j] += w * po[64 * j + lane];
        }
    }
    const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
    // row = (batch, query, head): the output row of the same index, D floats
    float *out = reinterpret_cast<float *>(a.o) + row * D;
#pragma unroll
    for (int j = 0; j < D / 64; ++j) out[64 * j + lane] = acc[j] * inv;
}

// f32 MultiHeadAttention on prefill_f32_kernel: head dim 128 or 64, at least 16 query
// rows, causal or not, with or without a sliding window and ALiBi.
static bool launch_prefill_f32(const MhaArgs &m, hipStream_t s, int *status) {
    if (m.dim != 128 && m.dim != 64) return false;
    if (m.seq_q < 16) return false;
    if (m.seq_q > 0x3FFFFFFF || m.seq_k > 0x3FFFFFFF || m.shift > 0x3FFFFFFF || m.shift < -0x3FFFFFFF) return false;
    if (m.kv_heads > 32768) return false;   // a 32-row K/V tile spans < 2^31 bytes
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
    // a window of seq_q or more hides no key (a query's distance to a visible key is
    // below seq_q): run it as no window
    a.window = (m.window > 0 && m.window < m.seq_q) ? (int)m.window : 0;
    a.alibi_s = m.alibi != 0.0f ? m.alibi / m.scale : 0.0f;
    a.xcd_map = ((a.batch * a.kv_heads) % 8 == 0) ? 1 : 0;
    a.scale_log2 = m.scale * 1.4426950408889634f;
    const bool gen = a.window > 0 || a.alibi_s != 0.0f;   // the kernel with the window / ALiBi code
    const int64_t blocks = (int64_t)a.qtiles * a.batch * a.heads;
    if (blocks > 0x7FFFFFFF) return false;
    const int64_t cus = device_cus();
    const int64_t ktiles = (m.seq_k + 31) / 32;
    hipStreamCaptureStatus cst = hipStreamCaptureStatusNone;
    const bool capturing = hipStreamIsCapturing(s, &cst) != hipSuccess || cst != hipStreamCaptureStatusNone;
    // Grids of fewer than 24 blocks stay on the general kernel (one block per query
    // row and head) unless they are causal over at least 8 key tiles and can split
    // them (below): config 1's 128 queries x 8 heads of 64 (8 blocks) 9.2 us there
    // against 14.2 here even split; 256 x 8 x 128 (16 blocks) 33.1 against 24.1 split
    // (43 unsplit), 640 x 4 x 64 47.5 against 22.1.  From 24 blocks this kernel wins
    // unsplit too (384 x 8 x 64: 32.9 against 36.0, 4 x 128 x 8 x 64: 15.0 against 24.5)
    if (blocks < 24 && (!a.causal || ktiles < 8 || capturing)) return false;
    // Small grids split each block's key range over blockIdx.y, partials in the
    // library's scratch: the longest block's key loop, the critical path, shrinks with
    // the split count.  Causal grids of under two blocks per CU aim at four blocks per
    // CU in runs of at least 8 key tiles (2 under 24 blocks) (the triangle leaves most
    // CUs idle while the last query tiles run: B1 S4096 8 x 64 causal 296 -> 221 us,
    // S2048 8 x 128 154 -> 146 us), other grids of under one block per CU at two, in
    // runs of at least 16 (B1 S2048 8 x 64, 150 -> 88 us; more splits lose there).  A
    // stream that is capturing a graph keeps the unsplit kernel (the scratch cannot
    // grow there)
    int64_t splits = 1;
    if (a.causal && blocks < 2 * cus)
        splits = std::max<int64_t>(1, std::min<int64_t>((4 * cus + blocks - 1) / blocks, ktiles / (blocks < 24 ? 2 : 8)));
    else if (!a.causal && blocks < cus)
        splits = std::max<int64_t>(1, std::min<int64_t>((2 * cus + blocks - 1) / blocks, ktiles / 16));
    if (capturing) splits = 1;
    if (splits > 1) {
        a.split_tiles = (int)((ktiles + splits - 1) / splits);
        splits = (ktiles + a.split_tiles - 1) / a.split_tiles;
        const int64_t rows = m.batch * m.seq_q * m.heads;
        const size_t need = (size_t)(splits * rows) * (sizeof(float2) + (size_t)m.dim * sizeof(float));
        ScratchLease lease(need, s);
        if (lease.status()) {
            *status = lease.status();
            return true;
        }
        // outputs first: splits * rows * D floats keep the (max, sum) pairs 16-byte aligned
        a.part_o = static_cast<float *>(lease.ptr());
        a.part_ml = reinterpret_cast<float2 *>(a.part_o + splits * rows * m.dim);
        const dim3 grid((unsigned)blocks, (unsigned)splits);
        const unsigned cblocks = (unsigned)((rows + 3) / 4);
        if (m.dim == 128) {
            if (gen) prefill_f32_kernel<128, true><<<grid, 256, 0, s>>>(a);
            else prefill_f32_kernel<128, false><<<grid, 256, 0, s>>>(a);
            prefill_f32_combine_kernel<128><<<cblocks, 256, 0, s>>>(a, (int)splits, rows);
        } else {
            if (gen) prefill_f32_kernel<64, true><<<grid, 256, 0, s>>>(a);
            else prefill_f32_kernel<64, false><<<grid, 256, 0, s>>>(a);
            prefill_f32_combine_kernel<64><<<cblocks, 256, 0, s>>>(a, (int)splits, rows);
        }
        const int rc = check_launch("prefill f32 mfma split");
        const int fin = lease.finish();
        *status = rc ? rc : fin;
        return true;
    }
    if (m.dim == 128) {
        if (gen) prefill_f32_kernel<128, true><<<(unsigned)blocks, 256, 0, s>>>(a);
        else prefill_f32_kernel<128, false><<<(unsigned)blocks, 256, 0, s>>>(a);
    } else {
        if (gen) prefill_f32_kernel<64, true><<<(unsigned)blocks, 256, 0, s>>>(a);
        else prefill_f32_kernel<64, false><<<(unsigned)blocks, 256, 0, s>>>(a);
    }
    *status = check_launch("prefill f32 mfma");
    return true;
}

bool launch_prefill_mfma(const MhaArgs &m, int dtype, hipStream_t s, int *status) {
    if (dtype == PUTER_F32) return launch_prefill_f32(m, s, status);
    if ((dtype != PUTER_BF16 && dtype != PUTER_F16) || (m.dim != 128 && m.dim != 64)) return false;
    if (m.dim == 64 && m.seq_q == 1) return false;   // one query row: the general kernel (no 127 padding rows)
    if (m.seq_q > 0x3FFFFFFF || m.seq_k > 0x3FFFFFFF || m.shift > 0x3FFFFFFF || m.shift < -0x3FFFFFFF)
        return false;
    // 32-bit buffer offsets: one 64-row tile of K/V must span < 2^31 bytes
    if (m.kv_heads > 65536) return false;
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
    // a window of seq_q or more hides no key (a query's distance to a visible key
    // is below seq_q): run it as no window
    a.window = (m.window > 0 && m.window < m.seq_q) ? (int)m.window : 0;
    a.alibi_s = m.alibi != 0.0f ? m.alibi / m.scale : 0.0f;
    a.xcd_map = ((a.batch * a.kv_heads) % 8 == 0) ? 1 : 0;
    a.scale_log2 = m.scale * 1.4426950408889634f;
    const int64_t blocks = (int64_t)a.qtiles * a.batch * a.heads;
    if (blocks > 0x7FFFFFFF) return false;
    const bool bf = dtype == PUTER_BF16, win = a.window > 0 || a.alibi_s != 0.0f;
    const dim3 grid((unsigned)blocks);
    if (m.dim == 128) {
        if (win) {
            if (bf) prefill_kernel<PUTER_BF16, 128, true><<<grid, 256, 0, s>>>(a);
            else prefill_kernel<PUTER_F16, 128, true><<<grid, 256, 0, s>>>(a);
        } else {
            if (bf) prefill_kernel<PUTER_BF16, 128, false><<<grid, 256, 0, s>>>(a);
            else prefill_kernel<PUTER_F16, 128, false><<<grid, 256, 0, s>>>(a);
        }
    } else {
        if (win) {
            if (bf) prefill_kernel<PUTER_BF16, 64, true><<<grid, 256, 0, s>>>(a);
            else prefill_kernel<PUTER_F16, 64, true><<<grid, 256, 0, s>>>(a);
        } else {
            if (bf) prefill_kernel<PUTER_BF16, 64, false><<<grid, 256, 0, s>>>(a);
            else prefill_kernel<PUTER_F16, 64, false><<<grid, 256, 0, s>>>(a);
        }
    }
    *status = check_launch("prefill mfma");
    return true;
}

}  // namespace puter
