/*
 * puter_hip.h -- C ABI of the MI355X (gfx950) device backend for puter.
 *
 * Every entry point mirrors one method of the reference's Go contract
 * (device/interface.go) or one optional execution hook, and is what a cgo
 * package `device/hip` binds.  The
 * conventions follow the reference's call conventions:
 *
 *   - plain pointers (device addresses) and 64-bit sizes; no C++ or HIP types;
 *   - the Go methods return nothing and panic on misuse: here every entry point
 *     returns an int status (0 = ok) that the Go wrapper turns into panic(err),
 *     with puter_hip_last_error() giving the message (thread-local);
 *   - zero-sized work returns 0 without launching (device/cpu/layernorm/compute.go:19-21);
 *   - `stream` is a hipStream_t passed as void* (NULL = the default stream).
 *     Launches are asynchronous: no compute entry point synchronises the host,
 *     matching the zero-host-sync rule the reference's interface documents;
 *   - the caller owns every buffer (workspaces included, see
 *     puter_hip_paged_decode_workspace_bytes).  The one allocation the library
 *     makes itself is a split-K scratch shared by puter_hip_matmul (16-bit
 *     formats with at most 512 rows or under two rounds of 128x128 tiles, F32
 *     outputs of fewer 128x128 tiles than the device has CUs, when K is split
 *     across blocks rather than inside them) and
 *     puter_hip_multi_head_attention[_batched] with seq_q == 1 (bf16 / f16 at
 *     head dim 128 without ALiBi, or any row over more than 768 keys) or in F32
 *     with at least 16 query rows, head dim 128 or 64, and
 *     fewer 128-query blocks than two per CU (causal) or one per CU (not
 *     causal): one buffer per device, allocated on first use and grown on
 *     demand (Matmul: at most 16 MiB; one-row attention: the paged decode
 *     workspace size, or batch x heads x ceil(seq_k / 256) x (head_dim + 2)
 *     floats; F32 attention: key splits x batch x seq_q x heads x (head_dim +
 *     2) floats, at most about 100 MB).  A growth is stream-ordered on the calling
 *     stream (hipFreeAsync of the old buffer after its last user, then
 *     hipMallocAsync): it never blocks the host.  On a stream that is capturing
 *     a HIP graph these calls allocate, free, wait on and record nothing: they
 *     use the buffer held if it is large enough (the graph keeps its address,
 *     so that buffer is never freed: a later growth keeps it and allocates
 *     beside it) and otherwise return PUTER_ERR_INVALID before launching; make
 *     the same call, or a larger one, outside the capture first (F32 attention
 *     takes its unsplit kernel under capture and uses no scratch).  Replays share
 *     the buffer with eager scratch-using calls until such a growth, so the
 *     caller orders them (one stream, or its own events).
 *
 * Status codes follow the reference's CUDA bridge (device/cuda/internal/bridge/status.c):
 *   -2 nil buffer, -6 invalid dtype / shape / config, -7 device unavailable,
 *   -8 launch or runtime error.
 */
#ifndef PUTER_HIP_H
#define PUTER_HIP_H

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define PUTER_API __attribute__((visibility("default")))
#else
#define PUTER_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes (manifesto/dtype values are Go-side; the cgo wrapper maps them) */
enum puter_dtype {
    PUTER_F32 = 0,
    PUTER_F16 = 1,
    PUTER_BF16 = 2,
    PUTER_F8E4M3 = 3, /* OCP E4M3FN: bias 7, no Inf, NaN = S.1111.111 */
    PUTER_F8E5M2 = 4, /* OCP E5M2: bias 15, IEEE-like Inf/NaN */
    PUTER_I32 = 5,
    PUTER_I8 = 6,
    PUTER_I4 = 7,     /* packed signed nibbles: element 2k = low nibble of byte k, 2k+1 = high */
    PUTER_F64 = 8,
};

enum puter_status {
    PUTER_OK = 0,
    PUTER_ERR_NIL = -2,
    PUTER_ERR_INVALID = -6,
    PUTER_ERR_UNAVAILABLE = -7,
    PUTER_ERR_LAUNCH = -8,
};

/* ------------------------------------------------------------------------ */
/* Runtime: the tensor.Backend side (device/cuda/backend.go:101-234 is the   */
/* reference memory backend these replace: Upload/Download/Close).           */
/* ------------------------------------------------------------------------ */
PUTER_API const char *puter_hip_last_error(void);
PUTER_API int puter_hip_version(void);
PUTER_API int puter_hip_device_count(int *count);
PUTER_API int puter_hip_set_device(int device);
/* device memory is 256-byte aligned (>= the 128-byte NativeAlignment of
 * device/cuda/backend.go Capabilities) */
PUTER_API int puter_hip_malloc(void **ptr, size_t bytes);
PUTER_API int puter_hip_free(void *ptr);
PUTER_API int puter_hip_memcpy_htod(void *dst, const void *src, size_t bytes, void *stream);
PUTER_API int puter_hip_memcpy_dtoh(void *dst, const void *src, size_t bytes, void *stream);
PUTER_API int puter_hip_memcpy_dtod(void *dst, const void *src, size_t bytes, void *stream);
PUTER_API int puter_hip_stream_create(void **stream);
PUTER_API int puter_hip_stream_destroy(void *stream);
PUTER_API int puter_hip_stream_synchronize(void *stream);

/* ------------------------------------------------------------------------ */
/* LayerNorm family: device/interface.go:355-379                             */
/* ------------------------------------------------------------------------ */
/* RMSNorm(config RMSNormConfig{Epsilon}, input, scale, output, rows, lastDim, format)
 * interface.go:373-378; CPU semantics device/cpu/layernorm/compute.go:350-385.
 * dtypes: F32, BF16, F16.  epsilon must be > 0 (device/config.go:86-92). */
PUTER_API int puter_hip_rmsnorm(const void *input, const void *scale, void *output, int64_t rows,
                      int64_t last_dim, double epsilon, int dtype, void *stream);

/* LayerNorm(input, scale, bias, output, rows, lastDim, format) interface.go:362-366;
 * epsilon is fixed at 1e-5 as in device/cpu/layernorm/compute.go:11. */
PUTER_API int puter_hip_layernorm(const void *input, const void *scale, const void *bias, void *output,
                        int64_t rows, int64_t last_dim, int dtype, void *stream);

/* AdaptiveRMSNorm(config, input, modulation, output, rows, lastDim, rowsPerBatch,
 * modulationCols, format) interface.go:356-361; y = x*inv*(1+scale)+shift with
 * scale at modulation[b*cols + c], shift at + lastDim (compute.go:387-433). */
PUTER_API int puter_hip_adaptive_rmsnorm(const void *input, const void *modulation, void *output,
                               int64_t rows, int64_t last_dim, int64_t rows_per_batch,
                               int64_t modulation_cols, double epsilon, int dtype, void *stream);

/* ModulatedLayerNorm(config{Epsilon, Set}, ...) interface.go:367-372; shift at
 * set*3H, scale at set*3H + H (compute.go:513-570,646-660). */
PUTER_API int puter_hip_modulated_layernorm(const void *input, const void *modulation, void *output,
                                  int64_t rows, int64_t last_dim, int64_t rows_per_batch,
                                  int64_t modulation_cols, double epsilon, int set, int dtype,
                                  void *stream);

/* GatedResidual: optional hook execution/math_gated_residual_intrinsic.go:11-17,
 * called at :268-279.  out = residual + gate * branch with
 * gate = modulation[(r/rowsPerBatch)*modulationCols + 3*set*H + 2H + c]. */
PUTER_API int puter_hip_gated_residual(const void *residual, const void *branch, const void *modulation,
                             void *output, int64_t rows, int64_t last_dim,
                             int64_t rows_per_batch, int64_t modulation_cols, int set,
                             int dtype, void *stream);

/* Fused GatedResidual -> RMSNorm / LayerNorm (extension hook; no reference
 * method exists).  Result equals GatedResidual(residual, branch, modulation,
 * hidden) followed by RMSNorm(hidden, scale, normed) / LayerNorm(hidden, scale,
 * bias, normed): the norm reads the stored (dtype-rounded) hidden values.
 * Both outputs are written; one HBM pass instead of three. */
PUTER_API int puter_hip_gated_residual_rmsnorm(const void *residual, const void *branch,
                                     const void *modulation, const void *scale, void *hidden,
                                     void *normed, int64_t rows, int64_t last_dim,
                                     int64_t rows_per_batch, int64_t modulation_cols, int set,
                                     double epsilon, int dtype, void *stream);
PUTER_API int puter_hip_gated_residual_layernorm(const void *residual, const void *branch,
                                       const void *modulation, const void *scale,
                                       const void *bias, void *hidden, void *normed,
                                       int64_t rows, int64_t last_dim, int64_t rows_per_batch,
                                       int64_t modulation_cols, int set, int dtype,
                                       void *stream);

/* ------------------------------------------------------------------------ */
/* RoPE family: device/interface.go:592-610, config device/config.go:125-213  */
/* ------------------------------------------------------------------------ */
typedef struct puter_rope_config {
    double base_freq;         /* RoPEConfig.BaseFreq */
    int64_t start_position;   /* RoPEConfig.StartPosition */
    int32_t mode;             /* 0 RoPEModeInterleaved, 1 RoPEModeHalf */
    int32_t scaling;          /* 0 RoPEScalingNone, 1 RoPEScalingLlama3 */
    double scaling_factor;
    double low_freq_factor;
    double high_freq_factor;
    int64_t original_context;
} puter_rope_config;

/* RoPE(config, input, output, seqLen, numHeads, headDim, format) interface.go:599-604.
 * Layout [seqLen, numHeads, headDim]; angles in float64 as
 * device/cpu/rope/compute.go:55-126.  input may equal output. */
PUTER_API int puter_hip_rope(const puter_rope_config *config, const void *input, void *output,
                   int64_t seq_len, int64_t num_heads, int64_t head_dim, int dtype,
                   void *stream);

typedef struct puter_multi_axis_rope_config {
    double base_freq;
    int64_t latent_seq_len;
    int64_t latent_side;
    int32_t axis_count;
    int32_t pad_;
    int64_t axis_dims[4];
} puter_multi_axis_rope_config;

/* MultiAxisRoPE(config, input, output, batch, seqLen, numHeads, headDim, format)
 * interface.go:593-598; compute.go:195-330. */
PUTER_API int puter_hip_multi_axis_rope(const puter_multi_axis_rope_config *config, const void *input,
                              void *output, int64_t batch, int64_t seq_len, int64_t num_heads,
                              int64_t head_dim, int dtype, void *stream);

/* RoPEPairs(output, input, cosBuffer, sinBuffer, halfDim, format) interface.go:605-609;
 * device/cpu/rope/ops.go:25-38 -> RopePairsGeneric f32_generic.go:3-11.  F32 only
 * (any other dtype is PUTER_ERR_INVALID, where the reference panics, ops.go:10-14):
 * output[2i] = in[2i]*cos[i] - in[2i+1]*sin[i], output[2i+1] = in[2i]*sin[i] +
 * in[2i+1]*cos[i] for i < half_dim, each operation rounded to f32. */
PUTER_API int puter_hip_rope_pairs(void *output, const void *input, const void *cos_buffer,
                                   const void *sin_buffer, int64_t half_dim, int dtype, void *stream);

/* ------------------------------------------------------------------------ */
/* Activation family (gated subset + Silu/Gelu): device/interface.go:18-74   */
/* ------------------------------------------------------------------------ */
enum puter_gate_kind {
    PUTER_GATE_SWIGLU = 0,     /* silu(gate) * up   (FastSwiGLU32) */
    PUTER_GATE_GEGLU = 1,      /* gate * gelu(up)   (FastGeGLU32)  */
    PUTER_GATE_GEGLU_TANH = 2, /* gate * gelu_tanh(up) */
    PUTER_GATE_SIGLU = 3,      /* sigmoid(gate) * up */
    PUTER_GATE_GLU = 4,        /* gate * sigmoid(up) */
    PUTER_GATE_REGLU = 5,      /* gate * relu(up) */
    PUTER_GATE_LINGLU = 6,     /* gate * up */
    PUTER_GATE_SEGLU = 7,      /* up * sigmoid(gate)   (FastSeGLU32, math/extra_activation.go:88-90) */
};
/* <Kind>Tensors(dst, gate, up, count, format): interface.go:28,35,52,57,62 ...
 * device/cpu/activation/gated.go:59-136 */
PUTER_API int puter_hip_gated_tensors(int kind, void *dst, const void *gate, const void *up,
                            int64_t count, int dtype, void *stream);
/* <Kind>(dst, packed, batch, halfCount, format): rows [gate | up] -> [half];
 * device/cpu/activation/gated.go:10-57, compute.go:72-116 */
PUTER_API int puter_hip_gated_packed(int kind, void *dst, const void *packed, int64_t batch,
                           int64_t half_count, int dtype, void *stream);
enum puter_unary_kind { PUTER_UNARY_SILU = 0, PUTER_UNARY_GELU = 1 };
/* Silu / Gelu(dst, src, count, format): interface.go:30,61; activation/ops.go:37-51 */
PUTER_API int puter_hip_unary(int kind, void *dst, const void *src, int64_t count, int dtype,
                    void *stream);

/* ------------------------------------------------------------------------ */
/* Casts: convert/ package (BFloat16ToFloat32 bf16_f32.go:11, Float32ToBFloat16   */
/* :21, Float16ToFloat32/Float32ToFloat16 f16_f32.go:10-42,                   */
/* Float8E4M3ToFloat32/Float32ToFloat8E4M3/E5M2 fp8_f32.go:8-65,              */
/* Int8ToFloat32 / Float32ToInt8 / Int4ToFloat32 int_f32.go:14-77,             */
/* Float32ToFloat64 / Float64ToFloat32 f32_f64.go:8-17).                       */
/* One of src_dtype / dst_dtype must be F32 (I4 only as a source; count is    */
/* the element count, the I4 source holds (count+1)/2 bytes).  Bit-exact      */
/* element-wise rules: RNE narrowing; fp8 saturating; NaN kept as NaN; int8   */
/* saturating then truncating toward zero, NaN -> 0.                          */
/* ------------------------------------------------------------------------ */
PUTER_API int puter_hip_cast(void *dst, int dst_dtype, const void *src, int src_dtype, int64_t count,
                   void *stream);

/* ------------------------------------------------------------------------ */
/* Paged KV: optional hooks execution/page_intrinsic.go:13-24 (called at      */
/* :199-211 and :334-344).  storage is [pages, pageSize, inner] starting      */
/* storage_offset elements into the buffer.                                   */
/*                                                                            */
/* Ids are validated on the device (the host cannot read them without a      */
/* synchronisation).  Where the reference's CPU path rejects the whole call   */
/* with ErrShapeMismatch (device/cpu/shape/page.go:139-146,191-203), a row    */
/* whose page id or slot is out of range is skipped (write) or zero-filled    */
/* (gather), no access leaves the storage, and PUTER_ERR_INVALID is stored    */
/* into *status, a caller-owned 4-byte-aligned device int32 (NULL: not        */
/* reported).  The library never clears it: the caller zeroes it, reads it at */
/* its next synchronisation and panics when it is non-zero.                   */
/* Write order matches the reference's sequential copy: among rows that       */
/* target one (page, slot) the last row wins (page_generic.go:23-27).         */
/* ------------------------------------------------------------------------ */
PUTER_API int puter_hip_kv_page_write(const void *storage, const void *values, const int32_t *page_ids,
                            const int32_t *offsets, void *output, int64_t page_count,
                            int64_t page_size, int64_t inner, int64_t value_rows,
                            int64_t storage_offset, int dtype, int32_t *status, void *stream);
/* out_rows must not exceed len(page_table) * page_size: the reference caller caps
 * it there before the call (execution/page_intrinsic.go:326-330). */
PUTER_API int puter_hip_kv_page_gather(const void *storage, const int32_t *page_table, void *output,
                             int64_t page_count, int64_t page_size, int64_t inner,
                             int64_t out_rows, int64_t storage_offset, int dtype, int32_t *status,
                             void *stream);

/* Extension (no reference method): KVPageWrite into an fp8-E4M3 pool with
 * quantisation.  The reference writes rows in the storage dtype
 * (execution/page_intrinsic.go:135-215, device/cpu/shape/page_generic.go:5-43);
 * this hook takes bf16 / f16 / f32 value rows [value_rows, kv_heads * head_dim]
 * and stores byte = E4M3(value / scale[kv head]) (IEEE f32 division, then the
 * library's saturating round-to-nearest-even narrowing) at page page_ids[r],
 * slot offsets[r] of the pool [pages, page_size, kv_heads, head_dim] that starts
 * storage_offset bytes into `storage`.  It is the inverse of the paged decode's
 * dequantisation decode(byte) * scale.  Written in place (the device caller's
 * output == storage, page_intrinsic.go:199-205); out-of-range rows, duplicate
 * slots and *status as puter_hip_kv_page_write. */
PUTER_API int puter_hip_kv_page_write_fp8(void *storage, const void *values, const int32_t *page_ids,
                                          const int32_t *offsets, int64_t page_count, int64_t page_size,
                                          int64_t kv_heads, int64_t head_dim, int64_t value_rows,
                                          int64_t storage_offset, const float *scales, int value_dtype,
                                          int32_t *status, void *stream);

/* ------------------------------------------------------------------------ */
/* Attention: device/interface.go:91-110                                      */
/* ------------------------------------------------------------------------ */
typedef struct puter_mha_config {
    int64_t num_heads;     /* MultiHeadAttentionConfig.NumHeads */
    int64_t head_dim;      /* .HeadDim */
    int32_t causal;        /* .Causal (bottom-right aligned: k > q + seqK - seqQ masked) */
    int32_t pad_;
    int64_t window_size;   /* .WindowSize (0 = off) */
    float alibi_slope;     /* .ALiBiSlope (0 = off) */
    int32_t pad2_;
    int64_t kv_head_count; /* .KVHeadCount (0 = NumHeads) */
} puter_mha_config;

/* MultiHeadAttention(config, q, k, v, out, seqQ, seqK, format) interface.go:98-103.
 * Q/O [seqQ, H*D], K/V [seqK, Hkv*D]. */
PUTER_API int puter_hip_multi_head_attention(const puter_mha_config *config, const void *query,
                                   const void *key, const void *value, void *output,
                                   int64_t seq_q, int64_t seq_k, int dtype, void *stream);
/* Same contract over `batch` independent [seq, heads*D] slabs laid out back to
 * back (the reference runs one MultiHeadAttention call per batch element). */
PUTER_API int puter_hip_multi_head_attention_batched(const puter_mha_config *config, const void *query,
                                           const void *key, const void *value, void *output,
                                           int64_t batch, int64_t seq_q, int64_t seq_k,
                                           int dtype, void *stream);

/* FlashAttentionConfig, device/config.go:278-281. */
typedef struct puter_flash_config {
    int64_t block_size; /* .BlockSize (accepted and unused, as in device/cpu/attention) */
    int32_t causal;     /* .Causal (top-left aligned: key k > query row masked) */
    int32_t pad_;
} puter_flash_config;

/* ScaledDotProductAttention(config, q, k, v, out, seqQ, seqK, depth, valueDim, format)
 * interface.go:104-109: one head, Q [seqQ, depth], K [seqK, depth], V [seqK, valueDim],
 * O [seqQ, valueDim]; online softmax through FastExp32 (cpu/attention/typed_compute.go:31-97).
 * depth <= 8192, valueDim <= 1024 (beyond: PUTER_ERR_INVALID). */
PUTER_API int puter_hip_scaled_dot_product_attention(const puter_flash_config *config,
                                           const void *query, const void *key, const void *value,
                                           void *output, int64_t seq_q, int64_t seq_k,
                                           int64_t depth, int64_t value_dim, int dtype,
                                           void *stream);
/* FlashAttention(...) interface.go:92-97: the same computation
 * (cpu/attention/ops.go:21-31 forwards to ScaledDotProductAttention). */
PUTER_API int puter_hip_flash_attention(const puter_flash_config *config, const void *query,
                                        const void *key, const void *value, void *output,
                                        int64_t seq_q, int64_t seq_k, int64_t depth,
                                        int64_t value_dim, int dtype, void *stream);

/* Paged decode (extension: the reference runs KVPageGather then
 * MultiHeadAttention with seqQ = 1, page_intrinsic.go:217-352 + bind_router.go:640-684).
 * K/V pools [pages, page_size, Hkv, D] of kv_dtype: BF16 or F16 (query and
 * output [batch, Hq*D] in the same format), or F8E4M3 with fp32 k_scale/v_scale
 * per kv head, value = decode(byte) * scale (query and output bf16);
 * D = 128, Hq/Hkv from 1 to 16; page_table [batch, max_pages_per_seq] int32;
 * context_lens [batch] int32 (clamped to max_context); num_pages = pool size:
 * a token whose page id is outside [0, num_pages) is masked, never read.
 * workspace: caller-owned device buffer of
 * puter_hip_paged_decode_workspace_bytes(...) bytes.  query, both pools and
 * the workspace must be 16-byte aligned (PUTER_ERR_INVALID otherwise). */
PUTER_API size_t puter_hip_paged_decode_workspace_bytes(int64_t batch, int64_t num_heads,
                                              int64_t head_dim, int64_t max_context);
PUTER_API int puter_hip_paged_decode_attention(const void *query, const void *key_pages,
                                     const void *value_pages, const int32_t *page_table,
                                     const int32_t *context_lens, int64_t batch,
                                     int64_t max_pages_per_seq, int64_t page_size,
                                     int64_t num_pages, int64_t num_heads, int64_t kv_heads,
                                     int64_t head_dim,
                                     int64_t max_context, const float *k_scale,
                                     const float *v_scale, int kv_dtype, void *output,
                                     void *workspace, size_t workspace_bytes, void *stream);

/* ------------------------------------------------------------------------ */
/* Integer quantisation: Dequant / Dequant4 device/interface.go:196-199,       */
/* Quant :580-582 (config = DequantInt8Config{Scale, ZeroPoint} by value,     */
/* device/config.go:268-276; zero_point must fit int8).                       */
/* ------------------------------------------------------------------------ */
/* Dequant: F32 <- I8 only (device/cpu/dequant/ops.go:11-37):
 * dst[i] = float32(src[i] - zero_point) * scale. */
PUTER_API int puter_hip_dequant(void *dst, const void *src, int64_t count, float scale,
                                int32_t zero_point, int dst_dtype, int src_dtype, void *stream);
/* Dequant4: F32 <- I4 only (dequant/ops.go:39-58): pair_count elements read
 * from (pair_count+1)/2 packed bytes, dst[i] = float32(nibble(i) - zero_point) * scale. */
PUTER_API int puter_hip_dequant4(void *dst, const void *src, int64_t pair_count, float scale,
                                 int32_t zero_point, int dst_dtype, int src_dtype, void *stream);
/* Quant: I8 <- F32 only (device/cpu/quant/ops.go:10-37, int8_generic.go:5-18):
 * round-half-away-from-zero(src / scale) + zero_point, saturated to [-128, 127]
 * (f32 division; NaN -> 0). */
PUTER_API int puter_hip_quant(void *dst, const void *src, int64_t count, float scale,
                              int32_t zero_point, int dst_dtype, int src_dtype, void *stream);

/* ------------------------------------------------------------------------ */
/* Matmul: device/interface.go:409-415 (F32), device/cpu/matmul/compute.go:46-62 */
/* ------------------------------------------------------------------------ */
/* out[rows, cols] = left[rows, inner] . right[inner, cols], row-major, in F32, F64,
 * BF16 or F16 (16-bit formats accumulate in f32 and round once).  BF16 / F16 with
 * cols % 8 == 0, inner % 8 == 0 and 16-byte aligned buffers run on MFMA; with at
 * most 512 rows they split `inner` across blocks and keep f32 partials in the
 * library's per-device scratch (calls on different streams are ordered on the
 * device by an event); so does F32 when the output has fewer than 256 64x64
 * tiles.  inner == 0 writes zeros. */
PUTER_API int puter_hip_matmul(void *out, const void *left, const void *right, int64_t rows,
                     int64_t inner, int64_t cols, int dtype, void *stream);

/* Allocation-free Matmul.  No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  Same contract, formats and
 * kernels as puter_hip_matmul, but the split-K partials go to a fixed 16 MiB
 * device array per GPU (held until the process ends) instead of the growable
 * scratch, so the call never allocates or frees.  That array is the most any
 * split-K launch needs; a larger need would be PUTER_ERR_INVALID.  Every call on
 * one GPU shares the array: calls that overlap on one GPU race, so issue them on
 * one stream (or order them).  Calls on different GPUs are independent. */
PUTER_API int puter_hip_matmul_noalloc(void *out, const void *left, const void *right, int64_t rows,
                                       int64_t inner, int64_t cols, int dtype, void *stream);

/* ------------------------------------------------------------------------ */
/* Diagnostic (no counterpart in the reference): HBM stream probe with the   */
/* fused GatedResidual+norm's traffic (read a and b, write c and d; vectors  */
/* of 16 bytes each) and no arithmetic, so its rate is the norm kernels'     */
/* practical ceiling on the same device.  shape 0: one vector of each input  */
/* per thread; 1: a 1024-thread block per 1024-vector row with a block-wide  */
/* sum between the stores; 2: a wave per 1024-vector row, 16 vectors per     */
/* lane.  Shapes 1 and 2 need vectors % 1024 == 0; all buffers 16-byte       */
/* aligned.                                                                  */
/* ------------------------------------------------------------------------ */
PUTER_API int puter_hip_stream_probe(const void *a, const void *b, void *c, void *d, int64_t vectors,
                                     int shape, void *stream);

/* Diagnostic (no counterpart in the reference): MFMA rate probe.  blocks     */
/* 256-thread blocks (two per CU), each wave running iters iterations of 32   */
/* v_mfma_f32_32x32x16_bf16 on operands read once from operands (16 KiB of    */
/* bf16, 16-byte aligned): mode 0 the MFMAs alone on 4 accumulator chains;    */
/* mode 1 the prefill's 64-key tile dataflow (S = K.Q^T, exp2 softmax with    */
/* the row sum and bf16 narrowing, O += V^T.P^T) with no memory traffic.      */
/* out receives blocks * 256 floats.  Flops per launch: blocks * 4 * iters *  */
/* 32 * 32768.                                                                */
PUTER_API int puter_hip_mfma_probe(const void *operands, void *out, int64_t blocks, int iters, int mode,
                                   void *stream);

#ifdef __cplusplus
}
#endif
#endif /* PUTER_HIP_H */
