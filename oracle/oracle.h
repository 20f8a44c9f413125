/*
 * CPU oracle: a plain-C restatement of the reference's device/cpu arithmetic for
 * the hot path (norms, gated residual, RoPE, gated activations, dtype casts,
 * paged KV, multi-head attention, f32 matmul, integer quantisation).
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the shipped library (puter_amd/) links,
 * loads or calls this code. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, as the checker and as the timed CPU baseline.
 *
 * Floating-point contract: compiled with -ffp-contract=off and without
 * -ffast-math, so every float expression rounds per operation like Go on amd64
 * (Go does not fuse x*y+z into FMA on amd64).  f64 helpers (sqrt, cos, sin,
 * pow, exp, erf) are libm's correctly-rounded-or-nearly versions, matching Go's
 * math package to within 1 ulp of f64 (invisible after the f32 narrowing in
 * all but measure-zero cases).
 *
 * Parity pinning (see tests/test_oracle_*.py):
 *   - casts: OCP FP8 decode tables, torch's bf16/f16/e4m3fn/e5m2 casts for
 *     finite in-range values, IEEE special values; NaN payload and overflow
 *     saturation rules are fixed by documented rule (parity unpinned at the
 *     manifesto/dtype boundary, see header of numeric.c).
 *   - norms/rope/activations/attention: reference known-answer tests, closed
 *     forms, and f64 brute force on tiny shapes.
 *   - every gate kind (ReGLU / LinGLU / SeGLU included), the fp8 paged-decode
 *     branch (torch's E4M3 decode, distinct per-head K and V scales), Matmul in
 *     F32 / F64 / BF16 / F16 (exact sums, single-rounding sums) and the f16
 *     attention dot rounding each have a check that does not restate their
 *     formula (tests/test_oracle_pins_glu_decode_matmul.py).
 */
#ifndef PUTER_ORACLE_H
#define PUTER_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes: identical to include/puter_hip.h */
enum {
    OR_F32 = 0,
    OR_F16 = 1,
    OR_BF16 = 2,
    OR_F8E4M3 = 3,
    OR_F8E5M2 = 4,
    OR_I32 = 5,
    OR_I8 = 6,
    OR_I4 = 7,   /* packed signed nibbles: element 2k = low nibble of byte k */
    OR_F64 = 8,
};

void oracle_set_threads(int threads);
int oracle_get_threads(void);

/* ---- numeric.c: scalar codecs (element-wise, bit-exact rules) ---- */
float or_bf16_to_f32(uint16_t bits);
uint16_t or_f32_to_bf16(float value);
float or_f16_to_f32(uint16_t bits);
uint16_t or_f32_to_f16(float value);
float or_e4m3_to_f32(uint8_t bits);
uint8_t or_f32_to_e4m3(float value);
float or_e5m2_to_f32(uint8_t bits);
uint8_t or_f32_to_e5m2(float value);
float or_fast_exp32(float value);
float or_load(const void *base, size_t index, int dtype);
void or_store(void *base, size_t index, float value, int dtype);

/* bulk casts: src dtype -> f32, f32 -> dst dtype */
int or_cast_to_f32(float *dst, const void *src, size_t count, int src_dtype);
int or_cast_from_f32(void *dst, const float *src, size_t count, int dst_dtype);

/* ---- quant.c: integer (de)quantisation, int8 / int4 / f64 casts ---- */
float or_dequant_int8_one(int8_t code, float scale, int8_t zero_point);
int or_int4_nibble(const uint8_t *src, size_t index);
int8_t or_quant_int8_one(float value, float scale, int8_t zero_point);
int8_t or_f32_to_int8(float value);
int or_dequant_int8(float *dst, const int8_t *src, size_t count, float scale, int zero_point);
int or_dequant_int4(float *dst, const uint8_t *src, size_t count, float scale, int zero_point);
int or_quant_int8(int8_t *dst, const float *src, size_t count, float scale, int zero_point);
int or_cast_ext(void *dst, int dst_dtype, const void *src, int src_dtype, size_t count);
int or_cast_pair(void *dst, int dst_dtype, const void *src, int src_dtype, size_t count);

/* ---- norm.c ---- */
int or_rmsnorm(const void *input, const void *scale, void *output,
               int64_t rows, int64_t last_dim, double epsilon, int dtype);
int or_layernorm(const void *input, const void *scale, const void *bias, void *output,
                 int64_t rows, int64_t last_dim, int dtype);
int or_adaptive_rmsnorm(const void *input, const void *modulation, void *output,
                        int64_t rows, int64_t last_dim, int64_t rows_per_batch,
                        int64_t modulation_cols, double epsilon, int dtype);
int or_modulated_layernorm(const void *input, const void *modulation, void *output,
                           int64_t rows, int64_t last_dim, int64_t rows_per_batch,
                           int64_t modulation_cols, double epsilon, int set, int dtype);
int or_gated_residual(const void *residual, const void *branch, const void *modulation,
                      void *output, int64_t rows, int64_t last_dim, int64_t rows_per_batch,
                      int64_t modulation_cols, int set, int dtype);

/* ---- rope.c ---- */
typedef struct {
    double base_freq;
    int64_t start_position;
    int mode;     /* 0 interleaved, 1 half */
    int scaling;  /* 0 none, 1 llama3 */
    double scaling_factor;
    double low_freq_factor;
    double high_freq_factor;
    int64_t original_context;
} or_rope_config;

int or_rope(const or_rope_config *config, const void *input, void *output,
            int64_t seq_len, int64_t num_heads, int64_t head_dim, int dtype);

typedef struct {
    double base_freq;
    int64_t latent_seq_len;
    int64_t latent_side;
    int axis_count;
    int64_t axis_dims[4];
} or_multi_axis_rope_config;

int or_multi_axis_rope(const or_multi_axis_rope_config *config, const void *input, void *output,
                       int64_t batch, int64_t seq_len, int64_t num_heads, int64_t head_dim,
                       int dtype);

int or_rope_pairs(float *output, const float *input, const float *cos_buffer, const float *sin_buffer,
                  int64_t half_dim);

/* ---- activation.c ---- */
enum { OR_GATE_SWIGLU = 0, OR_GATE_GEGLU = 1, OR_GATE_GEGLU_TANH = 2, OR_GATE_SIGLU = 3,
       OR_GATE_GLU = 4, OR_GATE_REGLU = 5, OR_GATE_LINGLU = 6, OR_GATE_SEGLU = 7 };
int or_gated_tensors(int kind, void *dst, const void *gate, const void *up,
                     int64_t count, int dtype);
int or_gated_packed(int kind, void *dst, const void *packed,
                    int64_t batch, int64_t half_count, int dtype);
int or_unary(int kind, void *dst, const void *src, int64_t count, int dtype);
/* scalar helpers, exported for the pins: FastExp64, FastTanh32, FastSigmoid32,
 * float32(FastSilu64(x)) */
double or_fast_exp64(double x);
float or_fast_tanh32(float x);
float or_fast_sigmoid32(float x);
float or_fast_silu64(float x);
enum { OR_UNARY_SILU = 0, OR_UNARY_GELU = 1 };

/* ---- page.c ---- */
int or_page_write(const void *storage, const void *values, const int32_t *page_ids,
                  const int32_t *offsets, void *output, int64_t page_count, int64_t page_size,
                  int64_t inner, int64_t value_rows, int64_t storage_offset, int elem_size);
int or_page_gather(const void *storage, const int32_t *page_table, void *output,
                   int64_t page_count, int64_t page_size, int64_t inner, int64_t out_rows,
                   int64_t storage_offset, int64_t table_len, int elem_size);
int or_page_write_fp8(uint8_t *storage, const void *values, const int32_t *page_ids,
                      const int32_t *offsets, int64_t page_count, int64_t page_size,
                      int64_t kv_heads, int64_t head_dim, int64_t value_rows,
                      int64_t storage_offset, const float *scales, int value_dtype);

/* ---- attention.c ---- */
typedef struct {
    int64_t num_heads;
    int64_t head_dim;
    int causal;
    int64_t window_size;
    float alibi_slope;
    int64_t kv_head_count;
} or_mha_config;

int or_mha(const or_mha_config *config, const void *query, const void *key, const void *value,
           void *output, int64_t seq_q, int64_t seq_k, int dtype);
/* one (head) of or_mha, restricted to query rows [q_begin, q_end): the subset
 * form used to time and check the large prefill config on the CPU */
int or_mha_rows(const or_mha_config *config, const void *query, const void *key,
                const void *value, void *output, int64_t seq_q, int64_t seq_k,
                int64_t head_begin, int64_t head_end, int64_t q_begin, int64_t q_end,
                int dtype);
/* paged decode as the reference executes it: KVPageGather of K and V, then
 * MultiHeadAttention with seqQ = 1.  fp8 caches are dequantised with a per-kv-head
 * scale before the bf16 path (value = decode(byte) * scale, rounded to bf16). */
int or_paged_decode(const void *query, const void *key_pages, const void *value_pages,
                    const int32_t *page_table, const int32_t *context_lens,
                    int64_t batch, int64_t max_pages_per_seq, int64_t page_size,
                    int64_t num_heads, int64_t kv_heads, int64_t head_dim,
                    const float *k_scale, const float *v_scale, int kv_dtype,
                    void *output);

/* ScaledDotProductAttention / FlashAttention: one head, Q/K [seq, depth],
 * V/O [seq, value_dim], sequential online softmax through FastExp32; causal
 * hides key > row (top-left aligned, unlike or_mha). */
int or_flash_attention(int causal, const void *query, const void *key, const void *value,
                       void *output, int64_t seq_q, int64_t seq_k, int64_t depth,
                       int64_t value_dim, int dtype);

/* ---- matmul.c ---- */
int or_matmul_f32(float *out, const float *left, const float *right,
                  int64_t rows, int64_t inner, int64_t cols);
int or_matmul(void *out, const void *left, const void *right, int64_t rows, int64_t inner,
              int64_t cols, int dtype);

#ifdef __cplusplus
}
#endif
#endif
