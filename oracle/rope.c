/*
 * RoPE and MultiAxisRoPE for the CPU oracle (test infrastructure only; see
 * oracle.h).  Restates device/cpu/rope/compute.go.
 */
#include "oracle.h"

#include <math.h>

/* ropeInverseFrequency compute.go:98-107, llama3ScaledInverseFrequency :109-126 */
static double inverse_frequency(const or_rope_config *c, int64_t pair, int64_t head_dim) {
    double exponent = -(double)(2 * pair) / (double)head_dim;
    double inv = pow(c->base_freq, exponent);
    if (c->scaling != 1) return inv;
    double wavelength = (2.0 * M_PI) / inv;
    double low = (double)c->original_context / c->low_freq_factor;
    double high = (double)c->original_context / c->high_freq_factor;
    if (wavelength > low) return inv / c->scaling_factor;
    if (wavelength < high) return inv;
    double smooth = ((double)c->original_context / wavelength - c->low_freq_factor) /
                    (c->high_freq_factor - c->low_freq_factor);
    return (1.0 - smooth) * (inv / c->scaling_factor) + smooth * inv;
}

/* RoPEConfig.Validate device/config.go:215-258 */
static int rope_config_ok(const or_rope_config *c) {
    if (!(c->base_freq > 0)) return 0;
    if (c->mode != 0 && c->mode != 1) return 0;
    if (c->scaling == 0) return 1;
    if (c->scaling != 1) return 0;
    if (!(c->scaling_factor > 0) || !(c->low_freq_factor > 0)) return 0;
    if (!(c->high_freq_factor > c->low_freq_factor)) return 0;
    return c->original_context > 0;
}

/* dispatchRoPE compute.go:11-31 -> runRoPE :55-96 -> ropePairsTyped :171-189,
 * RopePairsGeneric f32_generic.go:3-11, ropePairsHalfFloat32 :150-169 */
int or_rope(const or_rope_config *config, const void *input, void *output,
            int64_t seq_len, int64_t num_heads, int64_t head_dim, int dtype) {
    if (seq_len == 0 || num_heads == 0 || head_dim == 0 || head_dim % 2 != 0) return 0;
    if (!rope_config_ok(config)) return -6;
    if (dtype != OR_F32 && dtype != OR_BF16 && dtype != OR_F16) return -6;
    int64_t half = head_dim / 2;
    if (half > 4096) return -6; /* oracle limit: per-position angle buffers */
#pragma omp parallel for schedule(static) num_threads(oracle_get_threads())
    for (int64_t s = 0; s < seq_len; ++s) {
        float cosb[4096], sinb[4096];
        double position = (double)(s + config->start_position);
        for (int64_t p = 0; p < half; ++p) {
            double theta = position * inverse_frequency(config, p, head_dim);
            cosb[p] = (float)cos(theta);
            sinb[p] = (float)sin(theta);
        }
        for (int64_t h = 0; h < num_heads; ++h) {
            size_t row = (size_t)((s * num_heads + h) * head_dim);
            for (int64_t p = 0; p < half; ++p) {
                size_t ei, oi;
                if (config->mode == 1) {
                    ei = row + (size_t)p;
                    oi = row + (size_t)(half + p);
                } else {
                    ei = row + (size_t)(2 * p);
                    oi = ei + 1;
                }
                float c = cosb[p], sn = sinb[p];
                float e = or_load(input, ei, dtype);
                float o = or_load(input, oi, dtype);
                or_store(output, ei, e * c - o * sn, dtype);
                or_store(output, oi, e * sn + o * c, dtype);
            }
        }
    }
    return 0;
}

/* MultiAxisRoPEConfig.Validate/ValidateHeadDim device/config.go:148-213 */
static int multi_axis_ok(const or_multi_axis_rope_config *c, int64_t head_dim) {
    if (!(c->base_freq > 0) || c->latent_seq_len <= 0 || c->latent_side <= 0) return 0;
    if (c->axis_count <= 0 || c->axis_count > 4) return 0;
    int64_t total = 0;
    for (int a = 0; a < 4; ++a) {
        if (a >= c->axis_count) {
            if (c->axis_dims[a] != 0) return 0;
            continue;
        }
        if (c->axis_dims[a] <= 0 || c->axis_dims[a] % 2 != 0) return 0;
        total += c->axis_dims[a];
    }
    return total == head_dim;
}

/* runMultiAxisRoPE compute.go:195-215, axis plan :223-251, angle :276-300,
 * positions :302-330 */
int or_multi_axis_rope(const or_multi_axis_rope_config *config, const void *input, void *output,
                       int64_t batch, int64_t seq_len, int64_t num_heads, int64_t head_dim,
                       int dtype) {
    if (batch == 0 || seq_len == 0 || num_heads == 0 || head_dim == 0 || head_dim % 2 != 0)
        return 0;
    if (!multi_axis_ok(config, head_dim)) return -6;
    if (dtype != OR_F32 && dtype != OR_BF16 && dtype != OR_F16) return -6;
    int64_t half = head_dim / 2;
    int64_t starts[5] = {0, 0, 0, 0, 0};
    for (int a = 0; a < config->axis_count; ++a) starts[a + 1] = starts[a] + config->axis_dims[a] / 2;
    int64_t text_len = seq_len - config->latent_seq_len;
    if (text_len < 0) text_len = 0;
    int64_t pair_count = batch * seq_len * num_heads * half;
#pragma omp parallel for schedule(static) num_threads(oracle_get_threads())
    for (int64_t po = 0; po < pair_count; ++po) {
        int64_t pair = po % half;
        int64_t head = (po / half) % num_heads;
        int64_t seq = (po / (half * num_heads)) % seq_len;
        int64_t b = po / (half * num_heads * seq_len);
        size_t even = (size_t)(((b * seq_len + seq) * num_heads + head) * head_dim + pair * 2);
        int axis = 0;
        int64_t local = pair, axis_pairs = 0;
        for (int a = 0; a < config->axis_count; ++a) {
            if (pair < starts[a + 1]) {
                axis = a;
                local = pair - starts[a];
                axis_pairs = starts[a + 1] - starts[a];
                break;
            }
        }
        int64_t position;
        if (seq < text_len) {
            if (config->axis_count == 4 && axis == 3) position = seq;
            else if (config->axis_count < 4 && axis == 0) position = seq;
            else position = 0;
        } else {
            int64_t img = seq - text_len;
            position = axis == 1 ? img / config->latent_side : axis == 2 ? img % config->latent_side : 0;
        }
        float c = 1.0f, sn = 0.0f;
        double axis_dim = (double)(axis_pairs * 2);
        if (axis_dim != 0) {
            double exponent = -2.0 * (double)local / axis_dim;
            double angle = (double)position * pow(config->base_freq, exponent);
            c = (float)cos(angle);
            sn = (float)sin(angle);
        }
        float e = or_load(input, even, dtype);
        float o = or_load(input, even + 1, dtype);
        or_store(output, even, e * c - o * sn, dtype);
        or_store(output, even + 1, e * sn + o * c, dtype);
    }
    return 0;
}

/* RoPEPairs: device/cpu/rope/ops.go:25-38 -> RopePairsGeneric f32_generic.go:3-11 */
int or_rope_pairs(float *output, const float *input, const float *cos_buffer, const float *sin_buffer,
                  int64_t half_dim) {
    for (int64_t i = 0; i < half_dim; ++i) {
        float c = cos_buffer[i], sn = sin_buffer[i];
        float e = input[2 * i], o = input[2 * i + 1];
        output[2 * i] = e * c - o * sn;
        output[2 * i + 1] = e * sn + o * c;
    }
    return 0;
}
