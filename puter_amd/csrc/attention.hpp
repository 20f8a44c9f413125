// Shared argument block of the attention kernels (attention.hip dispatches,
// prefill.hip holds the MFMA flash kernel).
#pragma once

#include "common.hpp"

namespace puter {

struct MhaArgs {
    const void *q, *k, *v;
    void *o;
    int64_t batch, seq_q, seq_k, heads, kv_heads, dim;
    int causal;
    int64_t window;
    float alibi;
    float scale;
    int64_t shift;  // causal: key k is visible to query row q iff k <= q + shift
    // one-row split of the general kernel: per (batch, head, split) the chunk's
    // (max, sum) and unnormalised output row; null otherwise
    float2 *part_ml = nullptr;
    float *part_o = nullptr;
};

// MFMA flash prefill (prefill.hip).  Returns true and sets *status when the
// shape is one it serves (bf16 / f16, head_dim 128 or 64, causal or not, sliding window, ALiBi;
// head dim 64 only for more than one query row; f32, head_dim 128 or 64, at least 16
// query rows, causal or not, sliding window, ALiBi).
bool launch_prefill_mfma(const MhaArgs &a, int dtype, hipStream_t s, int *status);
// one query row per sequence (bf16 / f16, head_dim 128): the paged decode kernels
bool launch_decode_contiguous(const MhaArgs &m, int dtype, hipStream_t s, int *status);

}  // namespace puter
