// MFMA flash-attention prefill for bf16 (placeholder: the general kernel in
// attention.hip serves every shape until the MFMA path lands).
#include "common.hpp"

namespace puter {
struct MhaArgs;
bool launch_prefill_mfma(const MhaArgs &, int, hipStream_t, int *) { return false; }
}  // namespace puter
