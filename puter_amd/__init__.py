"""puter_amd: MI355X (gfx950) device backend for the puter hot path.

The compute lives in libputer_hip.so (hand-written HIP kernels behind the C
ABI of include/puter_hip.h).  `Backend` mirrors the reference's
device.Backend method names for the norm / RoPE / gated activation / cast /
paged-KV / attention / matmul / quantisation path.
"""
from .backend import (  # noqa: F401
    Backend, DeviceBuffer, PuterError, RMSNormConfig, ModulatedLayerNormConfig, RoPEConfig,
    MultiAxisRoPEConfig, MultiHeadAttentionConfig, FlashAttentionConfig, DequantInt8Config, DequantInt4Config,
    F32, F16, BF16, F8E4M3, F8E5M2, I32, I8, I4, F64,
    RoPEModeInterleaved, RoPEModeHalf, RoPEScalingNone, RoPEScalingLlama3, dtype_of,
)

__all__ = ["Backend", "PuterError"]
