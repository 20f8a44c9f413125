"""ctypes binding of libputer_hip.so (the C ABI declared in include/puter_hip.h).

There is no fallback: if the library is missing or fails to load, importing
the backend raises, so no caller can silently run anything but the HIP path.
"""
import ctypes as C
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY = os.path.join(HERE, "libputer_hip.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "puter_hip.h")

OK, ERR_NIL, ERR_INVALID, ERR_UNAVAILABLE, ERR_LAUNCH = 0, -2, -6, -7, -8

vp, i64, i32, dbl, sz = C.c_void_p, C.c_int64, C.c_int, C.c_double, C.c_size_t


class PuterError(RuntimeError):
    """Raised for a non-zero status (the Go wrapper panics with the same message)."""

    def __init__(self, status: int, message: str):
        super().__init__(f"puter_hip status {status}: {message}")
        self.status = status


class RopeConfig(C.Structure):
    _fields_ = [("base_freq", C.c_double), ("start_position", C.c_int64), ("mode", C.c_int32),
                ("scaling", C.c_int32), ("scaling_factor", C.c_double),
                ("low_freq_factor", C.c_double), ("high_freq_factor", C.c_double),
                ("original_context", C.c_int64)]


class MultiAxisRopeConfig(C.Structure):
    _fields_ = [("base_freq", C.c_double), ("latent_seq_len", C.c_int64),
                ("latent_side", C.c_int64), ("axis_count", C.c_int32), ("pad_", C.c_int32),
                ("axis_dims", C.c_int64 * 4)]


class MHAConfig(C.Structure):
    _fields_ = [("num_heads", C.c_int64), ("head_dim", C.c_int64), ("causal", C.c_int32),
                ("pad_", C.c_int32), ("window_size", C.c_int64), ("alibi_slope", C.c_float),
                ("pad2_", C.c_int32), ("kv_head_count", C.c_int64)]


class FlashConfig(C.Structure):
    _fields_ = [("block_size", C.c_int64), ("causal", C.c_int32), ("pad_", C.c_int32)]


SIGNATURES = {
    "puter_hip_last_error": ([], C.c_char_p),
    "puter_hip_version": ([], i32),
    "puter_hip_device_count": ([C.POINTER(C.c_int)], i32),
    "puter_hip_set_device": ([i32], i32),
    "puter_hip_malloc": ([C.POINTER(C.c_void_p), sz], i32),
    "puter_hip_free": ([vp], i32),
    "puter_hip_memcpy_htod": ([vp, vp, sz, vp], i32),
    "puter_hip_memcpy_dtoh": ([vp, vp, sz, vp], i32),
    "puter_hip_memcpy_dtod": ([vp, vp, sz, vp], i32),
    "puter_hip_stream_create": ([C.POINTER(C.c_void_p)], i32),
    "puter_hip_stream_destroy": ([vp], i32),
    "puter_hip_stream_synchronize": ([vp], i32),
    "puter_hip_rmsnorm": ([vp, vp, vp, i64, i64, dbl, i32, vp], i32),
    "puter_hip_layernorm": ([vp, vp, vp, vp, i64, i64, i32, vp], i32),
    "puter_hip_adaptive_rmsnorm": ([vp, vp, vp, i64, i64, i64, i64, dbl, i32, vp], i32),
    "puter_hip_modulated_layernorm": ([vp, vp, vp, i64, i64, i64, i64, dbl, i32, i32, vp], i32),
    "puter_hip_gated_residual": ([vp, vp, vp, vp, i64, i64, i64, i64, i32, i32, vp], i32),
    "puter_hip_gated_residual_rmsnorm": ([vp] * 6 + [i64] * 4 + [i32, dbl, i32, vp], i32),
    "puter_hip_gated_residual_layernorm": ([vp] * 7 + [i64] * 4 + [i32, i32, vp], i32),
    "puter_hip_rope": ([C.POINTER(RopeConfig), vp, vp, i64, i64, i64, i32, vp], i32),
    "puter_hip_rope_pairs": ([vp, vp, vp, vp, i64, i32, vp], i32),
    "puter_hip_multi_axis_rope": ([C.POINTER(MultiAxisRopeConfig), vp, vp, i64, i64, i64, i64,
                                   i32, vp], i32),
    "puter_hip_gated_tensors": ([i32, vp, vp, vp, i64, i32, vp], i32),
    "puter_hip_gated_packed": ([i32, vp, vp, i64, i64, i32, vp], i32),
    "puter_hip_unary": ([i32, vp, vp, i64, i32, vp], i32),
    "puter_hip_cast": ([vp, i32, vp, i32, i64, vp], i32),
    "puter_hip_kv_page_write": ([vp] * 5 + [i64] * 5 + [i32, vp, vp], i32),
    "puter_hip_kv_page_gather": ([vp] * 3 + [i64] * 5 + [i32, vp, vp], i32),
    "puter_hip_kv_page_write_fp8": ([vp] * 4 + [i64] * 6 + [vp, i32, vp, vp], i32),
    "puter_hip_multi_head_attention": ([C.POINTER(MHAConfig), vp, vp, vp, vp, i64, i64, i32, vp],
                                       i32),
    "puter_hip_multi_head_attention_batched": ([C.POINTER(MHAConfig), vp, vp, vp, vp, i64, i64,
                                                i64, i32, vp], i32),
    "puter_hip_scaled_dot_product_attention": ([C.POINTER(FlashConfig), vp, vp, vp, vp, i64, i64,
                                                i64, i64, i32, vp], i32),
    "puter_hip_flash_attention": ([C.POINTER(FlashConfig), vp, vp, vp, vp, i64, i64, i64, i64,
                                   i32, vp], i32),
    "puter_hip_paged_decode_workspace_bytes": ([i64, i64, i64, i64], sz),
    "puter_hip_paged_decode_attention": ([vp] * 5 + [i64] * 8 + [vp, vp, i32, vp, vp, sz, vp],
                                         i32),
    "puter_hip_dequant": ([vp, vp, i64, C.c_float, i32, i32, i32, vp], i32),
    "puter_hip_dequant4": ([vp, vp, i64, C.c_float, i32, i32, i32, vp], i32),
    "puter_hip_quant": ([vp, vp, i64, C.c_float, i32, i32, i32, vp], i32),
    "puter_hip_matmul": ([vp, vp, vp, i64, i64, i64, i32, vp], i32),
    "puter_hip_stream_probe": ([vp, vp, vp, vp, i64, i32, vp], i32),
    "puter_hip_mfma_probe": ([vp, vp, i64, i32, i32, vp], i32),
    "puter_hip_matmul_noalloc": ([vp, vp, vp, i64, i64, i64, i32, vp], i32),
}

_lib = None


def header_symbols() -> list:
    """Every function name declared in include/puter_hip.h."""
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(puter_hip_\w+)\s*\(", text)))


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIBRARY):
            raise ImportError(f"{LIBRARY} is not built; run __graft_entry__.build()")
        lib = C.CDLL(LIBRARY)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        _lib = lib
    return _lib


def check(status: int) -> None:
    if status != OK:
        msg = load().puter_hip_last_error().decode(errors="replace")
        raise PuterError(status, msg)
