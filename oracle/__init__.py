"""ctypes front-end of the CPU oracle (test infrastructure only).

The oracle is a C restatement of the reference's device/cpu arithmetic
(see oracle/*.c for the file:line each function follows).  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg import this package,
as the checker; the shipped library (puter_amd/) never calls it.

Arrays are numpy: f32 -> float32, bf16/f16 -> uint16 bit patterns,
fp8 -> uint8 bit patterns, indices -> int32.
"""
import ctypes as C
import os

import numpy as np

from .build import LIBRARY, build

F32, F16, BF16, F8E4M3, F8E5M2, I32, I8, I4, F64 = 0, 1, 2, 3, 4, 5, 6, 7, 8
(GATE_SWIGLU, GATE_GEGLU, GATE_GEGLU_TANH, GATE_SIGLU, GATE_GLU, GATE_REGLU, GATE_LINGLU,
 GATE_SEGLU) = range(8)
UNARY_SILU, UNARY_GELU = 0, 1

_lib = None


class RopeConfig(C.Structure):
    _fields_ = [("base_freq", C.c_double), ("start_position", C.c_int64), ("mode", C.c_int),
                ("scaling", C.c_int), ("scaling_factor", C.c_double),
                ("low_freq_factor", C.c_double), ("high_freq_factor", C.c_double),
                ("original_context", C.c_int64)]


class MultiAxisRopeConfig(C.Structure):
    _fields_ = [("base_freq", C.c_double), ("latent_seq_len", C.c_int64),
                ("latent_side", C.c_int64), ("axis_count", C.c_int),
                ("axis_dims", C.c_int64 * 4)]


class MHAConfig(C.Structure):
    _fields_ = [("num_heads", C.c_int64), ("head_dim", C.c_int64), ("causal", C.c_int),
                ("window_size", C.c_int64), ("alibi_slope", C.c_float),
                ("kv_head_count", C.c_int64)]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIBRARY):
            build()
        _lib = C.CDLL(LIBRARY)
        _lib.or_fast_exp32.restype = C.c_float
        _lib.or_fast_exp32.argtypes = [C.c_float]
        _lib.or_fast_exp64.restype = C.c_double
        _lib.or_fast_exp64.argtypes = [C.c_double]
        for name in ("or_fast_tanh32", "or_fast_sigmoid32", "or_fast_silu64"):
            getattr(_lib, name).restype = C.c_float
            getattr(_lib, name).argtypes = [C.c_float]
        _lib.or_rmsnorm.argtypes = [C.c_void_p] * 3 + [C.c_int64, C.c_int64, C.c_double, C.c_int]
        _lib.or_layernorm.argtypes = [C.c_void_p] * 4 + [C.c_int64, C.c_int64, C.c_int]
        _lib.or_adaptive_rmsnorm.argtypes = [C.c_void_p] * 3 + [C.c_int64] * 4 + [C.c_double, C.c_int]
        _lib.or_modulated_layernorm.argtypes = ([C.c_void_p] * 3 + [C.c_int64] * 4 +
                                                [C.c_double, C.c_int, C.c_int])
        _lib.or_gated_residual.argtypes = [C.c_void_p] * 4 + [C.c_int64] * 4 + [C.c_int, C.c_int]
        _lib.or_rope.argtypes = [C.POINTER(RopeConfig), C.c_void_p, C.c_void_p,
                                 C.c_int64, C.c_int64, C.c_int64, C.c_int]
        _lib.or_multi_axis_rope.argtypes = [C.POINTER(MultiAxisRopeConfig), C.c_void_p, C.c_void_p,
                                            C.c_int64, C.c_int64, C.c_int64, C.c_int64, C.c_int]
        _lib.or_rope_pairs.argtypes = [C.c_void_p] * 4 + [C.c_int64]
        _lib.or_gated_tensors.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64, C.c_int]
        _lib.or_gated_packed.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_int64, C.c_int64, C.c_int]
        _lib.or_unary.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_int64, C.c_int]
        _lib.or_page_write.argtypes = [C.c_void_p] * 5 + [C.c_int64] * 5 + [C.c_int]
        _lib.or_page_gather.argtypes = [C.c_void_p] * 3 + [C.c_int64] * 6 + [C.c_int]
        _lib.or_page_write_fp8.argtypes = [C.c_void_p] * 4 + [C.c_int64] * 6 + [C.c_void_p, C.c_int]
        _lib.or_mha.argtypes = [C.POINTER(MHAConfig)] + [C.c_void_p] * 4 + [C.c_int64, C.c_int64, C.c_int]
        _lib.or_mha_rows.argtypes = ([C.POINTER(MHAConfig)] + [C.c_void_p] * 4 +
                                     [C.c_int64] * 6 + [C.c_int])
        _lib.or_flash_attention.argtypes = ([C.c_int] + [C.c_void_p] * 4 + [C.c_int64] * 4 +
                                            [C.c_int])
        _lib.or_paged_decode.argtypes = ([C.c_void_p] * 5 + [C.c_int64] * 6 +
                                         [C.c_void_p, C.c_void_p, C.c_int, C.c_void_p])
        _lib.or_matmul_f32.argtypes = [C.c_void_p] * 3 + [C.c_int64] * 3
        _lib.or_cast_to_f32.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        _lib.or_cast_from_f32.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        for name in ("or_dequant_int8", "or_dequant_int4", "or_quant_int8"):
            getattr(_lib, name).argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_float, C.c_int]
        _lib.or_cast_ext.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_size_t]
        _lib.or_cast_pair.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_size_t]
        _lib.or_matmul.argtypes = [C.c_void_p] * 3 + [C.c_int64] * 3 + [C.c_int]
        _lib.oracle_set_threads.argtypes = [C.c_int]
        _lib.oracle_get_threads.restype = C.c_int
    return _lib


def set_threads(n: int) -> None:
    lib().oracle_set_threads(int(n))


def get_threads() -> int:
    return lib().oracle_get_threads()


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _check(rc, what):
    if rc != 0:
        raise ValueError(f"oracle {what}: status {rc}")


STORAGE = {F32: np.float32, F16: np.uint16, BF16: np.uint16, F8E4M3: np.uint8, F8E5M2: np.uint8}


def _c(a, dtype=None):
    a = np.ascontiguousarray(a)
    if dtype is not None:
        assert a.dtype == dtype, (a.dtype, dtype)
    return a


# ---- casts ----
def to_f32(bits: np.ndarray, dtype: int) -> np.ndarray:
    bits = _c(bits, STORAGE[dtype])
    out = np.empty(bits.shape, np.float32)
    _check(lib().or_cast_to_f32(_p(out), _p(bits), bits.size, dtype), "cast_to_f32")
    return out


def from_f32(values: np.ndarray, dtype: int) -> np.ndarray:
    values = _c(values, np.float32)
    out = np.empty(values.shape, STORAGE[dtype])
    _check(lib().or_cast_from_f32(_p(out), _p(values), values.size, dtype), "cast_from_f32")
    return out


def fast_exp32(x: float) -> float:
    return lib().or_fast_exp32(float(x))


def fast_exp64(x: float) -> float:
    """FastExp64 (device/cpu/math/f64.go:10-32)."""
    return lib().or_fast_exp64(float(x))


def fast_tanh32(x: float) -> float:
    """FastTanh32 (device/cpu/math/f32.go:73-86)."""
    return lib().or_fast_tanh32(float(x))


def fast_sigmoid32(x: float) -> float:
    """FastSigmoid32 (device/cpu/math/f32.go:88-95)."""
    return lib().or_fast_sigmoid32(float(x))


def fast_silu64(x: float) -> float:
    """float32(FastSilu64(float64(x))) (device/cpu/math/f64.go:90-92): one entry of
    the 16-bit Silu tables (device/cpu/activation/lut.go:14-62) before narrowing."""
    return lib().or_fast_silu64(float(x))


# ---- norms ----
def rmsnorm(x, scale, eps, dtype):
    x = _c(x, STORAGE[dtype]); scale = _c(scale, STORAGE[dtype])
    rows, h = x.shape
    out = np.empty_like(x)
    _check(lib().or_rmsnorm(_p(x), _p(scale), _p(out), rows, h, eps, dtype), "rmsnorm")
    return out


def layernorm(x, scale, bias, dtype):
    x = _c(x, STORAGE[dtype]); scale = _c(scale, STORAGE[dtype]); bias = _c(bias, STORAGE[dtype])
    rows, h = x.shape
    out = np.empty_like(x)
    _check(lib().or_layernorm(_p(x), _p(scale), _p(bias), _p(out), rows, h, dtype), "layernorm")
    return out


def adaptive_rmsnorm(x, modulation, rows_per_batch, eps, dtype):
    x = _c(x, STORAGE[dtype]); modulation = _c(modulation, STORAGE[dtype])
    rows, h = x.shape
    out = np.empty_like(x)
    _check(lib().or_adaptive_rmsnorm(_p(x), _p(modulation), _p(out), rows, h, rows_per_batch,
                                     modulation.shape[-1], eps, dtype), "adaptive_rmsnorm")
    return out


def modulated_layernorm(x, modulation, rows_per_batch, eps, set_index, dtype):
    x = _c(x, STORAGE[dtype]); modulation = _c(modulation, STORAGE[dtype])
    rows, h = x.shape
    out = np.empty_like(x)
    _check(lib().or_modulated_layernorm(_p(x), _p(modulation), _p(out), rows, h, rows_per_batch,
                                        modulation.shape[-1], eps, set_index, dtype),
           "modulated_layernorm")
    return out


def gated_residual(residual, branch, modulation, rows_per_batch, set_index, dtype):
    residual = _c(residual, STORAGE[dtype]); branch = _c(branch, STORAGE[dtype])
    modulation = _c(modulation, STORAGE[dtype])
    h = residual.shape[-1]
    rows = residual.size // h
    out = np.empty_like(residual)
    _check(lib().or_gated_residual(_p(residual), _p(branch), _p(modulation), _p(out), rows, h,
                                   rows_per_batch, modulation.shape[-1], set_index, dtype),
           "gated_residual")
    return out


# ---- rope ----
def rope(x, base_freq=10000.0, start_position=0, mode=0, scaling=0, scaling_factor=1.0,
         low_freq_factor=0.0, high_freq_factor=0.0, original_context=0, dtype=F32):
    x = _c(x, STORAGE[dtype])
    seq, heads, dim = x.shape
    cfg = RopeConfig(base_freq, start_position, mode, scaling, scaling_factor, low_freq_factor,
                     high_freq_factor, original_context)
    out = np.empty_like(x)
    _check(lib().or_rope(C.byref(cfg), _p(x), _p(out), seq, heads, dim, dtype), "rope")
    return out


def multi_axis_rope(x, base_freq, latent_seq_len, latent_side, axis_dims, dtype):
    x = _c(x, STORAGE[dtype])
    batch, seq, heads, dim = x.shape
    dims = (C.c_int64 * 4)(*(list(axis_dims) + [0] * (4 - len(axis_dims))))
    cfg = MultiAxisRopeConfig(base_freq, latent_seq_len, latent_side, len(axis_dims), dims)
    out = np.empty_like(x)
    _check(lib().or_multi_axis_rope(C.byref(cfg), _p(x), _p(out), batch, seq, heads, dim, dtype),
           "multi_axis_rope")
    return out


def rope_pairs(x, cos, sin):
    """RoPEPairs (f32): x holds 2*len(cos) values."""
    x = _c(x, np.float32); cos = _c(cos, np.float32); sin = _c(sin, np.float32)
    out = np.empty_like(x)
    _check(lib().or_rope_pairs(_p(out), _p(x), _p(cos), _p(sin), cos.size), "rope_pairs")
    return out


# ---- activations ----
def gated_tensors(kind, gate, up, dtype):
    gate = _c(gate, STORAGE[dtype]); up = _c(up, STORAGE[dtype])
    out = np.empty_like(gate)
    _check(lib().or_gated_tensors(kind, _p(out), _p(gate), _p(up), gate.size, dtype), "gated")
    return out


def gated_packed(kind, packed, dtype):
    packed = _c(packed, STORAGE[dtype])
    batch, width = packed.shape
    out = np.empty((batch, width // 2), packed.dtype)
    _check(lib().or_gated_packed(kind, _p(out), _p(packed), batch, width // 2, dtype), "gated_packed")
    return out


def unary(kind, x, dtype):
    x = _c(x, STORAGE[dtype])
    out = np.empty_like(x)
    _check(lib().or_unary(kind, _p(out), _p(x), x.size, dtype), "unary")
    return out


# ---- paged kv ----
def page_write(storage, values, page_ids, offsets, page_size, inner, storage_offset=0,
               page_count=None):
    """Returns a new storage array (the reference copies storage to the output first)."""
    storage = _c(storage); values = _c(values)
    page_ids = _c(page_ids, np.int32); offsets = _c(offsets, np.int32)
    out = storage.copy()
    es = storage.dtype.itemsize
    if page_count is None:
        page_count = (storage.size - storage_offset) // (page_size * inner)
    _check(lib().or_page_write(_p(storage), _p(values), _p(page_ids), _p(offsets), _p(out),
                               page_count, page_size, inner, page_ids.size, storage_offset, es),
           "page_write")
    return out


def page_write_fp8(storage, values, page_ids, offsets, page_size, kv_heads, head_dim, scales,
                   value_dtype, storage_offset=0, page_count=None):
    """fp8-E4M3 quantising page write (library extension): returns a new uint8
    storage with byte = E4M3(x / scale[head]) written at each row's page slot."""
    storage = _c(storage, np.uint8); values = _c(values)
    page_ids = _c(page_ids, np.int32); offsets = _c(offsets, np.int32)
    scales = _c(scales, np.float32)
    out = storage.copy()
    inner = kv_heads * head_dim
    if page_count is None:
        page_count = (storage.size - storage_offset) // (page_size * inner)
    _check(lib().or_page_write_fp8(_p(out), _p(values), _p(page_ids), _p(offsets), page_count,
                                   page_size, kv_heads, head_dim, page_ids.size, storage_offset,
                                   _p(scales), value_dtype), "page_write_fp8")
    return out


def page_gather(storage, page_table, page_size, inner, out_rows, storage_offset=0, page_count=None):
    storage = _c(storage); page_table = _c(page_table, np.int32)
    es = storage.dtype.itemsize
    if page_count is None:
        page_count = (storage.size - storage_offset) // (page_size * inner)
    rows = min(out_rows, page_table.size * page_size)
    out = np.zeros((out_rows, inner), storage.dtype)
    _check(lib().or_page_gather(_p(storage), _p(page_table), _p(out), page_count, page_size, inner,
                                rows, storage_offset, page_table.size, es), "page_gather")
    return out


# ---- attention ----
def mha(q, k, v, num_heads, head_dim, causal=True, kv_heads=0, window=0, alibi=0.0, dtype=F32):
    q = _c(q, STORAGE[dtype]); k = _c(k, STORAGE[dtype]); v = _c(v, STORAGE[dtype])
    seq_q = q.shape[0]; seq_k = k.shape[0]
    cfg = MHAConfig(num_heads, head_dim, int(causal), window, alibi, kv_heads)
    out = np.zeros_like(q)
    _check(lib().or_mha(C.byref(cfg), _p(q), _p(k), _p(v), _p(out), seq_q, seq_k, dtype), "mha")
    return out


def mha_rows(q, k, v, num_heads, head_dim, heads, rows, causal=True, kv_heads=0, dtype=F32,
             out=None):
    q = _c(q, STORAGE[dtype]); k = _c(k, STORAGE[dtype]); v = _c(v, STORAGE[dtype])
    seq_q = q.shape[0]; seq_k = k.shape[0]
    cfg = MHAConfig(num_heads, head_dim, int(causal), 0, 0.0, kv_heads)
    if out is None:
        out = np.zeros_like(q)
    _check(lib().or_mha_rows(C.byref(cfg), _p(q), _p(k), _p(v), _p(out), seq_q, seq_k,
                             heads[0], heads[1], rows[0], rows[1], dtype), "mha_rows")
    return out


def flash_attention(q, k, v, causal=True, dtype=F32):
    """ScaledDotProductAttention / FlashAttention on one head: q [seqQ, depth],
    k [seqK, depth], v [seqK, valueDim] -> [seqQ, valueDim]."""
    q = _c(q, STORAGE[dtype]); k = _c(k, STORAGE[dtype]); v = _c(v, STORAGE[dtype])
    seq_q, depth = q.shape
    seq_k, value_dim = v.shape
    out = np.zeros((seq_q, value_dim), STORAGE[dtype])
    _check(lib().or_flash_attention(int(causal), _p(q), _p(k), _p(v), _p(out), seq_q, seq_k,
                                    depth, value_dim, dtype), "flash_attention")
    return out


def paged_decode(q, key_pages, value_pages, page_table, context_lens, page_size, num_heads,
                 kv_heads, head_dim, kv_dtype, k_scale=None, v_scale=None):
    q = _c(q, np.uint16); key_pages = _c(key_pages); value_pages = _c(value_pages)
    page_table = _c(page_table, np.int32); context_lens = _c(context_lens, np.int32)
    if k_scale is not None:
        k_scale = _c(k_scale, np.float32); v_scale = _c(v_scale, np.float32)
    batch, max_pages = page_table.shape
    out = np.zeros((batch, num_heads * head_dim), np.uint16)
    _check(lib().or_paged_decode(_p(q), _p(key_pages), _p(value_pages), _p(page_table),
                                 _p(context_lens), batch, max_pages, page_size, num_heads, kv_heads,
                                 head_dim, _p(k_scale), _p(v_scale), kv_dtype, _p(out)),
           "paged_decode")
    return out


def dequant_int8(codes, scale, zero_point):
    """Dequant (F32 <- Int8): device/cpu/dequant/int8_generic.go:3-7."""
    codes = _c(codes, np.int8)
    out = np.empty(codes.shape, np.float32)
    _check(lib().or_dequant_int8(_p(out), _p(codes), codes.size, scale, zero_point), "dequant_int8")
    return out


def dequant_int4(packed, count, scale, zero_point):
    """Dequant4 (F32 <- Int4): `count` signed nibbles, element 2k = low nibble of byte k."""
    packed = _c(packed, np.uint8)
    assert packed.size >= (count + 1) // 2
    out = np.empty(count, np.float32)
    _check(lib().or_dequant_int4(_p(out), _p(packed), count, scale, zero_point), "dequant_int4")
    return out


def quant_int8(values, scale, zero_point):
    """Quant (Int8 <- F32): device/cpu/quant/int8_generic.go:5-18."""
    values = _c(values, np.float32)
    out = np.empty(values.shape, np.int8)
    _check(lib().or_quant_int8(_p(out), _p(values), values.size, scale, zero_point), "quant_int8")
    return out


_EXT_NP = {F32: np.float32, I8: np.int8, I4: np.uint8, F64: np.float64}


def cast_ext(src, src_dtype, dst_dtype, count=None):
    """convert/int_f32.go and convert/f32_f64.go casts (one side is F32)."""
    src = _c(src, _EXT_NP[src_dtype])
    n = src.size if count is None else count
    out = np.empty(n, _EXT_NP[dst_dtype])
    _check(lib().or_cast_ext(_p(out), dst_dtype, _p(src), src_dtype, n), "cast_ext")
    return out


_PAIR_NP = {F16: np.uint16, BF16: np.uint16, F8E4M3: np.uint8, F8E5M2: np.uint8, F64: np.float64}


def cast_pair(src, src_dtype, dst_dtype):
    """shape.cast between two float formats without an f32 side
    (execution/shape_cast_intrinsic.go:56-115): f64 widening, float32(v), narrowing."""
    src = _c(src, _PAIR_NP[src_dtype])
    out = np.empty(src.size, _PAIR_NP[dst_dtype])
    _check(lib().or_cast_pair(_p(out), dst_dtype, _p(src), src_dtype, src.size), "cast_pair")
    return out


def matmul_f32(left, right):
    left = _c(left, np.float32); right = _c(right, np.float32)
    rows, inner = left.shape
    cols = right.shape[1]
    out = np.empty((rows, cols), np.float32)
    _check(lib().or_matmul_f32(_p(out), _p(left), _p(right), rows, inner, cols), "matmul")
    return out


def matmul(left, right, dtype):
    """Matmul in F32 / F64 / BF16 / F16 (bf16 and f16 as uint16 bit patterns)."""
    npt = {F32: np.float32, F64: np.float64, BF16: np.uint16, F16: np.uint16}[dtype]
    left = _c(left, npt); right = _c(right, npt)
    rows, inner = left.shape
    cols = right.shape[1]
    out = np.empty((rows, cols), npt)
    _check(lib().or_matmul(_p(out), _p(left), _p(right), rows, inner, cols, dtype), "matmul")
    return out


# ---- seeded inputs: SplitMix64 -> Box-Muller (implementation-independent) ----
def splitmix64(seed: int, n: int) -> np.ndarray:
    """n uint64 outputs of SplitMix64 starting from `seed` (vectorised)."""
    with np.errstate(over="ignore"):
        idx = np.arange(1, n + 1, dtype=np.uint64)
        z = np.uint64(seed) + idx * np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def normal(seed: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    """n N(mean, std^2) float32 values from SplitMix64 + Box-Muller."""
    m = (n + 1) // 2
    bits = splitmix64(seed, 2 * m)
    u1 = ((bits[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)
    u2 = (bits[1::2] >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * m, np.float64)
    z[0::2] = r * np.cos(2 * np.pi * u2)
    z[1::2] = r * np.sin(2 * np.pi * u2)
    return (z[:n] * std + mean).astype(np.float32)
