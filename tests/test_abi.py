"""CPU tier: the C-ABI library loads, exports every symbol include/puter_hip.h
declares, and rejects invalid arguments with the reference's status codes
before touching a device (device/cuda/internal/bridge/status.c: -2 nil buffer,
-6 invalid dtype/shape/config).  No compute call is made here."""
import ctypes as C
import subprocess

import pytest

from puter_amd import _lib

FAKE = 0x1000  # a non-null address that is never dereferenced on these paths


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_every_header_symbol_is_exported(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIBRARY], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    declared = _lib.header_symbols()
    assert declared, "no declarations parsed"
    missing = [s for s in declared if s not in exported]
    assert not missing, missing
    assert set(_lib.SIGNATURES) == set(declared), set(_lib.SIGNATURES) ^ set(declared)
    # nothing but the C ABI leaks out of the library
    extra = sorted(s for s in exported if s.startswith("puter") and s not in declared)
    assert not extra, extra


def test_library_links_no_torch(lib):
    out = subprocess.run(["ldd", _lib.LIBRARY], capture_output=True, text=True).stdout
    assert "torch" not in out and "python" not in out


def err(lib):
    return lib.puter_hip_last_error().decode()


def test_norm_validation(lib):
    rc = lib.puter_hip_rmsnorm(FAKE, FAKE, FAKE, 4, 8, 0.0, 0, None)
    assert rc == _lib.ERR_INVALID and "epsilon" in err(lib)
    assert lib.puter_hip_rmsnorm(FAKE, FAKE, FAKE, 4, 8, 1e-5, 3, None) == _lib.ERR_INVALID   # fp8 norm
    assert lib.puter_hip_rmsnorm(None, FAKE, FAKE, 4, 8, 1e-5, 0, None) == _lib.ERR_NIL
    assert lib.puter_hip_rmsnorm(None, None, None, 0, 8, 1e-5, 0, None) == _lib.OK         # zero rows: no-op
    assert lib.puter_hip_layernorm(FAKE, FAKE, FAKE, FAKE, -1, 8, 0, None) == _lib.ERR_INVALID
    # rows % rowsPerBatch != 0 (compute.go:636-638) and too-narrow modulation
    assert lib.puter_hip_adaptive_rmsnorm(FAKE, FAKE, FAKE, 6, 8, 4, 16, 1e-6, 0, None) == _lib.ERR_INVALID
    assert lib.puter_hip_adaptive_rmsnorm(FAKE, FAKE, FAKE, 8, 8, 4, 15, 1e-6, 0, None) == _lib.ERR_INVALID
    assert lib.puter_hip_modulated_layernorm(FAKE, FAKE, FAKE, 8, 8, 4, 39, 1e-6, 1, 0, None) == _lib.ERR_INVALID
    assert lib.puter_hip_modulated_layernorm(FAKE, FAKE, FAKE, 8, 8, 4, 40, 1e-6, -1, 0, None) == _lib.ERR_INVALID
    # gated residual layout: modCols >= (3*set+3)*H (math_gated_residual_intrinsic.go:135-137)
    assert lib.puter_hip_gated_residual(FAKE, FAKE, FAKE, FAKE, 4, 8, 2, 23, 0, 2, None) == _lib.ERR_INVALID
    assert lib.puter_hip_gated_residual(FAKE, FAKE, FAKE, FAKE, 4, 8, 3, 24, 0, 2, None) == _lib.ERR_INVALID
    assert lib.puter_hip_gated_residual_rmsnorm(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 4, 8, 4, 24, 0, 0.0, 2,
                                                None) == _lib.ERR_INVALID


def test_rope_validation(lib):
    c = _lib.RopeConfig(0.0, 0, 0, 0, 1.0, 0, 0, 0)
    assert lib.puter_hip_rope(C.byref(c), FAKE, FAKE, 4, 2, 8, 0, None) == _lib.ERR_INVALID
    c = _lib.RopeConfig(1e4, 0, 2, 0, 1.0, 0, 0, 0)
    assert lib.puter_hip_rope(C.byref(c), FAKE, FAKE, 4, 2, 8, 0, None) == _lib.ERR_INVALID
    c = _lib.RopeConfig(1e4, 0, 0, 1, 8.0, 4.0, 1.0, 8192)   # high <= low
    assert lib.puter_hip_rope(C.byref(c), FAKE, FAKE, 4, 2, 8, 0, None) == _lib.ERR_INVALID
    c = _lib.RopeConfig(1e4, 0, 0, 0, 1.0, 0, 0, 0)
    # odd head dim / empty: silent no-op (rope/compute.go:17-19)
    assert lib.puter_hip_rope(C.byref(c), None, None, 4, 2, 7, 0, None) == _lib.OK
    assert lib.puter_hip_rope(C.byref(c), None, None, 0, 2, 8, 0, None) == _lib.OK
    dims = (C.c_int64 * 4)(4, 6, 0, 0)
    m = _lib.MultiAxisRopeConfig(1e4, 2, 2, 2, 0, dims)
    assert lib.puter_hip_multi_axis_rope(C.byref(m), FAKE, FAKE, 1, 4, 1, 12, 0, None) == _lib.ERR_INVALID


def test_cast_activation_page_validation(lib):
    assert lib.puter_hip_cast(FAKE, 2, FAKE, 5, 16, None) == _lib.ERR_INVALID      # int32 -> bf16
    assert lib.puter_hip_cast(FAKE, 1, FAKE, 6, 16, None) == _lib.ERR_INVALID      # int8 -> f16: no f32 side
    assert lib.puter_hip_cast(None, 0, FAKE, 2, 16, None) == _lib.ERR_NIL
    assert lib.puter_hip_cast(None, 0, None, 2, 0, None) == _lib.OK
    assert lib.puter_hip_gated_tensors(9, FAKE, FAKE, FAKE, 16, 0, None) == _lib.ERR_INVALID
    assert lib.puter_hip_gated_packed(0, FAKE, FAKE, 2, 8, 3, None) == _lib.ERR_INVALID
    assert lib.puter_hip_kv_page_write(FAKE, FAKE, FAKE, FAKE, FAKE, 4, 0, 8, 2, 0, 0, None, None) == _lib.ERR_INVALID
    assert lib.puter_hip_kv_page_gather(FAKE, FAKE, FAKE, 4, 16, 8, 2, 0, 9, None, None) == _lib.ERR_INVALID
    # the device status word must be a 4-byte aligned int32
    assert lib.puter_hip_kv_page_write(FAKE, FAKE, FAKE, FAKE, FAKE, 4, 16, 8, 2, 0, 0, FAKE + 2, None) == _lib.ERR_INVALID
    assert lib.puter_hip_kv_page_gather(FAKE, FAKE, FAKE, 4, 16, 8, 2, 0, 0, FAKE + 1, None) == _lib.ERR_INVALID
    assert lib.puter_hip_kv_page_write_fp8(FAKE, FAKE, FAKE, FAKE, 4, 16, 2, 128, 2, 0, FAKE, 2, FAKE + 2,
                                           None) == _lib.ERR_INVALID
    # stream probe: shapes 0-2 only, rows of 1024 vectors for the row shapes
    assert lib.puter_hip_stream_probe(FAKE, FAKE, FAKE, FAKE, 1024, 3, None) == _lib.ERR_INVALID
    assert lib.puter_hip_stream_probe(FAKE, FAKE, FAKE, FAKE, 1000, 1, None) == _lib.ERR_INVALID
    assert lib.puter_hip_stream_probe(None, None, None, None, 0, 0, None) == _lib.OK
    # MFMA probe: modes 0-1, non-negative sizes; no blocks is a no-op
    assert lib.puter_hip_mfma_probe(FAKE, FAKE, 8, 4, 2, None) == _lib.ERR_INVALID
    assert lib.puter_hip_mfma_probe(FAKE, FAKE, -1, 4, 0, None) == _lib.ERR_INVALID
    assert lib.puter_hip_mfma_probe(None, None, 0, 4, 0, None) == _lib.OK
    # RoPEPairs is F32 only (device/cpu/rope/ops.go:10-14); zero pairs is a no-op
    assert lib.puter_hip_rope_pairs(FAKE, FAKE, FAKE, FAKE, 8, 2, None) == _lib.ERR_INVALID
    assert lib.puter_hip_rope_pairs(None, None, None, None, 0, 0, None) == _lib.OK
    assert lib.puter_hip_rope_pairs(None, FAKE, FAKE, FAKE, 8, 0, None) == _lib.ERR_NIL


def test_attention_validation(lib):
    cfg = _lib.MHAConfig(6, 64, 1, 0, 0, 0.0, 0, 4)   # 6 heads not divisible by 4 kv heads
    assert lib.puter_hip_multi_head_attention(C.byref(cfg), FAKE, FAKE, FAKE, FAKE, 8, 8, 2, None) == _lib.ERR_INVALID
    cfg = _lib.MHAConfig(4, 512, 1, 0, 0, 0.0, 0, 0)
    assert lib.puter_hip_multi_head_attention(C.byref(cfg), FAKE, FAKE, FAKE, FAKE, 8, 8, 2, None) == _lib.ERR_INVALID
    assert lib.puter_hip_multi_head_attention(None, FAKE, FAKE, FAKE, FAKE, 8, 8, 2, None) == _lib.ERR_NIL
    # paged decode: workspace sizing and argument checks
    ws = lib.puter_hip_paged_decode_workspace_bytes(64, 32, 128, 8192)
    assert ws == 64 * 32 * (8192 // 256) * 130 * 4   # 256-token splits, (m, l, o[128]) per slot
    args = [FAKE] * 5 + [2, 4, 16, 100, 32, 8, 128, 64, None, None, 2, FAKE, FAKE, ws, None]
    assert lib.puter_hip_paged_decode_attention(*args[:-4], FAKE, FAKE, 16, None) == _lib.ERR_INVALID  # workspace too small
    bad = list(args)
    bad[11] = 64                                                    # head_dim 64 unsupported
    assert lib.puter_hip_paged_decode_attention(*bad) == _lib.ERR_INVALID
    bad = list(args)
    bad[12] = 65                                                    # max_context > pages*page_size
    assert lib.puter_hip_paged_decode_attention(*bad) == _lib.ERR_INVALID
    bad = list(args)
    bad[9], bad[10] = 34, 2                                         # 17 query heads per kv head (at most 16)
    assert lib.puter_hip_paged_decode_attention(*bad) == _lib.ERR_INVALID
    bad = list(args)
    bad[15] = 3                                                     # fp8 without scales
    assert lib.puter_hip_paged_decode_attention(*bad) == _lib.ERR_NIL
    # Matmul takes F32 / F64 / BF16 / F16 (compute.go:46-62); fp8 is rejected
    assert lib.puter_hip_matmul(FAKE, FAKE, FAKE, 4, 4, 4, 3, None) == _lib.ERR_INVALID
    assert lib.puter_hip_matmul(FAKE, FAKE, FAKE, -1, 4, 4, 2, None) == _lib.ERR_INVALID


def test_backend_class_requires_the_library():
    import puter_amd
    be = puter_amd.Backend()
    assert be.lib is _lib.load()
    with pytest.raises(puter_amd.PuterError) as e:
        be.RMSNorm(puter_amd.RMSNormConfig(-1.0), FAKE, FAKE, FAKE, 4, 8, puter_amd.F32)
    assert e.value.status == _lib.ERR_INVALID


def test_flash_attention_validation(lib):
    fc = _lib.FlashConfig(0, 1, 0)
    for fn in (lib.puter_hip_scaled_dot_product_attention, lib.puter_hip_flash_attention):
        assert fn(None, FAKE, FAKE, FAKE, FAKE, 4, 4, 8, 8, 0, None) == _lib.ERR_NIL
        assert fn(C.byref(fc), FAKE, FAKE, FAKE, FAKE, 4, 4, 8, 8, 3, None) == _lib.ERR_INVALID   # fp8
        assert fn(C.byref(fc), None, None, None, None, 0, 4, 8, 8, 0, None) == _lib.OK            # seqQ 0
        assert fn(C.byref(fc), None, None, None, None, 4, 0, 8, 8, 0, None) == _lib.OK            # seqK 0
        assert fn(C.byref(fc), FAKE, FAKE, FAKE, FAKE, 4, 4, 0, 8, 0, None) == _lib.ERR_INVALID   # depth 0
        assert fn(C.byref(fc), FAKE, FAKE, FAKE, FAKE, 4, 4, 8192 + 1, 8, 0, None) == _lib.ERR_INVALID
        assert fn(C.byref(fc), FAKE, FAKE, FAKE, FAKE, 4, 4, 8, 1025, 0, None) == _lib.ERR_INVALID
        assert fn(C.byref(fc), FAKE, None, FAKE, FAKE, 4, 4, 8, 8, 0, None) == _lib.ERR_NIL
