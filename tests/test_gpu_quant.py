"""GPU tier: Dequant / Dequant4 / Quant and the int8 / int4 / f64 casts,
bit-exact against the pinned oracle (oracle/quant.c) through the C ABI."""
import numpy as np
import pytest

import oracle as O
from helpers import empty_dev, to_dev, to_host

pytestmark = pytest.mark.gpu

SIZES = [1, 3, 4, 5, 17, 1000, (1 << 20) + 7]


def _bits_equal(a, b):
    a, b = np.asarray(a), np.asarray(b)
    w = {4: np.uint32, 8: np.uint64, 1: np.uint8}[a.dtype.itemsize]
    return np.array_equal(a.view(w), b.view(w))


def _f32_values(n, seed, scale=10.0):
    """Gaussians, random bit patterns (NaNs, denormals, infinities) and exact ties."""
    rng = np.random.default_rng(seed)
    g = (rng.standard_normal(n) * scale).astype(np.float32)
    bits = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32).view(np.float32)
    ties = ((rng.integers(-140, 140, n) + 0.5) * 0.125).astype(np.float32)
    pick = rng.integers(0, 3, n)
    x = np.where(pick == 0, g, np.where(pick == 1, bits, ties)).astype(np.float32)
    x[: min(n, 8)] = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 1e9, -1e9, 1e-45], np.float32)[: min(n, 8)]
    return x


def _dev_slice(arr, offset):
    """Device copy of arr starting `offset` elements into a larger buffer (unaligned pointers)."""
    pad = np.zeros(offset, arr.dtype)
    return to_dev(np.concatenate([pad, arr]))[offset:]


@pytest.mark.parametrize("scale,zp", [(0.0875, -13), (0.0625, 3), (0.1, 0), (-3.0, 127), (1e-3, -128)])
@pytest.mark.parametrize("n", SIZES)
def test_dequant_int8(backend, scale, zp, n):
    import puter_amd
    codes = np.random.default_rng(1000 * n + zp + 128).integers(-128, 128, n).astype(np.int8)
    ref = O.dequant_int8(codes, scale, zp)
    for off in (0, 1):
        out = empty_dev((n + off,), np.float32)[off:]
        backend.Dequant(out, _dev_slice(codes, off), n, puter_amd.DequantInt8Config(scale, zp),
                        puter_amd.F32, puter_amd.I8)
        assert _bits_equal(to_host(out, np.float32), ref), (n, off)


@pytest.mark.parametrize("scale,zp", [(0.0625, 3), (0.3, -8), (2.0, 0)])
@pytest.mark.parametrize("n", SIZES)
def test_dequant4(backend, scale, zp, n):
    import puter_amd
    packed = np.random.default_rng(n).integers(0, 256, (n + 1) // 2).astype(np.uint8)
    ref = O.dequant_int4(packed, n, scale, zp)
    for off in (0, 1):
        out = empty_dev((n + off,), np.float32)[off:]
        backend.Dequant4(out, _dev_slice(packed, off), n, puter_amd.DequantInt4Config(scale, zp),
                         puter_amd.F32, puter_amd.I4)
        assert _bits_equal(to_host(out, np.float32), ref), (n, off)


@pytest.mark.parametrize("scale,zp", [(0.125, 7), (0.1, 0), (3.0, -128), (-0.5, 127), (0.0, 5)])
@pytest.mark.parametrize("n", SIZES)
def test_quant(backend, scale, zp, n):
    import puter_amd
    x = _f32_values(n, 11 + n)
    ref = O.quant_int8(x, scale, zp)
    for off in (0, 1):
        out = empty_dev((n + off,), np.int8)[off:]
        backend.Quant(out, _dev_slice(x, off), n, puter_amd.DequantInt8Config(scale, zp),
                      puter_amd.I8, puter_amd.F32)
        assert np.array_equal(to_host(out, np.int8), ref), (n, off)


@pytest.mark.parametrize("n", SIZES)
def test_int_and_f64_casts(backend, n):
    import puter_amd as P
    rng = np.random.default_rng(100 + n)
    codes = rng.integers(-128, 128, n).astype(np.int8)
    x = _f32_values(n, 200 + n)
    packed = rng.integers(0, 256, (n + 1) // 2).astype(np.uint8)
    f64 = rng.integers(0, 2**64, n, dtype=np.uint64).view(np.float64).copy()
    f64[: min(n, 4)] = np.array([1.0 + 2.0 ** -24, 2.0 ** -150, 3 * 2.0 ** -150,
                                 (2 - 2.0 ** -25) * 2.0 ** 127])[: min(n, 4)]
    cases = [
        (codes, P.I8, P.F32, np.float32, None),
        (x, P.F32, P.I8, np.int8, None),
        (packed, P.I4, P.F32, np.float32, n),
        (x, P.F32, P.F64, np.float64, None),
        (f64, P.F64, P.F32, np.float32, None),
    ]
    for src, sdt, ddt, np_out, count in cases:
        ref = O.cast_ext(src, sdt, ddt, count=count)
        for off in (0, 1):
            out = empty_dev((n + off,), np_out)[off:]
            backend.Cast(out, ddt, _dev_slice(src, off), sdt, n)
            assert _bits_equal(to_host(out, np_out), ref), (sdt, ddt, n, off)


def test_quant_dequant_round_trip_full_size(backend):
    """Size-independent property at 32M elements: Quant(Dequant(c)) == c for every
    code when the scale is a power of two."""
    import puter_amd as P
    import torch
    n = 1 << 25
    codes = torch.randint(-128, 128, (n,), dtype=torch.int8, device="cuda")
    mid = torch.empty(n, dtype=torch.float32, device="cuda")
    back = torch.empty(n, dtype=torch.int8, device="cuda")
    cfg = P.DequantInt8Config(0.25, -7)
    backend.Dequant(mid, codes, n, cfg, P.F32, P.I8)
    backend.Quant(back, mid, n, cfg, P.I8, P.F32)
    assert torch.equal(back, codes)
    # f32 -> f64 -> f32 is the identity on finite values
    x = torch.randn(n, device="cuda") * 1e3
    d = torch.empty(n, dtype=torch.float64, device="cuda")
    y = torch.empty(n, dtype=torch.float32, device="cuda")
    backend.Cast(d, P.F64, x, P.F32, n)
    backend.Cast(y, P.F32, d, P.F64, n)
    assert torch.equal(x.view(torch.int32), y.view(torch.int32))


def test_quant_errors(backend):
    import puter_amd as P
    a = empty_dev((16,), np.float32)
    b = empty_dev((16,), np.int8)
    with pytest.raises(P.PuterError):
        backend.Dequant(a, b, 16, P.DequantInt8Config(1.0, 0), P.BF16, P.I8)   # unsupported pair
    with pytest.raises(P.PuterError):
        backend.Quant(b, a, 16, P.DequantInt8Config(1.0, 200), P.I8, P.F32)    # zero point outside int8
    with pytest.raises(P.PuterError):
        backend.Cast(a, P.I4, b, P.F32, 16)                                     # int4 only as a source
    backend.Quant(b, a, 0, P.DequantInt8Config(1.0, 0), P.I8, P.F32)            # zero count: no-op


# ------------------------------ shape.cast between float formats, one launch --
PAIR_NP = {O.F16: np.uint16, O.BF16: np.uint16, O.F8E4M3: np.uint8, O.F8E5M2: np.uint8, O.F64: np.float64}
PAIR_FORMATS = [O.BF16, O.F16, O.F8E4M3, O.F8E5M2, O.F64]


def _pair_source(dt, n, seed):
    rng = np.random.default_rng(seed)
    if dt == O.F64:
        v = np.concatenate([rng.standard_normal(n) * 300.0, [1 + 2**-8 + 2**-30, np.inf, -np.inf, np.nan,
                                                            0.0, -0.0, 1e-39, 1e300, 5e-324]])
        return v[:n].astype(np.float64) if n < 9 else v
    es = np.dtype(PAIR_NP[dt]).itemsize
    return rng.integers(0, 1 << (8 * es), n).astype(PAIR_NP[dt])   # every bit pattern class


@pytest.mark.parametrize("src", PAIR_FORMATS)
@pytest.mark.parametrize("dst", PAIR_FORMATS)
@pytest.mark.parametrize("n,off", [(1, 0), (13, 0), (4096, 0), ((1 << 18) + 5, 0), (1000, 1)])
def test_cast_float_pair(backend, src, dst, n, off):
    """Any two of bf16 / f16 / fp8 / f64 in one pass (execution/shape_cast_intrinsic.go:56-115),
    bit-exact against the oracle (NaN codes compared as NaN), aligned and unaligned."""
    x = _pair_source(src, n, 100 * src + dst + n)
    n = x.size
    ref = x.copy() if src == dst else O.cast_pair(x, src, dst)
    out_np = PAIR_NP[dst]
    if off:
        d_out = to_dev(np.zeros(n + off, out_np))[off:]
        d_in = _dev_slice(x, off)
    else:
        d_out, d_in = empty_dev((n,), out_np), to_dev(x)
    backend.Cast(d_out, dst, d_in, src, n)
    got = to_host(d_out, out_np)
    if dst == O.F64:
        nan = np.isnan(ref)
        assert np.array_equal(np.isnan(got), nan) and _bits_equal(got[~nan], ref[~nan])
    else:
        nan = np.isnan(O.to_f32(ref, dst))
        assert np.array_equal(np.isnan(O.to_f32(got, dst)), nan)
        assert np.array_equal(got[~nan], ref[~nan])
