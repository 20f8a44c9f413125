"""CPU tier: pin the quantisation oracle (oracle/quant.c) before it checks the GPU.

Every check is something other than the oracle's own formula: numpy's IEEE
f32 arithmetic on the reference's test parameters, exact rational arithmetic,
explicit bit patterns, round-trip invariants, and cases chosen so that a
plausible mistake (nibble order swapped, ties to even, the zero point added
before rounding, a reciprocal multiply instead of the division, truncation
instead of saturation) fails one of them."""
from fractions import Fraction

import numpy as np

import oracle as O

CODES = np.arange(-128, 128, dtype=np.int8)


# --------------------------------------------------------------- Dequant --
def test_dequant_int8_reference_parameters_and_exact_form():
    # dequant_int8_generic_parity_test.go:29-30 (scale 0.0875, zero point -13)
    got = O.dequant_int8(CODES, 0.0875, -13)
    want = (CODES.astype(np.int32) + 13).astype(np.float32) * np.float32(0.0875)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # power-of-two scale: exact rational value for every code
    got = O.dequant_int8(CODES, 0.0625, 3)
    for c, g in zip(CODES.tolist(), got.tolist()):
        assert Fraction(g) == Fraction(c - 3, 16)


def test_dequant_int4_nibble_order_and_sign():
    # element 2k = low nibble of byte k, 2k+1 = high nibble, signed
    # (device/cpu/dequant/dequant_int4_neon_arm64.s:4-6)
    packed = np.array([0x8F, 0x17, 0x70], np.uint8)
    assert O.dequant_int4(packed, 6, 1.0, 0).tolist() == [-1.0, -8.0, 7.0, 1.0, 0.0, 7.0]
    # an odd count ignores the last high nibble
    assert O.dequant_int4(packed, 5, 1.0, 0).tolist() == [-1.0, -8.0, 7.0, 1.0, 0.0]
    # all 256 bytes against a bit-twiddled sign extension
    b = np.arange(256, dtype=np.uint8)
    lo = ((b & 15).astype(np.int32) ^ 8) - 8
    hi = ((b >> 4).astype(np.int32) ^ 8) - 8
    want = np.stack([lo, hi], 1).reshape(-1)
    # reference parameters: dequant_int4_generic_parity_test.go:51-52
    got = O.dequant_int4(b, 512, 0.0625, 3)
    assert np.array_equal(got, ((want - 3).astype(np.float32) * np.float32(0.0625)))


# ----------------------------------------------------------------- Quant --
def test_quant_ties_go_away_from_zero_and_zero_point_after_rounding():
    x = np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 0.49999997], np.float32)
    assert O.quant_int8(x, 1.0, 0).tolist() == [1, 2, 3, -1, -2, -3, 0]
    # round(-0.5) + 1 = 0, whereas rounding after adding the zero point gives 1
    assert O.quant_int8(np.array([-0.5], np.float32), 1.0, 1).tolist() == [0]


def test_quant_saturates_and_maps_nan_to_zero():
    x = np.array([1e9, -1e9, np.inf, -np.inf, np.nan, 127.4, 127.6, -128.4, -128.6], np.float32)
    assert O.quant_int8(x, 1.0, 0).tolist() == [127, -128, 127, -128, 0, 127, 127, -128, -128]
    # scale 0: x / 0 is +-inf (saturates) and 0 / 0 is NaN (0)
    assert O.quant_int8(np.array([2.0, -2.0, 0.0], np.float32), 0.0, 5).tolist() == [127, -128, 0]


def test_quant_divides_rather_than_multiplying_by_the_reciprocal():
    # find (x, scale) where x / scale and x * (1 / scale) round to different int8
    rng = np.random.default_rng(7)
    s = np.float32(0.1)
    inv = np.float32(1.0) / s
    found = None
    for _ in range(200):
        k = rng.integers(-100, 100, 4096)
        x = ((k + 0.5) * s).astype(np.float32)
        x = np.concatenate([x, np.nextafter(x, np.float32(np.inf)), np.nextafter(x, np.float32(-np.inf))])
        qd = x / s
        qr = x * inv
        r_d = np.sign(qd) * np.floor(np.abs(qd).astype(np.float64) + 0.5)
        r_r = np.sign(qr) * np.floor(np.abs(qr).astype(np.float64) + 0.5)
        idx = np.nonzero(r_d != r_r)[0]
        if idx.size:
            found = (x[idx[0]], int(r_d[idx[0]]), int(r_r[idx[0]]))
            break
    assert found is not None
    xv, want, other = found
    assert want != other
    assert O.quant_int8(np.array([xv], np.float32), float(s), 0).tolist() == [want]


def test_quant_reference_parameters_against_numpy_formulation():
    # quant_int8_generic_parity_test.go:27-35: N(0,1) * 10, scale 0.125, zero point 7
    x = (O.normal(0x55AA, 1 << 16) * 10).astype(np.float32)
    q = (x / np.float32(0.125)).astype(np.float64)
    want = np.clip(np.sign(q) * np.floor(np.abs(q) + 0.5) + 7, -128, 127).astype(np.int8)
    assert np.array_equal(O.quant_int8(x, 0.125, 7), want)


def test_quant_dequant_round_trip_every_code():
    for zp in (-128, -13, 0, 3, 127):
        for scale in (0.0625, 4.0, 0.5):
            x = O.dequant_int8(CODES, scale, zp)
            assert np.array_equal(O.quant_int8(x, scale, zp), CODES)


# ----------------------------------------------------------------- casts --
def test_int8_and_int4_casts():
    assert np.array_equal(O.cast_ext(CODES, O.I8, O.F32), CODES.astype(np.float32))
    x = np.array([2.9, -2.9, 127.9, 128.0, -128.9, -129.0, 1e10, np.nan, np.inf, -np.inf, -0.0, 0.99],
                 np.float32)
    # convert/int_f32.go:30-52: saturate, else truncate toward zero
    assert O.cast_ext(x, O.F32, O.I8).tolist() == [2, -2, 127, 127, -128, -128, 127, 0, 127, -128, 0, 0]
    assert O.cast_ext(np.array([0x8F, 0x17], np.uint8), O.I4, O.F32, count=3).tolist() == [-1.0, -8.0, 7.0]


def _f64(bits):
    return np.array(bits, np.uint64).view(np.float64)


def test_f64_to_f32_rounding_underflow_overflow_nan():
    cases = {
        1.0 / 3.0: 0x3EAAAAAB,
        1.0 + 2.0 ** -24: 0x3F800000,            # tie -> even (down)
        1.0 + 3 * 2.0 ** -24: 0x3F800002,        # tie -> even (up)
        2.0 ** -150: 0x00000000,                 # tie between 0 and the least denormal -> 0
        3 * 2.0 ** -150: 0x00000002,             # tie -> even: 2 * 2^-149
        2.0 ** -149 * 1.25: 0x00000001,
        (2 - 2.0 ** -23) * 2.0 ** 127: 0x7F7FFFFF,
        (2 - 2.0 ** -25) * 2.0 ** 127: 0x7F800000,  # rounds up past the largest finite
        2.0 ** 128: 0x7F800000,
        -0.0: 0x80000000,
    }
    src = np.array(list(cases), np.float64)
    got = O.cast_ext(src, O.F64, O.F32).view(np.uint32)
    assert got.tolist() == list(cases.values())
    special = _f64([0x7FF0000000000001, 0x7FF4000000000000, 0xFFF8000000000123, 0x0000000000000001,
                    0x7FF0000000000000, 0x7FEFFFFFFFFFFFFF])
    got = O.cast_ext(special, O.F64, O.F32).view(np.uint32)
    # signalling NaNs are quieted keeping the payload's top bits; f64 denormals -> 0
    assert [hex(v) for v in got] == ['0x7fc00000', '0x7fe00000', '0xffc00000', '0x0', '0x7f800000',
                                     '0x7f800000']


def test_f32_to_f64_exact_and_nan_quieting():
    src = np.array([0x00000001, 0x007FFFFF, 0x80000000, 0x7F800001, 0x3F800000, 0x7F7FFFFF],
                   np.uint32).view(np.float32)
    got = O.cast_ext(src, O.F32, O.F64).view(np.uint64)
    assert [hex(v) for v in got] == ['0x36a0000000000000', '0x380fffffc0000000', '0x8000000000000000',
                                     '0x7ff8000020000000', '0x3ff0000000000000', '0x47efffffe0000000']
    # every finite f32 survives the round trip
    rng = np.random.default_rng(3)
    bits = rng.integers(0, 2**32, 1 << 18, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[np.isfinite(x)]
    back = O.cast_ext(O.cast_ext(x, O.F32, O.F64), O.F64, O.F32)
    assert np.array_equal(back.view(np.uint32), x.view(np.uint32))


# ------------------------------------------- shape.cast between float formats --
def _all16(dtype):
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    return bits[~np.isnan(O.to_f32(bits, dtype))]


def test_cast_pair_16bit_each_way_matches_torch():
    """bf16 <-> f16 for every non-NaN pattern: widen, narrow with RNE (torch
    converts through float32 too; f16 overflow goes to infinity)."""
    import torch
    b = _all16(O.BF16)
    want = torch.from_numpy(b.view(np.int16)).view(torch.bfloat16).to(torch.float16).view(torch.int16)
    assert np.array_equal(O.cast_pair(b, O.BF16, O.F16), want.numpy().view(np.uint16))
    h = _all16(O.F16)
    want = torch.from_numpy(h.view(np.int16)).view(torch.float16).to(torch.bfloat16).view(torch.int16)
    assert np.array_equal(O.cast_pair(h, O.F16, O.BF16), want.numpy().view(np.uint16))


def test_cast_pair_fp8_sides():
    import torch
    codes = np.arange(256, dtype=np.uint8)
    finite = ~np.isnan(O.to_f32(codes, O.F8E4M3))
    for dst in (O.BF16, O.F16):          # every finite e4m3 value is exact in bf16 / f16
        got = O.cast_pair(codes, O.F8E4M3, dst)
        assert np.array_equal(O.to_f32(got, dst)[finite], O.to_f32(codes, O.F8E4M3)[finite])
    b = _all16(O.BF16)
    x = O.to_f32(b, O.BF16)
    inr = np.abs(x) <= 448
    ref = torch.from_numpy(x[inr]).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = O.cast_pair(b, O.BF16, O.F8E4M3)
    assert np.array_equal(got[inr], ref)
    assert np.all(got[~inr & np.isfinite(x)] & 0x7F == 0x7E)    # saturating (convert/fp8_f32.go:20-23)


def test_cast_pair_f64_rounds_through_float32():
    """shape_cast_intrinsic.go:83-114: float32(v) first, then the narrowing.  1 +
    2^-8 + 2^-30 rounds to 1 + 2^-8 in f32, an exact bf16 tie that goes to even
    (1.0); rounded straight from f64 it would be 1 + 2^-7."""
    x = np.array([1 + 2**-8 + 2**-30], np.float64)
    assert O.cast_pair(x, O.F64, O.BF16)[0] == 0x3F80
    rng = np.random.default_rng(5)
    v = np.concatenate([rng.standard_normal(1 << 16) * 100, rng.standard_normal(1000) * 1e-39,
                        [np.inf, -np.inf, 0.0, -0.0, 1e300, -1e300, 5e-324]])
    for dst in (O.BF16, O.F16, O.F8E4M3, O.F8E5M2):
        with np.errstate(over="ignore"):
            assert np.array_equal(O.cast_pair(v, O.F64, dst), O.from_f32(v.astype(np.float32), dst))
    for src in (O.BF16, O.F16):
        b = _all16(src)
        assert np.array_equal(O.cast_pair(b, src, O.F64), O.to_f32(b, src).astype(np.float64))
