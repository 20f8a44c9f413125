"""GPU parity: casts (bit-exact), the LayerNorm family and the gated residual
(fused and unfused) against the CPU oracle on the same seeded inputs.

Reference behaviour: convert/*.go, device/cpu/layernorm/compute.go,
execution/math_gated_residual_intrinsic.go:206-223."""
import numpy as np
import pytest

import oracle as O
from helpers import REDUCE_ELEM_TOL, TOL, assert_close, decode, empty_dev, encode, seeded, to_dev, to_host

pytestmark = pytest.mark.gpu
NP = {O.F32: np.float32, O.F16: np.uint16, O.BF16: np.uint16, O.F8E4M3: np.uint8, O.F8E5M2: np.uint8}


# ------------------------------------------------------------------ casts --
@pytest.mark.parametrize("dt,n", [(O.BF16, 1 << 16), (O.F16, 1 << 16), (O.F8E4M3, 256), (O.F8E5M2, 256)])
def test_widen_every_pattern_bit_exact(backend, dt, n):
    bits = np.arange(n, dtype=np.uint32).astype(NP[dt])
    ref = O.to_f32(bits, dt).view(np.uint32)
    src = to_dev(bits)
    dst = empty_dev((n,), np.float32)
    backend.Cast(dst, O.F32, src, dt, n)
    got = to_host(dst, np.float32).view(np.uint32)
    assert np.array_equal(got, ref), f"first mismatch at {np.nonzero(got != ref)[0][:5]}"


def special_f32_bits():
    vals = [0, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000, 0xFFC00000, 0x7F800001, 0x7FBFFFFF,
            0x00000001, 0x807FFFFF, 0x7F7FFFFF, 0xFF7FFFFF]
    # every exponent with mantissas at rounding boundaries of each narrow format
    mants = [0, 1, 0x7FFF, 0x8000, 0x8001, 0x18000, 0x0FFF, 0x1000, 0x1001, 0x3000,
             0x7FFFF, 0x80000, 0x80001, 0x180000, 0xFFFFF, 0x100000, 0x100001, 0x300000, 0x7FFFFF]
    for e in range(256):
        for m in mants:
            for s in (0, 1):
                vals.append((s << 31) | (e << 23) | m)
    return np.array(vals, dtype=np.uint32)


@pytest.mark.parametrize("dt", [O.BF16, O.F16, O.F8E4M3, O.F8E5M2])
def test_narrow_bit_exact(backend, dt):
    rng = np.random.default_rng(1234 + dt)
    bits = np.concatenate([special_f32_bits(), rng.integers(0, 2**32, size=1 << 22, dtype=np.uint64).astype(np.uint32)])
    x = bits.view(np.float32)
    ref = O.from_f32(x, dt)
    src = to_dev(x)
    dst = empty_dev((x.size,), NP[dt])
    backend.Cast(dst, dt, src, O.F32, x.size)
    got = to_host(dst, NP[dt])
    bad = np.nonzero(got != ref)[0]
    assert bad.size == 0, f"{bad.size} mismatches, e.g. f32 {bits[bad[:4]]} -> {got[bad[:4]]} vs {ref[bad[:4]]}"


@pytest.mark.parametrize("n", [1, 7, 64, 1000, 8192 + 3])
def test_cast_ragged_and_unaligned(backend, n):
    x = seeded(77 + n, (n + 1,)) * np.float32(40)
    src = to_dev(x)
    dst = empty_dev((n + 1,), np.uint16)
    backend.Cast(dst[1:], O.BF16, src[1:], O.F32, n)   # offset views: unaligned by 4 / 2 bytes
    got = to_host(dst, np.uint16)[1:]
    assert np.array_equal(got, O.from_f32(x[1:], O.BF16))


# ------------------------------------------------------------------ norms --
NORM_SHAPES = [(1, 8), (7, 64), (5, 1000), (128, 512), (64, 2048), (33, 4096), (16, 8192)]


@pytest.mark.parametrize("dt", [O.F32, O.BF16, O.F16])
@pytest.mark.parametrize("rows,h", NORM_SHAPES)
def test_rmsnorm(backend, dt, rows, h):
    import puter_amd
    x = encode(seeded(1000 + rows + h, (rows, h)), dt)
    g = encode(seeded(2000 + h, (h,), 1.0, 0.02), dt)
    eps = 1e-6 if dt == O.F32 else 1e-5
    ref = decode(O.rmsnorm(x, g, eps, dt), dt)
    out = empty_dev((rows, h), NP[dt])
    backend.RMSNorm(puter_amd.RMSNormConfig(eps), to_dev(x), to_dev(g), out, rows, h, dt)
    assert_close(decode(to_host(out, NP[dt]), dt), ref, TOL[dt], REDUCE_ELEM_TOL[dt], what="rmsnorm")


@pytest.mark.parametrize("dt", [O.F32, O.BF16, O.F16])
@pytest.mark.parametrize("rows,h", NORM_SHAPES)
def test_layernorm(backend, dt, rows, h):
    x = encode(seeded(3000 + rows + h, (rows, h)), dt)
    g = encode(seeded(4000 + h, (h,), 1.0, 0.02), dt)
    b = encode(seeded(5000 + h, (h,), 0.0, 0.02), dt)
    ref = decode(O.layernorm(x, g, b, dt), dt)
    out = empty_dev((rows, h), NP[dt])
    backend.LayerNorm(to_dev(x), to_dev(g), to_dev(b), out, rows, h, dt)
    assert_close(decode(to_host(out, NP[dt]), dt), ref, TOL[dt], REDUCE_ELEM_TOL[dt], what="layernorm")


def gated_inputs(dt, rows, h, rpb, set_index, seed):
    batches = rows // rpb
    cols = (3 * set_index + 3) * h
    res = encode(seeded(seed, (rows, h)), dt)
    br = encode(seeded(seed + 1, (rows, h)), dt)
    mod = encode(seeded(seed + 2, (batches, cols)), dt)
    return res, br, mod, cols


@pytest.mark.parametrize("dt", [O.F32, O.BF16, O.F16])
@pytest.mark.parametrize("rows,h,rpb,set_index", [(4, 6, 2, 0), (64, 2048, 64, 0), (32, 4096, 8, 1), (9, 1000, 3, 0)])
def test_gated_residual(backend, dt, rows, h, rpb, set_index):
    res, br, mod, cols = gated_inputs(dt, rows, h, rpb, set_index, 600 + rows)
    ref = O.gated_residual(res, br, mod, rpb, set_index, dt)
    out = empty_dev((rows, h), NP[dt])
    backend.GatedResidual(to_dev(res), to_dev(br), to_dev(mod), out, rows, h, rpb, cols, set_index, dt)
    got = to_host(out, NP[dt])
    if dt == O.F32:
        assert_close(got, ref, TOL[dt], REDUCE_ELEM_TOL[dt], what="gated residual")
    else:  # one multiply-add then one rounding: must agree bit for bit
        assert np.array_equal(got, ref)


@pytest.mark.parametrize("dt", [O.BF16, O.F32, O.F16])
@pytest.mark.parametrize("kind", ["rms", "ln"])
@pytest.mark.parametrize("rows,h", [(64, 2048), (48, 4096), (16, 8192), (6, 1000)])
def test_fused_gated_residual_norm(backend, dt, kind, rows, h):
    """Fused op == GatedResidual then the norm on the stored hidden values."""
    import puter_amd
    res, br, mod, cols = gated_inputs(dt, rows, h, rows, 0, 900 + h)
    g = encode(seeded(950 + h, (h,), 1.0, 0.02), dt)
    b = encode(seeded(960 + h, (h,), 0.0, 0.02), dt)
    hid_ref = O.gated_residual(res, br, mod, rows, 0, dt)
    eps = 1e-5
    y_ref = O.rmsnorm(hid_ref, g, eps, dt) if kind == "rms" else O.layernorm(hid_ref, g, b, dt)
    hid = empty_dev((rows, h), NP[dt])
    y = empty_dev((rows, h), NP[dt])
    if kind == "rms":
        backend.GatedResidualRMSNorm(puter_amd.RMSNormConfig(eps), to_dev(res), to_dev(br), to_dev(mod),
                                     to_dev(g), hid, y, rows, h, rows, cols, 0, dt)
    else:
        backend.GatedResidualLayerNorm(to_dev(res), to_dev(br), to_dev(mod), to_dev(g), to_dev(b),
                                       hid, y, rows, h, rows, cols, 0, dt)
    hid_got = to_host(hid, NP[dt])
    if dt != O.F32:
        assert np.array_equal(hid_got, hid_ref)
    assert_close(decode(hid_got, dt), decode(hid_ref, dt), TOL[dt], REDUCE_ELEM_TOL[dt], what="hidden")
    assert_close(decode(to_host(y, NP[dt]), dt), decode(y_ref, dt), TOL[dt], REDUCE_ELEM_TOL[dt], what=kind)


@pytest.mark.parametrize("dt", [O.F32, O.BF16, O.F16])
@pytest.mark.parametrize("rows,h,rpb", [(8, 64, 4), (16, 2048, 8), (6, 1000, 2)])
def test_adaptive_and_modulated(backend, dt, rows, h, rpb):
    import puter_amd
    x = encode(seeded(70 + h, (rows, h)), dt)
    mod = encode(seeded(71 + h, (rows // rpb, 6 * h), 0.0, 0.5), dt)
    eps = 1e-6
    ref = decode(O.adaptive_rmsnorm(x, mod, rpb, eps, dt), dt)
    out = empty_dev((rows, h), NP[dt])
    backend.AdaptiveRMSNorm(puter_amd.RMSNormConfig(eps), to_dev(x), to_dev(mod), out, rows, h, rpb, 6 * h, dt)
    assert_close(decode(to_host(out, NP[dt]), dt), ref, TOL[dt], REDUCE_ELEM_TOL[dt], what="adaptive")
    for set_index in (0, 1):
        ref = decode(O.modulated_layernorm(x, mod, rpb, eps, set_index, dt), dt)
        backend.ModulatedLayerNorm(puter_amd.ModulatedLayerNormConfig(eps, set_index), to_dev(x), to_dev(mod),
                                   out, rows, h, rpb, 6 * h, dt)
        assert_close(decode(to_host(out, NP[dt]), dt), ref, TOL[dt], REDUCE_ELEM_TOL[dt], what=f"modulated set {set_index}")


def test_norm_errors_raise(backend):
    import puter_amd
    x = empty_dev((4, 8), np.float32)
    with pytest.raises(puter_amd.PuterError):
        backend.RMSNorm(puter_amd.RMSNormConfig(0.0), x, x, x, 4, 8, O.F32)  # epsilon must be > 0
    with pytest.raises(puter_amd.PuterError):
        backend.LayerNorm(x, x, x, x, 4, 8, O.F8E4M3)  # unsupported dtype
    # zero-sized work is a no-op, as compute.go:19-21
    backend.LayerNorm(x, x, x, x, 0, 8, O.F32)


# the block-per-row kernel (>= 4096 rows of >= 512 16-byte vectors): every norm
# op and dtype, the fused ops included, against the oracle
@pytest.mark.parametrize("dt,h", [(O.BF16, 4096), (O.BF16, 8192), (O.F16, 8192), (O.F32, 2048), (O.F32, 8192)])
def test_norms_block_per_row(backend, dt, h):
    import puter_amd
    rows, rpb = 4096, 1024
    x = encode(seeded(7100 + h + dt, (rows, h)), dt)
    g = encode(seeded(7200 + h, (h,), 1.0, 0.02), dt)
    b = encode(seeded(7300 + h, (h,), 0.0, 0.02), dt)
    out = empty_dev((rows, h), NP[dt])
    dx = to_dev(x)
    backend.RMSNorm(puter_amd.RMSNormConfig(1e-5), dx, to_dev(g), out, rows, h, dt)
    assert_close(decode(to_host(out, NP[dt]), dt), decode(O.rmsnorm(x, g, 1e-5, dt), dt), TOL[dt],
                 REDUCE_ELEM_TOL[dt], what="rmsnorm")
    backend.LayerNorm(dx, to_dev(g), to_dev(b), out, rows, h, dt)
    assert_close(decode(to_host(out, NP[dt]), dt), decode(O.layernorm(x, g, b, dt), dt), TOL[dt],
                 REDUCE_ELEM_TOL[dt], what="layernorm")
    mod = encode(seeded(7400 + h, (rows // rpb, 6 * h), 0.0, 0.5), dt)
    backend.AdaptiveRMSNorm(puter_amd.RMSNormConfig(1e-6), dx, to_dev(mod), out, rows, h, rpb, 6 * h, dt)
    assert_close(decode(to_host(out, NP[dt]), dt), decode(O.adaptive_rmsnorm(x, mod, rpb, 1e-6, dt), dt),
                 TOL[dt], REDUCE_ELEM_TOL[dt], what="adaptive")
    backend.ModulatedLayerNorm(puter_amd.ModulatedLayerNormConfig(1e-6, 1), dx, to_dev(mod), out, rows, h, rpb,
                               6 * h, dt)
    assert_close(decode(to_host(out, NP[dt]), dt), decode(O.modulated_layernorm(x, mod, rpb, 1e-6, 1, dt), dt),
                 TOL[dt], REDUCE_ELEM_TOL[dt], what="modulated")
    br = encode(seeded(7500 + h, (rows, h)), dt)
    gm = encode(seeded(7600 + h, (rows // rpb, 3 * h)), dt)
    hid = empty_dev((rows, h), NP[dt])
    hid_ref = O.gated_residual(x, br, gm, rpb, 0, dt)
    for kind in ("rms", "ln"):
        if kind == "rms":
            backend.GatedResidualRMSNorm(puter_amd.RMSNormConfig(1e-5), dx, to_dev(br), to_dev(gm), to_dev(g), hid,
                                         out, rows, h, rpb, 3 * h, 0, dt)
            y_ref = O.rmsnorm(hid_ref, g, 1e-5, dt)
        else:
            backend.GatedResidualLayerNorm(dx, to_dev(br), to_dev(gm), to_dev(g), to_dev(b), hid, out, rows, h,
                                           rpb, 3 * h, 0, dt)
            y_ref = O.layernorm(hid_ref, g, b, dt)
        got_h = to_host(hid, NP[dt])
        if dt != O.F32:
            assert np.array_equal(got_h, hid_ref), kind
        else:
            assert_close(got_h, hid_ref, TOL[dt], REDUCE_ELEM_TOL[dt], what="hidden")
        assert_close(decode(to_host(out, NP[dt]), dt), decode(y_ref, dt), TOL[dt], REDUCE_ELEM_TOL[dt],
                     what=f"fused {kind}")
