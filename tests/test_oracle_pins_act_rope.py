"""CPU tier: pins for the oracle's MultiAxisRoPE positions and the activation
helpers that only the C restatement checked before (FastTanh32 / GeGLUTanh,
FastSigmoid32 / SiGLU / GLU, unary Silu / Gelu, FastExp64).

Every expected value here comes from a formulation other than the oracle's:
MultiAxisRoPE positions from an explicit enumeration of the latent grid and the
rotation as a float64 complex product; tanh from Lambert's continued fraction and
math.tanh; sigmoid, SiLU and GeLU from float64 exp / erf.  Each test also shows
that the plausible slip it guards against (swapped image axes, text on the wrong
axis, gate/up swapped, FastSilu32 instead of the float64 table) would fail it."""
import math

import numpy as np
import pytest

import oracle as O
from helpers import seeded


# ------------------------------------------------------------ MultiAxisRoPE --
def _axis_positions(seq_len, latent_seq_len, latent_side, axis_count):
    """positions[seq, axis] from an explicit walk over the latent grid: text
    tokens first (their index on the text axis: 3 with four axes, else 0), then
    the image tokens in row-major order over rows of latent_side columns
    (row on axis 1, column on axis 2), rope/compute.go:302-330."""
    text_len = max(seq_len - latent_seq_len, 0)
    text_axis = 3 if axis_count == 4 else 0
    pos = np.zeros((seq_len, 4), np.int64)
    for s in range(text_len):
        pos[s, text_axis] = s
    cells = [(r, c) for r in range(seq_len) for c in range(latent_side)]
    for i, s in enumerate(range(text_len, seq_len)):
        pos[s, 1], pos[s, 2] = cells[i]
    return pos


def _multi_axis_rope64(x, base, latent_seq_len, latent_side, axis_dims, swap_image_axes=False):
    """float64 model: pair p of axis a (local index j of axis_dims[a]/2 pairs)
    rotates by position[a] * base^(-2j / axis_dims[a]) as a complex product."""
    b, s, h, d = x.shape
    pos = _axis_positions(s, latent_seq_len, latent_side, len(axis_dims))
    if swap_image_axes:
        pos[:, [1, 2]] = pos[:, [2, 1]]
    z = x.astype(np.float64).reshape(b, s, h, d // 2, 2)
    z = z[..., 0] + 1j * z[..., 1]
    angles = np.zeros((s, d // 2))
    p = 0
    for a, ad in enumerate(axis_dims):
        for j in range(ad // 2):
            angles[:, p] = pos[:, a] * base ** (-2.0 * j / ad)
            p += 1
    z = z * np.exp(1j * angles)[None, :, None, :]
    out = np.stack([z.real, z.imag], -1).reshape(b, s, h, d)
    return out


def _rope_err(x, got, ref):
    scale = np.maximum(np.abs(x.astype(np.float64)), 1e-30)
    pair = scale.reshape(*x.shape[:-1], -1, 2).max(-1).repeat(2, -1)
    return np.max(np.abs(got.astype(np.float64) - ref) / pair)


CASES = [
    # batch, seq, heads, base, latent, side, axis dims
    (1, 20, 2, 1e4, 12, 4, [4, 6, 6]),          # 3 axes, 3x4 image grid after 8 text tokens
    (2, 23, 3, 1e4, 15, 6, [2, 6, 4, 4]),        # 4 axes: text on axis 3, ragged last image row
    (1, 9, 1, 500.0, 9, 3, [4, 4, 4]),           # no text tokens
    (1, 5, 2, 1e4, 12, 4, [4, 4, 8]),            # seq < latent: every token is an image token
    (1, 640, 2, 1e4, 512, 32, [32, 32, 32, 32]),  # multi_axis_test.go:48-60 scaled down (16x32 grid)
]


@pytest.mark.parametrize("b,s,h,base,latent,side,dims", CASES)
def test_multi_axis_rope_matches_latent_grid_walk(b, s, h, base, latent, side, dims):
    x = seeded(100 + s, (b, s, h, sum(dims)))
    got = O.multi_axis_rope(x, base, latent, side, dims, O.F32)
    assert _rope_err(x, got, _multi_axis_rope64(x, base, latent, side, dims)) < 4e-6
    if any(r != c for r, c in _axis_positions(s, latent, side, len(dims))[:, 1:3]):
        # the row/column swap on axes 1/2 is caught
        assert _rope_err(x, got, _multi_axis_rope64(x, base, latent, side, dims, True)) > 1e-2


@pytest.mark.parametrize("n", [1, 7, 64, 1024])
def test_multi_axis_rope_reference_parity_config(n):
    """The reference test's own configuration (multi_axis_test.go:15-44,81-95):
    four axes (2, 6, 4, 4), base 2000, latent = max(n/2, 1), side =
    ceil(sqrt(latent)), batch 1, 2 heads of 16."""
    latent = max(n // 2, 1)
    side = int(math.ceil(math.sqrt(latent)))
    x = seeded(0x9500 + n, (1, n, 2, 16))
    got = O.multi_axis_rope(x, 2000.0, latent, side, [2, 6, 4, 4], O.F32)
    assert _rope_err(x, got, _multi_axis_rope64(x, 2000.0, latent, side, [2, 6, 4, 4])) < 4e-6


def test_multi_axis_rope_text_axis_depends_on_axis_count():
    """With four axes a text token rotates only axis 3 (axis 0 stays put); with
    three it rotates only axis 0 (rope/compute.go:318-330)."""
    x = seeded(3, (1, 6, 1, 16))
    four = O.multi_axis_rope(x, 1e4, 2, 2, [4, 4, 4, 4], O.F32)
    three = O.multi_axis_rope(x, 1e4, 2, 2, [4, 6, 6], O.F32)
    for s in range(1, 4):   # text tokens past position 0
        assert np.array_equal(four[0, s, 0, :12], x[0, s, 0, :12])
        assert not np.allclose(four[0, s, 0, 12:], x[0, s, 0, 12:])
        assert not np.allclose(three[0, s, 0, :4], x[0, s, 0, :4])
        assert np.array_equal(three[0, s, 0, 4:], x[0, s, 0, 4:])


def test_multi_axis_rope_16bit_is_f32_rotation_then_narrowing():
    """bf16 / f16: widen, rotate in f32, narrow (rope/dtype_load.go:9-53)."""
    x32 = seeded(4, (1, 20, 2, 16))
    for dt in (O.BF16, O.F16):
        xb = O.from_f32(x32, dt)
        got = O.multi_axis_rope(xb, 1e4, 12, 4, [2, 6, 4, 4], dt)
        ref = O.from_f32(O.multi_axis_rope(O.to_f32(xb, dt), 1e4, 12, 4, [2, 6, 4, 4], O.F32), dt)
        assert np.array_equal(got, ref)


# ------------------------------------------------------ FastTanh32 / GeGLU --
def _lambert_tanh(x, terms=7):
    """Lambert's continued fraction x / (1 + x^2 / (3 + x^2 / (5 + ...))),
    truncated after the partial denominator 2*terms - 1, in float64."""
    t = 2.0 * terms - 1
    for k in range(terms - 1, 0, -1):
        t = (2 * k - 1) + x * x / t
    return x / t


def test_fast_tanh32_is_lambert_fraction_and_close_to_tanh():
    xs = np.concatenate([np.linspace(-4.92, 4.92, 4001), seeded(5, (2000,), 0.0, 2.0)]).astype(np.float32)
    xs = xs[np.abs(xs) <= 4.92]
    got = np.array([O.fast_tanh32(v) for v in xs])
    cf = np.array([_lambert_tanh(float(v)) for v in xs])
    assert np.max(np.abs(got - cf)) < 4e-7        # f32 evaluation of the same rational function
    assert np.max(np.abs(got - np.tanh(xs.astype(np.float64)))) < 9.5e-5   # the approximant's own error
    # clamps at +-4.92 (math/f32.go:76-81): exactly +-1 beyond, the fraction at the edge
    assert O.fast_tanh32(4.9201) == 1.0 and O.fast_tanh32(-4.9201) == -1.0 and O.fast_tanh32(100) == 1.0
    assert O.fast_tanh32(np.float32(4.92)) != 1.0 and abs(O.fast_tanh32(np.float32(4.92)) - 1) < 1.1e-4
    assert O.fast_tanh32(0.0) == 0.0 and O.fast_tanh32(-0.5) == -O.fast_tanh32(0.5)


def test_geglu_tanh_f64():
    g = seeded(6, (4096,), 0.0, 3.0)
    u = seeded(7, (4096,), 0.0, 3.0)
    got = O.gated_tensors(O.GATE_GEGLU_TANH, g, u, O.F32).astype(np.float64)
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    gelu = 0.5 * u64 * (1 + np.tanh(math.sqrt(2 / math.pi) * (u64 + 0.044715 * u64 ** 3)))
    ref = g64 * gelu                                           # gate * gelu_tanh(up)
    assert np.max(np.abs(got - ref) / (np.abs(g64) * np.maximum(np.abs(u64), 1))) < 1.2e-4
    swapped = u64 * 0.5 * g64 * (1 + np.tanh(math.sqrt(2 / math.pi) * (g64 + 0.044715 * g64 ** 3)))
    assert np.max(np.abs(got - swapped)) > 0.1


# --------------------------------------------- FastSigmoid32 / SiGLU / GLU --
def _sigmoid64(v):
    v = np.asarray(v, np.float64)
    return np.where(v >= 0, 1 / (1 + np.exp(-np.abs(v))), np.exp(-np.abs(v)) / (1 + np.exp(-np.abs(v))))


def test_fast_sigmoid32_both_branches():
    xs = np.concatenate([np.linspace(-80, 80, 3201), seeded(8, (2000,), 0.0, 5.0)]).astype(np.float32)
    got = np.array([O.fast_sigmoid32(v) for v in xs], np.float64)
    ref = _sigmoid64(xs)
    assert np.max(np.abs(got - ref) / ref) < 1.2e-4           # FastExp32's relative error, both branches
    # v < 0 keeps relative precision (e / (1 + e)), not 1 - something: at -60 the
    # value is ~8.8e-27, far below f32's resolution near 1
    assert abs(O.fast_sigmoid32(-60.0) / math.exp(-60.0) - 1) < 1.2e-4
    # FastExp32 clamps: below -87.33654 exp is 0, so sigmoid is exactly 0; large
    # positive inputs give exactly 1
    assert O.fast_sigmoid32(-87.5) == 0.0 and O.fast_sigmoid32(100.0) == 1.0
    assert O.fast_sigmoid32(0.0) == 0.5


def test_siglu_and_glu_operand_order():
    g = seeded(9, (4096,), 0.5, 3.0)
    u = seeded(10, (4096,), -0.5, 2.0)
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    siglu = O.gated_tensors(O.GATE_SIGLU, g, u, O.F32).astype(np.float64)   # sigmoid(gate) * up
    glu = O.gated_tensors(O.GATE_GLU, g, u, O.F32).astype(np.float64)       # gate * sigmoid(up)
    want_siglu, want_glu = _sigmoid64(g64) * u64, g64 * _sigmoid64(u64)
    tol = 1.5e-4 * (np.abs(g64) + np.abs(u64) + 1)
    assert np.all(np.abs(siglu - want_siglu) < tol) and np.all(np.abs(glu - want_glu) < tol)
    assert np.max(np.abs(siglu - want_glu)) > 1.0 and np.max(np.abs(glu - want_siglu)) > 1.0


# ------------------------------------------------------- unary Silu / Gelu --
def test_unary_f32_silu_gelu_f64():
    x = seeded(11, (8192,), 0.0, 4.0)
    x64 = x.astype(np.float64)
    silu = O.unary(O.UNARY_SILU, x, O.F32).astype(np.float64)
    ref = x64 * _sigmoid64(x64)
    assert np.max(np.abs(silu - ref) / np.maximum(np.abs(ref), 1e-3)) < 2e-4
    gelu = O.unary(O.UNARY_GELU, x, O.F32).astype(np.float64)
    erf = np.vectorize(math.erf)
    ref = 0.5 * x64 * (1 + erf(x64 / math.sqrt(2)))
    assert np.max(np.abs(gelu - ref) / np.maximum(np.abs(ref), 1e-30)) < 1.2e-7   # f32 rounding only


def test_fast_exp64_error_bound_and_clamps():
    xs = np.concatenate([np.linspace(-700, 700, 14001), seeded(12, (4000,), 0.0, 10.0).astype(np.float64)])
    got = np.array([O.fast_exp64(v) for v in xs])
    # 2^f by its degree-5 Taylor polynomial: relative error < ln2^6/720 * 2^... ~ 8.7e-5
    assert np.max(np.abs(got / np.exp(xs) - 1)) < 9e-5
    assert O.fast_exp64(0.0) == 1.0
    assert O.fast_exp64(-708.4) == 0.0 and O.fast_exp64(710.0) == np.finfo(np.float64).max


def test_unary_16bit_silu_is_the_float64_table():
    """The reference's f16 / bf16 Silu reads a table filled with
    narrow(float32(FastSilu64(x))) (activation/lut.go:14-62).  Every bf16 input
    pattern: the oracle agrees with float64 x*sigmoid(x) to within FastExp64's
    error (one bf16 step at most), and it is the float64 table, not FastSilu32
    (those differ on some inputs after narrowing)."""
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    x = O.to_f32(bits, O.BF16)
    ok = np.isfinite(x)
    got = O.unary(O.UNARY_SILU, bits, O.BF16)
    x64 = x[ok].astype(np.float64)
    with np.errstate(over="ignore"):
        exact = O.from_f32((x64 * _sigmoid64(x64)).astype(np.float32), O.BF16)
    diff = np.abs(got[ok].astype(np.int64) - exact.astype(np.int64))
    assert np.max(diff) <= 1 and np.count_nonzero(diff) < 0.01 * diff.size
    table = O.from_f32(np.array([O.fast_silu64(v) for v in x[ok]], np.float32), O.BF16)
    assert np.array_equal(got[ok], table)
    via_f32 = O.unary(O.UNARY_SILU, x[ok], O.F32)       # FastSilu32
    assert not np.array_equal(O.from_f32(via_f32, O.BF16), table)
    # f16: same table rule with the IEEE half narrowing
    bits16 = np.arange(0, 0x7C00, 7, dtype=np.uint16)
    x16 = O.to_f32(bits16, O.F16)
    got16 = O.unary(O.UNARY_SILU, bits16, O.F16)
    assert np.array_equal(got16, O.from_f32(np.array([O.fast_silu64(v) for v in x16], np.float32), O.F16))


# -------------------------------------------------------------- RoPEPairs --
def test_rope_pairs_f64_and_closed_forms():
    """RopePairsGeneric (rope/f32_generic.go:3-11): pair i rotated by (cos[i], sin[i])."""
    x = seeded(13, (2 * 1024,))
    ang = seeded(14, (1024,), 0.0, 3.0).astype(np.float64)
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    got = O.rope_pairs(x, cos, sin).astype(np.float64)
    z = (x[0::2] + 1j * x[1::2]).astype(np.complex128) * (cos.astype(np.float64) + 1j * sin.astype(np.float64))
    ref = np.stack([z.real, z.imag], -1).ravel()
    assert np.max(np.abs(got - ref)) < 1e-6 * np.max(np.abs(x))
    one, zero = np.ones(1024, np.float32), np.zeros(1024, np.float32)
    assert np.array_equal(O.rope_pairs(x, one, zero), x)                     # identity
    q = O.rope_pairs(x, zero, one)                                            # quarter turn: (e, o) -> (-o, e)
    assert np.array_equal(q[0::2], -x[1::2]) and np.array_equal(q[1::2], x[0::2])
