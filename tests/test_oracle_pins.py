"""CPU tier: pin the oracle before trusting it as the GPU checker.

Each oracle function is checked against something that does not restate its
own formula: the reference's known-answer tests, library routines (torch /
numpy casts), closed forms, invariants, and float64 brute force on tiny
shapes chosen so that a dropped term, a wrong sign or a transposed operand
fails.  File:line citations point at the reference test or code each check
follows."""
import math

import numpy as np
import pytest
import torch

import oracle as O
from helpers import seeded

# ------------------------------------------------------------------ casts --


def _finite_samples(n, seed, scale):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(n) * scale).astype(np.float32)
    bits = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32).view(np.float32)
    return np.concatenate([x, bits[np.isfinite(bits)]])


def test_bf16_narrow_matches_torch_rne_for_non_nan():
    x = _finite_samples(1 << 20, 1, 100.0)
    x = np.concatenate([x, np.array([np.inf, -np.inf, 3.4e38, -3.4e38, 1e-45, 0.0, -0.0], np.float32)])
    ours = O.from_f32(x, O.BF16)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)


def test_bf16_tie_cases_round_to_even():
    # 1 + 2^-8 is exactly halfway between 1 and 1 + 2^-7: even mantissa wins
    ties = np.array([0x3F808000, 0x3F818000, 0xBF808000, 0x3F807FFF, 0x3F808001], np.uint32).view(np.float32)
    assert list(O.from_f32(ties, O.BF16)) == [0x3F80, 0x3F82, 0xBF80, 0x3F80, 0x3F81]


def test_nan_stays_nan_everywhere():
    nans = np.array([0x7FC00000, 0xFFC00000, 0x7F800001, 0x7FBFFFFF, 0xFFFFFFFF], np.uint32).view(np.float32)
    assert np.all(np.isnan(O.to_f32(O.from_f32(nans, O.BF16), O.BF16)))
    assert np.all(np.isnan(O.to_f32(O.from_f32(nans, O.F16), O.F16)))
    assert np.all(O.from_f32(nans, O.F8E4M3) & 0x7F == 0x7F)       # S.1111.111 (fp8_test.go:131-133)
    assert np.all(np.isnan(O.to_f32(O.from_f32(nans, O.F8E5M2), O.F8E5M2)))


def test_f16_narrow_matches_numpy_ieee():
    x = _finite_samples(1 << 20, 2, 3000.0)
    x = np.concatenate([x, np.array([65504, 65519.99, 65520, -65520, 6e-8, 3e-8, 2.98e-8, 1e-9], np.float32)])
    ours = O.from_f32(x, O.F16)
    ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, ref)


def test_f16_widen_every_pattern_matches_numpy():
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    ours = O.to_f32(bits, O.F16)
    ref = bits.view(np.float16).astype(np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(ours[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.array_equal(np.isnan(ours), np.isnan(ref)) and np.array_equal(np.isinf(ours), np.isinf(ref))


def test_bf16_widen_is_shift():
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    ref = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).float().numpy()
    ours = O.to_f32(bits, O.BF16)
    ok = ~np.isnan(ref)
    assert np.array_equal(ours[ok].view(np.uint32), ref[ok].view(np.uint32))
    assert np.all(np.isnan(ours[~ok]))


def test_fp8_decode_tables_ocp():
    codes = np.arange(256, dtype=np.uint8)
    e4 = O.to_f32(codes, O.F8E4M3)
    # OCP E4M3FN spot values: max 448, min normal 2^-6, min subnormal 2^-9, NaN at 0x7F/0xFF
    assert e4[0x7E] == 448 and e4[0xFE] == -448 and e4[0x08] == 2**-6 and e4[0x01] == 2**-9
    assert np.isnan(e4[0x7F]) and np.isnan(e4[0xFF]) and np.sum(np.isnan(e4)) == 2
    ref4 = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(np.isnan(e4), np.isnan(ref4)) and np.array_equal(e4[~np.isnan(e4)], ref4[~np.isnan(ref4)])
    e5 = O.to_f32(codes, O.F8E5M2)
    assert e5[0x7B] == 57344 and e5[0x04] == 2**-14 and e5[0x01] == 2**-16 and np.isinf(e5[0x7C])
    ref5 = torch.from_numpy(codes).view(torch.float8_e5m2).float().numpy()
    assert np.array_equal(np.isnan(e5), np.isnan(ref5)) and np.array_equal(e5[~np.isnan(e5)], ref5[~np.isnan(ref5)])


def test_fp8_narrow_matches_torch_in_range_and_saturates_outside():
    x = _finite_samples(1 << 20, 3, 60.0)
    for dt, tdt, top, maxcode in ((O.F8E4M3, torch.float8_e4m3fn, 448.0, 0x7E), (O.F8E5M2, torch.float8_e5m2, 57344.0, 0x7B)):
        ours = O.from_f32(x, dt)
        inr = np.abs(x) < top
        ref = torch.from_numpy(x[inr]).to(tdt).view(torch.uint8).numpy()
        assert np.array_equal(ours[inr], ref)
        big = np.array([top, top * 1.01, 1e30, np.inf, -top * 2, -np.inf], np.float32)
        got = O.from_f32(big, dt)
        assert np.all(got & 0x7F == maxcode) and np.array_equal(got >> 7, (big < 0).astype(np.uint8))


@pytest.mark.parametrize("n", [1, 7, 64, 1024, 8192])  # parity.Lengths (cpu/parity/parity.go:10)
def test_reference_round_trip_kats(n):
    """convert/convert_test.go:54-178 round-trip tolerances."""
    i = np.arange(n)
    a = (i % 19).astype(np.float32) * 0.5
    rt = O.to_f32(O.from_f32(a, O.BF16), O.BF16)
    assert np.all(np.abs(rt - a) <= np.abs(a) / 128)
    b = ((i % 13) - 6).astype(np.float32) * 0.25
    rt = O.to_f32(O.from_f32(b, O.F16), O.F16)
    assert np.all(np.abs(rt - b) <= np.maximum(np.abs(b) / 1024, 1e-45))
    c = ((i % 9) - 4).astype(np.float32) * 0.5
    rt = O.to_f32(O.from_f32(c, O.F8E4M3), O.F8E4M3)
    assert np.all(np.abs(rt - c) <= np.maximum(np.abs(c) / 8, 0.0625))


# ------------------------------------------------------------- FastExp32 --
def test_fast_exp32_error_bound_and_clamps():
    xs = np.linspace(-87.0, 88.0, 20001, dtype=np.float32)
    got = np.array([O.fast_exp32(v) for v in xs], np.float64)
    rel = np.abs(got - np.exp(xs.astype(np.float64))) / np.exp(xs.astype(np.float64))
    assert rel.max() < 1.0e-4                      # polynomial quality (f32.go:38-39)
    assert O.fast_exp32(0.0) == 1.0                # z = 0 -> k = 0, f = 0, poly = 1
    assert O.fast_exp32(-87.34) == 0.0 and O.fast_exp32(-1000.0) == 0.0
    assert O.fast_exp32(88.73) == np.finfo(np.float32).max
    # monotone on a fine grid (a transposed coefficient would break this)
    fine = np.array([O.fast_exp32(v) for v in np.linspace(-2, 2, 4001, dtype=np.float32)])
    assert np.all(np.diff(fine) >= 0)


# ------------------------------------------------------------------ norms --
def _rms_ref64(x, g, eps):
    x64 = x.astype(np.float64)
    inv = 1 / np.sqrt((x64 ** 2).mean(axis=-1, keepdims=True) + eps)
    return x64 * inv * g.astype(np.float64)


def test_rmsnorm_reference_inputs_and_f64():
    """Inputs of cpu/layernorm/compute_test.go:73-90 (index%67-33)/19 and
    1+(index%31-15)/128, rows=2, over parity.Lengths; f32 result within a few ulp
    of the float64 evaluation."""
    for n in (1, 7, 64, 1024, 8192):
        i = np.arange(2 * n)
        x = ((i % 67 - 33) / 19).astype(np.float32).reshape(2, n)
        g = (1 + (np.arange(n) % 31 - 15) / 128).astype(np.float32)
        got = O.rmsnorm(x, g, 1e-5, O.F32)
        ref = _rms_ref64(x, g, 1e-5)
        # sequential f32 sum of squares: error grows ~n*u; a missing eps, mean or
        # scale term would be off by far more
        assert np.max(np.abs(got - ref)) <= 2e-5 * max(1.0, np.max(np.abs(ref)))


def test_rmsnorm_closed_form_constant_row():
    for c in (0.5, -3.0, 1e-3):
        x = np.full((1, 32), c, np.float32)
        g = np.linspace(0.5, 1.5, 32).astype(np.float32)
        got = O.rmsnorm(x, g, 1e-6, O.F32)
        expect = g * (c / math.sqrt(c * c + 1e-6))
        assert np.allclose(got, expect, rtol=2e-7, atol=0)


def test_rmsnorm_bf16_rounds_sum_of_squares():
    """The bf16 dot returns a bf16 (dot/bf16_generic.go:9-21): with 3 ones and a
    value whose square pushes the f32 sum off the bf16 grid, the normaliser must
    use the rounded sum."""
    x = O.from_f32(np.array([[1, 1, 1, 1.0078125]], np.float32), O.BF16)   # sum sq 4.0157 -> bf16 4.03125
    g = O.from_f32(np.ones(4, np.float32), O.BF16)
    got = O.to_f32(O.rmsnorm(x, g, 1e-9, O.BF16), O.BF16)
    # worked by hand: inv = 1/sqrt(4.03125/4) -> [0.99609375]*3 + [1.0]; with the
    # unrounded sum the last element would stay 1.0078125
    assert got.ravel().tolist() == [0.99609375, 0.99609375, 0.99609375, 1.0]


def test_layernorm_closed_forms_and_f64():
    x = np.full((2, 16), 2.5, np.float32)
    g = seeded(1, (16,), 1.0, 0.1)
    b = seeded(2, (16,), 0.0, 0.1)
    assert np.allclose(O.layernorm(x, g, b, O.F32), np.broadcast_to(b, (2, 16)), atol=1e-6)   # constant row -> beta
    x = seeded(3, (5, 33), 1.0, 2.0)
    x64 = x.astype(np.float64)
    mu = x64.mean(-1, keepdims=True)
    ref = (x64 - mu) / np.sqrt(((x64 - mu) ** 2).mean(-1, keepdims=True) + 1e-5) * g[0] + b[0]
    got = O.layernorm(x, np.full(33, g[0], np.float32), np.full(33, b[0], np.float32), O.F32)
    assert np.max(np.abs(got - ref)) < 2e-6
    for dt in (O.BF16, O.F16):
        xb = O.from_f32(x, dt)
        gb = O.from_f32(np.full(33, g[0], np.float32), dt)
        bb = O.from_f32(np.full(33, b[0], np.float32), dt)
        got = O.to_f32(O.layernorm(xb, gb, bb, dt), dt)
        assert np.max(np.abs(got - ref)) < 0.05


def test_gated_residual_reference_kat():
    """execution/math_gated_residual_intrinsic_test.go:13-67."""
    res = np.arange(1, 13, dtype=np.float32).reshape(2, 2, 3)
    br = np.ones_like(res)
    mod = np.array([[0, 0, 0, 0, 0, 0, 0.5, 1, 2], [0, 0, 0, 0, 0, 0, 3, 4, 5]], np.float32)
    got = O.gated_residual(res, br, mod, 2, 0, O.F32)
    assert got.ravel().tolist() == [1.5, 3, 5, 4.5, 6, 8, 10, 12, 14, 13, 15, 17]
    # layout rules: modulation too narrow / rows not divisible -> error
    with pytest.raises(ValueError):
        O.gated_residual(res, br, mod[:, :8], 2, 0, O.F32)
    with pytest.raises(ValueError):
        O.gated_residual(res.reshape(4, 3), br.reshape(4, 3), mod, 3, 0, O.F32)


def test_adaptive_and_modulated_f64():
    x = seeded(9, (4, 24))
    mod = seeded(10, (2, 72), 0.0, 0.3)
    x64, m64 = x.astype(np.float64), mod.astype(np.float64)
    got = O.adaptive_rmsnorm(x, mod, 2, 1e-6, O.F32)
    inv = 1 / np.sqrt((x64 ** 2).mean(-1, keepdims=True) + 1e-6)
    sc = np.repeat(m64[:, :24], 2, 0)
    sh = np.repeat(m64[:, 24:48], 2, 0)
    assert np.max(np.abs(got - (x64 * inv * (1 + sc) + sh))) < 2e-6   # scale first, shift second
    mu = x64.mean(-1, keepdims=True)
    inv = 1 / np.sqrt(((x64 - mu) ** 2).mean(-1, keepdims=True) + 1e-6)
    base = 3 * 24                                                       # set 1: shift at 3H, scale at 4H
    sh = np.repeat(np.concatenate([m64, m64], 1)[:, base:base + 24], 2, 0)
    sc = np.repeat(np.concatenate([m64, m64], 1)[:, base + 24:base + 48], 2, 0)
    # modulation width 72 < (3*1+2)*24 = 120 for set 1 -> the oracle must refuse
    with pytest.raises(ValueError):
        O.modulated_layernorm(x, mod, 2, 1e-6, 1, O.F32)
    mod2 = np.concatenate([mod, mod], 1)   # 144 columns
    got = O.modulated_layernorm(x, mod2, 2, 1e-6, 1, O.F32)
    assert np.max(np.abs(got - ((x64 - mu) * inv * (1 + sc) + sh))) < 2e-6


# ------------------------------------------------------------------- rope --
def _rope64(x, base, start, mode):
    s, h, d = x.shape
    half = d // 2
    out = x.astype(np.float64).copy()
    for p in range(s):
        for i in range(half):
            th = (p + start) * base ** (-(2 * i) / d)
            c, sn = math.cos(th), math.sin(th)
            for hh in range(h):
                ei, oi = (i, i + half) if mode == 1 else (2 * i, 2 * i + 1)
                e, o = x[p, hh, ei], x[p, hh, oi]
                out[p, hh, ei] = e * c - o * sn
                out[p, hh, oi] = e * sn + o * c
    return out


@pytest.mark.parametrize("mode", [0, 1])
def test_rope_f64_and_identity_at_position_zero(mode):
    x = seeded(5, (6, 3, 8))
    got = O.rope(x, base_freq=1e4, start_position=0, mode=mode)
    assert np.array_equal(got[0], x[0])                       # cos 0 = 1, sin 0 = 0
    assert np.max(np.abs(got - _rope64(x, 1e4, 0, mode))) < 1e-5
    got = O.rope(x, base_freq=5e5, start_position=4000, mode=mode)
    assert np.max(np.abs(got - _rope64(x, 5e5, 4000, mode))) < 3e-5
    # rotation keeps each pair's norm
    n_in = np.sqrt(x[..., 0::2] ** 2 + x[..., 1::2] ** 2) if mode == 0 else np.sqrt(x[..., :4] ** 2 + x[..., 4:] ** 2)
    n_out = np.sqrt(got[..., 0::2] ** 2 + got[..., 1::2] ** 2) if mode == 0 else np.sqrt(got[..., :4] ** 2 + got[..., 4:] ** 2)
    assert np.allclose(n_in, n_out, rtol=1e-5)


def test_rope_llama3_scaling_regimes():
    """rope/compute.go:109-126: low-frequency pairs divided by the factor,
    high-frequency pairs untouched; the reference test's config
    (rope/compute_test.go:67-78)."""
    x = seeded(6, (4, 2, 8))
    kw = dict(base_freq=500000.0, start_position=3, mode=1, scaling=1, scaling_factor=32.0,
              low_freq_factor=1.0, high_freq_factor=4.0, original_context=8192)
    got = O.rope(x, **kw)
    d, half = 8, 4
    out = x.astype(np.float64).copy()
    for p in range(4):
        for i in range(half):
            inv = 500000.0 ** (-(2 * i) / d)
            wl = 2 * math.pi / inv
            if wl > 8192 / 1.0:
                inv = inv / 32.0
            elif wl >= 8192 / 4.0:
                sm = (8192 / wl - 1.0) / 3.0
                inv = (1 - sm) * inv / 32.0 + sm * inv
            th = (p + 3) * inv
            for hh in range(2):
                e, o = x[p, hh, i], x[p, hh, i + half]
                out[p, hh, i] = e * math.cos(th) - o * math.sin(th)
                out[p, hh, i + half] = e * math.sin(th) + o * math.cos(th)
    assert np.max(np.abs(got - out)) < 1e-5


def test_multi_axis_rope_text_tokens_match_plain_rope_on_axis0():
    """Text tokens (seq < S - latent) rotate axis 0 by the sequence index and
    leave the other axes at position 0 (rope/compute.go:302-330)."""
    x = seeded(7, (1, 6, 1, 8))
    got = O.multi_axis_rope(x, 1e4, 2, 1, [4, 2, 2], O.F32)
    for s in range(4):   # text tokens
        for i in range(2):
            th = s * 1e4 ** (-2 * i / 4)
            e, o = x[0, s, 0, 2 * i], x[0, s, 0, 2 * i + 1]
            assert abs(got[0, s, 0, 2 * i] - (e * math.cos(th) - o * math.sin(th))) < 1e-5
        assert np.array_equal(got[0, s, 0, 4:], x[0, s, 0, 4:])


# ------------------------------------------------------------ activations --
def test_gated_closed_forms_and_f64():
    g = seeded(8, (4096,), 0.0, 4.0)
    u = seeded(9, (4096,))
    sw = O.gated_tensors(O.GATE_SWIGLU, g, u, O.F32)
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    ref = g64 / (1 + np.exp(-g64)) * u64
    assert np.max(np.abs(sw - ref) / np.maximum(np.abs(ref), 1e-3)) < 3e-4   # FastExp32 error
    assert np.all(O.gated_tensors(O.GATE_SWIGLU, np.zeros(8, np.float32), u[:8], O.F32) == 0)
    ge = O.gated_tensors(O.GATE_GEGLU, g, u, O.F32)
    erf = np.vectorize(math.erf)
    ref = g64 * 0.5 * u64 * (1 + erf(u64 / math.sqrt(2)))                   # gate * gelu(up): asymmetric
    assert np.max(np.abs(ge - ref)) < 1e-5 * np.max(np.abs(ref))
    assert np.all(O.gated_tensors(O.GATE_GEGLU, g[:8], np.zeros(8, np.float32), O.F32) == 0)
    packed = np.concatenate([g.reshape(4, 1024), u.reshape(4, 1024)], 1)
    assert np.array_equal(O.gated_packed(O.GATE_SWIGLU, packed, O.F32), sw.reshape(4, 1024))


# ------------------------------------------------------------------ pages --
def test_page_write_reference_kat_and_chain():
    """execution/page_intrinsic_test.go:15-71 and the write->gather chain."""
    out = O.page_write(np.zeros(12, np.float32), np.array([7, 8], np.float32), np.array([1, 1], np.int32),
                       np.array([0, 1], np.int32), 2, 1, storage_offset=6, page_count=3)
    assert out[8] == 7 and out[9] == 8 and np.count_nonzero(out) == 2
    g = O.page_gather(out, np.array([1], np.int32), 2, 1, 5, storage_offset=6, page_count=3)
    assert g[:2].ravel().tolist() == [7, 8] and np.all(g[2:] == 0)   # rows capped at len(table)*pageSize
    with pytest.raises(ValueError):
        O.page_write(np.zeros(12, np.float32), np.ones(2, np.float32), np.array([3, 0], np.int32),
                     np.array([0, 0], np.int32), 2, 1, storage_offset=6, page_count=3)


def test_page_write_duplicate_slots_keep_the_highest_row():
    """page_generic.go:23-27 copies rows in order, so for every (page, slot) the
    stored row is the highest row index that targets it; slots no row targets
    keep the storage's bytes."""
    rng = np.random.default_rng(11)
    pages, ps, inner, rows = 3, 4, 5, 40          # 12 slots, 40 rows: many duplicates
    ids = rng.integers(0, pages, rows).astype(np.int32)
    offs = rng.integers(0, ps, rows).astype(np.int32)
    vals = rng.standard_normal((rows, inner)).astype(np.float32)
    st = rng.standard_normal(pages * ps * inner).astype(np.float32)
    got = O.page_write(st, vals, ids, offs, ps, inner).reshape(pages, ps, inner)
    winner = {}
    for r in range(rows):
        key = (int(ids[r]), int(offs[r]))
        winner[key] = max(winner.get(key, -1), r)
    base = st.reshape(pages, ps, inner)
    for p in range(pages):
        for s in range(ps):
            want = vals[winner[(p, s)]] if (p, s) in winner else base[p, s]
            assert np.array_equal(got[p, s], want), (p, s)


def test_page_gather_identity_is_copy():
    st = seeded(4, (8 * 4 * 6,))
    assert np.array_equal(O.page_gather(st, np.arange(8, dtype=np.int32), 4, 6, 32).ravel(), st)


# -------------------------------------------------------------- attention --
def test_mha_closed_forms():
    s, h, d = 6, 2, 4
    q = np.zeros((s, h * d), np.float32)          # all scores equal -> mean of visible V rows
    k = seeded(1, (s, h * d))
    v = seeded(2, (s, h * d))
    got = O.mha(q, k, v, h, d, causal=True)
    for i in range(s):
        assert np.allclose(got[i], v[:i + 1].mean(0), atol=1e-6)
    assert np.allclose(got[0], v[0])               # causal row 0 sees key 0 only
    one = O.mha(q[:1], k, v, h, d, causal=True)    # bottom-right alignment: decode sees all keys
    assert np.allclose(one[0], v.mean(0), atol=1e-6)


def test_mha_f64_gqa_window_alibi():
    sq, h, kvh, d = 7, 4, 2, 8
    q, k, v = seeded(3, (sq, h * d)), seeded(4, (sq, kvh * d)), seeded(5, (sq, kvh * d))
    got = O.mha(q, k, v, h, d, causal=True, kv_heads=kvh, window=3, alibi=0.5)
    ref = np.zeros((sq, h * d))
    for hh in range(h):
        kv = hh // (h // kvh)                      # contiguous head groups
        for i in range(sq):
            sc = np.array([q[i, hh * d:(hh + 1) * d].astype(np.float64) @ k[j, kv * d:(kv + 1) * d]
                           for j in range(sq)]) / math.sqrt(d)
            sc = sc + 0.5 * (np.arange(sq) - i)
            sc[np.arange(sq) > i] = -np.inf
            sc[i - np.arange(sq) >= 3] = -np.inf
            p = np.exp(sc - sc.max())
            p /= p.sum()
            ref[i, hh * d:(hh + 1) * d] = p @ v[:, kv * d:(kv + 1) * d]
    assert np.max(np.abs(got - ref)) < 2e-6


def test_mha_bf16_close_to_f64():
    s, h, d = 32, 2, 64
    qf, kf, vf = (seeded(i, (s, h * d), 0.0, 0.125) for i in (6, 7, 8))
    q, k, v = (O.from_f32(a, O.BF16) for a in (qf, kf, vf))
    got = O.to_f32(O.mha(q, k, v, h, d, causal=True, dtype=O.BF16), O.BF16)
    ref = O.mha(O.to_f32(q, O.BF16), O.to_f32(k, O.BF16), O.to_f32(v, O.BF16), h, d, causal=True)
    assert np.max(np.abs(got - ref)) / np.max(np.abs(ref)) < 1e-2


def _flash64(q, k, v, causal):
    """float64 softmax attention of one head, top-left causal (key > row hidden)."""
    sq, d = q.shape
    sk = k.shape[0]
    sc = (q.astype(np.float64) @ k.astype(np.float64).T) * np.float64(np.float32(1.0 / math.sqrt(d)))
    if causal:
        sc[np.arange(sk)[None, :] > np.arange(sq)[:, None]] = -np.inf
    p = np.exp(sc - sc.max(1, keepdims=True))
    return (p / p.sum(1, keepdims=True)) @ v.astype(np.float64)


def test_flash_closed_forms():
    s, d, vd = 6, 4, 3
    q = np.zeros((s, d), np.float32)               # equal scores: FastExp32(0) = 1 exactly
    k, v = seeded(11, (s, d)), seeded(12, (s, vd))
    got = O.flash_attention(q, k, v, causal=True)
    for i in range(s):
        assert np.allclose(got[i], v[:i + 1].mean(0), atol=1e-6)
    assert np.array_equal(got[0], v[0])            # row 0 sees key 0 only
    nc = O.flash_attention(q, k, v, causal=False)
    assert np.allclose(nc, np.broadcast_to(v.mean(0), nc.shape), atol=1e-6)


@pytest.mark.parametrize("sq,sk,causal", [(9, 9, True), (4, 11, True), (11, 4, True), (7, 13, False)])
def test_flash_f64_top_left_causal(sq, sk, causal):
    d, vd = 16, 5                                  # depth != valueDim
    q, k, v = seeded(13, (sq, d)), seeded(14, (sk, d)), seeded(15, (sk, vd))
    got = O.flash_attention(q, k, v, causal=causal)
    ref = _flash64(q, k, v, causal)
    assert np.max(np.abs(got - ref)) < 1e-4 * max(1.0, np.max(np.abs(ref)))  # FastExp32 error
    if causal and sq < sk:                         # bottom-right alignment would differ
        sc = (q.astype(np.float64) @ k.T.astype(np.float64)) / math.sqrt(d)
        sc[np.arange(sk)[None, :] > np.arange(sq)[:, None] + (sk - sq)] = -np.inf
        p = np.exp(sc - sc.max(1, keepdims=True))
        wrong = (p / p.sum(1, keepdims=True)) @ v
        assert np.max(np.abs(got - wrong)) > 1e-2


def test_flash_matches_single_head_mha_and_rounds_bf16_dot():
    s, d = 12, 8
    q, k, v = seeded(16, (s, d)), seeded(17, (s, d)), seeded(18, (s, d))
    a = O.flash_attention(q, k, v, causal=True)
    b = O.mha(q, k, v, 1, d, causal=True)          # independent restatement (f64 exp, 2 passes)
    assert np.max(np.abs(a - b)) < 1e-4
    qb, kb, vb = (O.from_f32(x, O.BF16) for x in (q, k, v))
    got = O.to_f32(O.flash_attention(qb, kb, vb, causal=False, dtype=O.BF16), O.BF16)
    qf, kf, vf = (O.to_f32(x, O.BF16).astype(np.float64) for x in (qb, kb, vb))
    dots = O.to_f32(O.from_f32((qf @ kf.T).astype(np.float32), O.BF16), O.BF16)  # dot -> bf16
    sc = dots.astype(np.float64) * np.float64(np.float32(1.0 / math.sqrt(d)))
    p = np.exp(sc - sc.max(1, keepdims=True))
    ref = (p / p.sum(1, keepdims=True)) @ vf
    assert np.max(np.abs(got - ref)) < 1e-2 * np.max(np.abs(ref))


@pytest.mark.parametrize("dt", [O.BF16, O.F16])
def test_paged_decode_matches_gather_then_mha(dt):
    rng = np.random.default_rng(3)
    ps, h, kvh, d = 4, 4, 2, 8
    pages = 10
    kp = O.from_f32(seeded(1, (pages, ps, kvh, d)), dt)
    vp = O.from_f32(seeded(2, (pages, ps, kvh, d)), dt)
    table = rng.permutation(pages)[:6].reshape(2, 3).astype(np.int32)
    ctx = np.array([9, 12], np.int32)
    q = O.from_f32(seeded(3, (2, h * d)), dt)
    got = O.paged_decode(q, kp, vp, table, ctx, ps, h, kvh, d, dt)
    for b in range(2):
        kk = O.page_gather(kp.reshape(-1), table[b], ps, kvh * d, int(ctx[b]))
        vv = O.page_gather(vp.reshape(-1), table[b], ps, kvh * d, int(ctx[b]))
        ref = O.mha(q[b:b + 1], kk, vv, h, d, causal=True, kv_heads=kvh, dtype=dt)
        assert np.array_equal(got[b], ref[0])


def test_matmul_f64():
    a, b = seeded(1, (9, 17)), seeded(2, (17, 5))
    assert np.max(np.abs(O.matmul_f32(a, b) - a.astype(np.float64) @ b)) < 1e-5


# ------------------------------------------------ fp8 quantising page write --
def _write_fp8_one(values_f32, scales, head_dim):
    """One row, one page of one slot: returns the written bytes."""
    kvh = len(scales)
    storage = np.zeros(kvh * head_dim, np.uint8)
    return O.page_write_fp8(storage, np.asarray(values_f32, np.float32).reshape(1, -1),
                            np.array([0], np.int32), np.array([0], np.int32), 1, kvh, head_dim,
                            np.asarray(scales, np.float32), O.F32)


def test_page_write_fp8_grid_points_are_exact():
    """x = e4m3 value * 2^k with scale 2^k quantises to exactly that code."""
    codes = np.array([0x00, 0x01, 0x08, 0x38, 0x39, 0x7E, 0x80, 0xB8, 0xFE], np.uint8)
    vals = O.to_f32(codes, O.F8E4M3)
    got = _write_fp8_one(vals * 0.25, [0.25], codes.size)
    assert np.array_equal(got, codes)


def test_page_write_fp8_saturates_and_selects_head_scale():
    """|x / s| beyond 448 stores the largest finite code (0x7E / 0xFE); head h of a
    row uses scales[h] (element / head_dim)."""
    got = _write_fp8_one([1e6, -1e6, 448.0 * 3.0, 1.0], [1.0, 3.0], 2)
    assert list(got) == [0x7E, 0xFE, 0x7E, 0x2B]   # 1/3 -> 0.34375 = 0x2B (RNE: 0.25 + 2.67 steps of 2^-5)


def test_page_write_fp8_divides_rather_than_multiplying_by_reciprocal():
    """0.341796875 / 7 = 0.048828125 exactly: the tie between codes 0x14 (0.046875)
    and 0x15 (0.05078125), which RNE sends to the even 0x14.  The product with
    f32(1/7) lands just above the tie and would give 0x15."""
    x, s = np.float32(0.341796875), np.float32(7.0)
    assert x / s == np.float32(0.048828125)
    assert x * (np.float32(1.0) / s) > np.float32(0.048828125)
    assert list(_write_fp8_one([x], [s], 1)) == [0x14]
