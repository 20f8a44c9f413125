"""CPU tier: pins for the oracle functions the other pin files leave open.

* ReGLU, LinGLU and SeGLU (device/cpu/math/activation.go:26-32,298-300,
  math/extra_activation.go:84-90) against numpy closed forms on asymmetric
  gate / up values, so that a relu applied to the gate, swapped operands or a
  sigmoid of the wrong operand fails.
* The fp8-E4M3 branch of the paged-decode oracle against torch's E4M3 decode,
  float64 softmax attention and distinct per-head K and V scales, so that
  swapped scale roles or a wrong kv-head index fail.
* Matmul in F64, BF16 and F16 (device/cpu/matmul/compute.go:46-92) against
  exact sums (math.fsum) and constructed sums that only a single rounding of
  the f32 total reproduces.
* The f16 MultiHeadAttention's score dot rounded to f16
  (device/cpu/attention/typed_compute.go:10-29) against a numpy emulation on
  inputs whose dots are exact in f32, so only the f16 rounding separates the
  two candidate answers.
"""
import math

import numpy as np
import pytest
import torch

import oracle as O
from helpers import seeded


def _bf16_torch(x32):
    """bf16 RNE narrowing by torch (a library, not the oracle)."""
    return torch.from_numpy(np.ascontiguousarray(x32, np.float32)).to(torch.bfloat16).view(torch.int16) \
        .numpy().view(np.uint16)


def _bf16_widen(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32)


# ------------------------------------------------------- ReGLU / LinGLU / SeGLU --
G = np.array([-2.0, 3.0, -1.5, 0.5, 2.0, -0.75, 4.0, 1.25, -3.5, 0.0], np.float32)
U = np.array([1.5, -2.0, -0.25, 4.0, 0.0, 2.5, -0.0, -1.0, 3.0, -2.0], np.float32)


def test_reglu_relu_acts_on_up_not_gate():
    """FastReGLU32(gate, up) = gate * FastReLU32(up), FastReLU32(v) = v if v > 0 else +0."""
    got = O.gated_tensors(O.GATE_REGLU, G, U, O.F32)
    ref = G * np.where(U > 0, U, np.float32(0.0)).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    # a relu on the gate instead gives a different answer at (-2, 1.5) and (0.5, 4) ...
    wrong = np.where(G > 0, G, np.float32(0.0)) * U
    assert not np.array_equal(got, wrong)
    assert got[0] == -3.0 and got[1] == 0.0 and got[3] == 2.0
    # ... and the sign of a zero product follows the gate: -1.5 * relu(-0.25) = -0
    assert np.signbit(got[2]) and not np.signbit(got[1])
    # NaN up: NaN > 0 is false, so relu gives 0 and the product is gate * 0
    nan = O.gated_tensors(O.GATE_REGLU, np.array([2.0, -2.0], np.float32),
                          np.array([np.nan, np.nan], np.float32), O.F32)
    assert nan[0] == 0.0 and not np.signbit(nan[0]) and np.signbit(nan[1])


def test_linglu_is_the_plain_product():
    """FastLinGLU32(gate, up) = gate * up: one f32 rounding."""
    g, u = seeded(61, (4096,), 0.0, 3.0), seeded(62, (4096,))
    got = O.gated_tensors(O.GATE_LINGLU, g, u, O.F32)
    assert np.array_equal(got.view(np.uint32), (g * u).view(np.uint32))
    assert np.array_equal(O.gated_tensors(O.GATE_LINGLU, G, U, O.F32), G * U)


def test_seglu_is_up_times_sigmoid_of_gate():
    """FastSeGLU32(gate, up) = up * FastSigmoid32(gate): the sigmoid takes the gate
    (within FastExp32's error of float64), and the f32 product commutes, so the
    result is SiGLU's bit for bit."""
    g, u = seeded(63, (4096,), 0.0, 4.0), seeded(64, (4096,))
    se = O.gated_tensors(O.GATE_SEGLU, g, u, O.F32)
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    ref = u64 / (1 + np.exp(-g64))
    assert np.max(np.abs(se - ref) / np.maximum(np.abs(ref), 1e-3)) < 3e-4
    wrong = g64 / (1 + np.exp(-u64))                 # sigmoid of up times gate
    assert np.max(np.abs(se - wrong)) > 0.5
    assert np.array_equal(se.view(np.uint32), O.gated_tensors(O.GATE_SIGLU, g, u, O.F32).view(np.uint32))


@pytest.mark.parametrize("kind", [O.GATE_REGLU, O.GATE_LINGLU, O.GATE_SEGLU])
def test_16bit_gates_widen_combine_narrow(kind):
    """16-bit forms (activation/compute.go:17-36,148-176): widen, combine in f32,
    narrow once; bf16 checked against torch's narrowing, f16 against numpy's."""
    g32, u32 = seeded(65, (2048,), 0.0, 3.0), seeded(66, (2048,))
    for dt in (O.BF16, O.F16):
        if dt == O.BF16:
            gb, ub = _bf16_torch(g32), _bf16_torch(u32)
            gw, uw = _bf16_widen(gb), _bf16_widen(ub)
        else:
            gb, ub = g32.astype(np.float16).view(np.uint16), u32.astype(np.float16).view(np.uint16)
            gw, uw = gb.view(np.float16).astype(np.float32), ub.view(np.float16).astype(np.float32)
        f32 = O.gated_tensors(kind, gw, uw, O.F32)   # the f32 combine, pinned above
        ref = _bf16_torch(f32) if dt == O.BF16 else f32.astype(np.float16).view(np.uint16)
        got = O.gated_tensors(kind, gb, ub, dt)
        assert np.array_equal(got, ref), (kind, dt)
        packed = np.concatenate([gb.reshape(2, 1024), ub.reshape(2, 1024)], 1)
        assert np.array_equal(O.gated_packed(kind, packed, dt), ref.reshape(2, 1024))


# --------------------------------------------------- fp8 paged-decode oracle --
def _e4m3_torch(codes):
    return torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()


def _paged_fp8_f64(q_bits, kp, vp, table, ctx, ps, h, kvh, d, k_scale, v_scale, head_of=None):
    """float64 attention over torch-decoded E4M3 rows times the per-head scales."""
    head_of = head_of or (lambda hh: hh // (h // kvh))
    kf = _e4m3_torch(kp).reshape(-1, ps, kvh, d).astype(np.float64)
    vf = _e4m3_torch(vp).reshape(-1, ps, kvh, d).astype(np.float64)
    q = _bf16_widen(q_bits).astype(np.float64).reshape(len(ctx), h, d)
    out = np.zeros((len(ctx), h, d))
    for b, n in enumerate(ctx):
        slots = [(table[b, r // ps], r % ps) for r in range(n)]
        for hh in range(h):
            g = head_of(hh)
            kk = np.array([kf[p, s, g] for p, s in slots]) * np.float64(k_scale[g])
            vv = np.array([vf[p, s, g] for p, s in slots]) * np.float64(v_scale[g])
            sc = kk @ q[b, hh] / math.sqrt(d)
            p = np.exp(sc - sc.max())
            out[b, hh] = (p / p.sum()) @ vv
    return out.reshape(len(ctx), h * d)


def test_paged_decode_fp8_branch_scales_and_heads():
    rng = np.random.default_rng(71)
    ps, h, kvh, d, pages = 4, 6, 3, 8, 14
    kp = rng.integers(0, 256, pages * ps * kvh * d, dtype=np.uint8)
    vp = rng.integers(0, 256, pages * ps * kvh * d, dtype=np.uint8)
    for c in (kp, vp):
        c[(c & 0x7F) == 0x7F] = 0x3A                  # no NaN codes
        c[(c & 0x78) >= 0x60] &= 0xBF                 # keep magnitudes moderate (|x| < 16)
    table = rng.permutation(pages)[:12].reshape(3, 4).astype(np.int32)
    ctx = np.array([5, 16, 11], np.int32)
    k_scale = np.array([0.05, 0.2, 0.11], np.float32)   # distinct per head and per role
    v_scale = np.array([1.5, 0.25, 3.0], np.float32)
    q = _bf16_torch(seeded(72, (3, h * d)))
    got = _bf16_widen(O.paged_decode(q, kp, vp, table, ctx, ps, h, kvh, d, O.F8E4M3, k_scale, v_scale))
    ref = _paged_fp8_f64(q, kp, vp, table, ctx, ps, h, kvh, d, k_scale, v_scale)
    tol = 2.0 ** -8 * np.abs(ref) + 1e-5 * np.max(np.abs(ref))   # one bf16 rounding of the output
    assert np.all(np.abs(got - ref) <= tol)
    # the check separates the plausible mistakes
    for wrong in (_paged_fp8_f64(q, kp, vp, table, ctx, ps, h, kvh, d, v_scale, k_scale),
                  _paged_fp8_f64(q, kp, vp, table, ctx, ps, h, kvh, d, k_scale, v_scale,
                                 head_of=lambda hh: hh % kvh),
                  _paged_fp8_f64(q, kp, vp, table, ctx, ps, h, kvh, d, k_scale[::-1].copy(), v_scale)):
        assert np.max(np.abs(got - wrong)) > 20 * np.max(tol)


def test_paged_decode_fp8_one_key_returns_the_scaled_value_row():
    """With one visible key the softmax weight is exactly 1: the output is the
    decoded V row times its head's scale, narrowed to bf16."""
    ps, h, kvh, d = 2, 4, 2, 8
    codes = np.arange(2 * ps * kvh * d, dtype=np.uint8) % 0x70
    table = np.array([[1, 0]], np.int32)
    v_scale = np.array([0.5, 3.0], np.float32)
    q = _bf16_torch(seeded(73, (1, h * d)))
    got = O.paged_decode(q, codes, codes, table, np.array([1], np.int32), ps, h, kvh, d, O.F8E4M3,
                         np.array([1.0, 2.0], np.float32), v_scale)
    row = _e4m3_torch(codes).reshape(2, ps, kvh, d)[1, 0]          # page 1, slot 0
    ref = np.concatenate([row[hh // 2] * v_scale[hh // 2] for hh in range(h)]).astype(np.float32)
    assert np.array_equal(got[0], _bf16_torch(ref))


# ----------------------------------------------------------------- Matmul --
def _fsum_matmul(a, b):
    return np.array([[math.fsum(float(x) * float(y) for x, y in zip(a[r], b[:, c]))
                      for c in range(b.shape[1])] for r in range(a.shape[0])])


def test_matmul_f64_against_exact_sums():
    a = seeded(74, (7, 19)).astype(np.float64) * 3.0
    b = seeded(75, (19, 5)).astype(np.float64)
    a += np.arange(7)[:, None] * 0.125                 # asymmetric rows / columns
    got = O.matmul(a, b, O.F64)
    exact = _fsum_matmul(a, b)
    bound = 19 * 2.0 ** -53 * (np.abs(a) @ np.abs(b))  # sequential f64 summation bound
    assert np.all(np.abs(got - exact) <= bound)
    assert got.shape == (7, 5)
    assert np.max(np.abs(got - _fsum_matmul(a[:, ::-1].copy(), b))) > 1.0  # operand order matters
    # f64 keeps what f32 rounds away: 1 + 2^-30 survives
    one = O.matmul(np.array([[1.0, 2.0 ** -30]]), np.array([[1.0], [1.0]]), O.F64)
    assert one[0, 0] == 1.0 + 2.0 ** -30


@pytest.mark.parametrize("dt", [O.BF16, O.F16])
def test_matmul_16bit_sums_in_f32_and_rounds_once(dt):
    """runMatmulReducedCols (compute.go:74-92): widened operands summed in f32, the
    total stored once.  Sixteen addends of half an ulp of 1 after a 1 reach
    1 + 16 half-ulps exactly; rounding each partial to the 16-bit format would
    leave 1 (every tie goes to the even 1)."""
    half_ulp = 2.0 ** -9 if dt == O.BF16 else 2.0 ** -11
    enc = (lambda x: _bf16_torch(np.asarray(x, np.float32))) if dt == O.BF16 else \
        (lambda x: np.asarray(x, np.float32).astype(np.float16).view(np.uint16))
    dec = _bf16_widen if dt == O.BF16 else (lambda bits: bits.view(np.float16).astype(np.float32))
    left = enc(np.array([[1.0] + [half_ulp] * 16]))
    right = enc(np.ones((17, 1)))
    got = dec(O.matmul(left, right, dt))
    assert got[0, 0] == 1.0 + 16 * half_ulp
    # random operands: the exact sum of the widened operands, then one rounding
    a32, b32 = seeded(76, (9, 33)), seeded(77, (33, 6), 0.0, 0.5)
    a, b = enc(a32), enc(b32)
    aw, bw = dec(a).astype(np.float64), dec(b).astype(np.float64)
    exact = _fsum_matmul(aw, bw)
    got = dec(O.matmul(a, b, dt)).astype(np.float64)
    ulp = 2.0 ** -8 if dt == O.BF16 else 2.0 ** -11
    bound = ulp * np.abs(exact) + 33 * 2.0 ** -24 * (np.abs(aw) @ np.abs(bw))
    assert np.all(np.abs(got - exact) <= bound)
    assert np.max(np.abs(got - _fsum_matmul(aw, bw[::-1].copy()))) > 0.1


# ------------------------------------------------- f16 MHA score-dot rounding --
def _mha64(q, k, v, h, kvh, d, dot_round, causal):
    sq, sk = q.shape[0], k.shape[0]
    out = np.zeros((sq, h * d))
    for hh in range(h):
        g = hh // (h // kvh)
        dots = q[:, hh * d:(hh + 1) * d] @ k[:, g * d:(g + 1) * d].T        # exact (see below)
        sc = dot_round(dots) * np.float64(np.float32(1.0 / math.sqrt(d)))
        if causal:
            sc[np.arange(sk)[None, :] > np.arange(sq)[:, None] + (sk - sq)] = -np.inf
        p = np.exp(sc - sc.max(1, keepdims=True))
        out[:, hh * d:(hh + 1) * d] = (p / p.sum(1, keepdims=True)) @ v[:, g * d:(g + 1) * d]
    return out


def test_mha_f16_rounds_each_score_dot_to_f16():
    """typedRowDot (typed_compute.go:10-29) rounds the f16 dot to f16 before the
    scale.  Q holds multiples of 1/4 near 2, K multiples of 1/4 near 30: every dot
    is a multiple of 1/16 near 960, exact in f32 in any order, where f16's spacing
    is 0.5, so the rounding moves scores by up to 1/16 (scale 1/4) while keys differ
    by about 2: the rounded and unrounded answers are far apart, and only the
    rounded one is within the output's f16 rounding."""
    rng = np.random.default_rng(78)
    sq, sk, h, kvh, d = 4, 12, 4, 2, 16
    q = (2.0 + rng.integers(-2, 3, (sq, h * d)) * 0.25).astype(np.float16)
    k = (30.0 + rng.integers(-8, 9, (sk, kvh * d)) * 0.25).astype(np.float16)
    v = rng.standard_normal((sk, kvh * d)).astype(np.float16)
    got = O.mha(q.view(np.uint16), k.view(np.uint16), v.view(np.uint16), h, d, causal=True,
                kv_heads=kvh, dtype=O.F16).view(np.float16).astype(np.float64)
    q64, k64, v64 = (x.astype(np.float64) for x in (q, k, v))
    rounded = _mha64(q64, k64, v64, h, kvh, d, lambda x: x.astype(np.float16).astype(np.float64), True)
    plain = _mha64(q64, k64, v64, h, kvh, d, lambda x: x, True)
    tol = 2.0 ** -10 * np.abs(rounded) + 1e-4
    assert np.all(np.abs(got - rounded) <= tol)
    assert np.max(np.abs(got - plain)) > 10 * np.max(tol)
