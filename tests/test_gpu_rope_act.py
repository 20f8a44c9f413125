"""GPU parity: RoPE / MultiAxisRoPE and the gated activations against the CPU
oracle (device/cpu/rope/compute.go, device/cpu/activation/gated.go)."""
import numpy as np
import pytest

import oracle as O
from helpers import TOL, assert_close, decode, empty_dev, encode, seeded, to_dev, to_host

pytestmark = pytest.mark.gpu
NP = {O.F32: np.float32, O.F16: np.uint16, O.BF16: np.uint16}


@pytest.mark.parametrize("dt", [O.F32, O.BF16, O.F16])
@pytest.mark.parametrize("seq,heads,dim,base,mode,start", [
    (128, 8, 64, 1e4, 0, 0),        # config 1 shape (interleaved default)
    (256, 32, 128, 5e5, 0, 0),      # config 3 Q, first 256 positions
    (300, 8, 128, 5e5, 0, 7900),    # config 3 K tail positions
    (64, 4, 128, 5e5, 1, 3),        # half mode
    (9, 3, 10, 1e4, 0, 0),          # ragged: scalar path
    (5, 2, 12, 1e4, 1, 0),
])
def test_rope(backend, dt, seq, heads, dim, base, mode, start):
    import puter_amd
    x = encode(seeded(11 + seq + dim, (seq, heads, dim)), dt)
    ref = decode(O.rope(x, base_freq=base, start_position=start, mode=mode, dtype=dt), dt)
    out = empty_dev(x.shape, NP[dt])
    cfg = puter_amd.RoPEConfig(BaseFreq=base, StartPosition=start, Mode=mode)
    backend.RoPE(cfg, to_dev(x), out, seq, heads, dim, dt)
    assert_close(decode(to_host(out, NP[dt]), dt), ref, TOL[dt], what="rope")


def test_rope_llama3_in_place(backend):
    import puter_amd
    dt = O.F32
    x = seeded(5, (64, 4, 128))
    kw = dict(base_freq=5e5, start_position=8000, mode=1, scaling=1, scaling_factor=8.0,
              low_freq_factor=1.0, high_freq_factor=4.0, original_context=8192)
    ref = O.rope(x, dtype=dt, **kw)
    t = to_dev(x)
    cfg = puter_amd.RoPEConfig(5e5, 8000, 1, 1, 8.0, 1.0, 4.0, 8192)
    backend.RoPE(cfg, t, t, 64, 4, 128, dt)   # input == output
    assert_close(to_host(t, np.float32), ref, TOL[dt], what="rope llama3")


@pytest.mark.parametrize("dt", [O.F32, O.BF16, O.F16])
@pytest.mark.parametrize("b,s,h,base,latent,side,dims", [
    (2, 20, 3, 1e4, 12, 4, [4, 6, 6]),            # 3 axes, 3x4 image grid after 8 text tokens
    (2, 23, 3, 1e4, 15, 6, [2, 6, 4, 4]),          # 4 axes: text on axis 3, ragged last image row
    (1, 5, 2, 1e4, 12, 4, [4, 4, 8]),              # every token an image token
    (1, 640, 4, 1e4, 512, 32, [32, 32, 32, 32]),   # multi_axis_test.go:48-60 scaled down
])
def test_multi_axis_rope(backend, dt, b, s, h, base, latent, side, dims):
    import puter_amd
    d = sum(dims)
    x = encode(seeded(31 + s, (b, s, h, d)), dt)
    ref = decode(O.multi_axis_rope(x, base, latent, side, dims, dt), dt)
    out = empty_dev(x.shape, NP[dt])
    cfg = puter_amd.MultiAxisRoPEConfig(base, latent, side, len(dims), *(list(dims) + [0] * (4 - len(dims))))
    backend.MultiAxisRoPE(cfg, to_dev(x), out, b, s, h, d, dt)
    assert_close(decode(to_host(out, NP[dt]), dt), ref, TOL[dt], what="multi-axis")


GATES = ["SwiGLU", "GeGLU", "GeGLUTanh", "SiGLU", "GLU", "ReGLU", "LinGLU", "SeGLU"]


# kinds whose arithmetic the kernel evaluates operation by operation as the oracle
# does (FastExp32, IEEE division and products), so every dtype is bit-exact
BIT_EXACT_KINDS = (0, 3, 4, 5, 6, 7)


def _same(got, ref, dt):
    return np.array_equal(got.view(np.uint32) if dt == O.F32 else got,
                          ref.view(np.uint32) if dt == O.F32 else ref)


@pytest.mark.parametrize("dt", [O.F32, O.BF16, O.F16])
@pytest.mark.parametrize("kind", range(len(GATES)))
@pytest.mark.parametrize("count", [1, 13, 4096, 14336 * 3 + 5])
def test_gated_tensors(backend, dt, kind, count):
    g = encode(seeded(40 + count + kind, (count,), 0.0, 3.0), dt)
    u = encode(seeded(41 + count, (count,)), dt)
    ref = O.gated_tensors(kind, g, u, dt)
    out = empty_dev((count,), NP[dt])
    getattr(backend, GATES[kind] + "Tensors")(out, to_dev(g), to_dev(u), count, dt)
    got = to_host(out, NP[dt])
    if kind in BIT_EXACT_KINDS:
        assert _same(got, ref, dt), GATES[kind]
    else:
        assert_close(decode(got, dt), decode(ref, dt), TOL[dt], what=GATES[kind])


@pytest.mark.parametrize("dt", [O.F32, O.BF16, O.F16])
@pytest.mark.parametrize("kind", range(len(GATES)))
@pytest.mark.parametrize("batch,half", [(6, 1024), (3, 37)])
def test_gated_packed(backend, dt, kind, batch, half):
    """Packed rows [gate | up] (half 1024: the 16-byte vector path; half 37: the
    element path, rows not vector-aligned)."""
    p = encode(seeded(50 + kind + half, (batch, 2 * half), 0.0, 2.0), dt)
    ref = O.gated_packed(kind, p, dt)
    out = empty_dev((batch, half), NP[dt])
    getattr(backend, GATES[kind])(out, to_dev(p), batch, half, dt)
    got = to_host(out, NP[dt])
    if kind in BIT_EXACT_KINDS:
        assert _same(got, ref, dt), GATES[kind]
    else:
        assert_close(decode(got, dt), decode(ref, dt), TOL[dt], what="packed " + GATES[kind])


def test_fast_exp_edges_through_swiglu(backend):
    # gate values around FastExp32's clamps (-87.33654, 88.72283) and the k-- branch
    g = np.array([-100, -88.72283, -88.7, -87.34, 0, -0.0, 1e-30, 87.3, 87.34, 100, -3.0, 3.0,
                  np.inf, -np.inf], np.float32)
    u = np.ones_like(g)
    ref = O.gated_tensors(0, g, u, O.F32)
    out = empty_dev(g.shape, np.float32)
    backend.SwiGLUTensors(out, to_dev(g), to_dev(u), g.size, O.F32)
    got = to_host(out, np.float32)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (got, ref)


@pytest.mark.parametrize("dt", [O.F32, O.BF16, O.F16])
def test_unary_silu_gelu(backend, dt):
    """f32: FastSilu32 bit-exact, FastGelu32 (float64 erf) to the f32 bar.
    f16 / bf16: every one of the 65536 input patterns, as the reference's
    tables hold them: Silu = narrow(float32(FastSilu64(x))) bit-exact; Gelu's
    float64 erf (the device library's vs libm's) may differ in the last f64
    bits, so at most one 16-bit step on a handful of inputs."""
    if dt == O.F32:
        x = encode(seeded(60, (5000,), 0.0, 4.0), dt)
    else:
        x = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    for kind, name in ((O.UNARY_SILU, "Silu"), (O.UNARY_GELU, "Gelu")):
        ref = O.unary(kind, x, dt)
        out = empty_dev(x.shape, NP[dt])
        getattr(backend, name)(out, to_dev(x), x.size, dt)
        got = to_host(out, NP[dt])
        if dt == O.F32:
            if kind == O.UNARY_SILU:
                assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), name
            else:
                assert_close(got, ref, TOL[dt], what=name)
            continue
        fin = ~np.isnan(decode(ref, dt))
        nan_ok = np.array_equal(np.isnan(decode(got, dt)), np.isnan(decode(ref, dt)))
        assert nan_ok, name
        if kind == O.UNARY_SILU:
            assert np.array_equal(got[fin], ref[fin]), name
        else:
            steps = np.abs(got[fin].astype(np.int64) - ref[fin].astype(np.int64))
            assert np.max(steps) <= 1 and np.count_nonzero(steps) <= 16, (name, np.count_nonzero(steps))


@pytest.mark.parametrize("half", [1, 7, 64, 1024, 8192, 4097])
def test_rope_pairs(backend, half):
    """RoPEPairs (device/interface.go:605-609), f32, bit-exact against the oracle's
    RopePairsGeneric restatement (parity.Lengths of the reference's pair tests)."""
    x = seeded(70 + half, (2 * half,))
    ang = seeded(71 + half, (half,), 0.0, 3.0).astype(np.float64)
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    ref = O.rope_pairs(x, cos, sin)
    out = empty_dev((2 * half,), np.float32)
    backend.RoPEPairs(out, to_dev(x), to_dev(cos), to_dev(sin), half, O.F32)
    assert np.array_equal(to_host(out, np.float32).view(np.uint32), ref.view(np.uint32))
    # unaligned views take the element-wise path
    xd, cd, sd = to_dev(np.concatenate([[0.0], x]).astype(np.float32)), to_dev(cos), to_dev(sin)
    out2 = empty_dev((2 * half + 1,), np.float32)
    backend.RoPEPairs(out2[1:], xd[1:], cd, sd, half, O.F32)
    assert np.array_equal(to_host(out2, np.float32)[1:].view(np.uint32), ref.view(np.uint32))


def test_rope_pairs_rejects_16bit(backend):
    import puter_amd
    x = empty_dev((8,), np.uint16)
    c = empty_dev((4,), np.float32)
    with pytest.raises(puter_amd.PuterError):
        backend.RoPEPairs(x, x, c, c, 4, O.BF16)   # rope/ops.go:10-14 panics for non-f32
