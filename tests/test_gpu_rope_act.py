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


def test_multi_axis_rope(backend):
    import puter_amd
    for dt in (O.F32, O.BF16):
        x = encode(seeded(31, (2, 20, 3, 16)), dt)
        ref = decode(O.multi_axis_rope(x, 1e4, 12, 4, [4, 6, 6], dt), dt)
        out = empty_dev(x.shape, NP[dt])
        cfg = puter_amd.MultiAxisRoPEConfig(1e4, 12, 4, 3, 4, 6, 6, 0)
        backend.MultiAxisRoPE(cfg, to_dev(x), out, 2, 20, 3, 16, dt)
        assert_close(decode(to_host(out, NP[dt]), dt), ref, TOL[dt], what="multi-axis")


GATES = ["SwiGLU", "GeGLU", "GeGLUTanh", "SiGLU", "GLU", "ReGLU", "LinGLU"]


@pytest.mark.parametrize("dt", [O.F32, O.BF16, O.F16])
@pytest.mark.parametrize("kind", range(7))
@pytest.mark.parametrize("count", [1, 13, 4096, 14336 * 3 + 5])
def test_gated_tensors(backend, dt, kind, count):
    g = encode(seeded(40 + count + kind, (count,), 0.0, 3.0), dt)
    u = encode(seeded(41 + count, (count,)), dt)
    ref = O.gated_tensors(kind, g, u, dt)
    out = empty_dev((count,), NP[dt])
    getattr(backend, GATES[kind] + "Tensors")(out, to_dev(g), to_dev(u), count, dt)
    got = to_host(out, NP[dt])
    if kind in (0, 3, 4, 5, 6):
        # FastExp32 / IEEE division evaluated op by op: identical to the oracle
        assert np.array_equal(got.view(np.uint32) if dt == O.F32 else got,
                              ref.view(np.uint32) if dt == O.F32 else ref), GATES[kind]
    else:
        assert_close(decode(got, dt), decode(ref, dt), TOL[dt], what=GATES[kind])


@pytest.mark.parametrize("dt", [O.F32, O.BF16])
@pytest.mark.parametrize("kind", [0, 1])
def test_gated_packed(backend, dt, kind):
    batch, half = 6, 1024
    p = encode(seeded(50 + kind, (batch, 2 * half)), dt)
    ref = decode(O.gated_packed(kind, p, dt), dt)
    out = empty_dev((batch, half), NP[dt])
    getattr(backend, GATES[kind])(out, to_dev(p), batch, half, dt)
    assert_close(decode(to_host(out, NP[dt]), dt), ref, TOL[dt], what="packed")


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


@pytest.mark.parametrize("dt", [O.F32, O.BF16])
def test_unary_silu_gelu(backend, dt):
    x = encode(seeded(60, (5000,), 0.0, 4.0), dt)
    for kind, name in ((O.UNARY_SILU, "Silu"), (O.UNARY_GELU, "Gelu")):
        ref = decode(O.unary(kind, x, dt), dt)
        out = empty_dev(x.shape, NP[dt])
        getattr(backend, name)(out, to_dev(x), x.size, dt)
        assert_close(decode(to_host(out, NP[dt]), dt), ref, TOL[dt], what=name)
