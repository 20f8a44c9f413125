"""GPU tier: kernels looked up in the registry mirror run on the device and
match the oracle; workspace slots (execution/workspace_resident.go:12-20) carry
views that kernels read and write in place."""
import numpy as np
import pytest

import oracle as O
from helpers import TOL, assert_close, seeded, to_dev, to_host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def reg(backend):
    from puter_amd import registry as R
    return R, R.register_hip_kernels(R.Registry(), backend)


def _lookup(reg, name, inputs, outputs):
    R, r = reg
    k, ok = r.LookupLocation(name, R.Signature(R.LAYOUT_DENSE, tuple(inputs), tuple(outputs)), R.LOCATION_DEVICE)
    assert ok, name
    return k.Run


def test_registry_page_write_gather_bf16(backend, reg):
    import torch
    R = reg[0]
    pages, ps, kvh, d = 12, 16, 2, 64
    rng = np.random.default_rng(1)
    storage = O.from_f32(seeded(2, (pages, ps, kvh, d)), O.BF16)
    vals = O.from_f32(seeded(3, (20, kvh, d)), O.BF16)
    ids = rng.integers(0, pages, 20).astype(np.int32)
    offs = rng.integers(0, ps, 20).astype(np.int32)
    st = to_dev(storage).view(torch.bfloat16)
    _lookup(reg, "page_write", [R.BF16, R.BF16, R.I32, R.I32, R.I32], [R.BF16])(
        st, to_dev(vals).view(torch.bfloat16), to_dev(ids), to_dev(offs),
        torch.tensor([ps], dtype=torch.int32), st)
    ref = O.page_write(storage.ravel(), vals.ravel(), ids, offs, ps, kvh * d)
    assert np.array_equal(to_host(st.view(torch.int16), np.uint16).ravel(), ref)
    table = rng.permutation(pages)[:5].astype(np.int32)
    out = torch.empty((5 * ps - 3, kvh, d), dtype=torch.bfloat16, device="cuda")
    _lookup(reg, "page_gather", [R.BF16, R.I32, R.I32], [R.BF16])(st, to_dev(table), ps, out)
    want = O.page_gather(ref, table, ps, kvh * d, 5 * ps - 3)
    assert np.array_equal(to_host(out.view(torch.int16), np.uint16).reshape(want.shape), want)
    backend.CheckStatus()


def test_registry_layernorm_swiglu_cast_matmul(backend, reg):
    import torch
    R = reg[0]
    x = O.from_f32(seeded(4, (6, 256)), O.BF16)
    g = O.from_f32(seeded(5, (256,), 1.0, 0.02), O.BF16)
    b = O.from_f32(seeded(6, (256,), 0.0, 0.02), O.BF16)
    out = torch.empty((6, 256), dtype=torch.bfloat16, device="cuda")
    bf = lambda a: to_dev(a).view(torch.bfloat16)  # noqa: E731
    _lookup(reg, "layernorm", [R.BF16] * 3, [R.BF16])(bf(x), bf(g), bf(b), out)
    assert_close(O.to_f32(to_host(out.view(torch.int16), np.uint16), O.BF16),
                 O.to_f32(O.layernorm(x, g, b, O.BF16), O.BF16), TOL[O.BF16], what="layernorm")
    up = O.from_f32(seeded(7, (6, 256)), O.BF16)
    act = torch.empty_like(out)
    _lookup(reg, "swiglu", [R.BF16, R.BF16], [R.BF16])(bf(x), bf(up), act)
    assert np.array_equal(to_host(act.view(torch.int16), np.uint16),
                          O.gated_tensors(O.GATE_SWIGLU, x, up, O.BF16))
    h = torch.empty((6, 256), dtype=torch.float16, device="cuda")
    _lookup(reg, "cast", [R.BF16], [R.F16])(bf(x), h)
    assert np.array_equal(to_host(h.view(torch.int16), np.uint16).ravel(), O.cast_pair(x.ravel(), O.BF16, O.F16))
    with pytest.raises(Exception):      # convert.ErrLenMismatch
        _lookup(reg, "cast", [R.BF16], [R.F16])(bf(x), h[:3])
    a, w = seeded(8, (128, 512)), seeded(9, (512, 64))
    c = torch.empty((128, 64), dtype=torch.float32, device="cuda")
    _lookup(reg, "matmul", [R.F32, R.F32], [R.F32])(to_dev(a), to_dev(w), c)
    assert_close(to_host(c, np.float32), O.matmul_f32(a, w), TOL[O.F32], elem_tol=1e-3, what="matmul")


@pytest.mark.parametrize("name,kw", [("multi_head_attention", dict(causal=False)),
                                     ("grouped_query_attention", dict(causal=False, kv_heads=2)),
                                     ("sliding_window_attention", dict(causal=True, window=128))])
@pytest.mark.parametrize("dt", [O.F32, O.BF16])
def test_registry_attention_defaults(backend, reg, name, kw, dt):
    """The reference's registered attention names with their default configs
    (8 heads of 64; GQA over 2 kv heads; causal sliding window 128), looked up
    and run on device tensors, against the oracle's MultiHeadAttention."""
    import torch
    R = reg[0]
    rdt = {O.F32: R.F32, O.BF16: R.BF16}[dt]
    tdt = {O.F32: torch.float32, O.BF16: torch.bfloat16}[dt]
    kvh = kw.get("kv_heads", 8)
    sq, sk = 200, 200
    q = O.from_f32(seeded(11, (sq, 8 * 64), 0.0, 0.5), dt)
    k = O.from_f32(seeded(12, (sk, kvh * 64), 0.0, 0.5), dt)
    v = O.from_f32(seeded(13, (sk, kvh * 64)), dt)
    dev = lambda a: to_dev(a).view(tdt)  # noqa: E731
    out = torch.empty((sq, 8 * 64), dtype=tdt, device="cuda")
    _lookup(reg, name, [rdt] * 3, [rdt])(dev(q), dev(k), dev(v), out)
    ref = O.to_f32(O.mha(q, k, v, 8, 64, causal=kw["causal"], kv_heads=kw.get("kv_heads", 0),
                         window=kw.get("window", 0), dtype=dt), dt)
    got = O.to_f32(to_host(out.view(torch.int16) if dt == O.BF16 else out,
                           np.uint16 if dt == O.BF16 else np.float32), dt)
    assert_close(got, ref, TOL[dt], elem_tol=None if dt == O.BF16 else 1e-3, what=name)
    with pytest.raises(Exception):      # a query width other than 8 x 64: ErrShapeMismatch
        _lookup(reg, name, [rdt] * 3, [rdt])(dev(q)[:, :256], dev(k), dev(v), out[:, :256])


def test_registry_flash_attention_and_quant(backend, reg):
    import torch
    R = reg[0]
    q, k, v = seeded(14, (37, 48)), seeded(15, (90, 48)), seeded(16, (90, 24))
    out = torch.empty((37, 24), dtype=torch.float32, device="cuda")
    for name in ("attention", "flash_attention"):
        _lookup(reg, name, [R.F32] * 3, [R.F32])(to_dev(q), to_dev(k), to_dev(v), out)
        assert_close(to_host(out, np.float32), O.flash_attention(q, k, v, causal=False), TOL[O.F32],
                     elem_tol=1e-3, what=name)
    x = (seeded(17, (4097,)) * 60.0).astype(np.float32)
    codes = torch.empty(4097, dtype=torch.int8, device="cuda")
    _lookup(reg, "int8_quant", [R.F32], [R.I8])(to_dev(x), codes)
    want = O.quant_int8(x, 1.0, 0)
    assert np.array_equal(to_host(codes, np.int8), want)
    back = torch.empty(4097, dtype=torch.float32, device="cuda")
    _lookup(reg, "int8_dequant", [R.I8], [R.F32])(codes, back)
    assert np.array_equal(to_host(back, np.float32), O.dequant_int8(want, 1.0, 0))
    packed = np.random.default_rng(18).integers(0, 256, 2049).astype(np.uint8)
    out4 = torch.empty(4097, dtype=torch.float32, device="cuda")
    _lookup(reg, "int4_dequant", [R.I4], [R.F32])(to_dev(packed), out4)
    assert np.array_equal(to_host(out4, np.float32), O.dequant_int4(packed, 4097, 1.0, 0))


def test_workspace_slot_views_stay_resident(backend):
    """AllocateWorkspaceSlot / ViewWorkspaceSlot: one device allocation carved
    into views of other shapes and formats; a fused GatedResidual+RMSNorm reads
    and writes views of the same slot, and the results download intact."""
    import puter_amd
    rows, h = 32, 1024
    nb = rows * h * 2
    slot = backend.AllocateWorkspaceSlot(4 * nb)
    try:
        res = O.from_f32(seeded(10, (rows, h)), O.BF16)
        br = O.from_f32(seeded(11, (rows, h)), O.BF16)
        mod = O.from_f32(seeded(12, (1, 3 * h)), O.BF16)
        g = O.from_f32(seeded(13, (h,), 1.0, 0.02), O.BF16)
        v_res = backend.ViewWorkspaceSlot(slot, [rows, h], puter_amd.BF16, nb)
        backend.Upload(v_res, np.concatenate([res.ravel(), br.ravel()]))      # two planned tensors, back to back
        v_br = puter_amd.DeviceBuffer(backend.lib, slot.ptr + nb, [rows, h], puter_amd.BF16, nb, False)
        v_hid = puter_amd.DeviceBuffer(backend.lib, slot.ptr + 2 * nb, [rows, h], puter_amd.BF16, nb, False)
        v_out = puter_amd.DeviceBuffer(backend.lib, slot.ptr + 3 * nb, [rows, h], puter_amd.BF16, nb, False)
        dm, dg = to_dev(mod), to_dev(g)
        backend.GatedResidualRMSNorm(puter_amd.RMSNormConfig(1e-5), v_res, v_br, dm, dg, v_hid, v_out,
                                     rows, h, rows, 3 * h, 0, puter_amd.BF16)
        whole = backend.ViewWorkspaceSlot(slot, [4 * rows * h], puter_amd.BF16, 4 * nb)
        got = backend.Download(whole, np.empty(4 * rows * h, np.uint16)).reshape(4, rows, h)
        hid_ref = O.gated_residual(res, br, mod, rows, 0, O.BF16)
        assert np.array_equal(got[0], res) and np.array_equal(got[1], br)
        assert np.array_equal(got[2], hid_ref)
        assert_close(O.to_f32(got[3], O.BF16), O.to_f32(O.rmsnorm(hid_ref, g, 1e-5, O.BF16), O.BF16),
                     TOL[O.BF16], what="rmsnorm in a workspace view")
        with pytest.raises(puter_amd.PuterError):
            backend.ViewWorkspaceSlot(slot, [1], puter_amd.BF16, 4 * nb + 1)   # beyond the slot
        with pytest.raises(puter_amd.PuterError):
            backend.AllocateWorkspaceSlot(0)
    finally:
        slot.Close()
