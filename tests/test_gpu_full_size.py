"""GPU tier at the full sizes of BASELINE.json's configs.  The oracle cannot recompute these whole
in a test's time, so each case checks sampled rows / sequences against the
oracle (every sampled row spans the tensor's full width, and the samples sit at
the ends and in the middle, where indexing past 2^31 bytes or a wrong block
order would show) and, where the domain gives one, a property of the whole
output: RoPE preserves every pair's norm, a cast round trip is the identity."""
import numpy as np
import pytest

import oracle as O
from helpers import TOL, assert_close, decode, empty_dev, to_dev, to_host

pytestmark = pytest.mark.gpu


def _dev_normal(torch, gen, n, dtype, mean=0.0, std=1.0):
    return (torch.randn(n, device="cuda", generator=gen) * std + mean).to(dtype)


def _rows_to_host(t, rows, width):
    import torch
    idx = torch.tensor(rows, device="cuda", dtype=torch.long)
    return t.view(-1, width).index_select(0, idx).cpu().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("kind", ["rms", "ln"])
def test_fused_gated_residual_norm_65536x8192(backend, kind):
    """configs[1]'s largest shape (4.3 GB per launch): the hidden rows bit-exact,
    the normed rows to the bf16 bar, on 8 rows from first to last."""
    import torch
    import puter_amd
    R, H = 65536, 8192
    gen = torch.Generator(device="cuda").manual_seed(0x5EED0101)
    bf = torch.bfloat16
    res, br = _dev_normal(torch, gen, R * H, bf), _dev_normal(torch, gen, R * H, bf)
    mod = _dev_normal(torch, gen, 3 * H, bf)
    gamma = _dev_normal(torch, gen, H, bf, 1.0, 0.02)
    beta = _dev_normal(torch, gen, H, bf, 0.0, 0.02)
    hid, out = torch.empty_like(res), torch.empty_like(res)
    if kind == "rms":
        backend.GatedResidualRMSNorm(puter_amd.RMSNormConfig(1e-5), res, br, mod, gamma, hid, out,
                                     R, H, R, 3 * H, 0, O.BF16)
    else:
        backend.GatedResidualLayerNorm(res, br, mod, gamma, beta, hid, out, R, H, R, 3 * H, 0, O.BF16)
    rows = [0, 1, 4095, 16384, 32767, 32768, 65534, 65535]
    r_h, b_h = _rows_to_host(res, rows, H), _rows_to_host(br, rows, H)
    m_h = _rows_to_host(mod, [0], 3 * H)
    g_h, be_h = _rows_to_host(gamma, [0], H)[0], _rows_to_host(beta, [0], H)[0]
    hid_ref = O.gated_residual(r_h, b_h, m_h, len(rows), 0, O.BF16)
    assert np.array_equal(_rows_to_host(hid, rows, H), hid_ref)
    y_ref = O.rmsnorm(hid_ref, g_h, 1e-5, O.BF16) if kind == "rms" else O.layernorm(hid_ref, g_h, be_h, O.BF16)
    assert_close(decode(_rows_to_host(out, rows, H), O.BF16), decode(y_ref, O.BF16), TOL[O.BF16],
                 1e-2, what=f"{kind} 65536x8192")
    del res, br, hid, out
    torch.cuda.empty_cache()


def test_rope_q_8192_tokens(backend):
    """configs[2]'s Q (8192 x 32 x 128 bf16, base 5e5) in place: sampled positions
    against the oracle, every pair's norm preserved over the whole tensor."""
    import torch
    import puter_amd
    S, Hn, D = 8192, 32, 128
    gen = torch.Generator(device="cuda").manual_seed(0x5EED0102)
    x = _dev_normal(torch, gen, S * Hn * D, torch.bfloat16)
    x0 = x.clone()
    backend.RoPE(puter_amd.RoPEConfig(BaseFreq=500000.0), x, x, S, Hn, D, O.BF16)
    for p in (0, 1, 777, 4096, 8191):
        src = _rows_to_host(x0, [p], Hn * D).reshape(1, Hn, D)
        ref = O.rope(src, base_freq=500000.0, start_position=p, dtype=O.BF16)
        got = _rows_to_host(x, [p], Hn * D).reshape(1, Hn, D)
        assert_close(decode(got, O.BF16), decode(ref, O.BF16), TOL[O.BF16], what=f"rope position {p}")
    a = x0.float().view(-1, 2)
    b = x.float().view(-1, 2)
    na, nb = a.norm(dim=1), b.norm(dim=1)
    # each output element is rounded to bf16 once: |Δ| <= 2^-8 |value| per element
    assert bool(((nb - na).abs() <= 2.0 ** -7 * na + 1e-30).all())
    del x, x0, a, b
    torch.cuda.empty_cache()


def test_swiglu_8192x14336(backend):
    """configs[2]'s SwiGLU over 8192 x 14336 bf16: sampled rows bit-exact."""
    import torch
    R, C = 8192, 14336
    gen = torch.Generator(device="cuda").manual_seed(0x5EED0103)
    g = _dev_normal(torch, gen, R * C, torch.bfloat16)
    u = _dev_normal(torch, gen, R * C, torch.bfloat16)
    out = torch.empty_like(g)
    backend.SwiGLUTensors(out, g, u, R * C, O.BF16)
    rows = [0, 2047, 4096, 8191]
    ref = O.gated_tensors(0, _rows_to_host(g, rows, C), _rows_to_host(u, rows, C), O.BF16)
    assert np.array_equal(_rows_to_host(out, rows, C), ref)
    del g, u, out
    torch.cuda.empty_cache()


def test_cast_f32_bf16_117m_round_trip(backend):
    """configs[2]'s cast size (117,440,512 elements): f32 -> bf16 bit-exact against
    the oracle over every element, and bf16 -> f32 -> bf16 is the identity."""
    import torch
    n = 8192 * 14336
    gen = torch.Generator(device="cuda").manual_seed(0x5EED0104)
    f = torch.randn(n, device="cuda", generator=gen)
    narrow = torch.empty(n, device="cuda", dtype=torch.int16)
    backend.Cast(narrow, O.BF16, f, O.F32, n)
    got = to_host(narrow, np.int16).view(np.uint16)
    assert np.array_equal(got, O.from_f32(f.cpu().numpy(), O.BF16))
    wide = torch.empty(n, device="cuda")
    backend.Cast(wide, O.F32, narrow, O.BF16, n)
    back = torch.empty_like(narrow)
    backend.Cast(back, O.BF16, wide, O.F32, n)
    assert bool(torch.equal(back, narrow))
    del f, narrow, wide, back
    torch.cuda.empty_cache()


def test_prefill_b4_s4096(backend):
    """configs[3] (B4 S4096 Hq32 Hkv8 D128 causal bf16): in every batch, three
    groups of 8 query rows (a different set per batch: the first, a middle and the
    last rows, and rows beside the 128-query block edges) of every head against
    the oracle."""
    import torch
    import puter_amd
    B, S, H, KV, D = 4, 4096, 32, 8, 128
    sc = 1.0 / np.sqrt(D)
    gen = torch.Generator(device="cuda").manual_seed(0x5EED0105)
    q = _dev_normal(torch, gen, B * S * H * D, torch.bfloat16, 0.0, sc)
    k = _dev_normal(torch, gen, B * S * KV * D, torch.bfloat16, 0.0, sc)
    v = _dev_normal(torch, gen, B * S * KV * D, torch.bfloat16, 0.0, sc)
    o = torch.empty_like(q)
    backend.MultiHeadAttentionBatched(puter_amd.MultiHeadAttentionConfig(H, D, True, 0, 0.0, KV),
                                      q, k, v, o, B, S, S, O.BF16)
    O.set_threads(8)
    rows = {0: (0, 1020, S - 8), 1: (124, S // 2, 3580), 2: (8, 2044, S - 132), 3: (0, S // 2, S - 8)}
    for b in range(B):
        host = lambda t, w: t.view(B, S * w)[b].cpu().view(torch.int16).numpy().view(np.uint16).reshape(S, w)  # noqa: E731
        qh, kh, vh, oh = host(q, H * D), host(k, KV * D), host(v, KV * D), host(o, H * D)
        for lo in rows[b]:
            ref = O.mha_rows(qh, kh, vh, H, D, (0, H), (lo, lo + 8), kv_heads=KV, dtype=O.BF16)
            assert_close(decode(oh[lo:lo + 8], O.BF16), decode(ref[lo:lo + 8], O.BF16), TOL[O.BF16],
                         elem_tol=None, what=f"prefill batch {b} rows {lo}..{lo + 7}")
    del q, k, v, o
    torch.cuda.empty_cache()


@pytest.mark.parametrize("kv_dt", [O.BF16, O.F8E4M3])
def test_paged_decode_b64_full_pool(backend, kv_dt):
    """configs[4] (B64, ctx ~ U[512, 8192], page 16, Hq32 Hkv8 D128, pages randomly
    permuted over the pool): six sequences (the shortest, the longest and four
    more) against the oracle over the same pool."""
    rng = np.random.default_rng(0x5EED0106)
    B, H, KV, D, PS = 64, 32, 8, 128, 16
    ctx = rng.integers(512, 8193, B).astype(np.int32)
    npg = (ctx + PS - 1) // PS
    total = int(npg.sum())
    perm = rng.permutation(total).astype(np.int32)
    table = np.zeros((B, int(npg.max())), np.int32)
    at = 0
    for i in range(B):
        table[i, :npg[i]] = perm[at:at + npg[i]]
        at += npg[i]
    n = total * PS * KV * D

    def bits():
        if kv_dt == O.BF16:   # values in (-2, 2): random sign and mantissa, exponent 126 or 127
            return ((rng.integers(0, 1 << 16, n, dtype=np.uint32) & 0x80FF) | 0x3F00).astype(np.uint16)
        c = rng.integers(0, 256, n, dtype=np.uint8)   # E4M3 codes without the NaN pattern
        c[(c & 0x7F) == 0x7F] = 0x10
        return c
    ks = vs = None
    if kv_dt == O.F8E4M3:     # per-head scales
        ks = (rng.random(KV).astype(np.float32) + 0.5) / 64
        vs = (rng.random(KV).astype(np.float32) + 0.5) / 64
    kp, vp = bits(), bits()
    q = O.from_f32(rng.standard_normal(B * H * D).astype(np.float32).reshape(B, H * D), O.BF16)
    max_ctx = int(ctx.max())
    ws_bytes = backend.PagedDecodeWorkspaceBytes(B, H, D, max_ctx)
    ws = empty_dev((ws_bytes // 4,), np.float32)
    out = empty_dev((B, H * D), np.uint16)
    backend.PagedDecodeAttention(to_dev(q), to_dev(kp), to_dev(vp), to_dev(table), to_dev(ctx), B,
                                 table.shape[1], PS, total, H, KV, D, max_ctx,
                                 None if ks is None else to_dev(ks), None if vs is None else to_dev(vs),
                                 kv_dt, out, ws, ws_bytes)
    got = to_host(out, np.uint16)
    pick = sorted({int(np.argmin(ctx)), int(np.argmax(ctx)), 0, 21, 42, 63})
    ref = O.paged_decode(q[pick], kp, vp, table[pick], ctx[pick], PS, H, KV, D, kv_dt, ks, vs)
    assert_close(O.to_f32(got[pick], O.BF16), O.to_f32(ref, O.BF16), TOL[O.BF16], elem_tol=None,
                 what=f"paged decode sequences {pick}")
