"""GPU: the hot path captured in HIP graphs and replayed.

A decode step (below) and a bf16 pre-norm transformer block (the last test) are
each captured once and replayed with new inputs; every replay must equal the same
calls made eagerly, bit for bit.

The decode step is the paged-KV path of one generated token: KVPageWrite (bf16 pool) or
KVPageWriteFP8 (fp8 pool) of the token's K and V rows at each sequence's next
slot, PagedDecodeAttention over the grown contexts, and the fused
GatedResidualRMSNorm of the attention output.  None of these entry points
allocates, synchronises or issues a memset, so a caller can capture them.  Each
replay runs with the step's inputs changed in place (new query, new K/V rows at
the next slot, contexts one longer), with eager work and synchronisation between
replays, and must equal the same calls made eagerly on a copy of the pools, bit
for bit (output, hidden, attention output and both pools); the last replay's
attention output is also checked against the oracle.

Reference path: execution/page_intrinsic.go:135-352 (page write, gather),
bind_router.go:640-684 (MultiHeadAttention), math_gated_residual_intrinsic.go."""
import numpy as np
import pytest

import oracle as O
import puter_amd
from puter_amd._lib import ERR_INVALID
from helpers import TOL, assert_close, seeded, to_dev, to_host

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kv_dt", [O.BF16, O.F8E4M3])
def test_decode_step_graph_replays_match_eager(backend, kv_dt):
    import torch

    B, H, KV, D, PS, STEPS = 4, 16, 4, 128, 16, 3
    inner, hid_dim = KV * D, H * D
    rng = np.random.default_rng(900 + kv_dt)
    ctx0 = rng.integers(100, 700, B).astype(np.int32)         # tokens already cached
    npages = (ctx0 + STEPS + PS - 1) // PS                      # room for STEPS more
    total = int(npages.sum())
    perm = rng.permutation(total).astype(np.int32)
    table = np.zeros((B, int(npages.max())), np.int32)
    at = 0
    for b in range(B):
        table[b, :npages[b]] = perm[at:at + npages[b]]
        at += npages[b]
    max_ctx = int(ctx0.max()) + STEPS                           # fixed in the captured call

    kf, vf = seeded(901, (total, PS, KV, D)), seeded(902, (total, PS, KV, D))
    if kv_dt == O.BF16:
        kp0, vp0, ks, vs = O.from_f32(kf, O.BF16), O.from_f32(vf, O.BF16), None, None
    else:
        ks = np.full(KV, 4.0 / 448.0, np.float32)
        vs = np.full(KV, 4.0 / 448.0, np.float32)
        kp0 = O.from_f32(kf / ks[0], O.F8E4M3)
        vp0 = O.from_f32(vf / vs[0], O.F8E4M3)
    kp, vp = to_dev(kp0), to_dev(vp0)
    d_ks = None if ks is None else to_dev(ks)
    d_vs = None if vs is None else to_dev(vs)
    d_table = to_dev(table)
    gamma = to_dev(O.from_f32(1.0 + 0.02 * seeded(903, (hid_dim,)), O.BF16))
    mod = to_dev(O.from_f32(seeded(904, (1, 3 * hid_dim)), O.BF16))
    ws_bytes = backend.PagedDecodeWorkspaceBytes(B, H, D, max_ctx)

    def inputs(step):
        pos = ctx0 + step                                       # the new token's index
        ids = table[np.arange(B), pos // PS].astype(np.int32)
        offs = (pos % PS).astype(np.int32)
        return dict(q=O.from_f32(seeded(910 + step, (B, hid_dim)), O.BF16),
                    knew=O.from_f32(seeded(920 + step, (B, inner)), O.BF16),
                    vnew=O.from_f32(seeded(930 + step, (B, inner)), O.BF16),
                    ids=ids, offs=offs, ctx=(pos + 1).astype(np.int32),
                    x=O.from_f32(seeded(940 + step, (B, hid_dim)), O.BF16))

    def buffers(inp):
        return {k: to_dev(v) for k, v in inp.items()}

    def outputs():
        return dict(attn=torch.empty((B, hid_dim), dtype=torch.int16, device="cuda"),
                    hid=torch.empty((B, hid_dim), dtype=torch.int16, device="cuda"),
                    y=torch.empty((B, hid_dim), dtype=torch.int16, device="cuda"),
                    ws=torch.empty(ws_bytes // 4, dtype=torch.float32, device="cuda"))

    def step_calls(buf, out, k_pool, v_pool):
        if kv_dt == O.BF16:
            backend.KVPageWrite(k_pool, buf["knew"], buf["ids"], buf["offs"], k_pool, total, PS, inner,
                                B, 0, O.BF16)
            backend.KVPageWrite(v_pool, buf["vnew"], buf["ids"], buf["offs"], v_pool, total, PS, inner,
                                B, 0, O.BF16)
        else:
            backend.KVPageWriteFP8(k_pool, buf["knew"], buf["ids"], buf["offs"], total, PS, KV, D, B, 0,
                                   d_ks, O.BF16)
            backend.KVPageWriteFP8(v_pool, buf["vnew"], buf["ids"], buf["offs"], total, PS, KV, D, B, 0,
                                   d_vs, O.BF16)
        backend.PagedDecodeAttention(buf["q"], k_pool, v_pool, d_table, buf["ctx"], B, table.shape[1], PS,
                                     total, H, KV, D, max_ctx, d_ks, d_vs, kv_dt, out["attn"], out["ws"],
                                     ws_bytes)
        backend.GatedResidualRMSNorm(puter_amd.RMSNormConfig(1e-5), buf["x"], out["attn"], mod, gamma,
                                     out["hid"], out["y"], B, hid_dim, B, 3 * hid_dim, 0, O.BF16)

    # static buffers the graph reads and writes; one eager step first (it also
    # creates the backend's status word outside the capture)
    static = buffers(inputs(0))
    sout = outputs()
    step_calls(static, sout, kp, vp)
    torch.cuda.synchronize()
    backend.CheckStatus()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step_calls(static, sout, kp, vp)

    for step in range(STEPS):
        inp = inputs(step)
        # eager reference on copies of the pools as they stand before this replay
        k_ref, v_ref = kp.clone(), vp.clone()
        eout = outputs()
        step_calls(buffers(inp), eout, k_ref, v_ref)
        torch.cuda.synchronize()
        # new inputs into the graph's static buffers, then replay
        for k, v in buffers(inp).items():
            static[k].copy_(v)
        graph.replay()
        torch.cuda.synchronize()
        backend.CheckStatus()
        for name in ("attn", "hid", "y"):
            assert torch.equal(sout[name], eout[name]), f"replay {step}: {name} differs from the eager step"
        assert torch.equal(kp, k_ref) and torch.equal(vp, v_ref), f"replay {step}: pools differ"
        # some unrelated eager work between replays
        (torch.randn(1 << 20, device="cuda") * 2).sum().item()

    # the last replay against the oracle (pools as the graph left them)
    kh = to_host(kp, np.uint16 if kv_dt == O.BF16 else np.uint8)
    vh = to_host(vp, np.uint16 if kv_dt == O.BF16 else np.uint8)
    last = inputs(STEPS - 1)
    ref = O.paged_decode(last["q"], kh.reshape(total, PS, KV, D), vh.reshape(total, PS, KV, D), table,
                         last["ctx"], PS, H, KV, D, kv_dt, ks, vs)
    got = to_host(sout["attn"], np.uint16)
    assert_close(O.to_f32(got, O.BF16), O.to_f32(ref, O.BF16), TOL[O.BF16], elem_tol=None,
                 what="graph-replayed paged decode")


@pytest.mark.parametrize("head_dim", [128, 64])
def test_prefill_block_graph_replays_match_eager(backend, head_dim):
    """A bf16 pre-norm transformer block (RMSNorm, Q/K/V projections, RoPE on Q
    and K, causal grouped-query MultiHeadAttention on the MFMA prefill kernel,
    output projection, gated residual, SwiGLU MLP with its projections, and an
    f32 cast of the result) captured once in a HIP graph and replayed three times
    with new activations each time; every replay equals the eager calls bit for
    bit.  Matmul goes through its allocation-free entry point."""
    import torch

    S, H, KVH, D = 256, 8, 2, head_dim
    HID, KVD, FF = H * D, KVH * D, 2 * H * D
    bf = O.BF16
    w = {n: to_dev(O.from_f32(seeded(1000 + i, shape, 0.0, 0.02), bf))
         for i, (n, shape) in enumerate([("wq", (HID, HID)), ("wk", (HID, KVD)), ("wv", (HID, KVD)),
                                         ("wo", (HID, HID)), ("wg", (HID, FF)), ("wu", (HID, FF)),
                                         ("wd", (FF, HID))])}
    gamma = to_dev(O.from_f32(1.0 + 0.02 * seeded(1010, (HID,)), bf))
    mod = to_dev(O.from_f32(seeded(1011, (1, 3 * HID)), bf))
    rope = puter_amd.RoPEConfig(BaseFreq=10000.0)
    mha = puter_amd.MultiHeadAttentionConfig(H, D, True, 0, 0.0, KVH)

    def buffers():
        e = lambda *shape: torch.empty(shape, dtype=torch.int16, device="cuda")  # noqa: E731
        return dict(h=e(S, HID), q=e(S, HID), k=e(S, KVD), v=e(S, KVD), o=e(S, HID), a=e(S, HID),
                    r=e(S, HID), g=e(S, FF), u=e(S, FF), f=e(S, FF), y=e(S, HID),
                    y32=torch.empty((S, HID), dtype=torch.float32, device="cuda"))

    def block(x, b):
        be = backend
        be.RMSNorm(puter_amd.RMSNormConfig(1e-6), x, gamma, b["h"], S, HID, bf)
        be.MatmulNoAlloc(b["q"], b["h"], w["wq"], S, HID, HID, bf)
        be.MatmulNoAlloc(b["k"], b["h"], w["wk"], S, HID, KVD, bf)
        be.MatmulNoAlloc(b["v"], b["h"], w["wv"], S, HID, KVD, bf)
        be.RoPE(rope, b["q"], b["q"], S, H, D, bf)
        be.RoPE(rope, b["k"], b["k"], S, KVH, D, bf)
        be.MultiHeadAttention(mha, b["q"], b["k"], b["v"], b["o"], S, S, bf)
        be.MatmulNoAlloc(b["a"], b["o"], w["wo"], S, HID, HID, bf)
        be.GatedResidual(x, b["a"], mod, b["r"], S, HID, S, 3 * HID, 0, bf)
        be.MatmulNoAlloc(b["g"], b["r"], w["wg"], S, HID, FF, bf)
        be.MatmulNoAlloc(b["u"], b["r"], w["wu"], S, HID, FF, bf)
        be.SwiGLUTensors(b["f"], b["g"], b["u"], S * FF, bf)
        be.MatmulNoAlloc(b["y"], b["f"], w["wd"], S, FF, HID, bf)
        be.Cast(b["y32"], O.F32, b["y"], bf, S * HID)

    x_static = to_dev(O.from_f32(seeded(1020, (S, HID)), bf))
    out_static = buffers()
    block(x_static, out_static)      # eager warm-up outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        block(x_static, out_static)
    for step in range(3):
        x = to_dev(O.from_f32(seeded(1030 + step, (S, HID)), bf))
        ref = buffers()
        block(x, ref)
        torch.cuda.synchronize()
        x_static.copy_(x)
        graph.replay()
        torch.cuda.synchronize()
        for name in ("h", "q", "k", "o", "r", "f", "y", "y32"):
            assert torch.equal(out_static[name], ref[name]), f"replay {step}: {name} differs from the eager block"
        (torch.randn(1 << 20, device="cuda") + 1).sum().item()   # eager work between replays


def _one_row_inputs(dt, b, h, kvh, d, seq_k, seed):
    q = encode_dt(seeded(seed, (b, h * d)), dt)
    k = encode_dt(seeded(seed + 1, (b * seq_k, kvh * d), 0.0, 0.5), dt)
    v = encode_dt(seeded(seed + 2, (b * seq_k, kvh * d)), dt)
    return q, k, v


def encode_dt(x, dt):
    return x if dt == O.F32 else O.from_f32(x, dt)


@pytest.mark.parametrize("dt,b,h,kvh,d,seq_k", [
    (O.BF16, 1, 8, 8, 64, 1000),     # the registered 8 x 64 heads: general kernel split over 256-key chunks
    (O.F32, 2, 4, 2, 64, 1500),      # f32, GQA: the same split path
    (O.F16, 3, 16, 4, 128, 3000),    # f16 at head dim 128: the decode kernels over contiguous K/V
])
def test_one_row_mha_graph_uses_the_held_scratch(backend, dt, b, h, kvh, d, seq_k):
    """One-row MultiHeadAttention (the reference's decode step after KVPageGather,
    bind_router.go:640-684) keeps its split partials in the library's scratch.
    Captured after an eager call of the same shape, the call reuses the held buffer
    (no allocation, event wait or record inside the capture); three replays with
    new inputs equal the eager calls bit for bit and the oracle to the dtype's
    bar.  An eager call that then needs a larger scratch retires the captured
    buffer instead of freeing it, and the graph still replays correctly."""
    import torch

    np_t = np.float32 if dt == O.F32 else np.uint16
    cfg = puter_amd.MultiHeadAttentionConfig(h, d, True, 0, 0.0, kvh)
    q0, k0, v0 = _one_row_inputs(dt, b, h, kvh, d, seq_k, 1100)
    sq, sk, sv = to_dev(q0), to_dev(k0), to_dev(v0)
    sout = torch.empty(sq.shape, dtype=sq.dtype, device="cuda")

    def call(q, k, v, o):
        backend.MultiHeadAttentionBatched(cfg, q, k, v, o, b, 1, seq_k, dt)

    call(sq, sk, sv, sout)                      # eager warm-up: sizes the scratch
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call(sq, sk, sv, sout)

    def replay_and_check(step):
        q, k, v = _one_row_inputs(dt, b, h, kvh, d, seq_k, 1110 + 10 * step)
        ref = torch.empty_like(sout)
        call(to_dev(q), to_dev(k), to_dev(v), ref)
        torch.cuda.synchronize()
        sq.copy_(to_dev(q)); sk.copy_(to_dev(k)); sv.copy_(to_dev(v))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(sout, ref), f"replay {step} differs from the eager call"
        got = to_host(sout, np_t)
        for bb in range(b):
            want = O.mha(q[bb:bb + 1], k[bb * seq_k:(bb + 1) * seq_k], v[bb * seq_k:(bb + 1) * seq_k], h, d,
                         causal=True, kv_heads=kvh, dtype=dt)
            g, w = (got[bb:bb + 1], want) if dt == O.F32 else (O.to_f32(got[bb:bb + 1], dt), O.to_f32(want, dt))
            assert_close(g, w, TOL[dt], elem_tol=None, what=f"replay {step} batch {bb}")
        (torch.randn(1 << 20, device="cuda") * 3).sum().item()   # eager work between replays

    for step in range(3):
        replay_and_check(step)
    # an eager call needing more scratch than the graph's buffer (135 MB of split
    # partials: 2040 heads x 64 chunks x (8 + 4*256) bytes, f32 general path)
    hh, dd, kk = 2040, 256, 64 * 256
    big = puter_amd.MultiHeadAttentionConfig(hh, dd, True, 0, 0.0, 1)
    bq = to_dev(seeded(1190, (1, hh * dd)))
    bk = to_dev(seeded(1191, (kk, dd), 0.0, 0.5))
    bo = torch.empty_like(bq)
    backend.MultiHeadAttentionBatched(big, bq, bk, bk, bo, 1, 1, kk, O.F32)
    torch.cuda.synchronize()
    del bq, bk, bo
    replay_and_check(3)


def test_f32_prefill_captured_runs_unsplit(backend):
    """f32 MultiHeadAttention on the f32 MFMA kernel splits the key range of small
    grids with partials in the library's scratch when called eagerly; under capture
    it takes the unsplit kernel and touches no scratch.  A capture with no eager
    call before it succeeds; its replays with new inputs match the oracle to the f32
    bar, and the eager (split) call on the same inputs agrees with them to the same
    bar."""
    import torch

    sq_, sk_, h, kvh, d = 1024, 1024, 4, 1, 64   # 32 blocks: 4 key runs when eager
    cfg = puter_amd.MultiHeadAttentionConfig(h, d, True, 0, 0.0, kvh)

    def inputs(seed):
        return (seeded(seed, (sq_, h * d)), seeded(seed + 1, (sk_, kvh * d)), seeded(seed + 2, (sk_, kvh * d)))

    q0, k0, v0 = inputs(1300)
    sq, sk, sv = to_dev(q0), to_dev(k0), to_dev(v0)
    sout = torch.empty(sq.shape, dtype=sq.dtype, device="cuda")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        backend.MultiHeadAttention(cfg, sq, sk, sv, sout, sq_, sk_, O.F32)
    for step in range(2):
        q, k, v = inputs(1310 + 10 * step)
        sq.copy_(to_dev(q)); sk.copy_(to_dev(k)); sv.copy_(to_dev(v))
        graph.replay()
        torch.cuda.synchronize()
        got = to_host(sout, np.float32)
        want = O.mha(q, k, v, h, d, causal=True, kv_heads=kvh, dtype=O.F32)
        assert_close(got, want, TOL[O.F32], elem_tol=1e-3, what=f"captured f32 prefill, replay {step}")
        eager = torch.empty_like(sout)
        backend.MultiHeadAttention(cfg, sq, sk, sv, eager, sq_, sk_, O.F32)
        torch.cuda.synchronize()
        assert_close(to_host(eager, np.float32), got, TOL[O.F32], elem_tol=1e-3, what="eager split against replay")


def test_capture_that_would_grow_the_scratch_fails_before_launching(backend):
    """A one-row MultiHeadAttention whose split partials exceed what the library's
    scratch holds cannot be captured: the call raises PUTER_ERR_INVALID inside the
    capture without allocating or launching (its output keeps the sentinel the
    capture's own fill wrote), the capture ends normally, and the same call made
    eagerly afterwards grows the scratch and matches the oracle on sampled heads."""
    import torch

    # 2040 heads x 256 chunks x (8 + 4*256) B = 539 MB of partials, more than
    # any other call in this suite makes the scratch hold
    b, h, kvh, d, seq_k = 1, 2040, 8, 256, 65536
    cfg = puter_amd.MultiHeadAttentionConfig(h, d, True, 0, 0.0, kvh)
    q = to_dev(O.from_f32(seeded(1200, (b, h * d)), O.BF16))
    k = to_dev(O.from_f32(seeded(1201, (seq_k, kvh * d), 0.0, 0.5), O.BF16))
    v = to_dev(O.from_f32(seeded(1202, (seq_k, kvh * d)), O.BF16))
    out = torch.empty(q.shape, dtype=q.dtype, device="cuda")
    marker = torch.empty(16, dtype=torch.float32, device="cuda")
    err = None
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out.fill_(0x3F80)                      # bf16 1.0 everywhere
        try:
            backend.MultiHeadAttentionBatched(cfg, q, k, v, out, b, 1, seq_k, O.BF16)
        except puter_amd.PuterError as e:
            err = e
        marker.fill_(2.0)
    assert err is not None and err.status == ERR_INVALID, err
    assert "capture" in str(err)
    out.zero_()
    graph.replay()
    torch.cuda.synchronize()
    assert bool((out == 0x3F80).all()) and bool((marker == 2.0).all())
    backend.MultiHeadAttentionBatched(cfg, q, k, v, out, b, 1, seq_k, O.BF16)
    torch.cuda.synchronize()
    got = to_host(out, np.uint16).reshape(h, d)
    qh, kh, vh = to_host(q, np.uint16), to_host(k, np.uint16), to_host(v, np.uint16)
    O.set_threads(8)
    heads = (0, 1, 777, 2039)
    for hd in heads:
        ref = O.mha_rows(qh, kh, vh, h, d, (hd, hd + 1), (0, 1), kv_heads=kvh, dtype=O.BF16)
        assert_close(O.to_f32(got[hd], O.BF16), O.to_f32(ref.reshape(h, d)[hd], O.BF16), TOL[O.BF16],
                     elem_tol=None, what=f"head {hd}")
