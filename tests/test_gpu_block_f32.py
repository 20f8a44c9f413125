"""BASELINE configs[0] end to end on the GPU: one pre-norm attention block in
f32 (seq 128, hidden 512, 8 heads x 64) chained through the backend exactly as
the reference's execution layer would call it (RMSNorm -> three Matmul
projections -> RoPE on Q and K -> causal MultiHeadAttention -> output Matmul),
checked against the same chain through the oracle."""
import numpy as np
import pytest

import oracle as O
from helpers import assert_close, empty_dev, to_dev, to_host

pytestmark = pytest.mark.gpu


def test_prenorm_attention_block_f32(backend):
    import puter_amd
    S, HID, H, D = 128, 512, 8, 64
    seed = 0x5EED0000
    x = O.normal(seed, S * HID).reshape(S, HID)
    g = O.normal(seed + 1, HID, 1.0, 0.02)
    W = [O.normal(seed + 2 + i, HID * HID, 0.0, 0.02).reshape(HID, HID) for i in range(4)]

    h = O.rmsnorm(x, g, 1e-6, O.F32)
    q, k, v = (O.matmul_f32(h, w) for w in W[:3])
    q = O.rope(q.reshape(S, H, D)).reshape(S, HID)
    k = O.rope(k.reshape(S, H, D)).reshape(S, HID)
    ref = O.matmul_f32(O.mha(q, k, v, H, D, causal=True), W[3])

    xd, gd = to_dev(x), to_dev(g)
    wd = [to_dev(w) for w in W]
    hd, qd, kd, vd, od, yd = (empty_dev((S, HID), np.float32) for _ in range(6))
    backend.RMSNorm(puter_amd.RMSNormConfig(1e-6), xd, gd, hd, S, HID, O.F32)
    for w, out in zip(wd[:3], (qd, kd, vd)):
        backend.Matmul(out, hd, w, S, HID, HID, O.F32)
    rc = puter_amd.RoPEConfig()
    backend.RoPE(rc, qd, qd, S, H, D, O.F32)
    backend.RoPE(rc, kd, kd, S, H, D, O.F32)
    backend.MultiHeadAttention(puter_amd.MultiHeadAttentionConfig(H, D, True, 0, 0.0, 0),
                               qd, kd, vd, od, S, S, O.F32)
    backend.Matmul(yd, od, wd[3], S, HID, HID, O.F32)
    assert_close(to_host(yd, np.float32), ref, 1e-5, elem_tol=1e-3, what="pre-norm block")


@pytest.mark.parametrize("S,HID,H,KV,D", [(128, 512, 8, 8, 64), (256, 512, 4, 2, 128)])
def test_prenorm_attention_block_bf16(backend, S, HID, H, KV, D):
    """The same chain in bf16 storage (f32 arithmetic inside each op), the
    second shape with grouped K/V heads and head dim 128: the projections run
    on the MFMA Matmul and the attention on the bf16 prefill kernel.  Each op
    rounds its output to bf16, as the reference's bf16 kernels do, so the
    chains agree to the bf16 bar."""
    import puter_amd
    BF = O.BF16
    seed = 0x5EED0100 + S
    KVW = KV * D
    enc = lambda a: O.from_f32(np.ascontiguousarray(a, np.float32), BF)  # noqa: E731
    x = enc(O.normal(seed, S * HID).reshape(S, HID))
    g = enc(O.normal(seed + 1, HID, 1.0, 0.02))
    wq = enc(O.normal(seed + 2, HID * HID, 0.0, 0.02).reshape(HID, HID))
    wk = enc(O.normal(seed + 3, HID * KVW, 0.0, 0.02).reshape(HID, KVW))
    wv = enc(O.normal(seed + 4, HID * KVW, 0.0, 0.02).reshape(HID, KVW))
    wo = enc(O.normal(seed + 5, HID * HID, 0.0, 0.02).reshape(HID, HID))

    h = O.rmsnorm(x, g, 1e-6, BF)
    q, k, v = O.matmul(h, wq, BF), O.matmul(h, wk, BF), O.matmul(h, wv, BF)
    q = O.rope(q.reshape(S, H, D), dtype=BF).reshape(S, HID)
    k = O.rope(k.reshape(S, KV, D), dtype=BF).reshape(S, KVW)
    ref = O.matmul(O.mha(q, k, v, H, D, causal=True, kv_heads=KV, dtype=BF), wo, BF)

    xd, gd, wqd, wkd, wvd, wod = (to_dev(a) for a in (x, g, wq, wk, wv, wo))
    hd, qd, od, yd = (empty_dev((S, HID), np.uint16) for _ in range(4))
    kd, vd = (empty_dev((S, KVW), np.uint16) for _ in range(2))
    backend.RMSNorm(puter_amd.RMSNormConfig(1e-6), xd, gd, hd, S, HID, BF)
    backend.Matmul(qd, hd, wqd, S, HID, HID, BF)
    backend.Matmul(kd, hd, wkd, S, HID, KVW, BF)
    backend.Matmul(vd, hd, wvd, S, HID, KVW, BF)
    rc = puter_amd.RoPEConfig()
    backend.RoPE(rc, qd, qd, S, H, D, BF)
    backend.RoPE(rc, kd, kd, S, KV, D, BF)
    backend.MultiHeadAttention(puter_amd.MultiHeadAttentionConfig(H, D, True, 0, 0.0, KV),
                               qd, kd, vd, od, S, S, BF)
    backend.Matmul(yd, od, wod, S, HID, HID, BF)
    got = O.to_f32(to_host(yd, np.uint16), BF)
    assert_close(got, O.to_f32(ref, BF), 1e-2, elem_tol=None, what=f"bf16 block S{S} H{HID}")
