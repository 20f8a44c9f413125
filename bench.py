"""Bench for the MI355X puter backend.  Prints ONE JSON line.

Primary metric: the bf16 RMSNorm / LayerNorm
bandwidth sweep fused with the gated-residual add, rows in {1024, 16384, 65536}
x hidden in {2048, 4096, 8192}.  One "step" = one pass over the 9 shapes, each
running the fused GatedResidual+RMSNorm and GatedResidual+LayerNorm once
(18 launches).  value = algorithmic bytes of the step (8 B/elem: read residual
and branch, write hidden and normed) / the step's GPU time, inputs resident in
HBM.  The other configs' figures are reported under "configs".

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--only norm,rope,...]
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
F32_PEAK_TFLOPS = 157.3   # dense f32 MFMA (and vector) peak
ROWS = (1024, 16384, 65536)
HIDDEN = (2048, 4096, 8192)


def log(msg):
    print(msg, file=sys.stderr, flush=True)


class Timer:
    """HIP events on the stream the kernels are launched on (torch's current)."""

    def __init__(self, torch):
        self.torch = torch

    def time(self, fn, iters, warmup=0):
        t = self.torch
        s, e = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
        for _ in range(warmup):
            fn()
        t.cuda.synchronize()
        s.record()
        for _ in range(iters):
            fn()
        e.record()
        e.synchronize()
        return s.elapsed_time(e) / iters  # ms

    def graph(self, fn, launches, reps=3):
        """ms per launch of fn, with `launches` calls captured in one HIP graph and
        the graph replayed: no host submission inside the timed region, so short
        kernels are timed by the device, not by the host's launch rate."""
        t = self.torch
        g = t.cuda.CUDAGraph()
        with t.cuda.graph(g):
            for _ in range(launches):
                fn()
        g.replay()
        t.cuda.synchronize()
        s, e = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(reps):
            g.replay()
        e.record()
        e.synchronize()
        del g
        return s.elapsed_time(e) / (reps * launches)


class NormPool:
    """residual / branch / hidden / normed pools of n bf16 elements for the norm
    sweep.  Each launch of a rows x hidden shape takes the next rows*hidden
    window of the pools (wrapping at the end), so no launch reads bytes that a
    recent launch left in the 256 MB last-level cache: every shape is timed from
    HBM, the small ones included."""

    def __init__(self, torch, n, gen):
        bf = torch.bfloat16
        self.n = n
        self.res = torch.randn(n, device="cuda", dtype=bf, generator=gen)
        self.br = torch.randn(n, device="cuda", dtype=bf, generator=gen)
        self.hid = torch.empty(n, device="cuda", dtype=bf)
        self.out = torch.empty(n, device="cuda", dtype=bf)
        self.base = [t.data_ptr() for t in (self.res, self.br, self.hid, self.out)]
        self.cur = 0

    def next(self, count):
        """Device addresses (res, br, hid, out) of the next count-element window."""
        if self.cur + count > self.n:
            self.cur = 0
        off = 2 * self.cur
        self.cur += count
        return [b + off for b in self.base]


def norm_sweep(torch, be, puter, steps, warmup):
    """returns (metric dict, dominant-kernel roofline dict)."""
    gen = torch.Generator(device="cuda").manual_seed(0x5EED0001)
    rmax, hmax = max(ROWS), max(HIDDEN)
    n = rmax * hmax
    bf = torch.bfloat16
    pool = NormPool(torch, n, gen)
    mod = torch.randn(3 * hmax, device="cuda", dtype=bf, generator=gen)
    gamma = 1 + 0.02 * torch.randn(hmax, device="cuda", dtype=torch.float32, generator=gen)
    gamma = gamma.to(bf)
    beta = (0.02 * torch.randn(hmax, device="cuda", dtype=torch.float32, generator=gen)).to(bf)
    cfg = puter.RMSNormConfig(1e-5)
    launches = []
    for r in ROWS:
        for h in HIDDEN:
            def rms(r=r, h=h):
                res, br, hid, out = pool.next(r * h)
                be.GatedResidualRMSNorm(cfg, res, br, mod, gamma, hid, out, r, h, r, 3 * h, 0, puter.BF16)

            def ln(r=r, h=h):
                res, br, hid, out = pool.next(r * h)
                be.GatedResidualLayerNorm(res, br, mod, gamma, beta, hid, out, r, h, r, 3 * h, 0, puter.BF16)
            launches.append((r, h, "rms", rms))
            launches.append((r, h, "ln", ln))
    step_bytes = sum(8 * r * h for r, h, _, _ in launches)

    def step():
        for _, _, _, fn in launches:
            fn()

    timer = Timer(torch)
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    ms = timer.time(step, steps)
    # per-shape figures (20 launches, each on the next pool window, captured in a
    # HIP graph and replayed) and the dominant kernel, timed live with events
    per = {}
    for r, h, kind, fn in launches:
        fn()
        t = timer.graph(fn, 20)
        per[f"{kind}_{r}x{h}"] = round(8 * r * h / (t * 1e-3) / 1e9, 1)
    dom = [x for x in launches if x[0] == rmax and x[1] == hmax and x[2] == "rms"][0]
    dom_ms = timer.time(dom[3], 50)
    # context, not this library: the same op in eager torch (h = res + gate * branch,
    # y = rms_norm(h)), charged the fused op's 8 B/elem
    r2, b2, h2 = pool.res.view(rmax, hmax), pool.br.view(rmax, hmax), pool.hid.view(rmax, hmax)
    gate, g2 = mod[2 * hmax:3 * hmax], gamma[:hmax]

    def torch_gr_rms():
        torch.add(r2, b2 * gate, out=h2)
        return torch.nn.functional.rms_norm(h2, (hmax,), g2, 1e-5)
    t_torch = timer.time(torch_gr_rms, 10, warmup=2)
    per["context_torch_gr_rmsnorm_%dx%d" % (rmax, hmax)] = round(8 * rmax * hmax / (t_torch * 1e-3) / 1e9, 1)
    dom_bytes = 8 * rmax * hmax
    achieved = dom_bytes / (dom_ms * 1e-3) / 1e9
    roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
            "kernel": "norm_row_kernel<bf16,RMS,GR,1> (fused gated residual + RMSNorm, a 1024-thread block per row)",
            "workload": f"{rmax}x{hmax} bf16, {dom_bytes} B/launch", "avg_launch_us": round(dom_ms * 1e3, 2)}
    del pool, r2, b2, h2
    torch.cuda.empty_cache()
    return ms, step_bytes, per, roof


def norm_legs(torch, be, puter):
    """The unfused legs of configs[1] at 65536 x 8192 bf16 (RMSNorm and LayerNorm
    alone: read x, write y, 4 B/elem; GatedResidual alone: read residual and
    branch, write hidden, 6 B/elem) and the 2-read/2-write stream ceiling of the
    fused op on the same device (puter_hip_stream_probe, 16 B/vector x 4
    streams over 1 GiB each), beside a 1 GiB device copy."""
    import ctypes as C
    rows, h = 65536, 8192
    n = rows * h
    bf = torch.bfloat16
    gen = torch.Generator(device="cuda").manual_seed(0x5EED0001)
    x = torch.randn(n, device="cuda", dtype=bf, generator=gen)
    br = torch.randn(n, device="cuda", dtype=bf, generator=gen)
    y = torch.empty_like(x)
    mod = torch.randn(3 * h, device="cuda", dtype=bf, generator=gen)
    gamma = (1 + 0.02 * torch.randn(h, device="cuda", generator=gen)).to(bf)
    beta = (0.02 * torch.randn(h, device="cuda", generator=gen)).to(bf)
    timer = Timer(torch)
    res = {}
    t = timer.time(lambda: be.RMSNorm(puter.RMSNormConfig(1e-5), x, gamma, y, rows, h, puter.BF16), 20, warmup=3)
    res["rmsnorm_65536x8192_GBs"] = round(4 * n / (t * 1e-3) / 1e9, 1)
    t = timer.time(lambda: be.LayerNorm(x, gamma, beta, y, rows, h, puter.BF16), 20, warmup=3)
    res["layernorm_65536x8192_GBs"] = round(4 * n / (t * 1e-3) / 1e9, 1)
    t = timer.time(lambda: be.GatedResidual(x, br, mod, y, rows, h, rows, 3 * h, 0, puter.BF16), 20, warmup=3)
    res["gated_residual_65536x8192_GBs"] = round(6 * n / (t * 1e-3) / 1e9, 1)
    # stream ceiling: four 1 GiB streams (x, br reused as a, b; y and a fourth as c, d)
    d = torch.empty_like(x)
    vectors = 2 * n // 16
    st = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731
    for shape, name in ((0, "flat"), (1, "block_row"), (2, "wave_row")):
        def probe(shape=shape):
            rc = be.lib.puter_hip_stream_probe(C.c_void_p(x.data_ptr()), C.c_void_p(br.data_ptr()),
                                               C.c_void_p(y.data_ptr()), C.c_void_p(d.data_ptr()), vectors, shape,
                                               C.c_void_p(st()))
            assert rc == 0, rc
        t = timer.time(probe, 20, warmup=3)
        res[f"stream_2r2w_{name}_GBs"] = round(4 * 16 * vectors / (t * 1e-3) / 1e9, 1)
    # the same 2-read/2-write stream at the sweep's 1024-row sizes (the ceiling of its
    # smallest shapes), timed as the sweep times them: 20 launches, each on the next
    # window of the 1 GiB buffers, captured in a HIP graph and replayed
    for hh in HIDDEN:
        vec = 1024 * hh * 2 // 16
        nwin = 2 * n // (16 * vec)
        for shape, name in ((0, "flat"), (2, "wave_row")):
            win = [0]

            def probe_small(shape=shape, vec=vec, nwin=nwin, win=win):
                off = (win[0] % nwin) * vec * 16
                win[0] += 1
                rc = be.lib.puter_hip_stream_probe(*(C.c_void_p(t.data_ptr() + off) for t in (x, br, y, d)), vec,
                                                   shape, C.c_void_p(st()))
                assert rc == 0, rc
            t = timer.graph(probe_small, 20)
            res[f"stream_2r2w_1024x{hh}_{name}_GBs"] = round(4 * 16 * vec / (t * 1e-3) / 1e9, 1)
    del x, br, y, d
    torch.cuda.empty_cache()
    return res


def rope_swiglu_casts(torch, be, puter):
    """RoPE on Q [8192,32,128] + K [8192,8,128] (theta 5e5), SwiGLU
    over [8192,14336], bf16/f16/fp8 <-> f32 casts over the same tensors."""
    gen = torch.Generator(device="cuda").manual_seed(0x5EED0002)
    bf = torch.bfloat16
    S = 8192
    q = torch.randn(S * 32 * 128, device="cuda", dtype=bf, generator=gen)
    k = torch.randn(S * 8 * 128, device="cuda", dtype=bf, generator=gen)
    gate = torch.randn(S * 14336, device="cuda", dtype=bf, generator=gen)
    up = torch.randn(S * 14336, device="cuda", dtype=bf, generator=gen)
    act = torch.empty_like(gate)
    cfg = puter.RoPEConfig(BaseFreq=500000.0)
    timer = Timer(torch)
    res = {}

    def rope():
        be.RoPE(cfg, q, q, S, 32, 128, puter.BF16)
        be.RoPE(cfg, k, k, S, 8, 128, puter.BF16)
    rope()
    t = timer.time(rope, 20)
    res["rope_qk_bf16_GBs"] = round(4 * (q.numel() + k.numel()) / (t * 1e-3) / 1e9, 1)

    def swiglu():
        be.SwiGLUTensors(act, gate, up, gate.numel(), puter.BF16)
    swiglu()
    t = timer.time(swiglu, 20)
    res["swiglu_bf16_GBs"] = round(6 * gate.numel() / (t * 1e-3) / 1e9, 1)
    f32 = torch.empty(gate.numel(), device="cuda", dtype=torch.float32)
    narrow = torch.empty(gate.numel(), device="cuda", dtype=torch.int16)
    n8 = torch.empty(gate.numel(), device="cuda", dtype=torch.uint8)
    for name, fmt, buf, eb in (("bf16", puter.BF16, narrow, 2), ("f16", puter.F16, narrow, 2),
                               ("fp8e4m3", puter.F8E4M3, n8, 1)):
        be.Cast(f32, puter.F32, gate, puter.BF16, gate.numel())
        t1 = timer.time(lambda: be.Cast(buf, fmt, f32, puter.F32, gate.numel()), 10)
        t2 = timer.time(lambda: be.Cast(f32, puter.F32, buf, fmt, gate.numel()), 10)
        res[f"cast_f32_to_{name}_GBs"] = round((4 + eb) * gate.numel() / (t1 * 1e-3) / 1e9, 1)
        res[f"cast_{name}_to_f32_GBs"] = round((4 + eb) * gate.numel() / (t2 * 1e-3) / 1e9, 1)
    # integer quantisation over the same 117 M elements: Quant (f32 -> int8, 5 B/elem),
    # Dequant (int8 -> f32, 5 B/elem), Dequant4 (packed int4 -> f32, 4.5 B/elem),
    # and the f32 <-> f64 casts (12 B/elem)
    n = gate.numel()
    i8 = n8.view(torch.int8)
    q8 = puter.DequantInt8Config(0.05, 3)
    # Quant's input: fresh N(0,1) f32 (the buffer above holds fp8-rounded values,
    # half of which divide to exact .5 ties that take the exact-division path)
    f32.normal_(generator=gen)
    t = timer.time(lambda: be.Quant(i8, f32, n, q8, puter.I8, puter.F32), 10, warmup=2)
    res["quant_f32_to_int8_GBs"] = round(5 * n / (t * 1e-3) / 1e9, 1)
    t = timer.time(lambda: be.Dequant(f32, i8, n, q8, puter.F32, puter.I8), 10, warmup=2)
    res["dequant_int8_to_f32_GBs"] = round(5 * n / (t * 1e-3) / 1e9, 1)
    t = timer.time(lambda: be.Dequant4(f32, n8, n, puter.DequantInt4Config(0.25, 0), puter.F32, puter.I4), 10, warmup=2)
    res["dequant4_int4_to_f32_GBs"] = round(4.5 * n / (t * 1e-3) / 1e9, 1)
    del narrow, n8, i8
    torch.cuda.empty_cache()
    f64 = torch.empty(n, device="cuda", dtype=torch.float64)
    t = timer.time(lambda: be.Cast(f64, puter.F64, f32, puter.F32, n), 10, warmup=2)
    res["cast_f32_to_f64_GBs"] = round(12 * n / (t * 1e-3) / 1e9, 1)
    t = timer.time(lambda: be.Cast(f32, puter.F32, f64, puter.F64, n), 10, warmup=2)
    res["cast_f64_to_f32_GBs"] = round(12 * n / (t * 1e-3) / 1e9, 1)
    del q, k, gate, up, act, f32, f64
    torch.cuda.empty_cache()
    return res


def prefill(torch, be, puter, return_fn=False):
    """causal GQA prefill bf16, B4 S4096 Hq32 Hkv8 D128, and the same
    step in f32 at S2048 (return_fn: only build the bf16 inputs and return the launch)."""
    gen = torch.Generator(device="cuda").manual_seed(0x5EED0003)
    B, S, H, KV, D = 4, 4096, 32, 8, 128
    sc = 1.0 / math.sqrt(D)
    q = (torch.randn(B * S * H * D, device="cuda", generator=gen) * sc).to(torch.bfloat16)
    k = (torch.randn(B * S * KV * D, device="cuda", generator=gen) * sc).to(torch.bfloat16)
    v = (torch.randn(B * S * KV * D, device="cuda", generator=gen) * sc).to(torch.bfloat16)
    o = torch.empty_like(q)
    cfg = puter.MultiHeadAttentionConfig(H, D, True, 0, 0.0, KV)
    fn = lambda: be.MultiHeadAttentionBatched(cfg, q, k, v, o, B, S, S, puter.BF16)  # noqa: E731
    if return_fn:
        return fn
    fn()
    # 20 warm-up launches (~10 ms) bring the shader clock to its loaded steady
    # state before the timed launches
    t = Timer(torch).time(fn, 20, warmup=20)
    flops = 4.0 * B * H * D * S * (S + 1) / 2
    tf = flops / (t * 1e-3) / 1e12
    res = {"prefill_ms": round(t, 3), "prefill_TFLOPs": round(tf, 1),
           "prefill_mfma_frac": round(tf / BF16_PEAK_TFLOPS, 4)}
    # context, not this library: torch's flash SDPA backend on the same shape
    # ([B, H, S, D], K/V heads repeated to 32); null if the backend is unavailable
    res["context_torch_sdpa_flash_TFLOPs"] = None
    try:
        import torch.nn.functional as F
        from torch.nn.attention import SDPBackend, sdpa_kernel
        qt = q.view(B, S, H, D).transpose(1, 2).contiguous()
        kt = k.view(B, S, KV, D).transpose(1, 2).repeat_interleave(H // KV, dim=1).contiguous()
        vt = v.view(B, S, KV, D).transpose(1, 2).repeat_interleave(H // KV, dim=1).contiguous()
        with sdpa_kernel(SDPBackend.FLASH_ATTENTION):
            t2 = Timer(torch).time(lambda: F.scaled_dot_product_attention(qt, kt, vt, is_causal=True), 10, warmup=3)
        res["context_torch_sdpa_flash_TFLOPs"] = round(flops / (t2 * 1e-3) / 1e12, 1)
        del qt, kt, vt
    except (RuntimeError, ImportError) as ex:
        log(f"torch flash SDPA unavailable: {ex}")
    del q, k, v, o
    # the same step in f32 (the reference's default format) at half the sequence, on
    # the f32 MFMA prefill kernel
    S2 = 2048
    q = torch.randn(B * S2 * H * D, device="cuda", generator=gen) * sc
    k = torch.randn(B * S2 * KV * D, device="cuda", generator=gen) * sc
    v = torch.randn(B * S2 * KV * D, device="cuda", generator=gen)
    o = torch.empty_like(q)
    fn32 = lambda: be.MultiHeadAttentionBatched(cfg, q, k, v, o, B, S2, S2, puter.F32)  # noqa: E731
    fn32()
    t = Timer(torch).time(fn32, 10, warmup=5)
    flops = 4.0 * B * H * D * S2 * (S2 + 1) / 2
    tf = flops / (t * 1e-3) / 1e12
    res.update({"prefill_f32_s2048_ms": round(t, 3), "prefill_f32_s2048_TFLOPs": round(tf, 1),
                "prefill_f32_s2048_frac": round(tf / F32_PEAK_TFLOPS, 4)})
    del q, k, v, o
    torch.cuda.empty_cache()
    return res


def decode(torch, be, puter, fp8, return_fn=False):
    """paged decode, B64, ctx ~ U[512, 8192], page 16, Hq32 Hkv8 D128
    (return_fn: only build the inputs and return the launch)."""
    import numpy as np
    rng = np.random.default_rng(0x5EED0004)
    B, H, KV, D, PS = 64, 32, 8, 128, 16
    ctx = rng.integers(512, 8193, B).astype(np.int32)
    npages = (ctx + PS - 1) // PS
    total = int(npages.sum())
    perm = rng.permutation(total).astype(np.int32)
    maxp = int(npages.max())
    table = np.zeros((B, maxp), np.int32)
    at = 0
    for i in range(B):
        table[i, :npages[i]] = perm[at:at + npages[i]]
        at += npages[i]
    gen = torch.Generator(device="cuda").manual_seed(0x5EED0005)
    q = torch.randn(B * H * D, device="cuda", generator=gen).to(torch.bfloat16)
    n = total * PS * KV * D
    if fp8:
        kp = (torch.randn(n, device="cuda", generator=gen) * 64).to(torch.float8_e4m3fn)
        vp = (torch.randn(n, device="cuda", generator=gen) * 64).to(torch.float8_e4m3fn)
        ks = torch.full((KV,), 1 / 64, device="cuda")
        vs = torch.full((KV,), 1 / 64, device="cuda")
        fmt, eb = puter.F8E4M3, 1
    else:
        kp = torch.randn(n, device="cuda", generator=gen).to(torch.bfloat16)
        vp = torch.randn(n, device="cuda", generator=gen).to(torch.bfloat16)
        ks = vs = None
        fmt, eb = puter.BF16, 2
    maxc = int(ctx.max())
    wsb = be.PagedDecodeWorkspaceBytes(B, H, D, maxc)
    ws = torch.empty(wsb, device="cuda", dtype=torch.uint8)
    out = torch.empty_like(q)
    tt = torch.from_numpy(table).cuda()
    cc = torch.from_numpy(ctx).cuda()
    fn = lambda: be.PagedDecodeAttention(q, kp, vp, tt, cc, B, maxp, PS, total, H, KV, D, maxc, ks, vs, fmt,  # noqa: E731
                                         out, ws, wsb)
    if return_fn:
        return fn
    fn()
    t = Timer(torch).time(fn, 20, warmup=3)
    kv_bytes = int(ctx.sum()) * KV * D * 2 * eb
    name = "fp8" if fp8 else "bf16"
    res = {f"decode_{name}_us": round(t * 1e3, 1),
           f"decode_{name}_GBs": round(kv_bytes / (t * 1e-3) / 1e9, 1),
           f"decode_{name}_hbm_frac": round(kv_bytes / (t * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
           "decode_sum_ctx": int(ctx.sum())}
    if not fp8:
        # the reference's own path for the same step (execution/page_intrinsic.go:277-352
        # then MultiHeadAttention with one query row, per sequence): KVPageGather of K
        # and V into contiguous rows, then attention over them
        kg = torch.empty(maxc * KV * D, device="cuda", dtype=torch.bfloat16)
        vg = torch.empty_like(kg)
        mcfg = puter.MultiHeadAttentionConfig(H, D, True, 0, 0.0, KV)

        def ref_path():
            for i in range(B):
                c = int(ctx[i])
                be.KVPageGather(kp, tt[i], kg, total, PS, KV * D, c, 0, fmt)
                be.KVPageGather(vp, tt[i], vg, total, PS, KV * D, c, 0, fmt)
                be.MultiHeadAttention(mcfg, q[i * H * D:(i + 1) * H * D], kg, vg,
                                      out[i * H * D:(i + 1) * H * D], 1, c, fmt)
        t2 = Timer(torch).time(ref_path, 3, warmup=1)
        res["decode_bf16_gather_then_mha_us"] = round(t2 * 1e3, 1)
        del kg, vg
    return res


def pages(torch, be, puter, return_fns=False):
    """The paged-KV hooks (execution/page_intrinsic.go:135-352) at configs[4]'s
    pool (B64, ctx ~ U[512, 8192], page 16, 8 kv heads x 128 bf16: 2 KiB rows,
    pages randomly permuted): KVPageWrite of one decode step (a row per
    sequence at its next slot), of 4096 and of 16384 prefill rows (consecutive
    tokens through a sequence's page table), and KVPageGather of every
    sequence's pages in one call.  Algorithmic bytes: rows x 2 KiB read + the
    same written, plus 8 B of (id, slot) per written row or 4 B of table per
    gathered page.  A plain device copy of the prefill write's bytes is timed
    beside it for context."""
    import numpy as np
    rng = np.random.default_rng(0x5EED0004)
    B, KV, D, PS = 64, 8, 128, 16
    inner, row_bytes = KV * D, KV * D * 2
    ctx = rng.integers(512, 8193, B).astype(np.int32)
    npages = (ctx + PS - 1) // PS
    total = int(npages.sum()) + 1024          # room for 16384 fresh rows
    perm = rng.permutation(total).astype(np.int32)
    gen = torch.Generator(device="cuda").manual_seed(0x5EED0007)
    pool = torch.randn(total * PS * inner, device="cuda", generator=gen).to(torch.bfloat16)
    t = Timer(torch)
    res, fns = {}, {}
    # decode step: sequence i writes its token ctx_i at its page table's slot
    first = np.concatenate([[0], np.cumsum(npages)[:-1]])
    dec_ids = perm[first + (ctx - 1) // PS].astype(np.int32)
    dec_offs = ((ctx - 1) % PS).astype(np.int32)
    cases = [("decode_b64", dec_ids, dec_offs)]
    for n in (4096, 16384):                   # a prefill's K rows into fresh pages
        fresh = perm[total - 1024:total - 1024 + n // PS]
        r = np.arange(n)
        cases.append((f"prefill_{n}", fresh[r // PS].astype(np.int32), (r % PS).astype(np.int32)))
    for name, ids, offs in cases:
        n = ids.size
        vals = torch.randn(n * inner, device="cuda", generator=gen).to(torch.bfloat16)
        di, do = torch.from_numpy(ids).cuda(), torch.from_numpy(offs).cuda()
        fn = (lambda v=vals, di=di, do=do, n=n:  # noqa: E731
              be.KVPageWrite(pool, v, di, do, pool, total, PS, inner, n, 0, puter.BF16))
        fns[f"page_write_{name}"] = fn
        if return_fns:
            continue
        fn()
        ms = t.graph(fn, 20) if n <= 4096 else t.time(fn, 20, warmup=3)
        nbytes = n * (2 * row_bytes + 8)
        res[f"page_write_{name}_us"] = round(ms * 1e3, 2)
        res[f"page_write_{name}_GBs"] = round(nbytes / (ms * 1e-3) / 1e9, 1)
        res[f"page_write_{name}_hbm_frac"] = round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
        if n == 16384:
            src = vals
            dst = torch.empty_like(src)
            ms = t.time(lambda: dst.copy_(src), 20, warmup=3)
            res["context_copy_prefill_16384_GBs"] = round(n * 2 * row_bytes / (ms * 1e-3) / 1e9, 1)
            del dst
    # gather: every sequence's pages back to back in one table
    table = torch.from_numpy(perm[:int(npages.sum())].copy()).cuda()
    out_rows = int(npages.sum()) * PS
    out = torch.empty(out_rows * inner, device="cuda", dtype=torch.bfloat16)
    fn = lambda: be.KVPageGather(pool, table, out, total, PS, inner, out_rows, 0, puter.BF16)  # noqa: E731
    fns["page_gather_b64"] = fn
    if return_fns:
        return fns
    fn()
    ms = t.time(fn, 20, warmup=3)
    nbytes = out_rows * 2 * row_bytes + table.numel() * 4
    res["page_gather_b64_us"] = round(ms * 1e3, 1)
    res["page_gather_b64_GBs"] = round(nbytes / (ms * 1e-3) / 1e9, 1)
    res["page_gather_b64_hbm_frac"] = round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
    be.CheckStatus()
    del pool, out
    torch.cuda.empty_cache()
    return res


def matmul_legs(torch, be, puter):
    """Matmul in bf16 (f32 accumulation): a square 8192^3 and the MLP
    up-projection shape rows 8192 x inner 4096 x cols 14336 (256 x 256 tiles),
    6144 x 4096 x 4096 (128 x 128 tiles), 2048^3 and 1024 x 8192 x 1024 (under one
    round of 128 x 128 tiles: the split-K kernel, unsplit and in four chunks), and
    decode-step projections of 64 rows (split-K path); in f32 (the reference's default
    format) 4096^3 and the MLP shape on the f32 MFMA kernel."""
    gen = torch.Generator(device="cuda").manual_seed(0x5EED0006)
    res = {}
    for name, (M, K, N) in (("8192c", (8192, 8192, 8192)), ("mlp", (8192, 4096, 14336)),
                            ("m6144_k4096_n4096", (6144, 4096, 4096)), ("2048c", (2048, 2048, 2048)),
                            ("m1024_k8192_n1024", (1024, 8192, 1024))):
        a = torch.randn(M * K, device="cuda", generator=gen).to(torch.bfloat16)
        b = torch.randn(K * N, device="cuda", generator=gen).to(torch.bfloat16)
        c = torch.empty(M * N, device="cuda", dtype=torch.bfloat16)
        t = Timer(torch).time(lambda: be.Matmul(c, a, b, M, K, N, puter.BF16), 10, warmup=3)
        tf = 2.0 * M * K * N / (t * 1e-3) / 1e12
        res[f"matmul_bf16_{name}_ms"] = round(t, 3)
        res[f"matmul_bf16_{name}_TFLOPs"] = round(tf, 1)
        res[f"matmul_bf16_{name}_mfma_frac"] = round(tf / BF16_PEAK_TFLOPS, 4)
        # context, not this library: torch.matmul on the same operands (hipBLASLt)
        a2, b2 = a.view(M, K), b.view(K, N)
        t = Timer(torch).time(lambda: torch.matmul(a2, b2), 10, warmup=3)
        res[f"context_torch_matmul_bf16_{name}_TFLOPs"] = round(2.0 * M * K * N / (t * 1e-3) / 1e12, 1)
        del a, b, c, a2, b2
    # f32 (the reference's default format) on the f32 MFMA kernel; context: torch.matmul
    # in f32 with TF32 off
    tf32 = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    for name, (M, K, N) in (("4096c", (4096, 4096, 4096)), ("mlp", (8192, 4096, 14336))):
        a = torch.randn(M * K, device="cuda", generator=gen)
        b = torch.randn(K * N, device="cuda", generator=gen)
        c = torch.empty(M * N, device="cuda")
        t = Timer(torch).time(lambda: be.Matmul(c, a, b, M, K, N, puter.F32), 10, warmup=3)
        tf = 2.0 * M * K * N / (t * 1e-3) / 1e12
        res[f"matmul_f32_{name}_ms"] = round(t, 3)
        res[f"matmul_f32_{name}_TFLOPs"] = round(tf, 1)
        res[f"matmul_f32_{name}_frac"] = round(tf / F32_PEAK_TFLOPS, 4)
        a2, b2 = a.view(M, K), b.view(K, N)
        t = Timer(torch).time(lambda: torch.matmul(a2, b2), 10, warmup=3)
        res[f"context_torch_matmul_f32_{name}_TFLOPs"] = round(2.0 * M * K * N / (t * 1e-3) / 1e12, 1)
        del a, b, c, a2, b2
    torch.backends.cuda.matmul.allow_tf32 = tf32
    # decode-step projections (batch 64 rows against a weight matrix): HBM-bound,
    # GB/s of operand + output bytes
    for M, K, N in ((64, 4096, 4096), (64, 4096, 14336), (64, 14336, 4096)):
        a = torch.randn(M * K, device="cuda", generator=gen).to(torch.bfloat16)
        b = torch.randn(K * N, device="cuda", generator=gen).to(torch.bfloat16)
        c = torch.empty(M * N, device="cuda", dtype=torch.bfloat16)
        t = Timer(torch).time(lambda: be.Matmul(c, a, b, M, K, N, puter.BF16), 20, warmup=3)
        name = f"matmul_bf16_m{M}_k{K}_n{N}"
        byt = 2 * (M * K + K * N + M * N)
        res[f"{name}_us"] = round(t * 1e3, 1)
        res[f"{name}_GBs"] = round(byt / (t * 1e-3) / 1e9, 1)
        a2, b2 = a.view(M, K), b.view(K, N)
        t = Timer(torch).time(lambda: torch.matmul(a2, b2), 20, warmup=3)
        res[f"context_torch_{name}_us"] = round(t * 1e3, 1)
        del a, b, c, a2, b2
    torch.cuda.empty_cache()
    return res


def block_bf16(torch, be, puter):
    """configs[0]'s block in bf16 storage (the same chain and shapes as block_f32,
    each op rounding its output to bf16): GPU latency per block."""
    S, HID, H, D = 128, 512, 8, 64
    gen = torch.Generator(device="cuda").manual_seed(0x5EED0007)
    bf = torch.bfloat16
    x = torch.randn(S * HID, device="cuda", generator=gen).to(bf)
    g = (1 + 0.02 * torch.randn(HID, device="cuda", generator=gen)).to(bf)
    W = [(0.02 * torch.randn(HID * HID, device="cuda", generator=gen)).to(bf) for _ in range(4)]
    h, q, k, v, o, y = (torch.empty(S * HID, device="cuda", dtype=bf) for _ in range(6))
    ncfg = puter.RMSNormConfig(1e-6)
    rcfg = puter.RoPEConfig(BaseFreq=10000.0)
    mcfg = puter.MultiHeadAttentionConfig(H, D, True, 0, 0.0, H)

    def chain():
        be.RMSNorm(ncfg, x, g, h, S, HID, puter.BF16)
        be.Matmul(q, h, W[0], S, HID, HID, puter.BF16)
        be.Matmul(k, h, W[1], S, HID, HID, puter.BF16)
        be.Matmul(v, h, W[2], S, HID, HID, puter.BF16)
        be.RoPE(rcfg, q, q, S, H, D, puter.BF16)
        be.RoPE(rcfg, k, k, S, H, D, puter.BF16)
        be.MultiHeadAttention(mcfg, q, k, v, o, S, S, puter.BF16)
        be.Matmul(y, o, W[3], S, HID, HID, puter.BF16)

    t = Timer(torch).time(chain, 50, warmup=3)

    # the same chain captured in a HIP graph (Matmul through the allocation-free
    # entry point) and replayed: the block's device latency without host submission
    def chain_graph():
        be.RMSNorm(ncfg, x, g, h, S, HID, puter.BF16)
        be.MatmulNoAlloc(q, h, W[0], S, HID, HID, puter.BF16)
        be.MatmulNoAlloc(k, h, W[1], S, HID, HID, puter.BF16)
        be.MatmulNoAlloc(v, h, W[2], S, HID, HID, puter.BF16)
        be.RoPE(rcfg, q, q, S, H, D, puter.BF16)
        be.RoPE(rcfg, k, k, S, H, D, puter.BF16)
        be.MultiHeadAttention(mcfg, q, k, v, o, S, S, puter.BF16)
        be.MatmulNoAlloc(y, o, W[3], S, HID, HID, puter.BF16)
    chain_graph()
    torch.cuda.synchronize()
    tg = Timer(torch).graph(chain_graph, 1, reps=50)
    return {"block_bf16_us": round(t * 1e3, 1), "block_bf16_graph_us": round(tg * 1e3, 1)}


def block_f32(torch, be, puter):
    """one pre-norm attention block in f32, batch 1, seq 128, hidden
    512, 8 heads x 64: RMSNorm (eps 1e-6, gamma 1+N(0,.02)) -> Q/K/V projections
    (weights N(0,.02)) -> RoPE (theta 1e4, the reference's default interleaved
    mode) -> causal MHA -> output projection (7 launches).  A latency / parity
    config: GPU latency per block, the same chain through the oracle on the host
    (one thread per op call as the oracle runs it), and the normwise difference."""
    import numpy as np
    import oracle as O
    S, HID, H, D = 128, 512, 8, 64
    seed = 0x5EED0000
    x = O.normal(seed, S * HID).reshape(S, HID)
    g = O.normal(seed + 1, HID, 1.0, 0.02)
    W = [O.normal(seed + 2 + i, HID * HID, 0.0, 0.02).reshape(HID, HID) for i in range(4)]

    def host_chain():
        h = O.rmsnorm(x, g, 1e-6, O.F32)
        q, k, v = (O.matmul_f32(h, w) for w in W[:3])
        q = O.rope(q.reshape(S, H, D)).reshape(S, HID)
        k = O.rope(k.reshape(S, H, D)).reshape(S, HID)
        o = O.mha(q, k, v, H, D, causal=True)
        return O.matmul_f32(o, W[3])

    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()  # noqa: E731
    xd, gd = dev(x), dev(g)
    wd = [dev(w) for w in W]
    h, q, k, v, o, y = (torch.empty(S * HID, device="cuda") for _ in range(6))
    ncfg = puter.RMSNormConfig(1e-6)
    rcfg = puter.RoPEConfig(BaseFreq=10000.0)
    mcfg = puter.MultiHeadAttentionConfig(H, D, True, 0, 0.0, H)

    def gpu_chain():
        be.RMSNorm(ncfg, xd, gd, h, S, HID, puter.F32)
        be.Matmul(q, h, wd[0], S, HID, HID, puter.F32)
        be.Matmul(k, h, wd[1], S, HID, HID, puter.F32)
        be.Matmul(v, h, wd[2], S, HID, HID, puter.F32)
        be.RoPE(rcfg, q, q, S, H, D, puter.F32)
        be.RoPE(rcfg, k, k, S, H, D, puter.F32)
        be.MultiHeadAttention(mcfg, q, k, v, o, S, S, puter.F32)
        be.Matmul(y, o, wd[3], S, HID, HID, puter.F32)

    gpu_chain()
    torch.cuda.synchronize()
    got = y.cpu().numpy().reshape(S, HID)
    t = Timer(torch).time(gpu_chain, 50)

    def graph_chain():   # captured in a HIP graph; Matmul through the allocation-free entry point
        be.RMSNorm(ncfg, xd, gd, h, S, HID, puter.F32)
        be.MatmulNoAlloc(q, h, wd[0], S, HID, HID, puter.F32)
        be.MatmulNoAlloc(k, h, wd[1], S, HID, HID, puter.F32)
        be.MatmulNoAlloc(v, h, wd[2], S, HID, HID, puter.F32)
        be.RoPE(rcfg, q, q, S, H, D, puter.F32)
        be.RoPE(rcfg, k, k, S, H, D, puter.F32)
        be.MultiHeadAttention(mcfg, q, k, v, o, S, S, puter.F32)
        be.MatmulNoAlloc(y, o, wd[3], S, HID, HID, puter.F32)
    graph_chain()
    torch.cuda.synchronize()
    tg = Timer(torch).graph(graph_chain, 1, reps=50)
    got_graph = y.cpu().numpy().reshape(S, HID)
    O.set_threads(1)
    ref = host_chain()
    reps, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < 2.0:
        host_chain()
        reps += 1
    cpu_ms = (time.perf_counter() - t0) / reps * 1e3
    err = float(np.max(np.abs(got - ref)) / np.max(np.abs(ref)))
    flops = 4 * 2 * S * HID * HID + 4 * H * D * S * (S + 1) / 2
    return {"block_f32_us": round(t * 1e3, 1), "block_f32_GFLOPs": round(flops / (t * 1e-3) / 1e9, 1),
            "block_f32_graph_us": round(tg * 1e3, 1), "block_f32_graph_equals_eager": bool(np.array_equal(got_graph, got)),
            "block_f32_normwise_err": err, "block_f32_cpu_us": round(cpu_ms * 1e3, 1),
            "block_f32_cpu_cores": 1}


def cpu_configs():
    """The oracle on bounded samples of configs[2..4] and of the bf16 Matmul, timed on the host cores
    (rope and casts are single-threaded in the oracle; SwiGLU, attention rows and
    norms thread over rows)."""
    import numpy as np
    import oracle as O
    cores = os.cpu_count() or 1
    O.set_threads(cores)
    res = {"cpu_cores": cores}

    def timed(fn, budget=2.0):
        reps, t0 = 0, time.perf_counter()
        while True:
            fn()
            reps += 1
            el = time.perf_counter() - t0
            if el > budget:
                return el / reps
    # RoPE on 512 tokens of Q and K, SwiGLU and casts on 512 x 14336
    S = 512
    q = O.from_f32(O.normal(21, S * 32 * 128).reshape(S, 32, 128), O.BF16)
    k = O.from_f32(O.normal(22, S * 8 * 128).reshape(S, 8, 128), O.BF16)
    t = timed(lambda: (O.rope(q, 500000.0, dtype=O.BF16), O.rope(k, 500000.0, dtype=O.BF16)))
    res["cpu_rope_qk_bf16_GBs"] = round(4 * (q.size + k.size) / t / 1e9, 3)
    gate = O.from_f32(O.normal(23, S * 14336), O.BF16)
    up = O.from_f32(O.normal(24, S * 14336), O.BF16)
    t = timed(lambda: O.gated_tensors(0, gate, up, O.BF16))
    res["cpu_swiglu_bf16_GBs"] = round(6 * gate.size / t / 1e9, 3)
    f = O.to_f32(gate, O.BF16)
    t = timed(lambda: O.from_f32(f, O.BF16))
    res["cpu_cast_f32_to_bf16_GBs"] = round(6 * f.size / t / 1e9, 3)
    # causal prefill, batch 0, all 32 heads, the last 64 query rows
    Sq, H, KV, D = 4096, 32, 8, 128
    sc = 1.0 / math.sqrt(D)
    qq = O.from_f32(O.normal(25, Sq * H * D, 0.0, sc).reshape(Sq, H * D), O.BF16)
    kk = O.from_f32(O.normal(26, Sq * KV * D, 0.0, sc).reshape(Sq, KV * D), O.BF16)
    vv = O.from_f32(O.normal(27, Sq * KV * D, 0.0, sc).reshape(Sq, KV * D), O.BF16)
    rows = (Sq - 64, Sq)
    t = timed(lambda: O.mha_rows(qq, kk, vv, H, D, (0, H), rows, kv_heads=KV, dtype=O.BF16))
    flops = 4.0 * H * D * sum(r + 1 for r in range(*rows))
    res["cpu_prefill_TFLOPs"] = round(flops / t / 1e12, 5)
    res["cpu_prefill_sample"] = "batch 0, 32 heads, query rows 4032..4095"
    # paged decode (bf16 pages) of 4 sequences, contexts ~ U[512, 8192]
    rng = np.random.default_rng(0x5EED0004)
    B, PS = 4, 16
    ctx = rng.integers(512, 8193, B).astype(np.int32)
    npg = (ctx + PS - 1) // PS
    total = int(npg.sum())
    perm = rng.permutation(total).astype(np.int32)
    table = np.zeros((B, int(npg.max())), np.int32)
    at = 0
    for i in range(B):
        table[i, :npg[i]] = perm[at:at + npg[i]]
        at += npg[i]
    kp = O.from_f32(O.normal(28, total * PS * KV * D), O.BF16)
    vp = O.from_f32(O.normal(29, total * PS * KV * D), O.BF16)
    qd = O.from_f32(O.normal(30, B * H * D).reshape(B, H * D), O.BF16)
    t = timed(lambda: O.paged_decode(qd, kp, vp, table, ctx, PS, H, KV, D, O.BF16))
    res["cpu_decode_bf16_GBs"] = round(int(ctx.sum()) * KV * D * 2 * 2 / t / 1e9, 3)
    res["cpu_decode_sample"] = f"4 sequences, sum ctx {int(ctx.sum())}"
    # Matmul bf16: one row of the 8192 x 4096 x 14336 MLP shape (the oracle is one
    # thread, f32 accumulation in index order)
    am = O.from_f32(O.normal(31, 4096).reshape(1, 4096), O.BF16)
    bm = O.from_f32(O.normal(32, 4096 * 14336).reshape(4096, 14336), O.BF16)
    t = timed(lambda: O.matmul(am, bm, O.BF16))
    res["cpu_matmul_bf16_TFLOPs"] = round(2.0 * 4096 * 14336 / t / 1e12, 6)
    res["cpu_matmul_sample"] = "rows 1 x inner 4096 x cols 14336, 1 thread"
    return res


def cpu_baseline():
    """The oracle's fused GatedResidual+RMSNorm (bf16) on a bounded sample of
    the primary workload, threaded over rows on all host cores."""
    import numpy as np
    import oracle as O
    cores = os.cpu_count() or 1
    O.set_threads(cores)
    rows, h = 2048, 8192
    res = O.from_f32(O.normal(11, rows * h).reshape(rows, h), O.BF16)
    br = O.from_f32(O.normal(12, rows * h).reshape(rows, h), O.BF16)
    mod = O.from_f32(O.normal(13, 3 * h).reshape(1, 3 * h), O.BF16)
    g = O.from_f32(O.normal(14, h, 1.0, 0.02), O.BF16)
    reps, t0 = 0, time.perf_counter()
    while True:
        hid = O.gated_residual(res, br, mod, rows, 0, O.BF16)
        O.rmsnorm(hid, g, 1e-5, O.BF16)
        reps += 1
        el = time.perf_counter() - t0
        if el > 10.0:
            break
    gbs = 8 * rows * h * reps / el / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"oracle fused GatedResidual+RMSNorm bf16, {rows}x{h}, {reps} reps in {el:.1f}s"}


def profile_dominant(torch, be, puter, launches):
    """Counter-collection workload: the dominant kernel (fused GatedResidual +
    RMSNorm, 65536 x 8192 bf16) `launches` times, then a plain device copy of
    1 GiB (torch copy_) whose FETCH_SIZE / WRITE_SIZE calibrate the counters
    (its algorithmic traffic is exactly 1 GiB read + 1 GiB written)."""
    rows, h = max(ROWS), max(HIDDEN)
    n = rows * h
    bf = torch.bfloat16
    gen = torch.Generator(device="cuda").manual_seed(0x5EED0001)
    res = torch.randn(n, device="cuda", dtype=bf, generator=gen)
    br = torch.randn(n, device="cuda", dtype=bf, generator=gen)
    hid = torch.empty(n, device="cuda", dtype=bf)
    out = torch.empty(n, device="cuda", dtype=bf)
    mod = torch.randn(3 * h, device="cuda", dtype=bf, generator=gen)
    gamma = torch.ones(h, device="cuda", dtype=bf)
    cfg = puter.RMSNormConfig(1e-5)
    for _ in range(launches):
        be.GatedResidualRMSNorm(cfg, res, br, mod, gamma, hid, out, rows, h, rows, 3 * h, 0, puter.BF16)
    src = torch.empty(1 << 28, device="cuda", dtype=torch.float32)   # 1 GiB
    dst = torch.empty_like(src)
    src.fill_(1.0)
    for _ in range(launches):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"profile workload done: {launches} x fused GR+RMSNorm {rows}x{h} bf16 "
        f"({8 * n} B algorithmic each), {launches} x 1 GiB copy")


def profile_matmul(torch, be, puter, launches):
    """Counter-collection workload for the bf16 GEMM: Matmul 8192^3 `launches`
    times (random normal operands)."""
    M = K = N = 8192
    gen = torch.Generator(device="cuda").manual_seed(0x5EED0006)
    a = torch.randn(M * K, device="cuda", generator=gen).to(torch.bfloat16)
    b = torch.randn(K * N, device="cuda", generator=gen).to(torch.bfloat16)
    c = torch.empty(M * N, device="cuda", dtype=torch.bfloat16)
    for _ in range(launches):
        be.Matmul(c, a, b, M, K, N, puter.BF16)
    torch.cuda.synchronize()
    log(f"profile workload done: {launches} x Matmul bf16 {M}x{K}x{N}")


def profile_workload(torch, be, puter, spec, launches):
    """Counter-collection workloads, one kernel family per run (`--profile-workload
    NAME --profile-launches N`): `norm:ROWSxHIDDEN` (fused GatedResidual+RMSNorm
    bf16 on one shape, each launch on the next window of 1 GiB pools so none is
    served from the 256 MB last-level cache, then one 1 GiB calibration copy),
    `stream` (the 2-read/2-write stream probe in its three launch shapes), `mfma`
    (the MFMA rate probe, alone and in the prefill's dataflow),
    `prefill`, `decode_bf16` / `decode_fp8`, `pages`
    (the page write / gather legs at configs[4]'s pool).  Each launch is preceded
    by nothing else on the stream."""
    if spec.startswith("norm:"):
        r, h = (int(x) for x in spec[5:].split("x"))
        gen = torch.Generator(device="cuda").manual_seed(0x5EED0001)
        pool = NormPool(torch, max(r * h, (1 << 30) // 2), gen)
        mod = torch.randn(3 * h, device="cuda", dtype=torch.bfloat16, generator=gen)
        gamma = torch.ones(h, device="cuda", dtype=torch.bfloat16)
        cfg = puter.RMSNormConfig(1e-5)
        for _ in range(launches):
            res, br, hid, out = pool.next(r * h)
            be.GatedResidualRMSNorm(cfg, res, br, mod, gamma, hid, out, r, h, r, 3 * h, 0, puter.BF16)
        # calibration for FETCH_SIZE / WRITE_SIZE: one 1 GiB device copy
        src = pool.res[: (1 << 30) // 2]
        pool.hid[: src.numel()].copy_(src)
    elif spec == "stream":
        # the 2-read/2-write stream ceiling: puter_hip_stream_probe over four 1 GiB
        # buffers in its three launch shapes (flat grid, block per 16 KiB row,
        # wave per 16 KiB row), `launches` times each
        import ctypes as C
        n = (1 << 30) // 2
        bufs = [torch.empty(n, device="cuda", dtype=torch.bfloat16).fill_(1.0) for _ in range(4)]
        vectors = 2 * n // 16
        stream = torch.cuda.current_stream().cuda_stream
        for shape in (0, 1, 2):
            for _ in range(launches):
                rc = be.lib.puter_hip_stream_probe(*(C.c_void_p(b.data_ptr()) for b in bufs), vectors, shape,
                                                   C.c_void_p(stream))
                assert rc == 0, rc
    elif spec == "mfma":
        # the matrix cores' rate on random bf16 operands (puter_hip_mfma_probe): mode 0
        # the MFMAs alone, mode 1 the prefill's 64-key tile dataflow with no memory
        # traffic; 2048 blocks held at two per CU, `launches` timed launches each
        import ctypes as C
        gen = torch.Generator(device="cuda").manual_seed(0x5EED0004)
        ops = torch.randn(8192, device="cuda", dtype=torch.bfloat16, generator=gen)
        blocks, iters = 2048, 256
        out = torch.empty(blocks * 256, device="cuda", dtype=torch.float32)
        stream = torch.cuda.current_stream().cuda_stream
        flops = blocks * 4 * iters * 32 * 32768.0
        for mode in (0, 1):
            def launch():
                rc = be.lib.puter_hip_mfma_probe(C.c_void_p(ops.data_ptr()), C.c_void_p(out.data_ptr()), blocks,
                                                 iters, mode, C.c_void_p(stream))
                assert rc == 0, rc
            launch()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(launches):
                launch()
            e1.record()
            e1.synchronize()
            ms = e0.elapsed_time(e1) / launches
            log(f"mfma probe mode {mode}: {ms * 1e3:.1f} us per launch, {flops / (ms * 1e-3) / 1e12:.1f} TFLOP/s "
                f"({flops / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS:.3f} of the dense bf16 peak)")
    elif spec == "prefill":
        fn = prefill(torch, be, puter, return_fn=True)
        for _ in range(launches):
            fn()
    elif spec in ("decode_bf16", "decode_fp8"):
        fn = decode(torch, be, puter, spec == "decode_fp8", return_fn=True)
        for _ in range(launches):
            fn()
    elif spec == "pages":
        for name, fn in pages(torch, be, puter, return_fns=True).items():
            for _ in range(launches):
                fn()
    else:
        raise SystemExit(f"unknown workload {spec}")
    torch.cuda.synchronize()
    log(f"profile workload done: {launches} x {spec}")


def measure_traffic():
    """HBM bytes per launch of the dominant kernel from two rocprofv3 --pmc
    passes (FETCH_SIZE, then WRITE_SIZE; KiB per dispatch) over
    `bench.py --profile-dominant 3`, each scaled by what the same counter reads
    for the 1 GiB calibration copy in that run.  Returns (bytes, detail) or
    (None, reason)."""
    import csv
    import shutil
    import subprocess
    import tempfile
    if not shutil.which("rocprofv3"):
        return None, "rocprofv3 not found"
    gib_kib = float(1 << 20)
    got = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        with tempfile.TemporaryDirectory() as tmp:
            cmd = ["timeout", "-s", "KILL", "120", "rocprofv3", "--pmc", counter, "--output-format", "csv",
                   "-d", tmp, "-o", "run", "--", sys.executable, os.path.abspath(__file__),
                   "--profile-dominant", "3"]
            r = subprocess.run(cmd, capture_output=True, text=True)
            files = [os.path.join(dp, f) for dp, _, fs in os.walk(tmp) for f in fs
                     if f.endswith("counter_collection.csv")]
            if not files:
                return None, f"{counter} pass failed (rc {r.returncode})"
            kern, copy = [], []
            for row in csv.DictReader(open(files[0])):
                if row.get("Counter_Name") != counter:
                    continue
                if "norm_wave_kernel" in row["Kernel_Name"] or "norm_row_kernel" in row["Kernel_Name"]:
                    kern.append(float(row["Counter_Value"]))
                elif "copyBuffer" in row["Kernel_Name"]:
                    copy.append(float(row["Counter_Value"]))
            if not kern or not copy:
                return None, f"{counter}: kernel or calibration copy missing"
            k_kib = sum(kern) / len(kern)
            c_kib = sum(copy) / len(copy)
            got[counter] = (k_kib, gib_kib / c_kib)
    fetch = got["FETCH_SIZE"][0] * got["FETCH_SIZE"][1] * 1024
    write = got["WRITE_SIZE"][0] * got["WRITE_SIZE"][1] * 1024
    detail = {"fetch_kib": round(got["FETCH_SIZE"][0], 1), "fetch_factor": round(got["FETCH_SIZE"][1], 4),
              "write_kib": round(got["WRITE_SIZE"][0], 1), "write_factor": round(got["WRITE_SIZE"][1], 4)}
    return int(fetch + write), detail


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--only", default="norm,rope,prefill,decode,pages,matmul,block,cpu,traffic")
    ap.add_argument("--profile-dominant", type=int, default=0, metavar="N",
                    help="only run the dominant kernel N times plus a 1 GiB calibration copy")
    ap.add_argument("--profile-workload", default="", metavar="NAME",
                    help="only run one counter-collection workload: norm:RxH, stream, prefill, decode_bf16, "
                         "decode_fp8, pages")
    ap.add_argument("--profile-launches", type=int, default=5, metavar="N")
    ap.add_argument("--profile-matmul", type=int, default=0, metavar="N",
                    help="only run the bf16 Matmul 8192^3 N times (counter collection)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); "
              "every kernel shards by rows/sequences with no exchange", file=sys.stderr)
        sys.exit(2)
    import torch
    import puter_amd as puter
    be = puter.Backend()
    if args.profile_dominant:
        profile_dominant(torch, be, puter, args.profile_dominant)
        return
    if args.profile_matmul:
        profile_matmul(torch, be, puter, args.profile_matmul)
        return
    if args.profile_workload:
        profile_workload(torch, be, puter, args.profile_workload, args.profile_launches)
        return
    only = set(args.only.split(","))
    ms, step_bytes, per, roof = norm_sweep(torch, be, puter, args.steps, args.warmup)
    log(f"norm sweep: {ms:.3f} ms/step, {step_bytes / (ms * 1e-3) / 1e9:.1f} GB/s")
    configs = {"norm_sweep_GBs": per}
    # context: a device-to-device copy of 1 GiB (read 1 GiB + write 1 GiB)
    src = torch.empty(1 << 28, device="cuda", dtype=torch.float32).fill_(1.0)
    dst = torch.empty_like(src)
    t = Timer(torch).time(lambda: dst.copy_(src), 10)
    configs["copy_1GiB_GBs"] = round(2 * (1 << 30) / (t * 1e-3) / 1e9, 1)
    del src, dst
    torch.cuda.empty_cache()
    configs.update(norm_legs(torch, be, puter))
    log(f"norm legs: rms {configs['rmsnorm_65536x8192_GBs']} ln {configs['layernorm_65536x8192_GBs']} "
        f"stream {configs['stream_2r2w_flat_GBs']} GB/s")
    if "rope" in only:
        configs.update(rope_swiglu_casts(torch, be, puter))
        log(f"rope/swiglu/casts: {configs}")
    if "prefill" in only:
        configs.update(prefill(torch, be, puter))
        log(f"prefill: {configs.get('prefill_TFLOPs')} TFLOP/s")
    if "decode" in only:
        configs.update(decode(torch, be, puter, False))
        configs.update(decode(torch, be, puter, True))
        log("decode done")
    if "pages" in only:
        configs.update(pages(torch, be, puter))
        log(f"pages: write 16384 rows {configs['page_write_prefill_16384_GBs']} GB/s, "
            f"gather {configs['page_gather_b64_GBs']} GB/s")
    if "matmul" in only:
        configs.update(matmul_legs(torch, be, puter))
        log(f"matmul bf16: {configs['matmul_bf16_8192c_TFLOPs']} TFLOP/s at 8192^3")
    if "block" in only:
        configs.update(block_f32(torch, be, puter))
        configs.update(block_bf16(torch, be, puter))
        log(f"block f32: {configs['block_f32_us']} us, err {configs['block_f32_normwise_err']:.2e}")
    cpu = cpu_baseline() if "cpu" in only else None
    if "cpu" in only:
        configs.update(cpu_configs())
        log("cpu configs done")
    if "traffic" in only:
        traffic, detail = measure_traffic()
        roof["traffic"] = traffic
        roof["traffic_detail"] = detail
        log(f"traffic: {traffic} B/launch ({detail})")
    value = step_bytes / (ms * 1e-3) / 1e9
    line = {
        "metric": "HBM GB/s for norm/RoPE/act; attention TFLOP/s; % of MI355X roofline",
        "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "fused GatedResidual+RMSNorm/LayerNorm bf16 sweep, rows {1024,16384,65536} "
                               "x hidden {2048,4096,8192}, eps 1e-5 (BASELINE configs[1])",
                   "bytes_per_step": step_bytes, "hbm_frac": round(value / HBM_PEAK_GBS, 4)},
        "roofline": roof,
        "cpu_baseline": cpu,
        "configs": configs,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
