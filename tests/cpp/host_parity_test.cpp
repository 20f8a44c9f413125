// GPU parity through the C++ host side: each case calls the device.Backend
// mirror (or a registered kernel's Run) on cuda device 0 and checks the result
// against the CPU oracle (oracle/liboracle.so, the checker) on the same seeded
// inputs, to the bars of the Python tests: bit-exact for casts, page write /
// gather, the gated residual's 16-bit output, SwiGLU and int8 quantisation;
// normwise 1e-5 for f32 and 1e-2 for bf16 / fp8 otherwise.
#include <algorithm>
#include <atomic>
#include <numeric>
#include <thread>

#include "backend.hpp"
#include "check.hpp"
#include "kernels.hpp"
#include "oracle.h"

using namespace puter::hip;
namespace K = puter::hip::kernels;
using check::normal;
using check::normwise;

namespace {

Backend &be() {
    static Backend b;   // the default stream
    return b;
}

// f32 values -> storage of `dt` (bits for the 16 / 8-bit formats)
std::vector<uint8_t> encode(const std::vector<float> &x, DType dt) {
    std::vector<uint8_t> out((size_t)ByteCount(dt, (int64_t)x.size()));
    or_cast_from_f32(out.data(), x.data(), x.size(), static_cast<int>(dt));
    return out;
}

std::vector<float> decode(const std::vector<uint8_t> &bits, DType dt, size_t n) {
    std::vector<float> out(n);
    or_cast_to_f32(out.data(), bits.data(), n, static_cast<int>(dt));
    return out;
}

template <class T> Tensor upload(const std::vector<T> &host, std::vector<int64_t> shape, DType dt) {
    Tensor t = be().AllocateTensor(std::move(shape), dt);
    be().Upload(t.data, host.data(), host.size() * sizeof(T));
    return t;
}

std::vector<uint8_t> download(const Tensor &t) {
    std::vector<uint8_t> out((size_t)t.byteCount);
    be().Download(out.data(), t.data, out.size());
    return out;
}

std::vector<float> download_f32(const Tensor &t, DType dt) { return decode(download(t), dt, (size_t)t.Numel()); }

}  // namespace

CASE(rmsnorm_bf16) {
    const int64_t rows = 64, h = 2048;
    const DType dt = DType::BFloat16;
    auto x = encode(normal(11, rows * h), dt);
    auto g = encode(normal(12, h, 1.0f, 0.02f), dt);
    Tensor dx = upload(x, {rows, h}, dt), dg = upload(g, {h}, dt), dy = be().AllocateTensor({rows, h}, dt);
    RMSNormConfig cfg;
    cfg.Epsilon = 1e-5;
    be().RMSNorm(cfg, dx.data, dg.data, dy.data, rows, h, dt);
    std::vector<uint8_t> ref(x.size());
    EXPECT(or_rmsnorm(x.data(), g.data(), ref.data(), rows, h, 1e-5, static_cast<int>(dt)) == 0, "oracle");
    const double e = normwise(download_f32(dy, dt), decode(ref, dt, rows * h));
    EXPECT(e <= 1e-2, "normwise %.3g", e);
}

CASE(layernorm_f32_ragged) {
    const int64_t rows = 33, h = 1000;
    const DType dt = DType::Float32;
    auto x = normal(21, rows * h, 0.5f, 2.0f), g = normal(22, h, 1.0f, 0.02f), b = normal(23, h, 0.0f, 0.02f);
    Tensor dx = upload(x, {rows, h}, dt), dg = upload(g, {h}, dt), db = upload(b, {h}, dt);
    Tensor dy = be().AllocateTensor({rows, h}, dt);
    be().LayerNorm(dx.data, dg.data, db.data, dy.data, rows, h, dt);
    std::vector<float> ref(x.size());
    EXPECT(or_layernorm(x.data(), g.data(), b.data(), ref.data(), rows, h, 0) == 0, "oracle");
    const double e = normwise(download_f32(dy, dt), ref);
    EXPECT(e <= 1e-5, "normwise %.3g", e);
}

CASE(gated_residual_rmsnorm_bf16) {
    // the fused hook: hidden bit-exact (math_gated_residual_intrinsic.go:206-223), then RMSNorm
    const int64_t rows = 64, h = 2048, cols = 3 * h;
    const DType dt = DType::BFloat16;
    auto res = encode(normal(31, rows * h), dt), br = encode(normal(32, rows * h), dt);
    auto mod = encode(normal(33, cols), dt), g = encode(normal(34, h, 1.0f, 0.02f), dt);
    Tensor dres = upload(res, {rows, h}, dt), dbr = upload(br, {rows, h}, dt), dmod = upload(mod, {1, cols}, dt);
    Tensor dg = upload(g, {h}, dt), dhid = be().AllocateTensor({rows, h}, dt), dy = be().AllocateTensor({rows, h}, dt);
    RMSNormConfig cfg;
    cfg.Epsilon = 1e-5;
    be().GatedResidualRMSNorm(cfg, dres.data, dbr.data, dmod.data, dg.data, dhid.data, dy.data, rows, h, rows, cols,
                              0, dt);
    std::vector<uint8_t> hid(res.size()), y(res.size());
    EXPECT(or_gated_residual(res.data(), br.data(), mod.data(), hid.data(), rows, h, rows, cols, 0,
                             static_cast<int>(dt)) == 0, "oracle gated residual");
    EXPECT(or_rmsnorm(hid.data(), g.data(), y.data(), rows, h, 1e-5, static_cast<int>(dt)) == 0, "oracle rmsnorm");
    EXPECT(download(dhid) == hid, "hidden rows differ from the oracle");
    const double e = normwise(download_f32(dy, dt), decode(y, dt, rows * h));
    EXPECT(e <= 1e-2, "normwise %.3g", e);
}

CASE(rope_bf16) {
    const int64_t seq = 64, heads = 8, d = 128;
    const DType dt = DType::BFloat16;
    auto x = encode(normal(41, seq * heads * d), dt);
    Tensor dx = upload(x, {seq, heads, d}, dt), dy = be().AllocateTensor({seq, heads, d}, dt);
    RoPEConfig cfg;
    cfg.BaseFreq = 500000.0;
    cfg.StartPosition = 3;
    be().RoPE(cfg, dx.data, dy.data, seq, heads, d, dt);
    or_rope_config oc{};
    oc.base_freq = 500000.0;
    oc.start_position = 3;
    oc.scaling_factor = 1.0;
    std::vector<uint8_t> ref(x.size());
    EXPECT(or_rope(&oc, x.data(), ref.data(), seq, heads, d, static_cast<int>(dt)) == 0, "oracle");
    const double e = normwise(download_f32(dy, dt), decode(ref, dt, seq * heads * d));
    EXPECT(e <= 1e-2, "normwise %.3g", e);
}

CASE(swiglu_bf16_bit_exact) {
    const int64_t n = 100003;
    const DType dt = DType::BFloat16;
    auto gate = encode(normal(51, n, 0.0f, 3.0f), dt), up = encode(normal(52, n), dt);
    Tensor dg = upload(gate, {n}, dt), du = upload(up, {n}, dt), dout = be().AllocateTensor({n}, dt);
    be().SwiGLUTensors(dout.data, dg.data, du.data, n, dt);
    std::vector<uint8_t> ref(gate.size());
    EXPECT(or_gated_tensors(OR_GATE_SWIGLU, ref.data(), gate.data(), up.data(), n, static_cast<int>(dt)) == 0,
           "oracle");
    EXPECT(download(dout) == ref, "SwiGLU differs from the oracle");
}

CASE(casts_bit_exact) {
    const int64_t n = 65537;
    auto x = normal(61, n, 0.0f, 40.0f);
    Tensor dx = upload(x, {n}, DType::Float32);
    for (DType dt : {DType::BFloat16, DType::Float16, DType::Float8E4M3, DType::Float8E5M2}) {
        Tensor narrow = be().AllocateTensor({n}, dt), wide = be().AllocateTensor({n}, DType::Float32);
        be().Cast(narrow.data, dt, dx.data, DType::Float32, n);
        be().Cast(wide.data, DType::Float32, narrow.data, dt, n);
        const auto ref = encode(x, dt);
        EXPECT(download(narrow) == ref, "f32 -> %s", Name(dt));
        std::vector<float> widened(n);
        or_cast_to_f32(widened.data(), ref.data(), n, static_cast<int>(dt));
        const auto got = download(wide);
        EXPECT(std::memcmp(got.data(), widened.data(), got.size()) == 0, "%s -> f32", Name(dt));
    }
    // narrow <-> narrow in one launch (shape.cast's device branch): bf16 -> f16
    auto b = encode(x, DType::BFloat16);
    Tensor db = upload(b, {n}, DType::BFloat16), dh = be().AllocateTensor({n}, DType::Float16);
    be().Cast(dh.data, DType::Float16, db.data, DType::BFloat16, n);
    std::vector<uint8_t> ref((size_t)(2 * n));
    EXPECT(or_cast_pair(ref.data(), OR_F16, b.data(), OR_BF16, n) == 0, "oracle pair");
    EXPECT(download(dh) == ref, "bf16 -> f16");
}

CASE(kv_page_write_gather_and_status) {
    const int64_t pages = 40, ps = 16, inner = 1024, rows = 37;
    const DType dt = DType::BFloat16;
    std::vector<uint16_t> storage((size_t)(pages * ps * inner));
    for (size_t i = 0; i < storage.size(); ++i) storage[i] = (uint16_t)(i * 2654435761u >> 16);
    std::vector<int32_t> ids(rows), offs(rows);
    for (int64_t r = 0; r < rows; ++r) {   // distinct (page, slot) targets
        const int64_t slot = (r * 97 + 5) % (pages * ps);
        ids[r] = (int32_t)(slot / ps);
        offs[r] = (int32_t)(slot % ps);
    }
    auto vals = encode(normal(71, rows * inner), dt);
    Tensor dst = upload(storage, {pages, ps, inner}, dt), dv = upload(vals, {rows, inner}, dt);
    Tensor di = upload(ids, {rows}, DType::Int32), doff = upload(offs, {rows}, DType::Int32);
    be().KVPageWrite(dst.data, dv.data, di.data, doff.data, dst.data, pages, ps, inner, rows, 0, dt);
    std::vector<uint16_t> ref(storage.size());
    EXPECT(or_page_write(storage.data(), vals.data(), ids.data(), offs.data(), ref.data(), pages, ps, inner, rows, 0,
                         2) == 0, "oracle write");
    auto got = download(dst);
    EXPECT(std::memcmp(got.data(), ref.data(), got.size()) == 0, "page write");
    std::vector<int32_t> table = {7, 3, 39, 0, 12};
    const int64_t out_rows = (int64_t)table.size() * ps - 5;
    Tensor dt_ = upload(table, {(int64_t)table.size()}, DType::Int32), dout = be().AllocateTensor({out_rows, inner}, dt);
    be().KVPageGather(dst.data, dt_.data, dout.data, pages, ps, inner, out_rows, 0, dt);
    std::vector<uint16_t> gref((size_t)(out_rows * inner));
    EXPECT(or_page_gather(ref.data(), table.data(), gref.data(), pages, ps, inner, out_rows, 0,
                          (int64_t)table.size(), 2) == 0, "oracle gather");
    got = download(dout);
    EXPECT(std::memcmp(got.data(), gref.data(), got.size()) == 0, "page gather");
    be().CheckStatus();   // clean so far
    // an out-of-range page id: nothing written, the status word flags it, and
    // EndBatch returns the reference's ErrShapeMismatch (page.go:139-146)
    std::vector<int32_t> bad = {(int32_t)pages};
    Tensor dbad = upload(bad, {1}, DType::Int32);
    be().KVPageWrite(dst.data, dv.data, dbad.data, doff.data, dst.data, pages, ps, inner, 1, 0, dt);
    MaybeError err = be().EndBatch();
    EXPECT(err && err->Status() == PUTER_ERR_INVALID, "bad page id not reported");
    EXPECT(!be().EndBatch(), "the status word is cleared once read");
    got = download(dst);
    EXPECT(std::memcmp(got.data(), ref.data(), got.size()) == 0, "a bad row touched the pool");
}

CASE(multi_head_attention_bf16_prefill_and_one_row) {
    // head dim 128 (prefill and one-row kernels) and 64 (the prefill kernel's other
    // layout); the registered sliding_window_attention's window, and a window with ALiBi
    const DType dt = DType::BFloat16;
    struct Shape { int64_t sq, sk, h, kvh, d; bool causal; int64_t window; float alibi; };
    for (Shape s : {Shape{256, 256, 8, 2, 128, true, 0, 0.0f}, Shape{1, 700, 32, 8, 128, true, 0, 0.0f},
                    Shape{96, 160, 4, 4, 128, false, 0, 0.0f}, Shape{300, 300, 8, 8, 64, true, 0, 0.0f},
                    Shape{512, 512, 8, 2, 64, true, 128, 0.0f}, Shape{200, 330, 4, 2, 128, true, 50, 0.25f}}) {
        const int64_t d = s.d;
        auto q = encode(normal(81, s.sq * s.h * d, 0.0f, 0.3f), dt);
        auto k = encode(normal(82, s.sk * s.kvh * d, 0.0f, 0.3f), dt), v = encode(normal(83, s.sk * s.kvh * d), dt);
        Tensor dq = upload(q, {s.sq, s.h * d}, dt), dk = upload(k, {s.sk, s.kvh * d}, dt), dv = upload(v, {s.sk, s.kvh * d}, dt);
        Tensor dout = be().AllocateTensor({s.sq, s.h * d}, dt);
        MultiHeadAttentionConfig cfg;
        cfg.NumHeads = s.h;
        cfg.HeadDim = d;
        cfg.Causal = s.causal;
        cfg.KVHeadCount = s.kvh;
        cfg.WindowSize = s.window;
        cfg.ALiBiSlope = s.alibi;
        be().MultiHeadAttention(cfg, dq.data, dk.data, dv.data, dout.data, s.sq, s.sk, dt);
        or_mha_config oc{s.h, d, s.causal ? 1 : 0, s.window, s.alibi, s.kvh};
        std::vector<uint8_t> ref(q.size());
        EXPECT(or_mha(&oc, q.data(), k.data(), v.data(), ref.data(), s.sq, s.sk, static_cast<int>(dt)) == 0, "oracle");
        const double e = normwise(download_f32(dout, dt), decode(ref, dt, s.sq * s.h * d));
        EXPECT(e <= 1e-2, "seqQ %lld seqK %lld: normwise %.3g", (long long)s.sq, (long long)s.sk, e);
    }
}

CASE(paged_decode_bf16_and_fp8) {
    const int64_t B = 4, H = 32, KV = 8, D = 128, PS = 16;
    const int32_t ctx_h[B] = {600, 17, 1300, 256};
    std::vector<int32_t> ctx(ctx_h, ctx_h + B);
    int64_t total = 0, maxp = 0;
    for (int32_t c : ctx) {
        total += (c + PS - 1) / PS;
        maxp = std::max<int64_t>(maxp, (c + PS - 1) / PS);
    }
    std::vector<int32_t> perm((size_t)total);
    std::iota(perm.begin(), perm.end(), 0);
    for (int64_t i = total - 1; i > 0; --i) std::swap(perm[i], perm[(i * 7919 + 13) % (i + 1)]);
    std::vector<int32_t> table((size_t)(B * maxp), 0);
    int64_t at = 0;
    for (int64_t b = 0; b < B; ++b)
        for (int64_t p = 0; p < (ctx[b] + PS - 1) / PS; ++p) table[b * maxp + p] = perm[at++];
    const int64_t max_ctx = *std::max_element(ctx.begin(), ctx.end());
    auto qf = normal(91, B * H * D);
    auto q = encode(qf, DType::BFloat16);
    auto kf = normal(92, total * PS * KV * D), vf = normal(93, total * PS * KV * D);
    Tensor dq = upload(q, {B, H * D}, DType::BFloat16), dtable = upload(table, {B, maxp}, DType::Int32);
    Tensor dctx = upload(ctx, {B}, DType::Int32);
    const size_t ws = be().PagedDecodeWorkspaceBytes(B, H, D, max_ctx);
    Tensor dws = be().AllocateTensor({(int64_t)ws}, DType::Int8), dout = be().AllocateTensor({B, H * D}, DType::BFloat16);
    for (DType kv : {DType::BFloat16, DType::Float8E4M3}) {
        std::vector<float> ks(KV, 1.0f), vs(KV, 1.0f);
        std::vector<float> kq = kf, vq = vf;
        if (kv == DType::Float8E4M3) {
            std::fill(ks.begin(), ks.end(), 4.0f / 448.0f);
            std::fill(vs.begin(), vs.end(), 4.0f / 448.0f);
            for (float &x : kq) x /= ks[0];
            for (float &x : vq) x /= vs[0];
        }
        auto kp = encode(kq, kv), vp = encode(vq, kv);
        Tensor dk = upload(kp, {total, PS, KV, D}, kv), dv = upload(vp, {total, PS, KV, D}, kv);
        Tensor dks = upload(ks, {KV}, DType::Float32), dvs = upload(vs, {KV}, DType::Float32);
        const bool f8 = kv == DType::Float8E4M3;
        be().PagedDecodeAttention(dq.data, dk.data, dv.data, dtable.data, dctx.data, B, maxp, PS, total, H, KV, D,
                                  max_ctx, f8 ? dks.data : nullptr, f8 ? dvs.data : nullptr, kv, dout.data, dws.data, ws);
        std::vector<uint8_t> ref((size_t)(B * H * D * 2));
        EXPECT(or_paged_decode(q.data(), kp.data(), vp.data(), table.data(), ctx.data(), B, maxp, PS, H, KV, D,
                               f8 ? ks.data() : nullptr, f8 ? vs.data() : nullptr, static_cast<int>(kv), ref.data()) == 0,
               "oracle");
        const double e = normwise(download_f32(dout, DType::BFloat16), decode(ref, DType::BFloat16, B * H * D));
        EXPECT(e <= 1e-2, "%s pools: normwise %.3g", Name(kv), e);
    }
}

CASE(matmul_bf16_f32_and_no_alloc) {
    struct Shape { int64_t m, k, n; DType dt; double tol; };
    for (Shape s : {Shape{256, 512, 384, DType::BFloat16, 1e-2}, Shape{128, 512, 512, DType::Float32, 1e-5},
                    Shape{64, 4096, 1024, DType::BFloat16, 1e-2}}) {
        auto a = encode(normal(101, s.m * s.k), s.dt), b = encode(normal(102, s.k * s.n, 0.0f, 0.05f), s.dt);
        Tensor da = upload(a, {s.m, s.k}, s.dt), db = upload(b, {s.k, s.n}, s.dt);
        Tensor dc = be().AllocateTensor({s.m, s.n}, s.dt), dc2 = be().AllocateTensor({s.m, s.n}, s.dt);
        be().Matmul(dc.data, da.data, db.data, s.m, s.k, s.n, s.dt);
        be().MatmulNoAlloc(dc2.data, da.data, db.data, s.m, s.k, s.n, s.dt);
        std::vector<uint8_t> ref((size_t)ByteCount(s.dt, s.m * s.n));
        EXPECT(or_matmul(ref.data(), a.data(), b.data(), s.m, s.k, s.n, static_cast<int>(s.dt)) == 0, "oracle");
        const double e = normwise(download_f32(dc, s.dt), decode(ref, s.dt, s.m * s.n));
        EXPECT(e <= s.tol, "%lldx%lldx%lld %s: normwise %.3g", (long long)s.m, (long long)s.k, (long long)s.n,
               Name(s.dt), e);
        EXPECT(download(dc) == download(dc2), "MatmulNoAlloc differs from Matmul");
    }
}

CASE(quant_dequant_int8_bit_exact) {
    const int64_t n = 50001;
    auto x = normal(111, n, 0.0f, 20.0f);
    Tensor dx = upload(x, {n}, DType::Float32), dq = be().AllocateTensor({n}, DType::Int8);
    Tensor dback = be().AllocateTensor({n}, DType::Float32);
    DequantInt8Config cfg;
    cfg.Scale = 0.125f;
    cfg.ZeroPoint = 7;
    be().Quant(dq.data, dx.data, n, cfg, DType::Int8, DType::Float32);
    be().Dequant(dback.data, dq.data, n, cfg, DType::Float32, DType::Int8);
    std::vector<int8_t> qref(n);
    std::vector<float> back(n);
    EXPECT(or_quant_int8(qref.data(), x.data(), n, 0.125f, 7) == 0, "oracle quant");
    EXPECT(or_dequant_int8(back.data(), qref.data(), n, 0.125f, 7) == 0, "oracle dequant");
    auto got = download(dq);
    EXPECT(std::memcmp(got.data(), qref.data(), n) == 0, "Quant");
    got = download(dback);
    EXPECT(std::memcmp(got.data(), back.data(), got.size()) == 0, "Dequant");
}

CASE(registered_kernels_run_on_device_tensors) {
    // a kernel looked up by (name, signature, location) runs the same kernels as
    // the backend method: page_write through Run with a device scalar page size
    K::Registry r;
    K::RegisterHIPKernels(r, be());
    const DType dt = DType::Float16;
    const int64_t pages = 6, ps = 4, inner = 24, rows = 5;
    std::vector<uint16_t> storage((size_t)(pages * ps * inner), 0x3C00);
    auto vals = encode(normal(121, rows * inner), dt);
    std::vector<int32_t> ids = {0, 5, 2, 2, 4}, offs = {3, 0, 1, 2, 3}, psz = {(int32_t)ps};
    Tensor dst = upload(storage, {pages, ps, inner}, dt), dv = upload(vals, {rows, inner}, dt);
    Tensor di = upload(ids, {rows}, DType::Int32), doff = upload(offs, {rows}, DType::Int32);
    Tensor dps = upload(psz, {1}, DType::Int32);
    auto k = r.LookupLocation("page_write", K::Signature{K::Layout::Dense, {dt, dt, DType::Int32, DType::Int32, DType::Int32}, {dt}},
                              Location::Device);
    EXPECT(k, "page_write f16 on the device");
    MaybeError err = k->Run({dst, dv, di, doff, dps, dst});
    EXPECT(!err, "%s", err ? err->what() : "");
    std::vector<uint16_t> ref(storage.size());
    EXPECT(or_page_write(storage.data(), vals.data(), ids.data(), offs.data(), ref.data(), pages, ps, inner, rows, 0,
                         2) == 0, "oracle");
    auto got = download(dst);
    EXPECT(std::memcmp(got.data(), ref.data(), got.size()) == 0, "page_write through Run");
    // matmul through Run against the backend method
    const DType bf = DType::BFloat16;
    auto a = encode(normal(122, 64 * 96), bf), b = encode(normal(123, 96 * 40), bf);
    Tensor da = upload(a, {64, 96}, bf), db = upload(b, {96, 40}, bf);
    Tensor c1 = be().AllocateTensor({64, 40}, bf), c2 = be().AllocateTensor({64, 40}, bf);
    auto mm = r.LookupLocation("matmul", K::Signature{K::Layout::Dense, {bf, bf}, {bf}}, Location::Device);
    EXPECT(mm && !mm->Run({da, db, c1}), "matmul Run");
    be().Matmul(c2.data, da.data, db.data, 64, 96, 40, bf);
    EXPECT(download(c1) == download(c2), "matmul through Run");
}

CASE(workspace_slots_stay_on_device) {
    // execution/workspace_resident.go: one slot, views of it with other shapes
    // and formats at the same address, bytes surviving between uses
    auto [slot, err] = be().AllocateWorkspaceSlot(1 << 20);
    EXPECT(!err && slot.data && slot.byteCount == (1 << 20), "slot");
    auto [view, verr] = be().ViewWorkspaceSlot(slot, {1024, 128}, DType::Float32, 1 << 19);
    EXPECT(!verr && view.data == slot.data, "view");
    auto x = normal(131, 1024 * 128);
    be().Upload(view.data, x.data(), x.size() * 4);
    auto [v16, e16] = be().ViewWorkspaceSlot(slot, {1024, 128}, DType::BFloat16, 1 << 18);
    EXPECT(!e16, "bf16 view");
    be().Cast(static_cast<char *>(slot.data) + (1 << 19), DType::BFloat16, view.data, DType::Float32, 1024 * 128);
    std::vector<uint8_t> got((size_t)(1 << 18));
    be().Download(got.data(), static_cast<char *>(slot.data) + (1 << 19), got.size());
    EXPECT(got == encode(x, DType::BFloat16), "cast inside the slot");
    slot.Close();   // the views still hold the allocation
    view.Close();
    v16.Close();
}

CASE(adaptive_and_modulated_norms_f32) {
    // AdaptiveRMSNorm: y = x inv (1 + scale) + shift; ModulatedLayerNorm with set 1
    // (shift at 3H, scale at 3H + H): device/cpu/layernorm/compute.go:387-433,513-570
    const int64_t rows = 12, h = 256, rpb = 4, batches = rows / rpb;
    const DType dt = DType::Float32;
    auto x = normal(141, rows * h, 0.2f, 1.5f);
    auto amod = normal(142, batches * 2 * h, 0.0f, 0.1f), mmod = normal(143, batches * 6 * h, 0.0f, 0.1f);
    Tensor dx = upload(x, {rows, h}, dt), da = upload(amod, {batches, 2 * h}, dt), dm = upload(mmod, {batches, 6 * h}, dt);
    Tensor dy = be().AllocateTensor({rows, h}, dt), dz = be().AllocateTensor({rows, h}, dt);
    RMSNormConfig rc;
    rc.Epsilon = 1e-6;
    be().AdaptiveRMSNorm(rc, dx.data, da.data, dy.data, rows, h, rpb, 2 * h, dt);
    ModulatedLayerNormConfig mc;
    mc.Epsilon = 1e-6;
    mc.Set = 1;
    be().ModulatedLayerNorm(mc, dx.data, dm.data, dz.data, rows, h, rpb, 6 * h, dt);
    std::vector<float> ry(x.size()), rz(x.size());
    EXPECT(or_adaptive_rmsnorm(x.data(), amod.data(), ry.data(), rows, h, rpb, 2 * h, 1e-6, 0) == 0, "oracle adaptive");
    EXPECT(or_modulated_layernorm(x.data(), mmod.data(), rz.data(), rows, h, rpb, 6 * h, 1e-6, 1, 0) == 0,
           "oracle modulated");
    double e = normwise(download_f32(dy, dt), ry);
    EXPECT(e <= 1e-5, "adaptive normwise %.3g", e);
    e = normwise(download_f32(dz, dt), rz);
    EXPECT(e <= 1e-5, "modulated normwise %.3g", e);
}

CASE(multi_axis_rope_and_rope_pairs) {
    // 4 axes (text on axis 3) over a ragged 6-wide image grid after 8 text tokens
    const int64_t b = 2, seq = 23, heads = 3, d = 16;
    const DType dt = DType::BFloat16;
    auto x = encode(normal(151, b * seq * heads * d), dt);
    Tensor dx = upload(x, {b, seq, heads, d}, dt), dy = be().AllocateTensor({b, seq, heads, d}, dt);
    MultiAxisRoPEConfig cfg;
    cfg.BaseFreq = 1e4;
    cfg.LatentSeqLen = 15;
    cfg.LatentSide = 6;
    cfg.AxisCount = 4;
    cfg.AxisDim0 = 2;
    cfg.AxisDim1 = 6;
    cfg.AxisDim2 = 4;
    cfg.AxisDim3 = 4;
    be().MultiAxisRoPE(cfg, dx.data, dy.data, b, seq, heads, d, dt);
    or_multi_axis_rope_config oc{1e4, 15, 6, 4, {2, 6, 4, 4}};
    std::vector<uint8_t> ref(x.size());
    EXPECT(or_multi_axis_rope(&oc, x.data(), ref.data(), b, seq, heads, d, static_cast<int>(dt)) == 0, "oracle");
    double e = normwise(download_f32(dy, dt), decode(ref, dt, b * seq * heads * d));
    EXPECT(e <= 1e-2, "multi-axis normwise %.3g", e);
    // RoPEPairs (F32): (x cos - y sin, x sin + y cos) per pair, rope/f32_generic.go:3-11
    const int64_t half = 1000;
    auto in = normal(152, 2 * half), ang = normal(153, half, 0.0f, 2.0f);
    std::vector<float> cs(half), sn(half);
    for (int64_t i = 0; i < half; ++i) {
        cs[i] = std::cos(ang[i]);
        sn[i] = std::sin(ang[i]);
    }
    Tensor di = upload(in, {2 * half}, DType::Float32), dc = upload(cs, {half}, DType::Float32);
    Tensor ds = upload(sn, {half}, DType::Float32), dout = be().AllocateTensor({2 * half}, DType::Float32);
    be().RoPEPairs(dout.data, di.data, dc.data, ds.data, half, DType::Float32);
    std::vector<float> pref(2 * half);
    EXPECT(or_rope_pairs(pref.data(), in.data(), cs.data(), sn.data(), half) == 0, "oracle pairs");
    e = normwise(download_f32(dout, DType::Float32), pref);
    EXPECT(e <= 1e-5, "pairs normwise %.3g", e);
}

CASE(activations_packed_and_unary) {
    // GeGLU packed rows [gate | up] (activation/gated.go) and Silu / Gelu in f32
    const int64_t batch = 37, half = 640;
    auto packed = normal(161, batch * 2 * half, 0.0f, 2.0f);
    Tensor dp = upload(packed, {batch, 2 * half}, DType::Float32), dout = be().AllocateTensor({batch, half}, DType::Float32);
    be().GeGLU(dout.data, dp.data, batch, half, DType::Float32);
    std::vector<float> ref((size_t)(batch * half));
    EXPECT(or_gated_packed(OR_GATE_GEGLU, ref.data(), packed.data(), batch, half, 0) == 0, "oracle geglu");
    double e = normwise(download_f32(dout, DType::Float32), ref);
    EXPECT(e <= 1e-5, "packed GeGLU normwise %.3g", e);
    const int64_t n = 4099;
    auto x = normal(162, n, 0.0f, 3.0f);
    Tensor dx = upload(x, {n}, DType::Float32), dy = be().AllocateTensor({n}, DType::Float32);
    be().Silu(dy.data, dx.data, n, DType::Float32);
    std::vector<float> uref(n);
    EXPECT(or_unary(OR_UNARY_SILU, uref.data(), x.data(), n, 0) == 0, "oracle silu");
    e = normwise(download_f32(dy, DType::Float32), uref);
    EXPECT(e <= 1e-5, "Silu normwise %.3g", e);
    be().Gelu(dy.data, dx.data, n, DType::Float32);
    EXPECT(or_unary(OR_UNARY_GELU, uref.data(), x.data(), n, 0) == 0, "oracle gelu");
    e = normwise(download_f32(dy, DType::Float32), uref);
    EXPECT(e <= 1e-5, "Gelu normwise %.3g", e);
}

CASE(scaled_dot_product_and_flash_attention) {
    // single head, top-left causal mask, FastExp32 online softmax
    // (device/cpu/attention/typed_compute.go:31-97)
    for (DType dt : {DType::Float32, DType::BFloat16}) {
        const int64_t sq = 70, sk = 90, d = 64, vd = 48;
        const float sd = dt == DType::Float32 ? 0.25f : 0.125f;
        auto q = encode(normal(171, sq * d, 0.0f, sd), dt), k = encode(normal(172, sk * d, 0.0f, sd), dt);
        auto v = encode(normal(173, sk * vd), dt);
        Tensor dq = upload(q, {sq, d}, dt), dk = upload(k, {sk, d}, dt), dv = upload(v, {sk, vd}, dt);
        Tensor do1 = be().AllocateTensor({sq, vd}, dt), do2 = be().AllocateTensor({sq, vd}, dt);
        FlashAttentionConfig cfg;
        cfg.BlockSize = 64;
        cfg.Causal = true;
        be().ScaledDotProductAttention(cfg, dq.data, dk.data, dv.data, do1.data, sq, sk, d, vd, dt);
        be().FlashAttention(cfg, dq.data, dk.data, dv.data, do2.data, sq, sk, d, vd, dt);
        std::vector<uint8_t> ref((size_t)ByteCount(dt, sq * vd));
        EXPECT(or_flash_attention(1, q.data(), k.data(), v.data(), ref.data(), sq, sk, d, vd, static_cast<int>(dt)) == 0,
               "oracle");
        const double tol = dt == DType::Float32 ? 1e-5 : 1e-2;
        const auto want = decode(ref, dt, sq * vd);
        double e = normwise(download_f32(do1, dt), want);
        EXPECT(e <= tol, "%s SDPA normwise %.3g", Name(dt), e);
        e = normwise(download_f32(do2, dt), want);
        EXPECT(e <= tol, "%s Flash normwise %.3g", Name(dt), e);
    }
}

CASE(kv_page_write_fp8_and_dequant4) {
    // the quantising page write: byte = E4M3(value / scale[kv head]), bit-exact
    const int64_t pages = 12, ps = 16, kvh = 4, hd = 128, inner = kvh * hd, rows = 30;
    std::vector<uint8_t> pool((size_t)(pages * ps * inner));
    for (size_t i = 0; i < pool.size(); ++i) pool[i] = (uint8_t)(i * 131 + 7);
    std::vector<int32_t> ids(rows), offs(rows);
    for (int64_t r = 0; r < rows; ++r) {
        ids[r] = (int32_t)((r * 5 + 1) % pages);
        offs[r] = (int32_t)((r * 3) % ps);
    }
    // distinct (page, slot) per row
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t q = 0; q < r; ++q) EXPECT(ids[r] != ids[q] || offs[r] != offs[q], "duplicate slot in the setup");
    std::vector<float> scales = {0.5f, 0.03f, 1.0f, 0.2f};
    auto vals = encode(normal(181, rows * inner, 0.0f, 30.0f), DType::BFloat16);
    Tensor dpool = upload(pool, {pages, ps, inner}, DType::Float8E4M3), dv = upload(vals, {rows, inner}, DType::BFloat16);
    Tensor di = upload(ids, {rows}, DType::Int32), doff = upload(offs, {rows}, DType::Int32);
    Tensor dsc = upload(scales, {kvh}, DType::Float32);
    be().KVPageWriteFP8(dpool.data, dv.data, di.data, doff.data, pages, ps, kvh, hd, rows, 0, dsc.data,
                        DType::BFloat16);
    std::vector<uint8_t> ref = pool;
    EXPECT(or_page_write_fp8(ref.data(), vals.data(), ids.data(), offs.data(), pages, ps, kvh, hd, rows, 0,
                             scales.data(), OR_BF16) == 0, "oracle");
    EXPECT(download(dpool) == ref, "fp8 page write");
    be().CheckStatus();
    // Dequant4: packed signed nibbles (low first), (code - zero point) * scale
    const int64_t n = 1001;
    std::vector<uint8_t> packed((size_t)((n + 1) / 2));
    for (size_t i = 0; i < packed.size(); ++i) packed[i] = (uint8_t)(i * 37 + 11);
    Tensor dpk = upload(packed, {n}, DType::Int4), dout = be().AllocateTensor({n}, DType::Float32);
    DequantInt4Config c4;
    c4.Scale = 0.75f;
    c4.ZeroPoint = -3;
    be().Dequant4(dout.data, dpk.data, n, c4, DType::Float32, DType::Int4);
    std::vector<float> dref(n);
    EXPECT(or_dequant_int4(dref.data(), packed.data(), n, 0.75f, -3) == 0, "oracle dequant4");
    const auto got = download(dout);
    EXPECT(std::memcmp(got.data(), dref.data(), got.size()) == 0, "Dequant4");
}

CASE(host_threads_with_their_own_streams) {
    // The shim must be thread-safe (one context, a stream per backend): four host
    // threads, each with its own stream and Backend, run the split-K Matmul and
    // one-row MultiHeadAttention at head dim 128 (the decode kernels) and 64 (the
    // general kernel split over key chunks) (all three lease the library's shared
    // split-K scratch, ordered across streams by its completion event) and RMSNorm, 12 rounds each,
    // all at once; every result equals the single-threaded one.  The scratch is
    // grown to its final size by the single-threaded pass first, so the threads
    // only share it.
    const DType bf = DType::BFloat16;
    const int64_t M = 64, K = 4096, N = 1024, H = 32, KVH = 8, D = 128, SK = 1500, R = 256, HID = 4096;
    auto a = encode(normal(191, M * K), bf), b = encode(normal(192, K * N, 0.0f, 0.05f), bf);
    auto q = encode(normal(193, H * D, 0.0f, 0.3f), bf), k = encode(normal(194, SK * KVH * D, 0.0f, 0.3f), bf);
    auto v = encode(normal(195, SK * KVH * D), bf), x = encode(normal(196, R * HID), bf);
    auto g = encode(normal(197, HID, 1.0f, 0.02f), bf);
    Tensor da = upload(a, {M, K}, bf), db = upload(b, {K, N}, bf), dq = upload(q, {1, H * D}, bf);
    Tensor dk = upload(k, {SK, KVH * D}, bf), dv = upload(v, {SK, KVH * D}, bf), dx = upload(x, {R, HID}, bf);
    Tensor dg = upload(g, {HID}, bf);
    MultiHeadAttentionConfig mha;
    mha.NumHeads = H;
    mha.HeadDim = D;
    mha.Causal = true;
    mha.KVHeadCount = KVH;
    MultiHeadAttentionConfig mha64 = mha;   // the same buffers as 64 heads of 64 over 16 kv heads
    mha64.NumHeads = 2 * H;
    mha64.HeadDim = D / 2;
    mha64.KVHeadCount = 2 * KVH;
    RMSNormConfig rc;
    rc.Epsilon = 1e-5;
    Tensor rmm = be().AllocateTensor({M, N}, bf), rat = be().AllocateTensor({1, H * D}, bf), rno = be().AllocateTensor({R, HID}, bf);
    be().Matmul(rmm.data, da.data, db.data, M, K, N, bf);
    be().MultiHeadAttention(mha, dq.data, dk.data, dv.data, rat.data, 1, SK, bf);
    Tensor r64 = be().AllocateTensor({1, H * D}, bf);
    be().MultiHeadAttention(mha64, dq.data, dk.data, dv.data, r64.data, 1, SK, bf);
    be().RMSNorm(rc, dx.data, dg.data, rno.data, R, HID, bf);
    const auto want_mm = download(rmm), want_at = download(rat), want_no = download(rno), want_64 = download(r64);
    constexpr int T = 4, ROUNDS = 12;
    std::atomic<int> failures{0};
    std::vector<std::string> why(T);
    std::vector<std::thread> threads;
    for (int t = 0; t < T; ++t) {
        threads.emplace_back([&, t] {
            void *stream = nullptr;
            try {
                Check(puter_hip_stream_create(&stream));
                Backend mine(stream);
                Tensor omm = mine.AllocateTensor({M, N}, bf), oat = mine.AllocateTensor({1, H * D}, bf);
                Tensor ono = mine.AllocateTensor({R, HID}, bf), o64 = mine.AllocateTensor({1, H * D}, bf);
                std::vector<uint8_t> got;
                for (int round = 0; round < ROUNDS; ++round) {
                    mine.Matmul(omm.data, da.data, db.data, M, K, N, bf);
                    mine.MultiHeadAttention(mha, dq.data, dk.data, dv.data, oat.data, 1, SK, bf);
                    mine.MultiHeadAttention(mha64, dq.data, dk.data, dv.data, o64.data, 1, SK, bf);
                    mine.RMSNorm(rc, dx.data, dg.data, ono.data, R, HID, bf);
                    got.resize(want_mm.size());
                    mine.Download(got.data(), omm.data, got.size());
                    if (got != want_mm) throw std::runtime_error("Matmul differs in round " + std::to_string(round));
                    got.resize(want_at.size());
                    mine.Download(got.data(), oat.data, got.size());
                    if (got != want_at) throw std::runtime_error("attention differs in round " + std::to_string(round));
                    got.resize(want_64.size());
                    mine.Download(got.data(), o64.data, got.size());
                    if (got != want_64) throw std::runtime_error("head-dim-64 attention differs in round " + std::to_string(round));
                    got.resize(want_no.size());
                    mine.Download(got.data(), ono.data, got.size());
                    if (got != want_no) throw std::runtime_error("RMSNorm differs in round " + std::to_string(round));
                }
            } catch (const std::exception &e) {
                why[t] = e.what();
                ++failures;
            }
            if (stream) {
                puter_hip_stream_synchronize(stream);
                puter_hip_stream_destroy(stream);
            }
        });
    }
    for (auto &th : threads) th.join();
    for (int t = 0; t < T; ++t) EXPECT(why[t].empty(), "thread %d: %s", t, why[t].c_str());
    EXPECT(failures == 0, "%d threads failed", failures.load());
}

int main(int argc, char **argv) {
    int count = 0;
    if (puter_hip_device_count(&count) != 0 || count < 1) {
        std::printf("no GPU\n");
        return 2;
    }
    return check::run_all(argc, argv);
}
