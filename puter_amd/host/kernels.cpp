// Kernel registry mirror and the HIP backend's registrations (see kernels.hpp).
#include "kernels.hpp"

#include <algorithm>
#include <cstring>

namespace puter::hip::kernels {

bool Signature::Equal(const Signature &other) const {
    return layout == other.layout && Inputs == other.Inputs && Outputs == other.Outputs;
}

std::string Signature::String() const {
    std::string s = "{dense [";
    for (size_t i = 0; i < Inputs.size(); ++i) s += (i ? " " : "") + std::string(Name(Inputs[i]));
    s += "] [";
    for (size_t i = 0; i < Outputs.size(); ++i) s += (i ? " " : "") + std::string(Name(Outputs[i]));
    return s + "]}";
}

namespace {

bool locations_overlap(const std::vector<Location> &a, const std::vector<Location> &b) {
    if (a.empty() || b.empty()) return true;
    return std::any_of(a.begin(), a.end(), [&](Location l) { return std::find(b.begin(), b.end(), l) != b.end(); });
}

Error mismatch() { return Error(PUTER_ERR_INVALID, "tensor: shape mismatch"); }

int64_t prod(const std::vector<int64_t> &dims, size_t from) {
    int64_t n = 1;
    for (size_t i = from; i < dims.size(); ++i) n *= dims[i];
    return n;
}

// int32ScalarTensor (device/cpu/shape/page.go): a one-element Int32 tensor; a
// device scalar is read back, as the reference reads its raw bytes
int64_t scalar_int(Backend &be, const Tensor &t) {
    if (t.Numel() != 1 || t.format != DType::Int32) throw Error(PUTER_ERR_INVALID, "tensor: shape mismatch (scalar expected)");
    int32_t v = 0;
    if (t.location == Location::Host) std::memcpy(&v, t.data, sizeof v);
    else be.Download(&v, t.data, sizeof v);
    return v;
}

// Run: the Go Run returns an error; a panic of the backend method it calls
// (Error) is returned as that error
template <class F> MaybeError guarded(F &&f) {
    try {
        f();
    } catch (const Error &e) {
        return e;
    }
    return std::nullopt;
}

using Args = std::vector<Tensor>;
using RunFn = std::function<MaybeError(const Args &)>;

// args: storage, values, pageIDs, offsets, pageSize, out (device/cpu/shape/page.go:14-44)
RunFn page_write(Backend &be, DType dt) {
    return [&be, dt](const Args &a) {
        return guarded([&] {
            if (a.size() != 6) throw mismatch();
            const Tensor &storage = a[0], &values = a[1], &ids = a[2], &offs = a[3], &ps = a[4], &out = a[5];
            const int64_t page_size = scalar_int(be, ps);
            const auto &sd = storage.shape;
            if (sd.size() < 2 || values.Rank() != sd.size() - 1 || out.shape != sd || sd[1] != page_size ||
                ids.Numel() != offs.Numel() || values.shape[0] < ids.Numel() || prod(values.shape, 1) != prod(sd, 2))
                throw mismatch();
            be.KVPageWrite(storage.data, values.data, ids.data, offs.data, out.data, sd[0], page_size, prod(sd, 2),
                           ids.Numel(), 0, dt);
        });
    };
}

// args: storage, pageTable, pageSize, out (device/cpu/shape/page.go:46-...)
RunFn page_gather(Backend &be, DType dt) {
    return [&be, dt](const Args &a) {
        return guarded([&] {
            if (a.size() != 4) throw mismatch();
            const Tensor &storage = a[0], &table = a[1], &ps = a[2], &out = a[3];
            const int64_t page_size = scalar_int(be, ps);
            const auto &sd = storage.shape;
            if (sd.size() < 2 || out.Rank() != sd.size() - 1 || sd[1] != page_size || prod(out.shape, 1) != prod(sd, 2))
                throw mismatch();
            const int64_t rows = std::min<int64_t>(out.shape[0], table.Numel() * page_size);
            be.KVPageGather(storage.data, table.data, out.data, sd[0], page_size, prod(sd, 2), rows, 0, dt);
        });
    };
}

// args: input, scale, bias, out; rows = all leading dims (layernorm/compute.go:14-33)
RunFn layernorm(Backend &be, DType dt) {
    return [&be, dt](const Args &a) {
        return guarded([&] {
            if (a.size() != 4 || a[0].shape.empty()) throw mismatch();
            const int64_t h = a[0].shape.back();
            if (a[3].shape != a[0].shape || a[1].Numel() != h || a[2].Numel() != h) throw mismatch();
            be.LayerNorm(a[0].data, a[1].data, a[2].data, a[3].data, h ? a[0].Numel() / h : 0, h, dt);
        });
    };
}

using GatedMethod = void (Backend::*)(void *, const void *, const void *, int64_t, DType);

// args: gate, up, dst (<Kind>Tensors(dst, gate, up, count), activation/gated.go:59-136)
RunFn gated(Backend &be, DType dt, GatedMethod m) {
    return [&be, dt, m](const Args &a) {
        return guarded([&] {
            if (a.size() != 3 || a[0].Numel() != a[1].Numel() || a[2].Numel() != a[0].Numel()) throw mismatch();
            (be.*m)(a[2].data, a[0].data, a[1].data, a[0].Numel(), dt);
        });
    };
}

using UnaryMethod = void (Backend::*)(void *, const void *, int64_t, DType);

RunFn unary(Backend &be, DType dt, UnaryMethod m) {
    return [&be, dt, m](const Args &a) {
        return guarded([&] {
            if (a.size() != 2 || a[0].Numel() != a[1].Numel()) throw mismatch();
            (be.*m)(a[1].data, a[0].data, a[0].Numel(), dt);
        });
    };
}

// args: src, dst; a length mismatch is convert.ErrLenMismatch (convert/errors.go:10-15)
RunFn cast(Backend &be, DType src, DType dst) {
    return [&be, src, dst](const Args &a) {
        return guarded([&] {
            if (a.size() != 2) throw mismatch();
            if (a[0].Numel() != a[1].Numel()) throw Error(PUTER_ERR_INVALID, "convert: length mismatch");
            be.Cast(a[1].data, dst, a[0].data, src, a[0].Numel());
        });
    };
}

// args: left [rows, inner], right [inner, cols], out [rows, cols] (matmul/ops.go:9-15)
RunFn matmul(Backend &be, DType dt) {
    return [&be, dt](const Args &a) {
        return guarded([&] {
            if (a.size() != 3) throw mismatch();
            const Tensor &l = a[0], &r = a[1], &o = a[2];
            if (l.Rank() != 2 || r.Rank() != 2 || l.shape[1] != r.shape[0] ||
                o.shape != std::vector<int64_t>{l.shape[0], r.shape[1]})
                throw mismatch();
            be.Matmul(o.data, l.data, r.data, l.shape[0], l.shape[1], r.shape[1], dt);
        });
    };
}

// the reference's default attention configs: NumHeads 8, HeadDim 64; KV heads 2
// for GQA; causal with window 128 for the sliding one
// (device/cpu/attention/attention_variants.go:27-60, attention_variants_dtype.go:14-25)
RunFn mha_default(Backend &be, DType dt, MultiHeadAttentionConfig cfg) {
    return [&be, dt, cfg](const Args &a) {
        return guarded([&] {
            if (a.size() != 4) throw mismatch();
            for (const Tensor &t : a)
                if (t.Rank() != 2) throw mismatch();
            const int64_t kvh = cfg.KVHeadCount > 0 ? cfg.KVHeadCount : cfg.NumHeads;
            const int64_t qf = cfg.NumHeads * cfg.HeadDim, kf = kvh * cfg.HeadDim;
            if (a[0].shape[1] != qf || a[1].shape[1] != kf || a[2].shape[1] != kf || a[3].shape[1] != qf)
                throw mismatch();
            be.MultiHeadAttention(cfg, a[0].data, a[1].data, a[2].data, a[3].data, a[0].shape[0], a[1].shape[0], dt);
        });
    };
}

// args: query [seqQ, depth], key [seqK, depth], value [seqK, valueDim], out
// [seqQ, valueDim]; BlockSize 64, not causal (attention.go:141-152)
RunFn flash_default(Backend &be, DType dt) {
    return [&be, dt](const Args &a) {
        return guarded([&] {
            if (a.size() != 4) throw mismatch();
            for (const Tensor &t : a)
                if (t.Rank() != 2) throw mismatch();
            const int64_t sq = a[0].shape[0], depth = a[0].shape[1], sk = a[1].shape[0], vd = a[2].shape[1];
            if (a[1].shape[1] != depth || a[2].shape[0] != sk || a[3].shape[0] != sq || a[3].shape[1] != vd)
                throw mismatch();
            FlashAttentionConfig cfg;
            cfg.BlockSize = 64;
            be.FlashAttention(cfg, a[0].data, a[1].data, a[2].data, a[3].data, sq, sk, depth, vd, dt);
        });
    };
}

}  // namespace

void Registry::Register(Kernel kernel) {
    std::lock_guard<std::mutex> lock(mu_);
    for (const Kernel &existing : kernels_[kernel.Name]) {
        if (existing.Signature.Equal(kernel.Signature) && locations_overlap(existing.Locations, kernel.Locations))
            throw Error(PUTER_ERR_INVALID, "kernels: duplicate registration for \"" + kernel.Name +
                                               "\" with signature " + kernel.Signature.String());
    }
    kernels_[kernel.Name].push_back(std::move(kernel));
}

std::optional<Kernel> Registry::Lookup(const std::string &name, const kernels::Signature &signature) const {
    std::lock_guard<std::mutex> lock(mu_);
    auto it = kernels_.find(name);
    if (it == kernels_.end()) return std::nullopt;
    for (const Kernel &k : it->second)
        if (k.Signature.Equal(signature)) return k;
    return std::nullopt;
}

std::optional<Kernel> Registry::LookupLocation(const std::string &name, const kernels::Signature &signature,
                                               Location location) const {
    std::lock_guard<std::mutex> lock(mu_);
    auto it = kernels_.find(name);
    if (it == kernels_.end()) return std::nullopt;
    for (const Kernel &k : it->second)
        if (k.Signature.Equal(signature) &&
            std::find(k.Locations.begin(), k.Locations.end(), location) != k.Locations.end())
            return k;
    return std::nullopt;
}

std::vector<Kernel> Registry::Snapshot() const {
    std::lock_guard<std::mutex> lock(mu_);
    std::vector<Kernel> all;
    for (const auto &entry : kernels_) all.insert(all.end(), entry.second.begin(), entry.second.end());
    return all;
}

Registry &Default() {
    static Registry registry;
    return registry;
}

void RegisterHIPKernels(Registry &registry, Backend &be) {
    using D = DType;
    auto reg = [&](const char *name, std::vector<D> in, std::vector<D> out, RunFn run) {
        Kernel k;
        k.Name = name;
        k.Signature = kernels::Signature{Layout::Dense, std::move(in), std::move(out)};
        k.Locations = {Location::Device};
        k.Run = std::move(run);
        registry.Register(std::move(k));
    };
    // the reference's registered names and signatures (slice_register.go:40-78), plus fp8 pools
    for (D dt : {D::Float32, D::BFloat16, D::Float16, D::Float8E4M3}) {
        reg("page_write", {dt, dt, D::Int32, D::Int32, D::Int32}, {dt}, page_write(be, dt));
        reg("page_gather", {dt, D::Int32, D::Int32}, {dt}, page_gather(be, dt));
    }
    const std::pair<const char *, GatedMethod> gated_kinds[] = {
        {"swiglu", &Backend::SwiGLUTensors}, {"geglu", &Backend::GeGLUTensors},
        {"geglu_tanh", &Backend::GeGLUTanhTensors}, {"siglu", &Backend::SiGLUTensors},
        {"glu", &Backend::GLUTensors}, {"reglu", &Backend::ReGLUTensors}, {"linglu", &Backend::LinGLUTensors},
        {"seglu", &Backend::SeGLUTensors}};
    for (D dt : {D::Float32, D::BFloat16, D::Float16}) {
        reg("layernorm", {dt, dt, dt}, {dt}, layernorm(be, dt));
        for (const auto &g : gated_kinds) reg(g.first, {dt, dt}, {dt}, gated(be, dt, g.second));
        reg("silu", {dt}, {dt}, unary(be, dt, &Backend::Silu));
        reg("gelu", {dt}, {dt}, unary(be, dt, &Backend::Gelu));
    }
    for (D dt : {D::Float32, D::BFloat16, D::Float16, D::Float64}) reg("matmul", {dt, dt}, {dt}, matmul(be, dt));
    const D floats[] = {D::Float32, D::BFloat16, D::Float16, D::Float8E4M3, D::Float8E5M2, D::Float64};
    for (D src : floats)
        for (D dst : floats)
            if (src != dst) reg("cast", {src}, {dst}, cast(be, src, dst));
    reg("cast", {D::Int8}, {D::Float32}, cast(be, D::Int8, D::Float32));
    reg("cast", {D::Float32}, {D::Int8}, cast(be, D::Float32, D::Int8));
    for (D dt : {D::Float32, D::BFloat16, D::Float16}) {
        MultiHeadAttentionConfig mha;
        mha.NumHeads = 8;
        mha.HeadDim = 64;
        reg("multi_head_attention", {dt, dt, dt}, {dt}, mha_default(be, dt, mha));
        MultiHeadAttentionConfig gqa = mha;
        gqa.KVHeadCount = 2;
        reg("grouped_query_attention", {dt, dt, dt}, {dt}, mha_default(be, dt, gqa));
        MultiHeadAttentionConfig sliding = mha;
        sliding.Causal = true;
        sliding.WindowSize = 128;
        reg("sliding_window_attention", {dt, dt, dt}, {dt}, mha_default(be, dt, sliding));
        reg("attention", {dt, dt, dt}, {dt}, flash_default(be, dt));
        reg("flash_attention", {dt, dt, dt}, {dt}, flash_default(be, dt));
    }
    // int8_dequant / int4_dequant / int8_quant: scale 1, zero point 0
    // (dequant/tensor.go:7-21,48-73, quant/tensor.go:8-14)
    reg("int8_dequant", {D::Int8}, {D::Float32}, [&be](const Args &a) {
        return guarded([&] {
            if (a.size() != 2 || a[0].Numel() != a[1].Numel()) throw mismatch();
            be.Dequant(a[1].data, a[0].data, a[0].Numel(), DequantInt8Config{}, D::Float32, D::Int8);
        });
    });
    reg("int4_dequant", {D::Int4}, {D::Float32}, [&be](const Args &a) {
        return guarded([&] {
            // packed input: its tensor counts elements (two per byte)
            if (a.size() != 2 || a[1].Numel() > a[0].Numel()) throw mismatch();
            be.Dequant4(a[1].data, a[0].data, a[1].Numel(), DequantInt4Config{}, D::Float32, D::Int4);
        });
    });
    reg("int8_quant", {D::Float32}, {D::Int8}, [&be](const Args &a) {
        return guarded([&] {
            if (a.size() != 2 || a[0].Numel() != a[1].Numel()) throw mismatch();
            be.Quant(a[1].data, a[0].data, a[0].Numel(), DequantInt8Config{}, D::Int8, D::Float32);
        });
    });
}

}  // namespace puter::hip::kernels
