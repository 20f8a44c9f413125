// CPU tier for the C++ host side: the kernel-registry mirror's semantics
// (kernels/registry.go:49-127), the HIP backend's registrations, and the Go
// contract's error behaviour for calls the library rejects before touching a
// device (a panic becomes puter::hip::Error with the bridge's status code; a Go
// `error` result becomes a MaybeError).  No GPU work: nothing here launches.
#include <algorithm>
#include <set>

#include "backend.hpp"
#include "check.hpp"
#include "kernels.hpp"

using namespace puter::hip;
namespace K = puter::hip::kernels;

static void *const FAKE = reinterpret_cast<void *>(0x1000);   // never dereferenced on these paths

static K::Kernel make(const char *name, std::vector<DType> in, std::vector<DType> out, std::vector<Location> locs) {
    K::Kernel k;
    k.Name = name;
    k.Signature = K::Signature{K::Layout::Dense, std::move(in), std::move(out)};
    k.Locations = std::move(locs);
    k.Run = [](const std::vector<Tensor> &) { return MaybeError{}; };
    return k;
}

template <class F> static int status_of(F &&f) {
    try {
        f();
    } catch (const Error &e) {
        return e.Status();
    }
    return 0;
}

CASE(registry_semantics_match_the_reference) {
    // duplicates (same name, equal signature, overlapping locations) panic; an
    // empty location list overlaps everything; LookupLocation needs the
    // location; Lookup returns the first match
    K::Registry r;
    using D = DType;
    r.Register(make("page_write", {D::Float32}, {D::Float32}, {Location::Host}));
    r.Register(make("page_write", {D::Float32}, {D::Float32}, {Location::Device}));     // other location
    r.Register(make("page_write", {D::BFloat16}, {D::BFloat16}, {Location::Device}));   // other signature
    EXPECT(status_of([&] { r.Register(make("page_write", {D::Float32}, {D::Float32}, {Location::Device})); }) ==
               PUTER_ERR_INVALID, "duplicate registration must panic");
    EXPECT(status_of([&] { r.Register(make("page_write", {D::BFloat16}, {D::BFloat16}, {})); }) == PUTER_ERR_INVALID,
           "an empty location list overlaps every other");
    const K::Signature sig{K::Layout::Dense, {D::Float32}, {D::Float32}};
    auto dev = r.LookupLocation("page_write", sig, Location::Device);
    EXPECT(dev && dev->Locations == std::vector<Location>{Location::Device}, "LookupLocation");
    auto first = r.Lookup("page_write", sig);
    EXPECT(first && first->Locations == std::vector<Location>{Location::Host}, "Lookup returns the first match");
    EXPECT(!r.LookupLocation("page_gather", sig, Location::Device), "unknown name");
    EXPECT(r.Snapshot().size() == 3, "snapshot holds %zu kernels", r.Snapshot().size());
}

CASE(hip_registrations) {
    Backend be;
    K::Registry r;
    K::RegisterHIPKernels(r, be);
    std::set<std::string> names;
    for (const K::Kernel &k : r.Snapshot()) {
        names.insert(k.Name);
        EXPECT(k.Locations == std::vector<Location>{Location::Device}, "%s registered off the device", k.Name.c_str());
    }
    for (const char *n : {"page_write", "page_gather", "layernorm", "swiglu", "geglu", "geglu_tanh", "siglu", "glu",
                          "reglu", "linglu", "seglu", "silu", "gelu", "cast", "matmul", "multi_head_attention",
                          "grouped_query_attention", "sliding_window_attention", "attention", "flash_attention",
                          "int8_dequant", "int4_dequant", "int8_quant"})
        EXPECT(names.count(n), "%s not registered", n);
    // page: 4 formats x 2; 3 formats x (layernorm + 8 gated + silu + gelu); matmul 4;
    // casts 6 x 5 float pairs + int8 <-> f32; attention 3 formats x 5; quantisation 3
    EXPECT(r.Snapshot().size() == 8 + 33 + 4 + 32 + 15 + 3, "%zu kernels", r.Snapshot().size());
    // the reference's own page signatures (slice_register.go:40-78) resolve to the
    // HIP kernels for device tensors, not for host ones
    for (DType dt : {DType::Float32, DType::BFloat16, DType::Float16}) {
        const K::Signature w{K::Layout::Dense, {dt, dt, DType::Int32, DType::Int32, DType::Int32}, {dt}};
        const K::Signature g{K::Layout::Dense, {dt, DType::Int32, DType::Int32}, {dt}};
        EXPECT(r.LookupLocation("page_write", w, Location::Device), "page_write %s", Name(dt));
        EXPECT(r.LookupLocation("page_gather", g, Location::Device), "page_gather %s", Name(dt));
        EXPECT(!r.LookupLocation("page_write", w, Location::Host), "page_write on host %s", Name(dt));
    }
    // the init() registers each kernel once: running it again panics
    EXPECT(status_of([&] { K::RegisterHIPKernels(r, be); }) == PUTER_ERR_INVALID, "second init() must panic");
    // CPU host registrations and the HIP device ones coexist in one registry
    K::Registry both;
    both.Register(make("page_write", {DType::Float32, DType::Float32, DType::Int32, DType::Int32, DType::Int32},
                       {DType::Float32}, {Location::Host}));
    K::RegisterHIPKernels(both, be);
}

CASE(run_wrappers_reject_bad_arguments) {
    // a Run wrapper returns the error the reference's Run returns; shape checks
    // come before any device call
    Backend be;
    K::Registry r;
    K::RegisterHIPKernels(r, be);
    const K::Signature cast_sig{K::Layout::Dense, {DType::Float32}, {DType::BFloat16}};
    auto cast = r.LookupLocation("cast", cast_sig, Location::Device);
    EXPECT(cast, "cast f32 -> bf16");
    MaybeError err = cast->Run({Wrap(FAKE, {4}, DType::Float32), Wrap(FAKE, {5}, DType::BFloat16)});
    EXPECT(err && std::string(err->what()) == "convert: length mismatch", "ErrLenMismatch expected");
    const K::Signature mm{K::Layout::Dense, {DType::BFloat16, DType::BFloat16}, {DType::BFloat16}};
    auto matmul = r.LookupLocation("matmul", mm, Location::Device);
    err = matmul->Run({Wrap(FAKE, {4, 3}, DType::BFloat16), Wrap(FAKE, {4, 5}, DType::BFloat16),
                       Wrap(FAKE, {4, 5}, DType::BFloat16)});
    EXPECT(err && err->Status() == PUTER_ERR_INVALID, "inner dimension mismatch");
    err = matmul->Run({Wrap(FAKE, {4, 3}, DType::BFloat16)});
    EXPECT(err && err->Status() == PUTER_ERR_INVALID, "argument count");
    const K::Signature pw{K::Layout::Dense, {DType::BFloat16, DType::BFloat16, DType::Int32, DType::Int32, DType::Int32},
                          {DType::BFloat16}};
    auto write = r.LookupLocation("page_write", pw, Location::Device);
    int32_t page_size = 16;   // a host scalar tensor: read without a device
    err = write->Run({Wrap(FAKE, {8, 4, 32}, DType::BFloat16), Wrap(FAKE, {2, 32}, DType::BFloat16),
                      Wrap(FAKE, {2}, DType::Int32), Wrap(FAKE, {2}, DType::Int32),
                      Wrap(&page_size, {1}, DType::Int32, Location::Host), Wrap(FAKE, {8, 4, 32}, DType::BFloat16)});
    EXPECT(err && err->Status() == PUTER_ERR_INVALID, "storage page size 4 against the scalar 16");
}

CASE(backend_panics_carry_the_bridge_codes) {
    Backend be;
    RMSNormConfig bad;
    bad.Epsilon = 0.0;   // device/config.go:86-92: epsilon must be > 0
    EXPECT(status_of([&] { be.RMSNorm(bad, FAKE, FAKE, FAKE, 4, 8, DType::Float32); }) == PUTER_ERR_INVALID, "eps");
    EXPECT(status_of([&] { be.RMSNorm(RMSNormConfig{}, nullptr, FAKE, FAKE, 4, 8, DType::Float32); }) == PUTER_ERR_NIL,
           "nil input");
    EXPECT(status_of([&] { be.RMSNorm(RMSNormConfig{}, FAKE, FAKE, FAKE, 4, 8, DType::Int8); }) == PUTER_ERR_INVALID,
           "unsupported dtype");
    // zero-sized work returns without launching (layernorm/compute.go:19-21)
    EXPECT(status_of([&] { be.RMSNorm(RMSNormConfig{}, nullptr, nullptr, nullptr, 0, 8, DType::Float32); }) == 0,
           "zero rows");
    MultiHeadAttentionConfig mha;
    mha.NumHeads = 6;
    mha.HeadDim = 64;
    mha.KVHeadCount = 4;   // 6 heads do not divide into 4 kv heads
    EXPECT(status_of([&] { be.MultiHeadAttention(mha, FAKE, FAKE, FAKE, FAKE, 4, 4, DType::BFloat16); }) ==
               PUTER_ERR_INVALID, "kv heads");
    EXPECT(status_of([&] { be.Matmul(FAKE, FAKE, FAKE, -1, 4, 4, DType::Float32); }) == PUTER_ERR_INVALID,
           "negative shape");
    try {
        be.Cast(FAKE, DType::Int32, FAKE, DType::Float32, 4);
        EXPECT(false, "an unsupported cast must panic");
    } catch (const Error &e) {
        EXPECT(e.Status() == PUTER_ERR_INVALID && std::string(e.what()).size() > 0, "message");
    }
}

CASE(workspace_slot_errors) {
    // execution/workspace_resident.go:12-20: both methods return (tensor, error)
    Backend be;
    auto [slot, err] = be.AllocateWorkspaceSlot(0);
    EXPECT(err && err->Status() == PUTER_ERR_INVALID, "byteCount 0 is tensor.ErrShapeInvalid");
    Tensor fake = Wrap(FAKE, {256}, DType::Int8);
    auto [view, verr] = be.ViewWorkspaceSlot(fake, {32}, DType::Float64, 256);
    EXPECT(!verr && view.data == FAKE && view.byteCount == 256 && view.format == DType::Float64, "view");
    auto [over, oerr] = be.ViewWorkspaceSlot(fake, {33}, DType::Float64, 264);
    EXPECT(oerr && oerr->Status() == PUTER_ERR_INVALID && !over.data, "view beyond the slot");
    EXPECT(!be.BeginBatch(), "BeginBatch");
}

int main(int argc, char **argv) { return check::run_all(argc, argv); }
