// C++ mirror of the reference's kernel registry (kernels/registry.go) and the HIP
// backend's registrations into it.
//
// The reference keys tensor-level kernels by name + Signature{Layout, Inputs,
// Outputs} + Locations (kernels/registry.go:15-29) in a process-wide registry
// (`Default`, :147); a duplicate name / signature with overlapping locations
// panics (:49-70), Lookup returns the first kernel of a name and signature
// (:75-87), LookupLocation the first that also lists a location (:107-127).  A
// device package registers from its init(); RegisterHIPKernels is that init()
// for this backend: the reference's own registered names and signatures
// (page_write / page_gather, device/cpu/shape/slice_register.go:9-78), the ops
// whose Run is fixed by its tensors (layernorm, the gated activations, silu /
// gelu, casts, matmul) and the names the reference's CPU backend registers with
// default configs on this path (multi_head_attention, grouped_query_attention,
// sliding_window_attention, attention, flash_attention, int8_dequant,
// int4_dequant, int8_quant), all under Location::Device.
#pragma once

#include <functional>
#include <mutex>
#include <optional>
#include <string>
#include <unordered_map>
#include <vector>

#include "backend.hpp"

namespace puter::hip::kernels {

enum class Layout { Dense };   // tensor.LayoutDense

struct Signature {   // kernels/registry.go:15-19
    Layout layout = Layout::Dense;
    std::vector<DType> Inputs;
    std::vector<DType> Outputs;

    bool Equal(const Signature &other) const;   // :129-140
    std::string String() const;
};

struct Kernel {   // :24-29
    std::string Name;
    kernels::Signature Signature;
    std::vector<Location> Locations;
    // func(args ...tensor.Tensor) error
    std::function<MaybeError(const std::vector<Tensor> &args)> Run;
};

class Registry {   // :34-127
public:
    // Duplicate name / signature with overlapping locations throws Error (the Go
    // registry panics); an empty location list overlaps every other.
    void Register(Kernel kernel);
    std::optional<Kernel> Lookup(const std::string &name, const kernels::Signature &signature) const;
    std::optional<Kernel> LookupLocation(const std::string &name, const kernels::Signature &signature,
                                         Location location) const;
    std::vector<Kernel> Snapshot() const;

private:
    mutable std::mutex mu_;
    std::unordered_map<std::string, std::vector<Kernel>> kernels_;
};

Registry &Default();   // kernels.Default

// The Go package's init(): every HIP kernel above under Location::Device, run on
// `backend` (which must outlive the registry's use of them).  Throws Error on a
// duplicate, as Register panics.
void RegisterHIPKernels(Registry &registry, Backend &backend);

}  // namespace puter::hip::kernels
