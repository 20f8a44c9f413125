"""CPU tier: the kernel-registry mirror (kernels/registry.go) and the HIP
backend's registrations into it (no GPU work: only loading the library)."""
import pytest

import puter_amd
from puter_amd import registry as R


def _k(name, inputs, outputs, locs):
    return R.Kernel(name, R.Signature(R.LAYOUT_DENSE, tuple(inputs), tuple(outputs)), locs, lambda *a: None)


def test_registry_semantics_match_the_reference():
    """kernels/registry.go:49-127: duplicates (same name, equal signature,
    overlapping locations) panic; an empty location list overlaps everything;
    LookupLocation needs the location; Lookup returns the first match."""
    r = R.Registry()
    r.Register(_k("page_write", [R.F32], [R.F32], [R.LOCATION_HOST]))
    r.Register(_k("page_write", [R.F32], [R.F32], [R.LOCATION_DEVICE]))      # other location: fine
    r.Register(_k("page_write", [R.BF16], [R.BF16], [R.LOCATION_DEVICE]))    # other signature: fine
    with pytest.raises(R.RegistryError):
        r.Register(_k("page_write", [R.F32], [R.F32], [R.LOCATION_DEVICE]))
    with pytest.raises(R.RegistryError):
        r.Register(_k("page_write", [R.BF16], [R.BF16], []))                 # empty overlaps all
    sig = R.Signature(R.LAYOUT_DENSE, (R.F32,), (R.F32,))
    k, ok = r.LookupLocation("page_write", sig, R.LOCATION_DEVICE)
    assert ok and k.Locations == [R.LOCATION_DEVICE]
    k, ok = r.Lookup("page_write", sig)
    assert ok and k.Locations == [R.LOCATION_HOST]
    assert not r.LookupLocation("page_gather", sig, R.LOCATION_DEVICE)[1]
    assert len(r.Snapshot()) == 3


def test_hip_registrations():
    r = R.register_hip_kernels(R.Registry(), puter_amd.Backend())
    names = {k.Name for k in r.Snapshot()}
    assert {"page_write", "page_gather", "layernorm", "swiglu", "geglu", "geglu_tanh", "siglu", "glu",
            "reglu", "linglu", "seglu", "silu", "gelu", "cast",
            "matmul", "multi_head_attention", "grouped_query_attention", "sliding_window_attention",
            "attention", "flash_attention", "int8_dequant", "int4_dequant", "int8_quant"} <= names
    assert all(k.Locations == [R.LOCATION_DEVICE] for k in r.Snapshot())
    # the reference's own page signatures (device/cpu/shape/slice_register.go:40-78)
    # resolve to the HIP kernels for device tensors
    for dt in (R.F32, R.BF16, R.F16):
        w = R.Signature(R.LAYOUT_DENSE, (dt, dt, R.I32, R.I32, R.I32), (dt,))
        g = R.Signature(R.LAYOUT_DENSE, (dt, R.I32, R.I32), (dt,))
        assert r.LookupLocation("page_write", w, R.LOCATION_DEVICE)[1]
        assert r.LookupLocation("page_gather", g, R.LOCATION_DEVICE)[1]
        assert not r.LookupLocation("page_write", w, R.LOCATION_HOST)[1]
    # the init() registers each kernel once: a second run panics on the first duplicate
    with pytest.raises(R.RegistryError):
        R.register_hip_kernels(r, puter_amd.Backend())
    # CPU host registrations and the HIP device ones coexist in one registry
    both = R.Registry()
    both.Register(_k("page_write", [R.F32, R.F32, R.I32, R.I32, R.I32], [R.F32], [R.LOCATION_HOST]))
    R.register_hip_kernels(both, puter_amd.Backend())
