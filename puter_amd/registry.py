"""Host-side mirror of the reference's kernel registry (kernels/registry.go) and
the HIP backend's registrations into it.

The reference keys tensor-level kernels by name + Signature{Layout, Inputs,
Outputs} + Locations (kernels/registry.go:15-29) in a process-wide registry
(`Default`, :147); a duplicate name/signature with overlapping locations
panics (:49-70).  The CPU backend registers page_write / page_gather / slice
for tensor.Host from an init() (device/cpu/shape/slice_register.go:9-78).  A Go
`device/hip` package registers its device kernels the same way; this module is
that registration for the Python host side, with the same names, signatures
and Run(args...) argument order, so a lookup by (name, signature, location)
finds the HIP kernel exactly where it would find the CPU one for host tensors.

Location: manifesto has no ROCm tensor.Location (pool/device_id.go:59-74), so the
HIP kernels register under the device location the dispatcher already routes
(`LOCATION_DEVICE`, the reference's tensor.CUDA) -- nothing else registers for it.

Only kernels whose behaviour is fixed by their tensors are registered (Run takes
tensors, no config): paged KV write / gather (the reference's own registered
names), LayerNorm (its epsilon is fixed at 1e-5, device/cpu/layernorm/compute.go:11),
the gated activations in tensor form, Silu / Gelu, the dtype casts, Matmul, and
the names the reference's CPU backend registers with default configs on this
path: multi_head_attention / grouped_query_attention / sliding_window_attention
(NumHeads 8, HeadDim 64; KV heads 2 for GQA; causal, window 128 for the sliding
one: device/cpu/attention/attention_variants.go:27-60,
attention_variants_dtype.go:14-25, registered at
device/cpu/neon/remaining_ops_dtype.go:252-290,737-777), attention /
flash_attention (single head, BlockSize 64, not causal: attention.go:141-152,
flash_attention.go:38-40,132-141), int8_dequant / int4_dequant / int8_quant
(scale 1, zero point 0: dequant/tensor.go:7-21, quant/tensor.go:8-14,
dequant/config.go:13-19; remaining_ops_dtype.go:647-665).  Ops that carry a
caller's config (RMSNorm epsilon, RoPE, MultiHeadAttention with other heads)
are reached through the device.Backend methods, as the reference's dispatcher
reaches them.
"""
from dataclasses import dataclass, field
import threading
from typing import Callable, List, Tuple

from . import backend as _be

LAYOUT_DENSE = "dense"          # tensor.LayoutDense
LOCATION_HOST = "host"          # tensor.Host
LOCATION_DEVICE = "cuda"        # tensor.CUDA: the device location HIP kernels register under

# dtype names of manifesto/dtype for the formats on the path, mapped to the
# library's codes
F32, F16, BF16, F8E4M3, F8E5M2, I32, I8, I4, F64 = ("float32", "float16", "bfloat16", "float8e4m3",
                                                   "float8e5m2", "int32", "int8", "int4", "float64")
_CODE = {F32: _be.F32, F16: _be.F16, BF16: _be.BF16, F8E4M3: _be.F8E4M3, F8E5M2: _be.F8E5M2,
         I32: _be.I32, I8: _be.I8, I4: _be.I4, F64: _be.F64}


class RegistryError(RuntimeError):
    """The Go registry panics; the mirror raises."""


@dataclass(frozen=True)
class Signature:  # kernels/registry.go:15-19
    Layout: str
    Inputs: Tuple[str, ...]
    Outputs: Tuple[str, ...]

    def Equal(self, other: "Signature") -> bool:  # :129-140
        return self.Layout == other.Layout and self.Inputs == other.Inputs and self.Outputs == other.Outputs


@dataclass
class Kernel:  # :24-29
    Name: str
    Signature: Signature
    Locations: List[str]
    Run: Callable = field(repr=False)


def _overlap(a, b):  # locationsOverlap :149-...: an empty list overlaps everything
    if not a or not b:
        return True
    return any(x in b for x in a)


class Registry:  # :34-127
    def __init__(self):
        self._mu = threading.RLock()
        self._kernels = {}

    def Register(self, kernel: Kernel) -> None:
        with self._mu:
            for existing in self._kernels.get(kernel.Name, []):
                if existing.Signature.Equal(kernel.Signature) and _overlap(existing.Locations, kernel.Locations):
                    raise RegistryError(f"kernels: duplicate registration for {kernel.Name!r} "
                                        f"with signature {kernel.Signature}")
            self._kernels.setdefault(kernel.Name, []).append(kernel)

    def Lookup(self, name: str, signature: Signature):
        with self._mu:
            for k in self._kernels.get(name, []):
                if k.Signature.Equal(signature):
                    return k, True
        return None, False

    def LookupLocation(self, name: str, signature: Signature, location: str):
        with self._mu:
            for k in self._kernels.get(name, []):
                if k.Signature.Equal(signature) and location in k.Locations:
                    return k, True
        return None, False

    def Snapshot(self) -> List[Kernel]:
        with self._mu:
            return [k for ks in self._kernels.values() for k in ks]


Default = Registry()


# ---- tensor helpers: torch device tensors carry shape and dtype ---------------
def _dtype_name(t) -> str:
    import torch
    return {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16, torch.float8_e4m3fn: F8E4M3,
            torch.float8_e5m2: F8E5M2, torch.int32: I32, torch.int8: I8, torch.float64: F64}[t.dtype]


def _scalar_int(t) -> int:
    """int32ScalarTensor (device/cpu/shape/page.go): a one-element Int32 tensor.
    A device scalar is read back (the reference's RawBytes read does the same)."""
    if isinstance(t, int):
        return t
    if t.numel() != 1:
        raise _be.PuterError(_be._lib.ERR_INVALID, "tensor: shape mismatch (scalar expected)")
    return int(t.reshape(()).item())


def _mismatch():
    return _be.PuterError(_be._lib.ERR_INVALID, "tensor: shape mismatch")


def _prod(dims):
    n = 1
    for d in dims:
        n *= int(d)
    return n


# ---- Run wrappers -------------------------------------------------------------
def _page_write(be, dt):
    """args: storage, values, pageIDs, offsets, pageSize, out (device/cpu/shape/page.go:14-44)."""
    def run(*args):
        if len(args) != 6:
            raise _mismatch()
        storage, values, ids, offs, ps, out = args
        page_size = _scalar_int(ps)
        sd = tuple(storage.shape)
        if (len(sd) < 2 or values.dim() != len(sd) - 1 or tuple(out.shape) != sd or sd[1] != page_size
                or ids.numel() != offs.numel() or values.shape[0] < ids.numel()
                or _prod(values.shape[1:]) != _prod(sd[2:])):
            raise _mismatch()
        be.KVPageWrite(storage, values, ids, offs, out, sd[0], page_size, _prod(sd[2:]), ids.numel(), 0,
                       _CODE[dt])
    return run


def _page_gather(be, dt):
    """args: storage, pageTable, pageSize, out (device/cpu/shape/page.go:46-...)."""
    def run(*args):
        if len(args) != 4:
            raise _mismatch()
        storage, table, ps, out = args
        page_size = _scalar_int(ps)
        sd = tuple(storage.shape)
        if len(sd) < 2 or out.dim() != len(sd) - 1 or sd[1] != page_size or _prod(out.shape[1:]) != _prod(sd[2:]):
            raise _mismatch()
        rows = min(int(out.shape[0]), table.numel() * page_size)
        be.KVPageGather(storage, table, out, sd[0], page_size, _prod(sd[2:]), rows, 0, _CODE[dt])
    return run


def _layernorm(be, dt):
    """args: input, scale, bias, out; rows = all leading dims (compute.go:14-33)."""
    def run(*args):
        if len(args) != 4:
            raise _mismatch()
        x, g, b, out = args
        h = int(x.shape[-1])
        if tuple(out.shape) != tuple(x.shape) or g.numel() != h or b.numel() != h:
            raise _mismatch()
        be.LayerNorm(x, g, b, out, x.numel() // h if h else 0, h, _CODE[dt])
    return run


def _gated(be, dt, method):
    """args: gate, up, dst (<Kind>Tensors(dst, gate, up, count), activation/gated.go:59-136)."""
    def run(*args):
        if len(args) != 3:
            raise _mismatch()
        gate, up, dst = args
        if gate.numel() != up.numel() or dst.numel() != gate.numel():
            raise _mismatch()
        getattr(be, method)(dst, gate, up, gate.numel(), _CODE[dt])
    return run


def _unary(be, dt, method):
    def run(*args):
        if len(args) != 2 or args[0].numel() != args[1].numel():
            raise _mismatch()
        getattr(be, method)(args[1], args[0], args[0].numel(), _CODE[dt])
    return run


def _cast(be, src, dst):
    """args: src, dst; len(dst) != len(src) is convert.ErrLenMismatch (convert/errors.go:10-15)."""
    def run(*args):
        if len(args) != 2:
            raise _mismatch()
        if args[0].numel() != args[1].numel():
            raise _be.PuterError(_be._lib.ERR_INVALID, _be.ErrLenMismatch)
        be.Cast(args[1], _CODE[dst], args[0], _CODE[src], args[0].numel())
    return run


def _matmul(be, dt):
    """args: left [rows, inner], right [inner, cols], out [rows, cols] (matmul/ops.go:9-15)."""
    def run(*args):
        if len(args) != 3:
            raise _mismatch()
        a, b, out = args
        if a.dim() != 2 or b.dim() != 2 or a.shape[1] != b.shape[0] or tuple(out.shape) != (a.shape[0], b.shape[1]):
            raise _mismatch()
        be.Matmul(out, a, b, int(a.shape[0]), int(a.shape[1]), int(b.shape[1]), _CODE[dt])
    return run


# the reference's default attention configs (attention_variants.go:27-60,
# attention_variants_dtype.go:14-25)
ATTENTION_VARIANTS = (("multi_head_attention", dict()),
                      ("grouped_query_attention", dict(KVHeadCount=2)),
                      ("sliding_window_attention", dict(Causal=True, WindowSize=128)))


def _mha_default(be, dt, overrides):
    """args: query [seqQ, 8*64], key, value [seqK, kvHeads*64], out [seqQ, 8*64]
    (multiHeadAttentionMixedDims, attention_variants_dtype.go:27-64)."""
    cfg = _be.MultiHeadAttentionConfig(NumHeads=8, HeadDim=64, **overrides)
    kvh = cfg.KVHeadCount if cfg.KVHeadCount > 0 else cfg.NumHeads

    def run(*args):
        if len(args) != 4:
            raise _mismatch()
        q, k, v, out = args
        if any(t.dim() != 2 for t in args):
            raise _mismatch()
        qf, kf = cfg.NumHeads * cfg.HeadDim, kvh * cfg.HeadDim
        if q.shape[1] != qf or k.shape[1] != kf or v.shape[1] != kf or out.shape[1] != qf:
            raise _mismatch()
        be.MultiHeadAttention(cfg, q, k, v, out, int(q.shape[0]), int(k.shape[0]), _CODE[dt])
    return run


def _flash_default(be, dt):
    """args: query [seqQ, depth], key [seqK, depth], value [seqK, valueDim], out
    [seqQ, valueDim]; BlockSize 64, not causal (attentionViews, attention.go:154-...)."""
    cfg = _be.FlashAttentionConfig(BlockSize=64, Causal=False)

    def run(*args):
        if len(args) != 4 or any(t.dim() != 2 for t in args):
            raise _mismatch()
        q, k, v, out = args
        sq, depth, sk, vd = int(q.shape[0]), int(q.shape[1]), int(k.shape[0]), int(v.shape[1])
        if k.shape[1] != depth or v.shape[0] != sk or out.shape[0] != sq or out.shape[1] != vd:
            raise _mismatch()
        be.FlashAttention(cfg, q, k, v, out, sq, sk, depth, vd, _CODE[dt])
    return run


def _int8_dequant(be):
    """args: quantized int8, output f32 of the same length; scale 1, zero point 0."""
    def run(*args):
        if len(args) != 2 or args[0].numel() != args[1].numel():
            raise _mismatch()
        be.Dequant(args[1], args[0], args[0].numel(), _be.DequantInt8Config(1.0, 0), _be.F32, _be.I8)
    return run


def _int4_dequant(be):
    """args: packed int4 (two codes per byte, low nibble first), output f32 of at
    most twice the byte count; scale 1, zero point 0 (dequant/tensor.go:48-73)."""
    def run(*args):
        if len(args) != 2 or args[1].numel() > 2 * args[0].numel():
            raise _mismatch()
        be.Dequant4(args[1], args[0], args[1].numel(), _be.DequantInt4Config(1.0, 0), _be.F32, _be.I4)
    return run


def _int8_quant(be):
    """args: input f32, output int8 of the same length; scale 1, zero point 0."""
    def run(*args):
        if len(args) != 2 or args[0].numel() != args[1].numel():
            raise _mismatch()
        be.Quant(args[1], args[0], args[0].numel(), _be.DequantInt8Config(1.0, 0), _be.I8, _be.F32)
    return run


GATED = (("swiglu", "SwiGLUTensors"), ("geglu", "GeGLUTensors"), ("geglu_tanh", "GeGLUTanhTensors"),
         ("siglu", "SiGLUTensors"), ("glu", "GLUTensors"), ("reglu", "ReGLUTensors"),
         ("linglu", "LinGLUTensors"), ("seglu", "SeGLUTensors"))


def register_hip_kernels(registry: Registry = None, backend=None) -> Registry:
    """The Go package's init(): register every HIP kernel above under
    LOCATION_DEVICE.  Raises RegistryError on a duplicate, as Register panics."""
    registry = Default if registry is None else registry
    be = backend if backend is not None else _be.Backend()
    dense = LAYOUT_DENSE

    def reg(name, inputs, outputs, run):
        registry.Register(Kernel(name, Signature(dense, tuple(inputs), tuple(outputs)), [LOCATION_DEVICE], run))

    # the reference's registered names and signatures (slice_register.go:40-78), plus fp8 pools
    for dt in (F32, BF16, F16, F8E4M3):
        reg("page_write", [dt, dt, I32, I32, I32], [dt], _page_write(be, dt))
        reg("page_gather", [dt, I32, I32], [dt], _page_gather(be, dt))
    for dt in (F32, BF16, F16):
        reg("layernorm", [dt, dt, dt], [dt], _layernorm(be, dt))
        for name, method in GATED:
            reg(name, [dt, dt], [dt], _gated(be, dt, method))
        reg("silu", [dt], [dt], _unary(be, dt, "Silu"))
        reg("gelu", [dt], [dt], _unary(be, dt, "Gelu"))
    for dt in (F32, BF16, F16, F64):
        reg("matmul", [dt, dt], [dt], _matmul(be, dt))
    floats = (F32, BF16, F16, F8E4M3, F8E5M2, F64)
    for src in floats:
        for dst in floats:
            if src != dst:
                reg("cast", [src], [dst], _cast(be, src, dst))
    reg("cast", [I8], [F32], _cast(be, I8, F32))
    reg("cast", [F32], [I8], _cast(be, F32, I8))
    for dt in (F32, BF16, F16):
        for name, overrides in ATTENTION_VARIANTS:
            reg(name, [dt, dt, dt], [dt], _mha_default(be, dt, overrides))
        reg("attention", [dt, dt, dt], [dt], _flash_default(be, dt))
        reg("flash_attention", [dt, dt, dt], [dt], _flash_default(be, dt))
    reg("int8_dequant", [I8], [F32], _int8_dequant(be))
    reg("int4_dequant", [I4], [F32], _int4_dequant(be))
    reg("int8_quant", [F32], [I8], _int8_quant(be))
    return registry
