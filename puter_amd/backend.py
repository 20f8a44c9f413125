"""Host-side mirror of the reference's device.Backend methods on the hot path.

Method names, argument order and meaning follow device/interface.go (and the
optional execution hooks GatedResidual / KVPageWrite / KVPageGather), so a
test written against this class reads like the reference's Go tests.  Buffers
are torch device tensors (or raw device addresses as ints); every call goes
through the C ABI of libputer_hip.so and raises PuterError where the Go method
would panic.  torch supplies device memory and the stream; all compute is the
HIP library's.
"""
from dataclasses import dataclass, field
import ctypes as C

from . import _lib
from ._lib import check, PuterError  # noqa: F401

F32, F16, BF16, F8E4M3, F8E5M2, I32, I8, I4, F64 = 0, 1, 2, 3, 4, 5, 6, 7, 8
(GATE_SWIGLU, GATE_GEGLU, GATE_GEGLU_TANH, GATE_SIGLU, GATE_GLU, GATE_REGLU, GATE_LINGLU,
 GATE_SEGLU) = range(8)
UNARY_SILU, UNARY_GELU = 0, 1

ErrLenMismatch = "convert: length mismatch"  # convert/errors.go:10-15


def dtype_of(t) -> int:
    import torch
    table = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16,
             torch.float8_e4m3fn: F8E4M3, torch.float8_e5m2: F8E5M2, torch.int32: I32,
             torch.int8: I8, torch.float64: F64}
    return table[t.dtype]


# --- config structs: device/config.go ---------------------------------------
@dataclass
class RMSNormConfig:  # config.go:82-92
    Epsilon: float = 1e-6


@dataclass
class ModulatedLayerNormConfig:  # config.go:94-109
    Epsilon: float = 1e-6
    Set: int = 0


RoPEModeInterleaved, RoPEModeHalf = 0, 1
RoPEScalingNone, RoPEScalingLlama3 = 0, 1


@dataclass
class RoPEConfig:  # config.go:125-134; DefaultRoPEConfig device/cpu/rope/config.go:7-15
    BaseFreq: float = 10000.0
    StartPosition: int = 0
    Mode: int = RoPEModeInterleaved
    Scaling: int = RoPEScalingNone
    ScalingFactor: float = 1.0
    LowFreqFactor: float = 0.0
    HighFreqFactor: float = 0.0
    OriginalContext: int = 0


@dataclass
class MultiAxisRoPEConfig:  # config.go:136-146
    BaseFreq: float = 10000.0
    LatentSeqLen: int = 0
    LatentSide: int = 0
    AxisCount: int = 0
    AxisDim0: int = 0
    AxisDim1: int = 0
    AxisDim2: int = 0
    AxisDim3: int = 0


@dataclass
class MultiHeadAttentionConfig:  # config.go:283-290
    NumHeads: int = 0
    HeadDim: int = 0
    Causal: bool = False
    WindowSize: int = 0
    ALiBiSlope: float = 0.0
    KVHeadCount: int = 0


@dataclass
class DequantInt8Config:  # config.go:268-271
    Scale: float = 1.0
    ZeroPoint: int = 0


@dataclass
class DequantInt4Config:  # config.go:273-276
    Scale: float = 1.0
    ZeroPoint: int = 0


@dataclass
class FlashAttentionConfig:  # config.go:278-281
    BlockSize: int = 0
    Causal: bool = False


def _ptr(x):
    if x is None:
        return None
    if isinstance(x, int):
        return x
    return x.data_ptr()


class DeviceBuffer:
    """A device allocation, or a view of one: the memory backend's device tensor
    (reference: device/metal/workspace_darwin.go:18-77, the backend that
    implements workspace slots).  A view shares its slot's device address with its
    own shape, element format and byte count, and owns nothing."""

    def __init__(self, lib, ptr, shape, element_format, byte_count, owns):
        self._lib, self.ptr, self.shape = lib, ptr, tuple(shape)
        self.element_format, self.byte_count, self.owns = element_format, byte_count, owns

    def data_ptr(self):
        return self.ptr

    def Close(self):
        if self.owns and self.ptr:
            check(self._lib.puter_hip_free(C.c_void_p(self.ptr)))
        self.ptr = 0


class Backend:
    """The MI355X device backend (device.Backend subset on the hot path)."""

    def __init__(self, stream=None):
        self.lib = _lib.load()
        self._stream = stream
        self._status = None   # device int32 status word of the paged-KV hooks
        import torch
        if torch.cuda.is_available():
            self._status_word()   # made here, so no hook call allocates (graph capture)

    def _status_word(self):
        """The backend's device status word (the Go wrapper keeps one per backend):
        the paged-KV hooks store PUTER_ERR_INVALID into it when a page id or slot
        is out of range.  The constructor makes it when a GPU is present."""
        if self._status is None:
            import torch
            self._status = torch.zeros(1, dtype=torch.int32, device="cuda")
        return self._status

    # ---- workspace slots: execution/workspace_resident.go:12-20 ----
    def AllocateWorkspaceSlot(self, byteCount):
        """One device allocation of byteCount bytes (shape [byteCount], Int8), which
        NewResidentWorkspace carves into planned views; it stays on the device
        until Close.  byteCount <= 0 is tensor.ErrShapeInvalid."""
        if byteCount <= 0:
            raise PuterError(_lib.ERR_INVALID, "tensor: invalid shape")
        p = C.c_void_p()
        check(self.lib.puter_hip_malloc(C.byref(p), byteCount))
        return DeviceBuffer(self.lib, p.value, [byteCount], I8, byteCount, True)

    def ViewWorkspaceSlot(self, slot, shape, elementFormat, byteCount):
        """A view of a slot with another shape / element format: the same device
        address, no copy.  byteCount outside [0, slot bytes] is
        tensor.ErrShapeMismatch."""
        if byteCount < 0 or byteCount > slot.byte_count:
            raise PuterError(_lib.ERR_INVALID, "tensor: shape mismatch")
        return DeviceBuffer(self.lib, slot.ptr, shape, elementFormat, byteCount, False)

    def Upload(self, dst, data):
        """Host bytes (a numpy array) into device memory on the backend's stream."""
        check(self.lib.puter_hip_memcpy_htod(_ptr(dst), data.ctypes.data_as(C.c_void_p), data.nbytes,
                                             self.stream()))
        check(self.lib.puter_hip_stream_synchronize(self.stream()))

    def Download(self, src, out):
        """Device memory into a host numpy array (synchronises the stream)."""
        check(self.lib.puter_hip_memcpy_dtoh(out.ctypes.data_as(C.c_void_p), _ptr(src), out.nbytes,
                                             self.stream()))
        check(self.lib.puter_hip_stream_synchronize(self.stream()))
        return out

    def CheckStatus(self):
        """Synchronise, read and clear the status word; raise PuterError with the
        reference's ErrShapeMismatch when a paged-KV call since the last check saw
        an out-of-range page id or slot (device/cpu/shape/page.go:139-146,191-203)."""
        if self._status is None:
            return
        v = int(self._status.item())
        self._status.zero_()
        if v != 0:
            raise PuterError(v, "tensor: shape mismatch (page id or slot out of range)")

    # execution/dispatch.go:120-123 (batchExecutionDevice): launches are already
    # asynchronous on the backend's stream, so BeginBatch does nothing; EndBatch
    # synchronises once and returns the status word's error (None when clear)
    def BeginBatch(self):
        return None

    def EndBatch(self):
        try:
            self.CheckStatus()
        except PuterError as e:
            return e
        return None

    # stream: explicit handle, else torch's current stream on the current device
    def stream(self):
        if self._stream is not None:
            return self._stream if isinstance(self._stream, int) else self._stream.cuda_stream
        try:
            import torch
            if torch.cuda.is_available():
                return torch.cuda.current_stream().cuda_stream
        except ImportError:
            pass
        return None

    # ---- LayerNorm family: device/interface.go:355-379 ----
    def RMSNorm(self, config, input, scale, output, rows, lastDim, format):
        check(self.lib.puter_hip_rmsnorm(_ptr(input), _ptr(scale), _ptr(output), rows, lastDim,
                                         float(config.Epsilon), format, self.stream()))

    def LayerNorm(self, input, scale, bias, output, rows, lastDim, format):
        check(self.lib.puter_hip_layernorm(_ptr(input), _ptr(scale), _ptr(bias), _ptr(output),
                                           rows, lastDim, format, self.stream()))

    def AdaptiveRMSNorm(self, config, input, modulation, output, rows, lastDim, rowsPerBatch,
                        modulationCols, format):
        check(self.lib.puter_hip_adaptive_rmsnorm(_ptr(input), _ptr(modulation), _ptr(output),
                                                  rows, lastDim, rowsPerBatch, modulationCols,
                                                  float(config.Epsilon), format, self.stream()))

    def ModulatedLayerNorm(self, config, input, modulation, output, rows, lastDim, rowsPerBatch,
                           modulationCols, format):
        check(self.lib.puter_hip_modulated_layernorm(_ptr(input), _ptr(modulation), _ptr(output),
                                                     rows, lastDim, rowsPerBatch, modulationCols,
                                                     float(config.Epsilon), int(config.Set),
                                                     format, self.stream()))

    # ---- optional hook: execution/math_gated_residual_intrinsic.go:11-17 ----
    def GatedResidual(self, residual, branch, modulation, output, rows, lastDim, rowsPerBatch,
                      modulationCols, set, format):
        check(self.lib.puter_hip_gated_residual(_ptr(residual), _ptr(branch), _ptr(modulation),
                                                _ptr(output), rows, lastDim, rowsPerBatch,
                                                modulationCols, set, format, self.stream()))

    # ---- extension hooks: fused gated residual + norm ----
    def GatedResidualRMSNorm(self, config, residual, branch, modulation, scale, hidden, output,
                             rows, lastDim, rowsPerBatch, modulationCols, set, format):
        check(self.lib.puter_hip_gated_residual_rmsnorm(
            _ptr(residual), _ptr(branch), _ptr(modulation), _ptr(scale), _ptr(hidden),
            _ptr(output), rows, lastDim, rowsPerBatch, modulationCols, set,
            float(config.Epsilon), format, self.stream()))

    def GatedResidualLayerNorm(self, residual, branch, modulation, scale, bias, hidden, output,
                               rows, lastDim, rowsPerBatch, modulationCols, set, format):
        check(self.lib.puter_hip_gated_residual_layernorm(
            _ptr(residual), _ptr(branch), _ptr(modulation), _ptr(scale), _ptr(bias), _ptr(hidden),
            _ptr(output), rows, lastDim, rowsPerBatch, modulationCols, set, format, self.stream()))

    # ---- RoPE family: device/interface.go:592-610 ----
    def RoPE(self, config, input, output, seqLen, numHeads, headDim, format):
        c = _lib.RopeConfig(config.BaseFreq, config.StartPosition, config.Mode, config.Scaling,
                            config.ScalingFactor, config.LowFreqFactor, config.HighFreqFactor,
                            config.OriginalContext)
        check(self.lib.puter_hip_rope(C.byref(c), _ptr(input), _ptr(output), seqLen, numHeads,
                                      headDim, format, self.stream()))

    def RoPEPairs(self, output, input, cosBuffer, sinBuffer, halfDim, format):
        """device/interface.go:605-609 (F32 only, as device/cpu/rope/ops.go:10-14)."""
        check(self.lib.puter_hip_rope_pairs(_ptr(output), _ptr(input), _ptr(cosBuffer), _ptr(sinBuffer),
                                            halfDim, format, self.stream()))

    def MultiAxisRoPE(self, config, input, output, batch, seqLen, numHeads, headDim, format):
        dims = (C.c_int64 * 4)(config.AxisDim0, config.AxisDim1, config.AxisDim2, config.AxisDim3)
        c = _lib.MultiAxisRopeConfig(config.BaseFreq, config.LatentSeqLen, config.LatentSide,
                                     config.AxisCount, 0, dims)
        check(self.lib.puter_hip_multi_axis_rope(C.byref(c), _ptr(input), _ptr(output), batch,
                                                 seqLen, numHeads, headDim, format, self.stream()))

    # ---- Activation family (gated + Silu/Gelu): device/interface.go:18-74 ----
    def _tensors(self, kind, dst, gate, up, count, format):
        check(self.lib.puter_hip_gated_tensors(kind, _ptr(dst), _ptr(gate), _ptr(up), count,
                                               format, self.stream()))

    def _packed(self, kind, dst, packed, batch, halfCount, format):
        check(self.lib.puter_hip_gated_packed(kind, _ptr(dst), _ptr(packed), batch, halfCount,
                                              format, self.stream()))

    def SwiGLUTensors(self, dst, gate, up, count, format):
        self._tensors(GATE_SWIGLU, dst, gate, up, count, format)

    def GeGLUTensors(self, dst, gate, up, count, format):
        self._tensors(GATE_GEGLU, dst, gate, up, count, format)

    def GeGLUTanhTensors(self, dst, gate, up, count, format):
        self._tensors(GATE_GEGLU_TANH, dst, gate, up, count, format)

    def SiGLUTensors(self, dst, gate, up, count, format):
        self._tensors(GATE_SIGLU, dst, gate, up, count, format)

    def GLUTensors(self, dst, gate, up, count, format):
        self._tensors(GATE_GLU, dst, gate, up, count, format)

    def ReGLUTensors(self, dst, gate, up, count, format):
        self._tensors(GATE_REGLU, dst, gate, up, count, format)

    def LinGLUTensors(self, dst, gate, up, count, format):
        self._tensors(GATE_LINGLU, dst, gate, up, count, format)

    def SeGLUTensors(self, dst, gate, up, count, format):
        self._tensors(GATE_SEGLU, dst, gate, up, count, format)

    def SwiGLU(self, dst, packed, batch, halfCount, format):
        self._packed(GATE_SWIGLU, dst, packed, batch, halfCount, format)

    def GeGLU(self, dst, packed, batch, halfCount, format):
        self._packed(GATE_GEGLU, dst, packed, batch, halfCount, format)

    def GeGLUTanh(self, dst, packed, batch, halfCount, format):
        self._packed(GATE_GEGLU_TANH, dst, packed, batch, halfCount, format)

    def SiGLU(self, dst, packed, batch, halfCount, format):
        self._packed(GATE_SIGLU, dst, packed, batch, halfCount, format)

    def GLU(self, dst, packed, batch, halfCount, format):
        self._packed(GATE_GLU, dst, packed, batch, halfCount, format)

    def ReGLU(self, dst, packed, batch, halfCount, format):
        self._packed(GATE_REGLU, dst, packed, batch, halfCount, format)

    def LinGLU(self, dst, packed, batch, halfCount, format):
        self._packed(GATE_LINGLU, dst, packed, batch, halfCount, format)

    def SeGLU(self, dst, packed, batch, halfCount, format):
        self._packed(GATE_SEGLU, dst, packed, batch, halfCount, format)

    def Silu(self, dst, src, count, format):
        check(self.lib.puter_hip_unary(UNARY_SILU, _ptr(dst), _ptr(src), count, format,
                                       self.stream()))

    def Gelu(self, dst, src, count, format):
        check(self.lib.puter_hip_unary(UNARY_GELU, _ptr(dst), _ptr(src), count, format,
                                       self.stream()))

    # ---- casts: convert/*.go (dst, src slices of equal length) ----
    def Cast(self, dst, dst_format, src, src_format, count):
        check(self.lib.puter_hip_cast(_ptr(dst), dst_format, _ptr(src), src_format, count,
                                      self.stream()))

    def _convert(self, dst, dst_format, src, src_format):
        if dst.numel() != src.numel():
            raise ValueError(ErrLenMismatch)
        self.Cast(dst, dst_format, src, src_format, src.numel())

    def BFloat16ToFloat32(self, dst, src):
        self._convert(dst, F32, src, BF16)

    def Float32ToBFloat16(self, dst, src):
        self._convert(dst, BF16, src, F32)

    def Float16ToFloat32(self, dst, src):
        self._convert(dst, F32, src, F16)

    def Float32ToFloat16(self, dst, src):
        self._convert(dst, F16, src, F32)

    def Float8E4M3ToFloat32(self, dst, src):
        self._convert(dst, F32, src, F8E4M3)

    def Float32ToFloat8E4M3(self, dst, src):
        self._convert(dst, F8E4M3, src, F32)

    def Float8E5M2ToFloat32(self, dst, src):
        self._convert(dst, F32, src, F8E5M2)

    def Float32ToFloat8E5M2(self, dst, src):
        self._convert(dst, F8E5M2, src, F32)

    def Int8ToFloat32(self, dst, src):  # convert/int_f32.go:14-25
        self._convert(dst, F32, src, I8)

    def Float32ToInt8(self, dst, src):  # convert/int_f32.go:30-52
        self._convert(dst, I8, src, F32)

    def Int4ToFloat32(self, dst, src):
        """convert/int_f32.go:59-77: dst.numel() nibbles from the packed bytes of src
        (len(dst) may be at most 2 * len(src))."""
        if dst.numel() > 2 * src.numel():
            raise ValueError(ErrLenMismatch)
        self.Cast(dst, F32, src, I4, dst.numel())

    def Float32ToFloat64(self, dst, src):  # convert/f32_f64.go:8-10
        self._convert(dst, F64, src, F32)

    def Float64ToFloat32(self, dst, src):  # convert/f32_f64.go:15-17
        self._convert(dst, F32, src, F64)

    # ---- paged KV hooks: execution/page_intrinsic.go:13-24 ----
    def KVPageWrite(self, storage, values, pageIDs, offsets, output, pageCount, pageSize, inner,
                    valueRows, storageOffset, format):
        check(self.lib.puter_hip_kv_page_write(_ptr(storage), _ptr(values), _ptr(pageIDs),
                                               _ptr(offsets), _ptr(output), pageCount, pageSize,
                                               inner, valueRows, storageOffset, format,
                                               _ptr(self._status_word()), self.stream()))

    def KVPageGather(self, storage, pageTable, output, pageCount, pageSize, inner, outRows,
                     storageOffset, format):
        check(self.lib.puter_hip_kv_page_gather(_ptr(storage), _ptr(pageTable), _ptr(output),
                                                pageCount, pageSize, inner, outRows,
                                                storageOffset, format, _ptr(self._status_word()),
                                                self.stream()))

    def KVPageWriteFP8(self, storage, values, pageIDs, offsets, pageCount, pageSize, kvHeads,
                       headDim, valueRows, storageOffset, scales, valueFormat):
        """Extension hook (no reference method): quantise bf16 / f16 / f32 rows into
        an fp8-E4M3 pool, byte = E4M3(value / scales[kv head]), in place."""
        check(self.lib.puter_hip_kv_page_write_fp8(_ptr(storage), _ptr(values), _ptr(pageIDs),
                                                   _ptr(offsets), pageCount, pageSize, kvHeads,
                                                   headDim, valueRows, storageOffset, _ptr(scales),
                                                   valueFormat, _ptr(self._status_word()), self.stream()))

    # ---- Attention: device/interface.go:91-110 ----
    @staticmethod
    def _mha(config):
        return _lib.MHAConfig(config.NumHeads, config.HeadDim, int(bool(config.Causal)), 0,
                              config.WindowSize, config.ALiBiSlope, 0, config.KVHeadCount)

    def MultiHeadAttention(self, config, query, key, value, output, seqQ, seqK, format):
        c = self._mha(config)
        check(self.lib.puter_hip_multi_head_attention(C.byref(c), _ptr(query), _ptr(key),
                                                      _ptr(value), _ptr(output), seqQ, seqK,
                                                      format, self.stream()))

    def MultiHeadAttentionBatched(self, config, query, key, value, output, batch, seqQ, seqK,
                                  format):
        c = self._mha(config)
        check(self.lib.puter_hip_multi_head_attention_batched(C.byref(c), _ptr(query), _ptr(key),
                                                              _ptr(value), _ptr(output), batch,
                                                              seqQ, seqK, format, self.stream()))

    # device/interface.go:92-109 (single head; FlashAttention forwards to
    # ScaledDotProductAttention as device/cpu/attention/ops.go:21-31 does)
    def ScaledDotProductAttention(self, config, query, key, value, output, seqQ, seqK, depth,
                                  valueDim, format):
        c = _lib.FlashConfig(config.BlockSize, 1 if config.Causal else 0, 0)
        check(self.lib.puter_hip_scaled_dot_product_attention(
            C.byref(c), _ptr(query), _ptr(key), _ptr(value), _ptr(output), seqQ, seqK, depth,
            valueDim, format, self.stream()))

    def FlashAttention(self, config, query, key, value, output, seqQ, seqK, depth, valueDim,
                       format):
        c = _lib.FlashConfig(config.BlockSize, 1 if config.Causal else 0, 0)
        check(self.lib.puter_hip_flash_attention(
            C.byref(c), _ptr(query), _ptr(key), _ptr(value), _ptr(output), seqQ, seqK, depth,
            valueDim, format, self.stream()))

    def PagedDecodeWorkspaceBytes(self, batch, numHeads, headDim, maxContext):
        return self.lib.puter_hip_paged_decode_workspace_bytes(batch, numHeads, headDim,
                                                               maxContext)

    def PagedDecodeAttention(self, query, keyPages, valuePages, pageTable, contextLens, batch,
                             maxPagesPerSeq, pageSize, numPages, numHeads, kvHeads, headDim,
                             maxContext, kScale, vScale, kvFormat, output, workspace,
                             workspaceBytes):
        check(self.lib.puter_hip_paged_decode_attention(
            _ptr(query), _ptr(keyPages), _ptr(valuePages), _ptr(pageTable), _ptr(contextLens),
            batch, maxPagesPerSeq, pageSize, numPages, numHeads, kvHeads, headDim, maxContext,
            _ptr(kScale), _ptr(vScale), kvFormat, _ptr(output), _ptr(workspace), workspaceBytes,
            self.stream()))

    # ---- Dequant / Quant: device/interface.go:196-199, 580-582 ----
    def Dequant(self, dst, src, count, config, dstFormat, srcFormat):
        """dequant/ops.go:11-37: F32 <- Int8, (src - ZeroPoint) * Scale."""
        check(self.lib.puter_hip_dequant(_ptr(dst), _ptr(src), count, config.Scale, config.ZeroPoint,
                                         dstFormat, srcFormat, self.stream()))

    def Dequant4(self, dst, src, pairCount, config, dstFormat, srcFormat):
        """dequant/ops.go:39-58: F32 <- Int4 (pairCount nibbles, low nibble first)."""
        check(self.lib.puter_hip_dequant4(_ptr(dst), _ptr(src), pairCount, config.Scale,
                                          config.ZeroPoint, dstFormat, srcFormat, self.stream()))

    def Quant(self, dst, src, count, config, dstFormat, srcFormat):
        """quant/ops.go:10-37: Int8 <- F32, round-half-away(src / Scale) + ZeroPoint, saturated."""
        check(self.lib.puter_hip_quant(_ptr(dst), _ptr(src), count, config.Scale, config.ZeroPoint,
                                       dstFormat, srcFormat, self.stream()))

    # ---- Matmul: device/interface.go:409-415 (F32, F64, BF16, F16) ----
    def Matmul(self, out, left, right, rows, inner, cols, format):
        check(self.lib.puter_hip_matmul(_ptr(out), _ptr(left), _ptr(right), rows, inner, cols,
                                        format, self.stream()))

    def MatmulNoAlloc(self, out, left, right, rows, inner, cols, format):
        """Extension (no reference method): Matmul that never allocates (its split-K
        partials use a fixed per-GPU device array); calls on one GPU must not overlap."""
        check(self.lib.puter_hip_matmul_noalloc(_ptr(out), _ptr(left), _ptr(right), rows, inner, cols,
                                                format, self.stream()))
