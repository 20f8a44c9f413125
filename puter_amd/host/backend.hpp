// C++ host side of the MI355X (gfx950) device backend for puter.
//
// The reference is compiled Go; its execution layer calls device.Backend methods
// (device/interface.go), three optional hooks it type-asserts
// (execution/math_gated_residual_intrinsic.go:11-17 GatedResidual,
// execution/page_intrinsic.go:13-24 KVPageWrite / KVPageGather,
// execution/dispatch.go:120-123 BeginBatch / EndBatch) and, for resident
// workspaces, the memory backend's AllocateWorkspaceSlot / ViewWorkspaceSlot
// (execution/workspace_resident.go:12-20).  This header mirrors those methods in
// C++ over the C ABI of libputer_hip.so (include/puter_hip.h): the same names,
// argument order and meaning, device buffers as raw device addresses (the
// unsafe.Pointer a cgo wrapper passes), sizes as int64_t.
//
// Error behaviour follows the Go contract: a method that panics in Go on a bad
// config, shape, dtype or nil buffer throws puter::hip::Error here (the library's
// status code and message); a method that returns a Go `error` returns
// MaybeError, empty on success.  Launches are asynchronous on the Backend's
// stream; only Upload, Download, CheckStatus and EndBatch synchronise it.
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <optional>
#include <stdexcept>
#include <string>
#include <vector>

#include "puter_hip.h"

namespace puter::hip {

// manifesto/dtype formats on the path, with the library's codes
enum class DType : int {
    Float32 = PUTER_F32,
    Float16 = PUTER_F16,
    BFloat16 = PUTER_BF16,
    Float8E4M3 = PUTER_F8E4M3,
    Float8E5M2 = PUTER_F8E5M2,
    Int32 = PUTER_I32,
    Int8 = PUTER_I8,
    Int4 = PUTER_I4,   // packed: element 2k is the low nibble of byte k
    Float64 = PUTER_F64,
};

// bytes of `count` elements of a format (Int4: two per byte, rounded up)
int64_t ByteCount(DType format, int64_t count);
const char *Name(DType format);   // the manifesto/dtype name ("bfloat16", ...)

// A panic of the Go contract: the library's status code (include/puter_hip.h:
// -2 nil buffer, -6 invalid dtype / shape / config, -7 unavailable, -8 launch)
// and its message.
class Error : public std::runtime_error {
public:
    Error(int status, const std::string &message) : std::runtime_error(message), status_(status) {}
    int Status() const { return status_; }

private:
    int status_;
};

// A Go `error` result: empty on success.
using MaybeError = std::optional<Error>;

// ---- config structs: device/config.go ----------------------------------------
struct RMSNormConfig {   // config.go:82-92
    double Epsilon = 1e-6;
};
struct ModulatedLayerNormConfig {   // config.go:94-109
    double Epsilon = 1e-6;
    int Set = 0;
};
enum RoPEMode { RoPEModeInterleaved = 0, RoPEModeHalf = 1 };
enum RoPEScaling { RoPEScalingNone = 0, RoPEScalingLlama3 = 1 };
struct RoPEConfig {   // config.go:125-134; DefaultRoPEConfig device/cpu/rope/config.go:7-15
    double BaseFreq = 10000.0;
    int64_t StartPosition = 0;
    int Mode = RoPEModeInterleaved;
    int Scaling = RoPEScalingNone;
    double ScalingFactor = 1.0;
    double LowFreqFactor = 0.0;
    double HighFreqFactor = 0.0;
    int64_t OriginalContext = 0;
};
struct MultiAxisRoPEConfig {   // config.go:136-146
    double BaseFreq = 10000.0;
    int64_t LatentSeqLen = 0;
    int64_t LatentSide = 0;
    int AxisCount = 0;
    int64_t AxisDim0 = 0, AxisDim1 = 0, AxisDim2 = 0, AxisDim3 = 0;
};
struct MultiHeadAttentionConfig {   // config.go:283-290
    int64_t NumHeads = 0;
    int64_t HeadDim = 0;
    bool Causal = false;
    int64_t WindowSize = 0;
    float ALiBiSlope = 0.0f;
    int64_t KVHeadCount = 0;
};
struct FlashAttentionConfig {   // config.go:278-281
    int64_t BlockSize = 0;
    bool Causal = false;
};
struct DequantInt8Config {   // config.go:268-271 (also Quant's config, interface.go:580-582)
    float Scale = 1.0f;
    int8_t ZeroPoint = 0;
};
struct DequantInt4Config {   // config.go:273-276
    float Scale = 1.0f;
    int8_t ZeroPoint = 0;
};

// ---- device tensors: the memory backend's tensor.Tensor ------------------------
// tensor.Host, and the device location the HIP backend's kernels register under
// (the reference's tensor.CUDA: manifesto has no ROCm location,
// pool/device_id.go:59-74).
enum class Location { Host, Device };

// A dense tensor: an address, a shape and an element format.  Allocations made
// by the memory backend own their memory through `holder` (freed when the last
// tensor sharing it goes away, or by Close); views and wrapped caller memory
// own nothing.  DispatchPointer is the raw address a backend method takes
// (device/cuda/resident.go:17-38 unwraps the same way).
struct Tensor {
    void *data = nullptr;
    std::vector<int64_t> shape;
    DType format = DType::Float32;
    Location location = Location::Device;
    int64_t byteCount = 0;
    std::shared_ptr<void> holder;

    void *DispatchPointer() const { return data; }
    int64_t Numel() const;
    size_t Rank() const { return shape.size(); }
    void Close();   // drops this tensor's share of an owned allocation
};

// Wrap memory the caller owns (device or host) as a Tensor.
Tensor Wrap(void *data, std::vector<int64_t> shape, DType format, Location location = Location::Device);

// ---- the backend ------------------------------------------------------------------
class Backend {
public:
    // stream: a hipStream_t (as void *); nullptr is the default stream
    explicit Backend(void *stream = nullptr);
    ~Backend();
    Backend(const Backend &) = delete;
    Backend &operator=(const Backend &) = delete;

    void *Stream() const { return stream_; }

    // -- memory backend (device/cuda/backend.go:101-234: Upload / Download),
    //    workspace slots (execution/workspace_resident.go:12-20)
    void Upload(void *dst, const void *host, size_t bytes);
    void Download(void *host, const void *src, size_t bytes);
    Tensor AllocateTensor(std::vector<int64_t> shape, DType format);
    std::pair<Tensor, MaybeError> AllocateWorkspaceSlot(int64_t byteCount);
    std::pair<Tensor, MaybeError> ViewWorkspaceSlot(const Tensor &slot, std::vector<int64_t> shape,
                                                    DType elementFormat, int64_t byteCount);

    // -- batch hooks (execution/dispatch.go:120-123).  Launches are already
    //    asynchronous, so BeginBatch does nothing; EndBatch synchronises once and
    //    returns the paged-KV status word's error.
    MaybeError BeginBatch();
    MaybeError EndBatch();
    // Synchronise, read and clear the status word; throw the reference's
    // ErrShapeMismatch (device/cpu/shape/page.go:139-146,191-203) if a paged-KV
    // call since the last check saw an out-of-range page id or slot.
    void CheckStatus();
    // The device int32 the paged-KV hooks flag bad ids in (created by the
    // constructor when a device is present, so the hooks can be captured).
    int32_t *StatusWord();

    // -- LayerNorm family: device/interface.go:355-379
    void RMSNorm(const RMSNormConfig &config, const void *input, const void *scale, void *output, int64_t rows,
                 int64_t lastDim, DType format);
    void LayerNorm(const void *input, const void *scale, const void *bias, void *output, int64_t rows,
                   int64_t lastDim, DType format);
    void AdaptiveRMSNorm(const RMSNormConfig &config, const void *input, const void *modulation, void *output,
                         int64_t rows, int64_t lastDim, int64_t rowsPerBatch, int64_t modulationCols,
                         DType format);
    void ModulatedLayerNorm(const ModulatedLayerNormConfig &config, const void *input, const void *modulation,
                            void *output, int64_t rows, int64_t lastDim, int64_t rowsPerBatch,
                            int64_t modulationCols, DType format);
    // GatedResidual hook (math_gated_residual_intrinsic.go:11-17) and its fused
    // norms (extension hooks: no reference method)
    void GatedResidual(const void *residual, const void *branch, const void *modulation, void *output,
                       int64_t rows, int64_t lastDim, int64_t rowsPerBatch, int64_t modulationCols, int set,
                       DType format);
    void GatedResidualRMSNorm(const RMSNormConfig &config, const void *residual, const void *branch,
                              const void *modulation, const void *scale, void *hidden, void *output,
                              int64_t rows, int64_t lastDim, int64_t rowsPerBatch, int64_t modulationCols,
                              int set, DType format);
    void GatedResidualLayerNorm(const void *residual, const void *branch, const void *modulation,
                                const void *scale, const void *bias, void *hidden, void *output, int64_t rows,
                                int64_t lastDim, int64_t rowsPerBatch, int64_t modulationCols, int set,
                                DType format);

    // -- RoPE family: device/interface.go:592-610
    void RoPE(const RoPEConfig &config, const void *input, void *output, int64_t seqLen, int64_t numHeads,
              int64_t headDim, DType format);
    void RoPEPairs(void *output, const void *input, const void *cosBuffer, const void *sinBuffer,
                   int64_t halfDim, DType format);
    void MultiAxisRoPE(const MultiAxisRoPEConfig &config, const void *input, void *output, int64_t batch,
                       int64_t seqLen, int64_t numHeads, int64_t headDim, DType format);

    // -- Activation family: device/interface.go:18-74 (tensor and packed forms)
    void SwiGLUTensors(void *dst, const void *gate, const void *up, int64_t count, DType format);
    void GeGLUTensors(void *dst, const void *gate, const void *up, int64_t count, DType format);
    void GeGLUTanhTensors(void *dst, const void *gate, const void *up, int64_t count, DType format);
    void SiGLUTensors(void *dst, const void *gate, const void *up, int64_t count, DType format);
    void GLUTensors(void *dst, const void *gate, const void *up, int64_t count, DType format);
    void ReGLUTensors(void *dst, const void *gate, const void *up, int64_t count, DType format);
    void LinGLUTensors(void *dst, const void *gate, const void *up, int64_t count, DType format);
    void SeGLUTensors(void *dst, const void *gate, const void *up, int64_t count, DType format);
    void SwiGLU(void *dst, const void *packed, int64_t batch, int64_t halfCount, DType format);
    void GeGLU(void *dst, const void *packed, int64_t batch, int64_t halfCount, DType format);
    void GeGLUTanh(void *dst, const void *packed, int64_t batch, int64_t halfCount, DType format);
    void SiGLU(void *dst, const void *packed, int64_t batch, int64_t halfCount, DType format);
    void GLU(void *dst, const void *packed, int64_t batch, int64_t halfCount, DType format);
    void ReGLU(void *dst, const void *packed, int64_t batch, int64_t halfCount, DType format);
    void LinGLU(void *dst, const void *packed, int64_t batch, int64_t halfCount, DType format);
    void SeGLU(void *dst, const void *packed, int64_t batch, int64_t halfCount, DType format);
    void Silu(void *dst, const void *src, int64_t count, DType format);
    void Gelu(void *dst, const void *src, int64_t count, DType format);

    // -- casts: convert/*.go on device buffers of `count` elements each, and the
    //    device branch of shape.cast (execution/shape_cast_intrinsic.go:13-115)
    void Cast(void *dst, DType dstFormat, const void *src, DType srcFormat, int64_t count);

    // -- paged KV hooks: execution/page_intrinsic.go:13-24
    void KVPageWrite(const void *storage, const void *values, const void *pageIDs, const void *offsets,
                     void *output, int64_t pageCount, int64_t pageSize, int64_t inner, int64_t valueRows,
                     int64_t storageOffset, DType format);
    void KVPageGather(const void *storage, const void *pageTable, void *output, int64_t pageCount,
                      int64_t pageSize, int64_t inner, int64_t outRows, int64_t storageOffset, DType format);
    // extension hook (no reference method): quantising write into an fp8-E4M3 pool
    void KVPageWriteFP8(void *storage, const void *values, const void *pageIDs, const void *offsets,
                        int64_t pageCount, int64_t pageSize, int64_t kvHeads, int64_t headDim, int64_t valueRows,
                        int64_t storageOffset, const void *scales, DType valueFormat);

    // -- Attention: device/interface.go:91-110
    void MultiHeadAttention(const MultiHeadAttentionConfig &config, const void *query, const void *key,
                            const void *value, void *output, int64_t seqQ, int64_t seqK, DType format);
    // extension: B independent [seqQ/seqK, heads*D] slabs back to back, one launch
    void MultiHeadAttentionBatched(const MultiHeadAttentionConfig &config, const void *query, const void *key,
                                   const void *value, void *output, int64_t batch, int64_t seqQ, int64_t seqK,
                                   DType format);
    void ScaledDotProductAttention(const FlashAttentionConfig &config, const void *query, const void *key,
                                   const void *value, void *output, int64_t seqQ, int64_t seqK, int64_t depth,
                                   int64_t valueDim, DType format);
    void FlashAttention(const FlashAttentionConfig &config, const void *query, const void *key,
                        const void *value, void *output, int64_t seqQ, int64_t seqK, int64_t depth,
                        int64_t valueDim, DType format);
    // extension: KVPageGather + one-row MultiHeadAttention fused over the page pools
    size_t PagedDecodeWorkspaceBytes(int64_t batch, int64_t numHeads, int64_t headDim, int64_t maxContext);
    void PagedDecodeAttention(const void *query, const void *keyPages, const void *valuePages,
                              const void *pageTable, const void *contextLens, int64_t batch,
                              int64_t maxPagesPerSeq, int64_t pageSize, int64_t numPages, int64_t numHeads,
                              int64_t kvHeads, int64_t headDim, int64_t maxContext, const void *kScale,
                              const void *vScale, DType kvFormat, void *output, void *workspace,
                              size_t workspaceBytes);

    // -- Dequant / Quant: device/interface.go:196-199,580-582
    void Dequant(void *dst, const void *src, int64_t count, const DequantInt8Config &config, DType dstFormat,
                 DType srcFormat);
    void Dequant4(void *dst, const void *src, int64_t pairCount, const DequantInt4Config &config,
                  DType dstFormat, DType srcFormat);
    void Quant(void *dst, const void *src, int64_t count, const DequantInt8Config &config, DType dstFormat,
               DType srcFormat);

    // -- Matmul: device/interface.go:409-415 (F32, F64, BF16, F16)
    void Matmul(void *out, const void *left, const void *right, int64_t rows, int64_t inner, int64_t cols,
                DType format);
    // extension: Matmul that never allocates (split-K partials in a fixed per-GPU
    // array); calls on one GPU must not overlap
    void MatmulNoAlloc(void *out, const void *left, const void *right, int64_t rows, int64_t inner,
                       int64_t cols, DType format);

private:
    void *stream_;
    int32_t *status_ = nullptr;
};

// Throw Error for a non-zero status of the C ABI (the Go wrapper's panic(err)).
void Check(int status);

}  // namespace puter::hip
