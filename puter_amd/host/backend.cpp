// C++ host side of the MI355X device backend: device.Backend methods over the C
// ABI of libputer_hip.so.  Every method forwards its arguments unchanged and
// turns a non-zero status into Error (the Go wrapper's panic(err)).
#include "backend.hpp"

#include <cstring>
#include <numeric>

namespace puter::hip {

namespace {

int code(DType f) { return static_cast<int>(f); }

std::string last_error(int status) {
    const char *m = puter_hip_last_error();
    return m && *m ? std::string(m) : "puter_hip: status " + std::to_string(status);
}

puter_mha_config mha_config(const MultiHeadAttentionConfig &c) {
    puter_mha_config m{};
    m.num_heads = c.NumHeads;
    m.head_dim = c.HeadDim;
    m.causal = c.Causal ? 1 : 0;
    m.window_size = c.WindowSize;
    m.alibi_slope = c.ALiBiSlope;
    m.kv_head_count = c.KVHeadCount;
    return m;
}

puter_flash_config flash_config(const FlashAttentionConfig &c) {
    puter_flash_config f{};
    f.block_size = c.BlockSize;
    f.causal = c.Causal ? 1 : 0;
    return f;
}

}  // namespace

void Check(int status) {
    if (status != PUTER_OK) throw Error(status, last_error(status));
}

int64_t ByteCount(DType format, int64_t count) {
    switch (format) {
    case DType::Float32:
    case DType::Int32: return 4 * count;
    case DType::Float16:
    case DType::BFloat16: return 2 * count;
    case DType::Float8E4M3:
    case DType::Float8E5M2:
    case DType::Int8: return count;
    case DType::Int4: return (count + 1) / 2;
    case DType::Float64: return 8 * count;
    }
    return 0;
}

const char *Name(DType format) {
    switch (format) {
    case DType::Float32: return "float32";
    case DType::Float16: return "float16";
    case DType::BFloat16: return "bfloat16";
    case DType::Float8E4M3: return "float8e4m3";
    case DType::Float8E5M2: return "float8e5m2";
    case DType::Int32: return "int32";
    case DType::Int8: return "int8";
    case DType::Int4: return "int4";
    case DType::Float64: return "float64";
    }
    return "unknown";
}

// ---- tensors ----------------------------------------------------------------------
int64_t Tensor::Numel() const {
    return std::accumulate(shape.begin(), shape.end(), (int64_t)1, [](int64_t a, int64_t b) { return a * b; });
}

void Tensor::Close() {
    holder.reset();
    data = nullptr;
}

Tensor Wrap(void *data, std::vector<int64_t> shape, DType format, Location location) {
    Tensor t;
    t.data = data;
    t.shape = std::move(shape);
    t.format = format;
    t.location = location;
    t.byteCount = ByteCount(format, t.Numel());
    return t;
}

// ---- backend ----------------------------------------------------------------------
// The paged-KV hooks' status word is made here, with a blocking upload of its
// zero, so that no hook call (which may sit inside a HIP-graph capture) allocates
// or synchronises; a host without a device makes it on first use instead.
Backend::Backend(void *stream) : stream_(stream) {
    int devices = 0;
    if (puter_hip_device_count(&devices) == PUTER_OK && devices > 0) StatusWord();
}

Backend::~Backend() {
    if (status_) puter_hip_free(status_);
}

void Backend::Upload(void *dst, const void *host, size_t bytes) {
    Check(puter_hip_memcpy_htod(dst, host, bytes, stream_));
    Check(puter_hip_stream_synchronize(stream_));
}

void Backend::Download(void *host, const void *src, size_t bytes) {
    Check(puter_hip_memcpy_dtoh(host, src, bytes, stream_));
    Check(puter_hip_stream_synchronize(stream_));
}

Tensor Backend::AllocateTensor(std::vector<int64_t> shape, DType format) {
    Tensor t = Wrap(nullptr, std::move(shape), format);
    void *p = nullptr;
    Check(puter_hip_malloc(&p, (size_t)std::max<int64_t>(t.byteCount, 1)));
    t.data = p;
    t.holder = std::shared_ptr<void>(p, [](void *q) { puter_hip_free(q); });
    return t;
}

// AllocateWorkspaceSlot: one device allocation of byteCount bytes, shape
// [byteCount] Int8, which NewResidentWorkspace carves into planned views; it
// stays on the device until its last tensor is closed.  byteCount <= 0 is
// tensor.ErrShapeInvalid.
std::pair<Tensor, MaybeError> Backend::AllocateWorkspaceSlot(int64_t byteCount) {
    if (byteCount <= 0) return {Tensor{}, Error(PUTER_ERR_INVALID, "tensor: invalid shape")};
    try {
        return {AllocateTensor({byteCount}, DType::Int8), std::nullopt};
    } catch (const Error &e) {
        return {Tensor{}, e};
    }
}

// ViewWorkspaceSlot: the slot's device address with another shape and element
// format, no copy; byteCount outside [0, slot bytes] is tensor.ErrShapeMismatch.
std::pair<Tensor, MaybeError> Backend::ViewWorkspaceSlot(const Tensor &slot, std::vector<int64_t> shape,
                                                         DType elementFormat, int64_t byteCount) {
    if (byteCount < 0 || byteCount > slot.byteCount || !slot.data)
        return {Tensor{}, Error(PUTER_ERR_INVALID, "tensor: shape mismatch")};
    Tensor v = Wrap(slot.data, std::move(shape), elementFormat, slot.location);
    v.byteCount = byteCount;
    v.holder = slot.holder;   // a view keeps the slot alive, owns nothing itself
    return {v, std::nullopt};
}

int32_t *Backend::StatusWord() {
    if (!status_) {
        void *p = nullptr;
        Check(puter_hip_malloc(&p, sizeof(int32_t)));
        status_ = static_cast<int32_t *>(p);
        const int32_t zero = 0;
        Upload(status_, &zero, sizeof zero);
    }
    return status_;
}

void Backend::CheckStatus() {
    if (!status_) return;
    int32_t v = 0;
    Download(&v, status_, sizeof v);
    if (v != 0) {
        const int32_t zero = 0;
        Upload(status_, &zero, sizeof zero);
        throw Error(v, "tensor: shape mismatch (page id or slot out of range)");
    }
}

MaybeError Backend::BeginBatch() { return std::nullopt; }

MaybeError Backend::EndBatch() {
    try {
        Check(puter_hip_stream_synchronize(stream_));
        CheckStatus();
    } catch (const Error &e) {
        return e;
    }
    return std::nullopt;
}

// ---- LayerNorm family ----------------------------------------------------------------
void Backend::RMSNorm(const RMSNormConfig &config, const void *input, const void *scale, void *output,
                      int64_t rows, int64_t lastDim, DType format) {
    Check(puter_hip_rmsnorm(input, scale, output, rows, lastDim, config.Epsilon, code(format), stream_));
}

void Backend::LayerNorm(const void *input, const void *scale, const void *bias, void *output, int64_t rows,
                        int64_t lastDim, DType format) {
    Check(puter_hip_layernorm(input, scale, bias, output, rows, lastDim, code(format), stream_));
}

void Backend::AdaptiveRMSNorm(const RMSNormConfig &config, const void *input, const void *modulation,
                              void *output, int64_t rows, int64_t lastDim, int64_t rowsPerBatch,
                              int64_t modulationCols, DType format) {
    Check(puter_hip_adaptive_rmsnorm(input, modulation, output, rows, lastDim, rowsPerBatch, modulationCols,
                                     config.Epsilon, code(format), stream_));
}

void Backend::ModulatedLayerNorm(const ModulatedLayerNormConfig &config, const void *input,
                                 const void *modulation, void *output, int64_t rows, int64_t lastDim,
                                 int64_t rowsPerBatch, int64_t modulationCols, DType format) {
    Check(puter_hip_modulated_layernorm(input, modulation, output, rows, lastDim, rowsPerBatch, modulationCols,
                                        config.Epsilon, config.Set, code(format), stream_));
}

void Backend::GatedResidual(const void *residual, const void *branch, const void *modulation, void *output,
                            int64_t rows, int64_t lastDim, int64_t rowsPerBatch, int64_t modulationCols, int set,
                            DType format) {
    Check(puter_hip_gated_residual(residual, branch, modulation, output, rows, lastDim, rowsPerBatch,
                                   modulationCols, set, code(format), stream_));
}

void Backend::GatedResidualRMSNorm(const RMSNormConfig &config, const void *residual, const void *branch,
                                   const void *modulation, const void *scale, void *hidden, void *output,
                                   int64_t rows, int64_t lastDim, int64_t rowsPerBatch, int64_t modulationCols,
                                   int set, DType format) {
    Check(puter_hip_gated_residual_rmsnorm(residual, branch, modulation, scale, hidden, output, rows, lastDim,
                                           rowsPerBatch, modulationCols, set, config.Epsilon, code(format),
                                           stream_));
}

void Backend::GatedResidualLayerNorm(const void *residual, const void *branch, const void *modulation,
                                     const void *scale, const void *bias, void *hidden, void *output,
                                     int64_t rows, int64_t lastDim, int64_t rowsPerBatch, int64_t modulationCols,
                                     int set, DType format) {
    Check(puter_hip_gated_residual_layernorm(residual, branch, modulation, scale, bias, hidden, output, rows,
                                             lastDim, rowsPerBatch, modulationCols, set, code(format), stream_));
}

// ---- RoPE family -----------------------------------------------------------------------
void Backend::RoPE(const RoPEConfig &config, const void *input, void *output, int64_t seqLen, int64_t numHeads,
                   int64_t headDim, DType format) {
    puter_rope_config c{};
    c.base_freq = config.BaseFreq;
    c.start_position = config.StartPosition;
    c.mode = config.Mode;
    c.scaling = config.Scaling;
    c.scaling_factor = config.ScalingFactor;
    c.low_freq_factor = config.LowFreqFactor;
    c.high_freq_factor = config.HighFreqFactor;
    c.original_context = config.OriginalContext;
    Check(puter_hip_rope(&c, input, output, seqLen, numHeads, headDim, code(format), stream_));
}

void Backend::RoPEPairs(void *output, const void *input, const void *cosBuffer, const void *sinBuffer,
                        int64_t halfDim, DType format) {
    Check(puter_hip_rope_pairs(output, input, cosBuffer, sinBuffer, halfDim, code(format), stream_));
}

void Backend::MultiAxisRoPE(const MultiAxisRoPEConfig &config, const void *input, void *output, int64_t batch,
                            int64_t seqLen, int64_t numHeads, int64_t headDim, DType format) {
    puter_multi_axis_rope_config c{};
    c.base_freq = config.BaseFreq;
    c.latent_seq_len = config.LatentSeqLen;
    c.latent_side = config.LatentSide;
    c.axis_count = config.AxisCount;
    c.axis_dims[0] = config.AxisDim0;
    c.axis_dims[1] = config.AxisDim1;
    c.axis_dims[2] = config.AxisDim2;
    c.axis_dims[3] = config.AxisDim3;
    Check(puter_hip_multi_axis_rope(&c, input, output, batch, seqLen, numHeads, headDim, code(format), stream_));
}

// ---- activations -----------------------------------------------------------------------
#define PUTER_TENSORS(NAME, KIND)                                                                          \
    void Backend::NAME(void *dst, const void *gate, const void *up, int64_t count, DType format) {          \
        Check(puter_hip_gated_tensors(KIND, dst, gate, up, count, code(format), stream_));                  \
    }
#define PUTER_PACKED(NAME, KIND)                                                                           \
    void Backend::NAME(void *dst, const void *packed, int64_t batch, int64_t halfCount, DType format) {     \
        Check(puter_hip_gated_packed(KIND, dst, packed, batch, halfCount, code(format), stream_));          \
    }
PUTER_TENSORS(SwiGLUTensors, PUTER_GATE_SWIGLU)
PUTER_TENSORS(GeGLUTensors, PUTER_GATE_GEGLU)
PUTER_TENSORS(GeGLUTanhTensors, PUTER_GATE_GEGLU_TANH)
PUTER_TENSORS(SiGLUTensors, PUTER_GATE_SIGLU)
PUTER_TENSORS(GLUTensors, PUTER_GATE_GLU)
PUTER_TENSORS(ReGLUTensors, PUTER_GATE_REGLU)
PUTER_TENSORS(LinGLUTensors, PUTER_GATE_LINGLU)
PUTER_TENSORS(SeGLUTensors, PUTER_GATE_SEGLU)
PUTER_PACKED(SwiGLU, PUTER_GATE_SWIGLU)
PUTER_PACKED(GeGLU, PUTER_GATE_GEGLU)
PUTER_PACKED(GeGLUTanh, PUTER_GATE_GEGLU_TANH)
PUTER_PACKED(SiGLU, PUTER_GATE_SIGLU)
PUTER_PACKED(GLU, PUTER_GATE_GLU)
PUTER_PACKED(ReGLU, PUTER_GATE_REGLU)
PUTER_PACKED(LinGLU, PUTER_GATE_LINGLU)
PUTER_PACKED(SeGLU, PUTER_GATE_SEGLU)
#undef PUTER_TENSORS
#undef PUTER_PACKED

void Backend::Silu(void *dst, const void *src, int64_t count, DType format) {
    Check(puter_hip_unary(PUTER_UNARY_SILU, dst, src, count, code(format), stream_));
}

void Backend::Gelu(void *dst, const void *src, int64_t count, DType format) {
    Check(puter_hip_unary(PUTER_UNARY_GELU, dst, src, count, code(format), stream_));
}

void Backend::Cast(void *dst, DType dstFormat, const void *src, DType srcFormat, int64_t count) {
    Check(puter_hip_cast(dst, code(dstFormat), src, code(srcFormat), count, stream_));
}

// ---- paged KV hooks ----------------------------------------------------------------------
void Backend::KVPageWrite(const void *storage, const void *values, const void *pageIDs, const void *offsets,
                          void *output, int64_t pageCount, int64_t pageSize, int64_t inner, int64_t valueRows,
                          int64_t storageOffset, DType format) {
    Check(puter_hip_kv_page_write(storage, values, static_cast<const int32_t *>(pageIDs),
                                  static_cast<const int32_t *>(offsets), output, pageCount, pageSize, inner,
                                  valueRows, storageOffset, code(format), StatusWord(), stream_));
}

void Backend::KVPageGather(const void *storage, const void *pageTable, void *output, int64_t pageCount,
                           int64_t pageSize, int64_t inner, int64_t outRows, int64_t storageOffset, DType format) {
    Check(puter_hip_kv_page_gather(storage, static_cast<const int32_t *>(pageTable), output, pageCount, pageSize,
                                   inner, outRows, storageOffset, code(format), StatusWord(), stream_));
}

void Backend::KVPageWriteFP8(void *storage, const void *values, const void *pageIDs, const void *offsets,
                             int64_t pageCount, int64_t pageSize, int64_t kvHeads, int64_t headDim,
                             int64_t valueRows, int64_t storageOffset, const void *scales, DType valueFormat) {
    Check(puter_hip_kv_page_write_fp8(storage, values, static_cast<const int32_t *>(pageIDs),
                                      static_cast<const int32_t *>(offsets), pageCount, pageSize, kvHeads, headDim,
                                      valueRows, storageOffset, static_cast<const float *>(scales),
                                      code(valueFormat), StatusWord(), stream_));
}

// ---- attention -------------------------------------------------------------------------------
void Backend::MultiHeadAttention(const MultiHeadAttentionConfig &config, const void *query, const void *key,
                                 const void *value, void *output, int64_t seqQ, int64_t seqK, DType format) {
    const puter_mha_config c = mha_config(config);
    Check(puter_hip_multi_head_attention(&c, query, key, value, output, seqQ, seqK, code(format), stream_));
}

void Backend::MultiHeadAttentionBatched(const MultiHeadAttentionConfig &config, const void *query,
                                        const void *key, const void *value, void *output, int64_t batch,
                                        int64_t seqQ, int64_t seqK, DType format) {
    const puter_mha_config c = mha_config(config);
    Check(puter_hip_multi_head_attention_batched(&c, query, key, value, output, batch, seqQ, seqK, code(format),
                                                 stream_));
}

void Backend::ScaledDotProductAttention(const FlashAttentionConfig &config, const void *query, const void *key,
                                        const void *value, void *output, int64_t seqQ, int64_t seqK,
                                        int64_t depth, int64_t valueDim, DType format) {
    const puter_flash_config c = flash_config(config);
    Check(puter_hip_scaled_dot_product_attention(&c, query, key, value, output, seqQ, seqK, depth, valueDim,
                                                 code(format), stream_));
}

void Backend::FlashAttention(const FlashAttentionConfig &config, const void *query, const void *key,
                             const void *value, void *output, int64_t seqQ, int64_t seqK, int64_t depth,
                             int64_t valueDim, DType format) {
    const puter_flash_config c = flash_config(config);
    Check(puter_hip_flash_attention(&c, query, key, value, output, seqQ, seqK, depth, valueDim, code(format),
                                    stream_));
}

size_t Backend::PagedDecodeWorkspaceBytes(int64_t batch, int64_t numHeads, int64_t headDim, int64_t maxContext) {
    return puter_hip_paged_decode_workspace_bytes(batch, numHeads, headDim, maxContext);
}

void Backend::PagedDecodeAttention(const void *query, const void *keyPages, const void *valuePages,
                                   const void *pageTable, const void *contextLens, int64_t batch,
                                   int64_t maxPagesPerSeq, int64_t pageSize, int64_t numPages, int64_t numHeads,
                                   int64_t kvHeads, int64_t headDim, int64_t maxContext, const void *kScale,
                                   const void *vScale, DType kvFormat, void *output, void *workspace,
                                   size_t workspaceBytes) {
    Check(puter_hip_paged_decode_attention(query, keyPages, valuePages, static_cast<const int32_t *>(pageTable),
                                           static_cast<const int32_t *>(contextLens), batch, maxPagesPerSeq,
                                           pageSize, numPages, numHeads, kvHeads, headDim, maxContext,
                                           static_cast<const float *>(kScale), static_cast<const float *>(vScale),
                                           code(kvFormat), output, workspace, workspaceBytes, stream_));
}

// ---- quantisation, matmul ---------------------------------------------------------------------
void Backend::Dequant(void *dst, const void *src, int64_t count, const DequantInt8Config &config, DType dstFormat,
                      DType srcFormat) {
    Check(puter_hip_dequant(dst, src, count, config.Scale, config.ZeroPoint, code(dstFormat), code(srcFormat),
                            stream_));
}

void Backend::Dequant4(void *dst, const void *src, int64_t pairCount, const DequantInt4Config &config,
                       DType dstFormat, DType srcFormat) {
    Check(puter_hip_dequant4(dst, src, pairCount, config.Scale, config.ZeroPoint, code(dstFormat), code(srcFormat),
                             stream_));
}

void Backend::Quant(void *dst, const void *src, int64_t count, const DequantInt8Config &config, DType dstFormat,
                    DType srcFormat) {
    Check(puter_hip_quant(dst, src, count, config.Scale, config.ZeroPoint, code(dstFormat), code(srcFormat),
                          stream_));
}

void Backend::Matmul(void *out, const void *left, const void *right, int64_t rows, int64_t inner, int64_t cols,
                     DType format) {
    Check(puter_hip_matmul(out, left, right, rows, inner, cols, code(format), stream_));
}

void Backend::MatmulNoAlloc(void *out, const void *left, const void *right, int64_t rows, int64_t inner,
                            int64_t cols, DType format) {
    Check(puter_hip_matmul_noalloc(out, left, right, rows, inner, cols, code(format), stream_));
}

}  // namespace puter::hip
