// forward_batch_device.cc -- see forward_batch_device.h.  Everything here is
// built on the reference's public types (Model, Context, Batch, CudaTensor,
// CudaCache) and on this library's batched entries (include/cuda_ops.h,
// include/cuda_forward.h); nothing reaches HIP directly.
#include "tests/dropin/forward_batch_device.h"

#include "include/cuda_forward.h"
#include "include/cuda_ops.h"
#include "include/forward.h"
#include "src/internal/cuda_stats.h"

#include <stdexcept>
#include <string>

namespace yan_lamma {

// src/forward.cc:425-431: final RmsNorm, lm_head, one logits download.  It has
// external linkage there; a maintainer adding this file's code to
// src/forward.cc needs no declaration.
Tensor ComputeLogitsDevice(const Model& model, CudaTensor& x);

namespace {

const CudaloadWeight* Find(const Model& model, const std::string& name, QuantType type) {
    for (const CudaloadWeight& w : model.cuda_weights->weights) {
        if (w.name == name && w.type == type) return &w;
    }
    return nullptr;
}

const void* Need(const Model& model, const std::string& name, QuantType type) {
    const CudaloadWeight* w = Find(model, name, type);
    if (w == nullptr) throw std::runtime_error("ForwardBatchDevice: CUDA weight not found: " + name);
    return w->buffer.GetData();
}

// A layer's device weights under the names UploadModelWeightToCuda gives them
// (src/model.cc:311-332).
CudaLayerWeights DeviceLayer(const Model& model, int i) {
    const Layer& L = model.n_layers_[i];
    const std::string p = "blk." + std::to_string(i) + ".";
    auto linear = [&](const char* name, const QuanTensor& t, const char* bias,
                      const Tensor& b) {
        CudaLinearWeight w;
        w.type = t.type;
        w.data = Need(model, p + name, t.type);
        if (!b.data.empty()) {
            w.bias = static_cast<const float*>(Need(model, p + bias, QuantType::kF32));
        }
        return w;
    };
    const Tensor none;
    CudaLayerWeights w;
    w.attention_norm = static_cast<const float*>(Need(model, p + "attention_norm", QuantType::kF32));
    w.ffn_norm = static_cast<const float*>(Need(model, p + "ffn_norm", QuantType::kF32));
    w.wq = linear("wq", L.wq, "bq", L.bq);
    w.wk = linear("wk", L.wk, "bk", L.bk);
    w.wv = linear("wv", L.wv, "bv", L.bv);
    w.wo = linear("wo", L.wo, nullptr, none);
    w.w_gate = linear("w_gate", L.w_gate, nullptr, none);
    w.w_up = linear("w_up", L.w_up, nullptr, none);
    w.w_down = linear("w_down", L.w_down, nullptr, none);
    return w;
}

bool Increasing(const std::vector<int>& poss) {
    for (size_t i = 1; i < poss.size(); ++i) {
        if (poss[i] <= poss[i - 1]) return false;
    }
    return true;
}

size_t BlockBytes(QuantType type) {
    switch (type) {
        case QuantType::kQ80: return kBytesPerQ80Block;
        case QuantType::kQ40: return kBytesPerQ40Block;
        case QuantType::kQ41: return kBytesPerQ41Block;
        default: return 0;
    }
}

const void* BlockData(const QuanTensor& t, size_t* count) {
    switch (t.type) {
        case QuantType::kQ80: *count = t.kQ80_data.size(); return t.kQ80_data.data();
        case QuantType::kQ40: *count = t.kQ40_data.size(); return t.kQ40_data.data();
        case QuantType::kQ41: *count = t.kQ41_data.size(); return t.kQ41_data.data();
        default: *count = 0; return nullptr;
    }
}

}  // namespace

const CudaloadWeight* DeviceTokenTable(const Model& model) {
    if (!model.cuda_weights) return nullptr;
    for (const CudaloadWeight& w : model.cuda_weights->weights) {
        if (w.name == "embedding_data_") return &w;
    }
    return nullptr;
}

void UploadTokenTableBlocks(Model& model, const QuanTensor& table) {
    const char* caller = "UploadTokenTableBlocks: ";
    if (!model.cuda_weights) {
        throw std::runtime_error(std::string(caller) + "CUDA weights are not loaded");
    }
    const size_t block_bytes = BlockBytes(table.type);
    if (block_bytes == 0) {
        throw std::runtime_error(std::string(caller) + "the table must be Q8_0, Q4_0 or Q4_1");
    }
    const ModelConfig& c = model.config;
    if (table.shape != std::vector<int>{c.vocab_size, c.dim}) {
        throw std::runtime_error(std::string(caller) + "the table must be [vocab_size, dim]");
    }
    size_t count = 0;
    const void* blocks = BlockData(table, &count);
    const size_t per_row = (static_cast<size_t>(c.dim) + kQuantBlockSize - 1) / kQuantBlockSize;
    if (count != per_row * static_cast<size_t>(c.vocab_size)) {
        throw std::runtime_error(std::string(caller) + "expected " +
                                 std::to_string(per_row * c.vocab_size) + " blocks, got " +
                                 std::to_string(count));
    }
    CudaModelWeights& arr = *model.cuda_weights;
    CudaloadWeight w;
    w.name = "embedding_data_";
    w.type = table.type;
    w.linear = false;
    w.shape = table.shape;
    w.block_count = count;
    w.buffer.Reset(count * block_bytes, arr.device_id);
    w.buffer.upload(blocks, count * block_bytes);
    for (auto it = arr.weights.begin(); it != arr.weights.end(); ++it) {
        if (it->name == "embedding_data_") {  // the F32 copy of src/model.cc:307
            arr.uploaded_bytes -= it->buffer.GetByteSize();
            --arr.uploaded_weight_count;
            arr.weights.erase(it);
            break;
        }
    }
    arr.uploaded_bytes += count * block_bytes;
    ++arr.uploaded_weight_count;
    arr.weights.push_back(std::move(w));
}

Tensor ForwardBatchDevice(const Model& model, Context& context, const Batch& batch) {
    // ForwardBatch's own checks (src/forward.cc:474-479)
    if (batch.tokens.size() == 0) {
        throw std::runtime_error("Empty Batch");
    }
    if (batch.tokens.size() != batch.poss.size()) {
        throw std::runtime_error("Tokens Pos Not Matched");
    }
    if (!model.cuda_weights || !Increasing(batch.poss)) {
        return ForwardBatch(model, context, batch);
    }
    // ForwardToken's checks for every token (src/forward.cc:433-447)
    const ModelConfig& c = model.config;
    if (!model.is_loaded) {
        throw std::runtime_error("Model Load Failed");
    }
    for (size_t i = 0; i < batch.tokens.size(); ++i) {
        if (batch.tokens[i] < 0 || batch.tokens[i] >= c.vocab_size) {
            throw std::out_of_range("ForwardToken: token out of range");
        }
        if (batch.poss[i] < 0 || batch.poss[i] >= c.max_seq_len) {
            throw std::out_of_range("ForwardToken position out of range");
        }
    }
    if (model.n_layers_.size() != static_cast<size_t>(c.layers)) {
        throw std::runtime_error("Layer Match Failed");
    }
    const int device = model.cuda_weights->device_id;
    if (context.cuda_cache_.Bytes_() == 0) {
        context.cuda_cache_.Reset(c.layers, c.max_seq_len, c.n_kv_heads, c.head_dim, device);
    }
    internal::CudaStatsScope scope(model.cuda_weights.get());

    // every token's row at once (EmbeddingDevice, src/forward.cc:206-212)
    const CudaloadWeight* table = DeviceTokenTable(model);
    if (table == nullptr) {
        throw std::runtime_error("ForwardBatchDevice: CUDA weight not found: embedding_data_");
    }
    CudaTensor x = table->type == QuantType::kF32
                       ? CudaEmbeddingBatchDevice(table->buffer.GetData(), table->shape,
                                                  batch.tokens, device)
                       : CudaEmbeddingQuantDevice(table->buffer.GetData(), table->type,
                                                  table->shape, batch.tokens, device);

    // every layer once over all rows (ForwardLayerDevice, src/forward.cc:337-384)
    CudaLayerConfig lc;
    lc.dim = c.dim;
    lc.hidden_dim = c.hidden_dim;
    lc.n_heads = c.n_heads;
    lc.n_kv_heads = c.n_kv_heads;
    lc.head_dim = c.head_dim;
    lc.rope_theta = c.rope_theta;
    lc.rms_norm_eps = c.rms_norm_eps;
    lc.rope_type = c.rope_type;
    for (int i = 0; i < c.layers; ++i) {
        CudaForwardLayerBatchDevice(lc, DeviceLayer(model, i), x, context.cuda_cache_, i,
                                    batch.poss, device);
    }

    // the last row's logits, as ForwardToken returns them for the last token
    const int T = static_cast<int>(batch.tokens.size());
    CudaTensor last({c.dim}, device);
    CudaMemcpy(last.GetData(),
               static_cast<const char*>(x.GetData()) + static_cast<size_t>(T - 1) * c.dim *
                   sizeof(float),
               static_cast<size_t>(c.dim) * sizeof(float), CudaMemoryKind::kDeviceDevice);
    Tensor logits = ComputeLogitsDevice(model, last);
    context.pos = static_cast<size_t>(batch.poss.back());
    context.token_id_.insert(context.token_id_.end(), batch.tokens.begin(), batch.tokens.end());
    return logits;
}

}  // namespace yan_lamma
