// cuda_forward.cc -- the batched layer (include/cuda_forward.h) over the C ABI
// of libminilamma_hip.so.  No HIP header is included here.
#include "include/cuda_forward.h"
#include "include/minilamma_hip.h"

#include <stdexcept>
#include <string>

namespace yan_lamma {

namespace {

[[noreturn]] void Throw(const std::string& reason) {
    throw std::runtime_error("CudaForwardLayerBatchDevice: " + reason);
}

mlk_linear_weight ToC(const CudaLinearWeight& w, const char* name) {
    mlk_linear_weight c{};
    switch (w.type) {
        case QuantType::kF32: c.type = MLK_WEIGHT_F32; break;
        case QuantType::kQ80: c.type = MLK_Q8_0; break;
        case QuantType::kQ40: c.type = MLK_Q4_0; break;
        case QuantType::kQ41: c.type = MLK_Q4_1; break;
        default: Throw(std::string("unsupported weight type for ") + name);
    }
    if (w.data == nullptr) Throw(std::string("weight ") + name + " is null");
    c.data = w.data;
    c.bias = w.bias;
    c.planar = w.planar;
    return c;
}

}  // namespace

namespace {

// Checks shared by both overloads; returns T.
int CheckCall(const CudaLayerConfig& config, const CudaTensor& x, const CudaCache& cache,
              int layer, int device_id) {
    if (x.IsEmpty() || x.num_dims() != 2 || x.shape()[1] != config.dim) {
        Throw("x must be a non-empty [T, dim] tensor");
    }
    if (x.DeviceId() != device_id || cache.device_id() != device_id) {
        Throw("x and the cache must be on device " + std::to_string(device_id));
    }
    if (cache.KData() == nullptr || cache.n_kv_heads() != config.n_kv_heads ||
        cache.head_dim() != config.head_dim) {
        Throw("cache must be initialized with the layer's n_kv_heads and head_dim");
    }
    if (layer < 0 || layer >= cache.n_layers()) {
        Throw("layer " + std::to_string(layer) + " out of range [0, " +
              std::to_string(cache.n_layers()) + ")");
    }
    return x.shape()[0];
}

// One mlk_forward_layer_batch call: tokens at d_positions[t] (device) or,
// when d_positions is null, at pos0 + t.
void Run(const CudaLayerConfig& config, const CudaLayerWeights& weights, CudaTensor& x,
         CudaCache& cache, int layer, const int32_t* d_positions, int pos0, int64_t max_ctx,
         int device_id) {
    const int T = x.shape()[0];
    mlk_layer_config c{};
    c.dim = config.dim;
    c.hidden_dim = config.hidden_dim;
    c.n_heads = config.n_heads;
    c.n_kv_heads = config.n_kv_heads;
    c.head_dim = config.head_dim;
    c.rope_type = config.rope_type == RopeType::kNeoX ? MLK_ROPE_NEOX : MLK_ROPE_NORMAL;
    c.rope_theta = config.rope_theta;
    c.rms_norm_eps = config.rms_norm_eps;
    mlk_layer_weights w{};
    w.attention_norm = weights.attention_norm;
    w.ffn_norm = weights.ffn_norm;
    w.wq = ToC(weights.wq, "wq");
    w.wk = ToC(weights.wk, "wk");
    w.wv = ToC(weights.wv, "wv");
    w.wo = ToC(weights.wo, "wo");
    w.w_gate = ToC(weights.w_gate, "w_gate");
    w.w_up = ToC(weights.w_up, "w_up");
    w.w_down = ToC(weights.w_down, "w_down");
    const int64_t bytes =
        mlk_forward_layer_workspace_bytes(&c, T, max_ctx, d_positions == nullptr ? 1 : 0);
    if (bytes <= 0) Throw("invalid layer configuration");
    SetCudaService(device_id);
    CudaDeviceBuffer ws(static_cast<size_t>(bytes), device_id);
    const mlk_status st = mlk_forward_layer_batch(
        &c, &w, static_cast<float*>(x.GetData()), T, d_positions, pos0,
        static_cast<float*>(const_cast<void*>(cache.KData())),
        static_cast<float*>(const_cast<void*>(cache.vData())), cache.n_layers(),
        cache.max_seq_len(), layer, max_ctx, ws.GetData(), ws.GetByteSize(), nullptr, nullptr);
    if (st != MLK_OK) Throw(mlk_last_error());
}

}  // namespace

void CudaForwardLayerBatchDevice(const CudaLayerConfig& config, const CudaLayerWeights& weights,
                                 CudaTensor& x, CudaCache& cache, int layer, int pos0,
                                 int device_id) {
    const int T = CheckCall(config, x, cache, layer, device_id);
    if (pos0 < 0 || static_cast<int64_t>(pos0) + T > cache.max_seq_len()) {
        Throw("positions " + std::to_string(pos0) + ".." + std::to_string(pos0 + T - 1) +
              " out of range [0, " + std::to_string(cache.max_seq_len()) + ")");
    }
    Run(config, weights, x, cache, layer, nullptr, pos0, static_cast<int64_t>(pos0) + T,
        device_id);
}

void CudaForwardLayerBatchDevice(const CudaLayerConfig& config, const CudaLayerWeights& weights,
                                 CudaTensor& x, CudaCache& cache, int layer,
                                 const std::vector<int>& positions, int device_id) {
    const int T = CheckCall(config, x, cache, layer, device_id);
    if (positions.size() != static_cast<size_t>(T)) {
        Throw("positions must hold one position per row of x (" + std::to_string(T) + "), got " +
              std::to_string(positions.size()));
    }
    bool consecutive = true;
    for (int t = 0; t < T; ++t) {
        if (positions[t] < 0 || positions[t] >= cache.max_seq_len()) {
            Throw("position " + std::to_string(positions[t]) + " out of range [0, " +
                  std::to_string(cache.max_seq_len()) + ")");
        }
        if (t > 0 && positions[t] <= positions[t - 1]) {
            Throw("positions must be strictly increasing");
        }
        consecutive = consecutive && positions[t] == positions[0] + t;
    }
    if (consecutive) {
        Run(config, weights, x, cache, layer, nullptr, positions[0],
            static_cast<int64_t>(positions[0]) + T, device_id);
        return;
    }
    SetCudaService(device_id);
    CudaDeviceBuffer d_pos(positions.size() * sizeof(int32_t), device_id);
    d_pos.upload(positions.data(), positions.size() * sizeof(int32_t));
    Run(config, weights, x, cache, layer, static_cast<const int32_t*>(d_pos.GetData()), 0,
        static_cast<int64_t>(positions.back()) + 1, device_id);
}

}  // namespace yan_lamma
