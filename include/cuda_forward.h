// cuda_forward.h -- one transformer layer over a batch of tokens on the
// device: the reference's ForwardLayerDevice (src/forward.cc:337-384 of the
// reference tree) for T tokens at once, so that ForwardBatch (:473-488) can
// run its prompt layer by layer instead of token by token.  No counterpart
// in the reference; a caller builds the weights from its own device buffers
// (FindLoadWeight in src/forward.cc).
// Implemented in cpp-minilamma_amd/host/cuda_forward.cc over
// mlk_forward_layer_batch.
#pragma once
#include "include/cuda_kvcache.h"
#include "include/cuda_tensor.h"
#include "include/model.h"
#include "include/quantized_tensor.h"

#include <vector>

namespace yan_lamma {

// A device linear weight [out, in]: fp32 (kF32) or packed Q8_0 / Q4_0 /
// Q4_1 blocks, borrowed; bias [out] (device) or null; planar: null, or the
// same Q8_0 / Q4_0 weight in the planar layout (mlk_quant_to_planar), which
// calls of 1..32 tokens then use (one token: the planar streaming GEMV;
// 2..32: the planar matrix-core kernel).
struct CudaLinearWeight {
    QuantType type = QuantType::kF32;
    const void* data = nullptr;
    const float* bias = nullptr;
    const void* planar = nullptr;
};

// The device weights of one layer (the reference's Layer, include/model.h).
struct CudaLayerWeights {
    const float* attention_norm = nullptr;  // [dim]
    CudaLinearWeight wq, wk, wv, wo;
    const float* ffn_norm = nullptr;        // [dim]
    CudaLinearWeight w_gate, w_up, w_down;
};

// The ModelConfig fields a layer uses.
struct CudaLayerConfig {
    int dim = 0;
    int hidden_dim = 0;
    int n_heads = 0;
    int n_kv_heads = 0;
    int head_dim = 0;
    float rope_theta = 10000.0f;
    float rms_norm_eps = 1e-5f;
    RopeType rope_type = RopeType::kNormal;
};

// x [T, dim] (device, updated in place) through layer `layer` for tokens at
// positions pos0 .. pos0 + T - 1: their K/V rows go to `cache`, each token
// attends to positions 0 .. its own.  Equal to T calls of the reference's
// ForwardLayerDevice at those positions.  The intermediates come from the
// caching device allocator.
void CudaForwardLayerBatchDevice(const CudaLayerConfig& config, const CudaLayerWeights& weights,
                                 CudaTensor& x, CudaCache& cache, int layer, int pos0,
                                 int device_id = 0);

// The same for tokens at positions[t] (the reference's Batch::poss,
// include/batch.h:5-8), positions.size() == T, strictly increasing and in
// [0, max_seq_len): all K/V rows are written before any token attends,
// which equals the reference's token loop only when each token's
// predecessors sit at lower positions.  Consecutive positions run as the
// pos0 overload (nothing copied); otherwise the positions are copied to the
// device once per call (one counted host-to-device copy of 4 T bytes).
void CudaForwardLayerBatchDevice(const CudaLayerConfig& config, const CudaLayerWeights& weights,
                                 CudaTensor& x, CudaCache& cache, int layer,
                                 const std::vector<int>& positions, int device_id = 0);

}  // namespace yan_lamma
