// cuda_ops.h -- the per-layer op surface forward.cc calls, on MI355X.
//
// The first block keeps the reference's declarations unchanged
// (include/cuda_ops.h:11-33 of the reference tree): same names (including
// "CudaRmsNromDevice"), arguments, defaults, ownership (each *Device op
// returns a new device tensor, RoPE works in place, weight pointers are
// borrowed device pointers) and error behaviour (std::runtime_error
// "<Caller>: <reason>" before any launch).  Implemented in
// cpp-minilamma_amd/host/cuda_ops.cc over the C ABI (minilamma_hip.h); all
// work is issued on the null stream, in order.
//
// The second block adds the batched and fused entries the reference lacks
// (its ops take one token per call): residual add fused with RMSNorm over
// [T, D], SwiGLU in one kernel, RoPE over T tokens with per-token positions,
// batched F32 and block-quantized token gathers, and the device quantizer.
#pragma once
#include "include/cuda_tensor.h"
#include "include/model.h"
#include "include/quantized_tensor.h"
#include "include/tensor.h"

#include <vector>

namespace yan_lamma {
// ---- reference surface (include/cuda_ops.h:11-33) -------------------------

// Always true in this build; equals CudaRuntimeBuilt().
bool CudaopsBuild();
// One embedding row: table [vocab, dim] (device, borrowed) -> new [dim].
CudaTensor CudaEmbeddingDevice(const void* embedding_data, const std::vector<int>& shape,
                               int token_id, int device_id = 0);
// RMSNorm of a 1-D host tensor through the device (upload, run, download).
Tensor CudaRmsNormHost(const Tensor& x, const Tensor& weight, float eps, int device_id = 0);
// RMSNorm of a 1-D device tensor; weight is a device pointer of shape x.shape().
CudaTensor CudaRmsNromDevice(const CudaTensor& x, const void* weight_data,
                             const std::vector<int>& shape, float eps, int device_id = 0);
Tensor CudaSilu(const Tensor& a, int device_id = 0);
CudaTensor CudaSiluDevice(const CudaTensor& a, int device_id = 0);
Tensor CudaElementwiseMul(const Tensor& a, const Tensor& b, int device_id = 0);
CudaTensor CudaElementwiseMulDevice(const CudaTensor& a, const CudaTensor& b, int device_id = 0);
// Residual add: a + b, same shapes.
CudaTensor CudaElementAddDevice(const CudaTensor& a, const CudaTensor& b, int device_id = 0);
// Bias add: a + b where b is a device pointer of the given shape.
CudaTensor OCudaElementAddDevice(const CudaTensor& a, const void* b, const std::vector<int>& shape,
                                 int device_id = 0);
// Softmax of a 1-D host tensor through the device.
Tensor CudaSoftmax(Tensor& x, int device_id = 0);
// RoPE of one token on host q [n_heads, head_dim] and k [n_kv_heads, head_dim].
void CudaRopeHost(Tensor& q, Tensor& k, int pos, float theta,
                  RopeType rope_type = RopeType::kNormal, int device_id = 0);
// RoPE of one token, in place on device q and k.
void CudaRopeDevice(CudaTensor& q, CudaTensor& k, int pos, int n_heads, int n_kv_heads,
                    int headdim, float theta, RopeType rope_type = RopeType::kNormal,
                    int device_id = 0);

// ---- batched and fused entries (no reference counterpart) ------------------

// residual [..., D] <- residual + delta (delta may be nullptr: no add, the
// residual is left as it is); returns RMSNorm(residual) * weight row by row.
// weight_data is a device pointer of shape weight_shape = {D}.  One kernel.
CudaTensor CudaAddRmsNormDevice(CudaTensor& residual, const CudaTensor* delta,
                                const void* weight_data, const std::vector<int>& weight_shape,
                                float eps, int device_id = 0);
// Row-wise RMSNorm of x [..., D] (any rank >= 1) into a new tensor.
CudaTensor CudaRmsNormRowsDevice(const CudaTensor& x, const void* weight_data,
                                 const std::vector<int>& weight_shape, float eps,
                                 int device_id = 0);
// SiLU(gate) * up in one kernel (ForwardSwiGlu without the silu round trip).
CudaTensor CudaSwiGluDevice(const CudaTensor& gate, const CudaTensor& up, int device_id = 0);
// RoPE over T = positions.size() tokens, in place: q holds T * n_heads *
// head_dim elements ([T, n_heads, head_dim]), k T * n_kv_heads * head_dim.
// positions are copied to the device (one counted host-to-device copy).
void CudaRopeBatchDevice(CudaTensor& q, CudaTensor& k, const std::vector<int>& positions,
                         int n_heads, int n_kv_heads, int head_dim, float theta,
                         RopeType rope_type = RopeType::kNormal, int device_id = 0);
// RoPE over T tokens at contiguous positions pos0 .. pos0 + T - 1 (prefill);
// T is q.NumEle() / (n_heads * head_dim).  No host-to-device copy.
void CudaRopeRangeDevice(CudaTensor& q, CudaTensor& k, int pos0, int n_heads, int n_kv_heads,
                         int head_dim, float theta, RopeType rope_type = RopeType::kNormal,
                         int device_id = 0);
// Embedding rows of token_ids from an F32 table [vocab, dim] -> [T, dim].
// One id is passed to the kernel as an argument; more are copied to the
// device (one counted host-to-device copy of 4 T bytes).  Likewise below.
CudaTensor CudaEmbeddingBatchDevice(const void* embedding_data, const std::vector<int>& shape,
                                    const std::vector<int>& token_ids, int device_id = 0);
// Embedding rows of token_ids from a block-quantized table (type kQ80, kQ40
// or kQ41; shape {vocab, dim}; rows of ceil(dim / 32) packed blocks as
// TensorToQ80/Q40/Q41 write them), dequantized on the fly -> [T, dim].
CudaTensor CudaEmbeddingQuantDevice(const void* blocks, QuantType type,
                                    const std::vector<int>& shape,
                                    const std::vector<int>& token_ids, int device_id = 0);
// Quantizes x [rows, cols] (last dimension = cols) into packed blocks on the
// device, byte-identical to TensorToQ80 / TensorToQ40 / TensorToQ41.
CudaDeviceBuffer CudaQuantizeDevice(const CudaTensor& x, QuantType type, int device_id = 0);
}  // namespace yan_lamma
