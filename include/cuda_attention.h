// cuda_attention.h -- decode attention over the device KV cache, on MI355X.
//
// Same declarations as the reference (include/cuda_attention.h:7-14 of the
// reference tree; src/cuda_attention.cu).  Query head i reads KV head
// i / (n_heads / n_kv_heads) over cache positions 0..pos of `layer`:
//   out_i = softmax_j(q_i . k_j / sqrt(head_dim)) . v_j   (src/forward.cc:265-298)
// Validation and messages follow the reference, before any allocation or
// launch.  The kernels (mlk_attention_decode_f32) split the positions over
// workgroups and read each K/V row once per KV head; head_dim <= 256.
// Implemented in cpp-minilamma_amd/host/cuda_attention.cc.
#pragma once
#include "include/cuda_kvcache.h"
#include "include/cuda_matmul.h"
#include "include/cuda_runtime.h"
#include "include/cuda_tensor.h"

namespace yan_lamma {
// True when the device kernels are built (always, in this build).
bool CudaAttentionBuilt();
// q and output: host [n_heads, head_dim].  Reads the populated cache prefix
// [0, pos]; uploads q, computes on the device and downloads the output.
Tensor CudaAttentionDecode(const Tensor& q, const CudaCache& cache, int layer, int pos,
                           int n_heads, int n_kv_head, int head_dim, int device_id = 0);
// q and output: device [n_heads, head_dim]; q and cache on device_id.
CudaTensor CudaAttentionDevice(const CudaTensor& q, const CudaCache& cache, int layer, int pos,
                               int n_heads, int n_kv_head, int head_dim, int device_id = 0);

// ---- additions (no reference counterpart) --------------------------------
// T query rows at once: q is device [T, n_heads, head_dim] (or
// [T, n_heads * head_dim]), row t at position pos0 + t attending to cache
// positions 0..pos0 + t (causal over the cache, as a prefill chunk after
// CudaKvWriteBatchDevice).  Returns device [T, n_heads, head_dim].
CudaTensor CudaAttentionBatchDevice(const CudaTensor& q, const CudaCache& cache, int layer,
                                    int pos0, int n_heads, int n_kv_heads, int head_dim,
                                    int device_id = 0);
}  // namespace yan_lamma
