// cuda_kvcache.h -- the device KV cache, on MI355X.
//
// Same declarations and member layout as the reference's device KV cache
// (include/cuda_kvcache.h:1-57 of the reference tree; src/cuda_kvcache.cc):
//   keys:   [n_layers, max_seq_len, n_kv_heads, head_dim] fp32
//   values: [n_layers, max_seq_len, n_kv_heads, head_dim] fp32
// Validation and messages follow the reference.  Differences a caller can
// see: Clear() zeroes the buffers on the device instead of uploading a host
// zero array (no H2D copies are counted for it), and WriteDevice is one
// kernel launch (mlk_kv_write_f32) instead of two device-to-device copies.
// Implemented in cpp-minilamma_amd/host/cuda_kvcache.cc.
#pragma once
#include "include/cuda_tensor.h"
#include "include/cuda_runtime.h"
#include "include/tensor.h"

namespace yan_lamma {
// True when the device cache is built (always, in this build).
bool CudaCacheBuild();
class CudaCache {
 public:
    CudaCache() = default;
    CudaCache(int n_layers, int max_seq_len, int n_kv_heads, int head_dim, int device_id = 0);
    ~CudaCache();
    CudaCache(const CudaCache&) = delete;
    CudaCache& operator=(const CudaCache&) = delete;
    CudaCache(CudaCache&&) noexcept = default;
    CudaCache& operator=(CudaCache&&) noexcept = default;
    void Reset();
    void Reset(int n_layers, int max_seq_len, int n_kv_heads, int head_dim, int device_id = 0);
    // k, v: host [n_kv_heads, head_dim] into slot (layer, pos)
    void WriteHost(int layer, int pos, const yan_lamma::Tensor& k, const Tensor& v) const;
    // k, v: device [n_kv_heads, head_dim] on the cache's device
    void WriteDevice(int layer, int pos, const CudaTensor& k, const CudaTensor& v) const;
    // slot (layer, pos) as host [n_kv_heads, head_dim]
    Tensor ReadKey(int layer, int pos) const;
    Tensor ReadVal(int layer, int pos) const;
    // one KV head of slot (layer, pos) as host [head_dim]
    Tensor ReadHeadKey(int layer, int pos, int head) const;
    Tensor ReadHeadVal(int layer, int pos, int head) const;
    // device addresses of the whole key / value buffers
    const void* KData() const;
    const void* vData() const;
    size_t Bytes_() const;
    int n_layers() const { return n_layers_; }
    int max_seq_len() const { return max_seq_len_; }
    int n_kv_heads() const { return n_kv_heads_; }
    int head_dim() const { return head_dim_; }
    int device_id() const { return device_id_; }
    void Clear();
    // byte offset of slot (layer, pos) [and of one KV head in it]
    size_t SlotOffsetBytes(int layer, int pos) const;
    size_t SlotOffsetBytes(int layer, int pos, int head) const;

 private:
    int n_layers_ = 0;
    int max_seq_len_ = 0;
    int n_kv_heads_ = 0;
    int head_dim_ = 0;
    int device_id_ = 0;
    yan_lamma::CudaDeviceBuffer k_;
    yan_lamma::CudaDeviceBuffer v_;
};

// ---- additions (no reference counterpart) --------------------------------
// Writes T rows at once: k and v are device [T, n_kv_heads, head_dim] (or
// [T, n_kv_heads * head_dim]) on the cache's device, row t going to slot
// (layer, pos0 + t).  One launch; the prefill path writes a whole chunk.
void CudaKvWriteBatchDevice(const CudaCache& cache, int layer, int pos0, const CudaTensor& k,
                            const CudaTensor& v);
}  // namespace yan_lamma
