// cuda_attention.cc -- decode attention (include/cuda_attention.h) over the
// C ABI of libminilamma_hip.so.  No HIP header is included here.
//
// Checks and messages follow the reference (src/cuda_attention.cu:23-73 and
// :178-264 of the reference tree), in its order: cache buffers, layer and
// pos ranges, positive head counts and head_dim, GQA divisibility, the
// cache's KV shape and device, size overflow, then q's shape (and, on the
// device path, q non-empty and on the cache's device).  The chunk
// workspace comes from the caching allocator, so a call costs no hipMalloc
// after the first.
#include "include/cuda_attention.h"
#include "include/minilamma_hip.h"

#include <limits>
#include <stdexcept>
#include <string>
#include <vector>

namespace yan_lamma {

bool CudaAttentionBuilt() { return CudaRuntimeBuilt(); }

namespace {

[[noreturn]] void Throw(const std::string& caller, const std::string& reason) {
    throw std::runtime_error(caller + ": " + reason);
}

void CheckIndex(int index, int limit, const char* caller) {
    if (index < 0 || index >= limit) {
        Throw(caller, "index " + std::to_string(index) + " out of range [0, " +
                          std::to_string(limit) + ")");
    }
}

void RequirePositive(int value, const char* caller) {
    if (value <= 0) Throw(caller, "value must be positive, got " + std::to_string(value));
}

void CheckMul(size_t a, size_t b, const char* caller) {
    if (a != 0 && b > std::numeric_limits<size_t>::max() / a) {
        Throw(caller, "size multiplication overflow for " + std::to_string(a) + " * " +
                          std::to_string(b));
    }
}

void CheckArgs(const CudaCache& cache, int layer, int pos, int n_heads, int n_kv_heads,
               int head_dim, int device_id, const char* caller) {
    if (cache.KData() == nullptr || cache.vData() == nullptr) {
        Throw(caller, "key and value cache buffers must both be initialized");
    }
    CheckIndex(layer, cache.n_layers(), caller);
    CheckIndex(pos, cache.max_seq_len(), caller);
    RequirePositive(n_heads, caller);
    RequirePositive(n_kv_heads, caller);
    RequirePositive(head_dim, caller);
    if (n_kv_heads == 0 || n_heads % n_kv_heads != 0) {
        Throw(caller, "n_kv_heads must be non-zero and divide n_heads, got n_heads=" +
                          std::to_string(n_heads) + ", n_kv_heads=" + std::to_string(n_kv_heads));
    }
    if (cache.n_kv_heads() != n_kv_heads) {
        Throw(caller, "cache n_kv_heads mismatch, expected " + std::to_string(n_kv_heads) +
                          ", got " + std::to_string(cache.n_kv_heads()));
    }
    if (cache.head_dim() != head_dim) {
        Throw(caller, "cache head_dim mismatch, expected " + std::to_string(head_dim) +
                          ", got " + std::to_string(cache.head_dim()));
    }
    if (cache.device_id() != device_id) {
        Throw(caller, "cache device_id mismatch, expected " + std::to_string(device_id) +
                          ", got " + std::to_string(cache.device_id()));
    }
    CheckMul(static_cast<size_t>(n_heads), static_cast<size_t>(head_dim), caller);
}

// Runs the kernels for T query rows at positions pos0..pos0+T-1 into out: a
// chunk of 16 or more rows with head_dim 64 / 128 takes the causal prefill
// kernel (no workspace), anything else the decode kernel.
void Attend(const float* q, float* out, int64_t T, const CudaCache& cache, int layer, int pos0,
            int n_heads, int n_kv_heads, int head_dim, int device_id, const char* caller) {
    if (T >= 16 && (head_dim == 64 || head_dim == 128)) {
        const mlk_status st = mlk_attention_prefill_f32(
            q, static_cast<int64_t>(n_heads) * head_dim, static_cast<const float*>(cache.KData()),
            static_cast<const float*>(cache.vData()), cache.n_layers(), cache.max_seq_len(),
            n_heads, n_kv_heads, head_dim, layer, pos0, T, out, nullptr);
        if (st != MLK_OK) Throw(caller, mlk_last_error());
        return;
    }
    const int64_t max_ctx = static_cast<int64_t>(pos0) + T;
    const int64_t ws_bytes =
        mlk_attention_workspace_bytes(T, n_heads, n_kv_heads, head_dim, max_ctx);
    CudaDeviceBuffer ws;
    if (ws_bytes > 0) ws.Reset(static_cast<size_t>(ws_bytes), device_id);
    const mlk_status st = mlk_attention_decode_f32(
        q, static_cast<int64_t>(n_heads) * head_dim, static_cast<const float*>(cache.KData()),
        static_cast<const float*>(cache.vData()), cache.n_layers(), cache.max_seq_len(), n_heads,
        n_kv_heads, head_dim, layer, nullptr, pos0, T, max_ctx, out, ws.GetData(),
        static_cast<size_t>(ws_bytes > 0 ? ws_bytes : 0), nullptr, nullptr);
    if (st != MLK_OK) Throw(caller, mlk_last_error());
}

}  // namespace

Tensor CudaAttentionDecode(const Tensor& q, const CudaCache& cache, int layer, int pos,
                           int n_heads, int n_kv_head, int head_dim, int device_id) {
    const char* caller = "CudaAttentionDecode";
    CheckArgs(cache, layer, pos, n_heads, n_kv_head, head_dim, device_id, caller);
    const size_t out_elements = static_cast<size_t>(n_heads) * head_dim;
    if (q.shape != std::vector<int>{n_heads, head_dim} || q.GetDataSize() != out_elements) {
        Throw(caller, "q shape and element count must match [n_heads, head_dim]");
    }
    SetCudaService(device_id);
    const size_t bytes = out_elements * sizeof(float);
    CudaDeviceBuffer qb(bytes, device_id);
    CudaDeviceBuffer ob(bytes, device_id);
    qb.upload(q.data.data(), bytes);
    Attend(static_cast<const float*>(qb.GetData()), static_cast<float*>(ob.GetData()), 1, cache,
           layer, pos, n_heads, n_kv_head, head_dim, device_id, caller);
    Tensor out({n_heads, head_dim});
    ob.download(out.data.data(), bytes);
    return out;
}

CudaTensor CudaAttentionDevice(const CudaTensor& q, const CudaCache& cache, int layer, int pos,
                               int n_heads, int n_kv_head, int head_dim, int device_id) {
    const char* caller = "CudaAttentionDevice";
    CheckArgs(cache, layer, pos, n_heads, n_kv_head, head_dim, device_id, caller);
    const size_t out_elements = static_cast<size_t>(n_heads) * head_dim;
    CheckMul(out_elements, sizeof(float), caller);
    if (q.shape() != std::vector<int>{n_heads, head_dim} || q.NumEle() != out_elements) {
        Throw(caller, "q shape and element count must match [n_heads, head_dim]");
    }
    if (q.IsEmpty()) Throw(caller, "q must not be empty");
    if (q.DeviceId() != cache.device_id()) {
        Throw(caller, "q and cache must be on the same CUDA device, got q device_id=" +
                          std::to_string(q.DeviceId()) + ", cache device_id=" +
                          std::to_string(cache.device_id()));
    }
    SetCudaService(device_id);
    CudaTensor out({n_heads, head_dim}, device_id);
    Attend(static_cast<const float*>(q.GetData()), static_cast<float*>(out.GetData()), 1, cache,
           layer, pos, n_heads, n_kv_head, head_dim, device_id, caller);
    return out;
}

CudaTensor CudaAttentionBatchDevice(const CudaTensor& q, const CudaCache& cache, int layer,
                                    int pos0, int n_heads, int n_kv_heads, int head_dim,
                                    int device_id) {
    const char* caller = "CudaAttentionBatchDevice";
    if (q.IsEmpty() || q.shape().empty()) Throw(caller, "q must not be empty");
    const int T = q.shape()[0];
    const int64_t last = static_cast<int64_t>(pos0) + T - 1;
    if (pos0 < 0 || last >= cache.max_seq_len()) {
        Throw(caller, "positions " + std::to_string(pos0) + ".." + std::to_string(last) +
                          " out of range [0, " + std::to_string(cache.max_seq_len()) + ")");
    }
    CheckArgs(cache, layer, static_cast<int>(last), n_heads, n_kv_heads, head_dim, device_id,
              caller);
    const size_t row = static_cast<size_t>(n_heads) * head_dim;
    if (q.NumEle() != static_cast<size_t>(T) * row) {
        Throw(caller, "q must hold [T, n_heads, head_dim] elements");
    }
    if (q.DeviceId() != cache.device_id()) {
        Throw(caller, "q and cache must be on the same device, got q device_id=" +
                          std::to_string(q.DeviceId()) + ", cache device_id=" +
                          std::to_string(cache.device_id()));
    }
    SetCudaService(device_id);
    CudaTensor out({T, n_heads, head_dim}, device_id);
    Attend(static_cast<const float*>(q.GetData()), static_cast<float*>(out.GetData()), T, cache,
           layer, pos0, n_heads, n_kv_heads, head_dim, device_id, caller);
    return out;
}

}  // namespace yan_lamma
