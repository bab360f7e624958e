// cuda_kvcache.cc -- the device KV cache (include/cuda_kvcache.h) over the C
// ABI of libminilamma_hip.so.  No HIP header is included here.
//
// Checks and messages follow the reference (src/cuda_kvcache.cc:16-335 of
// the reference tree): positive dimensions, size overflow, layer / pos /
// head ranges, the [n_kv_heads, head_dim] shape of written rows and the
// device match, all before any copy or launch.
#include "include/cuda_kvcache.h"
#include "include/minilamma_hip.h"

#include <limits>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace yan_lamma {

bool CudaCacheBuild() { return CudaRuntimeBuilt(); }

namespace {

[[noreturn]] void Throw(const std::string& msg) { throw std::runtime_error(msg); }

void RequireCacheBuffers(const CudaDeviceBuffer& k, const CudaDeviceBuffer& v,
                         const char* caller) {
    if (k.IsEmpty() || v.IsEmpty()) {
        Throw(std::string(caller) + ": key and value cache buffers must both be initialized");
    }
}

void RequirePositive(int value, const char* caller) {
    if (value <= 0) {
        Throw(std::string(caller) + ": value must be positive, got " + std::to_string(value));
    }
}

void CheckMul(size_t a, size_t b, const char* caller) {
    if (a == 0 || b == 0) {
        Throw(std::string(caller) + ": multiplication dimensions must be positive, got " +
              std::to_string(a) + " and " + std::to_string(b));
    }
    if (b > std::numeric_limits<size_t>::max() / a) {
        Throw(std::string(caller) + ": size multiplication overflow for " + std::to_string(a) +
              " * " + std::to_string(b));
    }
}

void CheckIndex(int index, int limit, const char* caller) {
    if (index < 0 || index >= limit) {
        Throw(std::string(caller) + ": index " + std::to_string(index) + " out of range [0, " +
              std::to_string(limit) + ")");
    }
}

void CheckHead(int head, int n_kv_heads, const char* caller) {
    if (head < 0 || head >= n_kv_heads) {
        Throw(std::string(caller) + ": KV head " + std::to_string(head) + " out of range [0, " +
              std::to_string(n_kv_heads) + ")");
    }
}

std::string ShapeToString(const std::vector<int>& shape) {
    std::string s = "[";
    for (size_t i = 0; i < shape.size(); ++i) s += (i ? ", " : "") + std::to_string(shape[i]);
    return s + "]";
}

void CheckKVShape(const std::vector<int>& shape, int n_kv_heads, int head_dim,
                  const char* caller) {
    RequirePositive(n_kv_heads, caller);
    RequirePositive(head_dim, caller);
    const std::string expected = ShapeToString({n_kv_heads, head_dim});
    if (shape.size() != 2) {
        Throw(std::string(caller) + ": expected 2D KV tensor with shape " + expected + ", got " +
              ShapeToString(shape));
    }
    if (shape[0] != n_kv_heads || shape[1] != head_dim) {
        Throw(std::string(caller) + ": expected shape " + expected + ", got " +
              ShapeToString(shape));
    }
}

void Launched(mlk_status st, const std::string& caller) {
    if (st != MLK_OK) Throw(caller + ": " + mlk_last_error());
}

}  // namespace

CudaCache::CudaCache(int n_layers, int max_seq_len, int n_kv_heads, int head_dim,
                     int device_id) {
    Reset(n_layers, max_seq_len, n_kv_heads, head_dim, device_id);
}

CudaCache::~CudaCache() = default;

void CudaCache::Clear() {
    if (k_.IsEmpty() || v_.IsEmpty()) return;
    SetCudaService(device_id_);
    Launched(mlk_zero_async(k_.GetData(), k_.GetByteSize(), nullptr), "CudaCache::Clear");
    Launched(mlk_zero_async(v_.GetData(), v_.GetByteSize(), nullptr), "CudaCache::Clear");
}

void CudaCache::Reset() {
    k_.ReSet();
    v_.ReSet();
    n_layers_ = 0;
    max_seq_len_ = 0;
    n_kv_heads_ = 0;
    head_dim_ = 0;
    device_id_ = 0;
}

void CudaCache::Reset(int n_layers, int max_seq_len, int n_kv_heads, int head_dim,
                      int device_id) {
    RequirePositive(n_layers, "CudaCache::Reset n_layers");
    RequirePositive(max_seq_len, "CudaCache::Reset max_seq_len");
    RequirePositive(n_kv_heads, "CudaCache::Reset n_kv_heads");
    RequirePositive(head_dim, "CudaCache::Reset head_dim");
    if (device_id < 0) {
        Throw("CudaCache::Reset: device_id must be non-negative, got " +
              std::to_string(device_id));
    }
    size_t bytes = static_cast<size_t>(n_layers);
    for (const int dimension : {max_seq_len, n_kv_heads, head_dim}) {
        CheckMul(bytes, static_cast<size_t>(dimension), "CudaCache::Reset");
        bytes *= static_cast<size_t>(dimension);
    }
    CheckMul(bytes, sizeof(float), "CudaCache::Reset bytes");
    bytes *= sizeof(float);
    CheckMul(bytes, 2, "CudaCache::Reset total K/V bytes");
    Reset();
    try {
        k_.Reset(bytes, device_id);
        v_.Reset(bytes, device_id);
        n_layers_ = n_layers;
        max_seq_len_ = max_seq_len;
        n_kv_heads_ = n_kv_heads;
        head_dim_ = head_dim;
        device_id_ = device_id;
        Clear();
    } catch (...) {
        try {
            Reset();
        } catch (...) {
            // keep the original allocation / clear error
        }
        throw;
    }
}

size_t CudaCache::SlotOffsetBytes(int layer, int pos) const {
    RequireCacheBuffers(k_, v_, "CudaCache::SlotOffsetBytes");
    CheckIndex(layer, n_layers_, "CudaCache::SlotOffsetBytes layer");
    CheckIndex(pos, max_seq_len_, "CudaCache::SlotOffsetBytes pos");
    return ((static_cast<size_t>(layer) * max_seq_len_ + pos) * n_kv_heads_ * head_dim_) *
           sizeof(float);
}

size_t CudaCache::SlotOffsetBytes(int layer, int pos, int head) const {
    const size_t slot = SlotOffsetBytes(layer, pos);
    CheckHead(head, n_kv_heads_, "CudaCache::SlotOffsetBytes head");
    return slot + static_cast<size_t>(head) * head_dim_ * sizeof(float);
}

void CudaCache::WriteHost(int layer, int pos, const Tensor& k, const Tensor& v) const {
    RequireCacheBuffers(k_, v_, "CudaCache::WriteHost");
    CheckIndex(layer, n_layers_, "CudaCache::WriteHost layer");
    CheckIndex(pos, max_seq_len_, "CudaCache::WriteHost pos");
    CheckKVShape(k.shape, n_kv_heads_, head_dim_, "CudaCache::WriteHost k");
    CheckKVShape(v.shape, n_kv_heads_, head_dim_, "CudaCache::WriteHost v");
    const size_t expected = static_cast<size_t>(n_kv_heads_) * head_dim_;
    if (expected != k.GetDataSize() || expected != v.GetDataSize()) {
        Throw("CudaCache::WriteHost: expected " + std::to_string(expected) +
              " elements in each K/V tensor, got K " + std::to_string(k.GetDataSize()) +
              " and V " + std::to_string(v.GetDataSize()));
    }
    const size_t bytes = expected * sizeof(float);
    const size_t offset = SlotOffsetBytes(layer, pos);
    SetCudaService(device_id_);
    CudaMemcpy(static_cast<char*>(const_cast<void*>(k_.GetData())) + offset, k.data.data(), bytes,
               CudaMemoryKind::kHostDevice);
    CudaMemcpy(static_cast<char*>(const_cast<void*>(v_.GetData())) + offset, v.data.data(), bytes,
               CudaMemoryKind::kHostDevice);
}

void CudaCache::WriteDevice(int layer, int pos, const CudaTensor& k, const CudaTensor& v) const {
    RequireCacheBuffers(k_, v_, "CudaCache::WriteDevice");
    CheckIndex(layer, n_layers_, "CudaCache::WriteDevice layer");
    CheckIndex(pos, max_seq_len_, "CudaCache::WriteDevice pos");
    CheckKVShape(k.shape(), n_kv_heads_, head_dim_, "CudaCache::WriteDevice k");
    CheckKVShape(v.shape(), n_kv_heads_, head_dim_, "CudaCache::WriteDevice v");
    if (k.DeviceId() != device_id_ || v.DeviceId() != device_id_) {
        Throw("CudaCache::WriteDevice: K and V must be on cache device " +
              std::to_string(device_id_) + ", got K device " + std::to_string(k.DeviceId()) +
              " and V device " + std::to_string(v.DeviceId()));
    }
    const size_t expected = static_cast<size_t>(n_kv_heads_) * head_dim_;
    if (expected != k.NumEle() || expected != v.NumEle()) {
        Throw("CudaCache::WriteDevice: expected " + std::to_string(expected) +
              " elements in each K/V tensor, got K " + std::to_string(k.NumEle()) + " and V " +
              std::to_string(v.NumEle()));
    }
    SetCudaService(device_id_);
    const int64_t row = static_cast<int64_t>(expected);
    Launched(mlk_kv_write_f32(static_cast<float*>(const_cast<void*>(k_.GetData())),
                              static_cast<float*>(const_cast<void*>(v_.GetData())), n_layers_,
                              max_seq_len_, n_kv_heads_, head_dim_, layer,
                              static_cast<const float*>(k.GetData()), row,
                              static_cast<const float*>(v.GetData()), row, nullptr, pos, 1,
                              nullptr, nullptr),
             "CudaCache::WriteDevice");
}

namespace {

Tensor ReadSlot(const CudaDeviceBuffer& buf, size_t offset, std::vector<int> shape, int device) {
    Tensor out(shape);
    SetCudaService(device);
    CudaMemcpy(out.data.data(), static_cast<const char*>(buf.GetData()) + offset,
               out.GetDataSize() * sizeof(float), CudaMemoryKind::kDeviceHost);
    return out;
}

}  // namespace

Tensor CudaCache::ReadKey(int layer, int pos) const {
    RequireCacheBuffers(k_, v_, "CudaCache::ReadKey");
    CheckIndex(layer, n_layers_, "CudaCache::ReadKey layer");
    CheckIndex(pos, max_seq_len_, "CudaCache::ReadKey pos");
    return ReadSlot(k_, SlotOffsetBytes(layer, pos), {n_kv_heads_, head_dim_}, device_id_);
}

Tensor CudaCache::ReadVal(int layer, int pos) const {
    RequireCacheBuffers(k_, v_, "CudaCache::ReadVal");
    CheckIndex(layer, n_layers_, "CudaCache::ReadVal layer");
    CheckIndex(pos, max_seq_len_, "CudaCache::ReadVal pos");
    return ReadSlot(v_, SlotOffsetBytes(layer, pos), {n_kv_heads_, head_dim_}, device_id_);
}

Tensor CudaCache::ReadHeadKey(int layer, int pos, int head) const {
    RequireCacheBuffers(k_, v_, "CudaCache::ReadHeadKey");
    CheckHead(head, n_kv_heads_, "CudaCache::ReadHeadKey head");
    CheckIndex(layer, n_layers_, "CudaCache::ReadHeadKey layer");
    CheckIndex(pos, max_seq_len_, "CudaCache::ReadHeadKey pos");
    return ReadSlot(k_, SlotOffsetBytes(layer, pos, head), {head_dim_}, device_id_);
}

Tensor CudaCache::ReadHeadVal(int layer, int pos, int head) const {
    RequireCacheBuffers(k_, v_, "CudaCache::ReadHeadVal");
    CheckHead(head, n_kv_heads_, "CudaCache::ReadHeadVal head");
    CheckIndex(layer, n_layers_, "CudaCache::ReadHeadVal layer");
    CheckIndex(pos, max_seq_len_, "CudaCache::ReadHeadVal pos");
    return ReadSlot(v_, SlotOffsetBytes(layer, pos, head), {head_dim_}, device_id_);
}

const void* CudaCache::KData() const {
    if (k_.IsEmpty()) Throw("CudaCache::KData: key cache is empty");
    return k_.GetData();
}

const void* CudaCache::vData() const {
    if (v_.IsEmpty()) Throw("CudaCache::vData: value cache is empty");
    return v_.GetData();
}

size_t CudaCache::Bytes_() const { return k_.GetByteSize() + v_.GetByteSize(); }

void CudaKvWriteBatchDevice(const CudaCache& cache, int layer, int pos0, const CudaTensor& k,
                            const CudaTensor& v) {
    const char* caller = "CudaKvWriteBatchDevice";
    const void* kc = cache.KData();
    const void* vc = cache.vData();
    CheckIndex(layer, cache.n_layers(), "CudaKvWriteBatchDevice layer");
    const size_t row = static_cast<size_t>(cache.n_kv_heads()) * cache.head_dim();
    if (k.IsEmpty() || v.IsEmpty() || k.shape() != v.shape() || k.shape().empty()) {
        Throw(std::string(caller) + ": k and v must be non-empty tensors of the same shape");
    }
    const int T = k.shape()[0];
    if (k.NumEle() != static_cast<size_t>(T) * row) {
        Throw(std::string(caller) + ": expected k, v of shape [T, " +
              std::to_string(cache.n_kv_heads()) + ", " + std::to_string(cache.head_dim()) +
              "], got " + ShapeToString(k.shape()));
    }
    if (pos0 < 0 || static_cast<int64_t>(pos0) + T > cache.max_seq_len()) {
        Throw(std::string(caller) + ": positions " + std::to_string(pos0) + ".." +
              std::to_string(static_cast<int64_t>(pos0) + T - 1) + " out of range [0, " +
              std::to_string(cache.max_seq_len()) + ")");
    }
    if (k.DeviceId() != cache.device_id() || v.DeviceId() != cache.device_id()) {
        Throw(std::string(caller) + ": k and v must be on the cache's device " +
              std::to_string(cache.device_id()));
    }
    SetCudaService(cache.device_id());
    Launched(mlk_kv_write_f32(static_cast<float*>(const_cast<void*>(kc)),
                              static_cast<float*>(const_cast<void*>(vc)), cache.n_layers(),
                              cache.max_seq_len(), cache.n_kv_heads(), cache.head_dim(), layer,
                              static_cast<const float*>(k.GetData()),
                              static_cast<int64_t>(row), static_cast<const float*>(v.GetData()),
                              static_cast<int64_t>(row), nullptr, pos0, T, nullptr, nullptr),
             caller);
}

}  // namespace yan_lamma
