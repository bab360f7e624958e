// cuda_kvcache.cc -- the device KV cache (include/cuda_kvcache.h) over the C
// ABI of libminilamma_hip.so.  No HIP header is included here.
//
// Keys and values are two buffers of [n_layers, max_seq_len, n_kv_heads,
// head_dim] floats.  Every accessor names a slot (layer, pos) or one head of
// it, so one routine here checks and locates all of them: the cache is
// initialized, then layer, pos and head are in range.  Writes check the
// rows' shape and element count (and device) first.  The checks and their
// phrases are the reference's (src/cuda_kvcache.cc:16-335), which its tests
// match on; the structure is this library's.  Clear zeroes the buffers on
// the device (no host transfers) and WriteDevice is one kernel launch.
#include "include/cuda_kvcache.h"
#include "include/minilamma_hip.h"

#include "host_checks.h"

#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace yan_lamma {

bool CudaCacheBuild() { return CudaRuntimeBuilt(); }

namespace {
using hostcheck::InRange;
using hostcheck::Raise;
using hostcheck::ShapeText;

void Launched(mlk_status st, const std::string& caller) {
    if (st != MLK_OK) Raise(caller, mlk_last_error());
}

// Byte offset of slot (layer, pos), or of KV head *head in it, after the
// checks every slot access shares.
size_t Locate(const CudaCache& c, const std::string& caller, int layer, int pos,
              const int* head = nullptr) {
    if (c.Bytes_() == 0) Raise(caller, "key and value cache buffers must both be initialized");
    InRange(layer, c.n_layers(), caller + " layer", "index");
    InRange(pos, c.max_seq_len(), caller + " pos", "index");
    size_t row = static_cast<size_t>(layer) * c.max_seq_len() + static_cast<size_t>(pos);
    row *= static_cast<size_t>(c.n_kv_heads());
    if (head != nullptr) {
        InRange(*head, c.n_kv_heads(), caller + " head", "KV head");
        row += static_cast<size_t>(*head);
    }
    return row * static_cast<size_t>(c.head_dim()) * sizeof(float);
}

// A K or V row written into a slot: shape [n_kv_heads, head_dim].
void CheckRowShape(const CudaCache& c, const std::vector<int>& shape, const std::string& caller) {
    const std::vector<int> want{c.n_kv_heads(), c.head_dim()};
    if (shape.size() != 2) {
        Raise(caller, "expected 2D KV tensor with shape " + ShapeText(want) + ", got " +
                          ShapeText(shape));
    }
    if (shape != want) Raise(caller, "expected shape " + ShapeText(want) + ", got " + ShapeText(shape));
}

void CheckRowCounts(const CudaCache& c, size_t k_count, size_t v_count, const char* caller) {
    const size_t want = static_cast<size_t>(c.n_kv_heads()) * static_cast<size_t>(c.head_dim());
    if (k_count == want && v_count == want) return;
    Raise(caller, "expected " + std::to_string(want) + " elements in each K/V tensor, got K " +
                      std::to_string(k_count) + " and V " + std::to_string(v_count));
}

float* At(const CudaDeviceBuffer& buf, size_t offset) {
    return reinterpret_cast<float*>(static_cast<char*>(const_cast<void*>(buf.GetData())) + offset);
}

// Host copy of `shape` floats at `offset` of `buf`.
Tensor Fetch(const CudaDeviceBuffer& buf, size_t offset, const std::vector<int>& shape,
             int device) {
    Tensor host(shape);
    SetCudaService(device);
    CudaMemcpy(host.data.data(), At(buf, offset), host.data.size() * sizeof(float),
               CudaMemoryKind::kDeviceHost);
    return host;
}

}  // namespace

CudaCache::CudaCache(int n_layers, int max_seq_len, int n_kv_heads, int head_dim,
                     int device_id) {
    Reset(n_layers, max_seq_len, n_kv_heads, head_dim, device_id);
}

CudaCache::~CudaCache() = default;

void CudaCache::Clear() {
    if (Bytes_() == 0) return;
    SetCudaService(device_id_);
    for (CudaDeviceBuffer* buf : {&k_, &v_}) {
        Launched(mlk_zero_async(buf->GetData(), buf->GetByteSize(), nullptr), "CudaCache::Clear");
    }
}

void CudaCache::Reset() { *this = CudaCache(); }

void CudaCache::Reset(int n_layers, int max_seq_len, int n_kv_heads, int head_dim,
                      int device_id) {
    const std::string caller = "CudaCache::Reset";
    const std::pair<const char*, int> dims[] = {{" n_layers", n_layers},
                                                {" max_seq_len", max_seq_len},
                                                {" n_kv_heads", n_kv_heads},
                                                {" head_dim", head_dim}};
    for (const auto& d : dims) {
        if (d.second <= 0) {
            Raise(caller + d.first, "value must be positive, got " + std::to_string(d.second));
        }
    }
    if (device_id < 0) {
        Raise(caller, "device_id must be non-negative, got " + std::to_string(device_id));
    }
    size_t elements = 1;
    for (const auto& d : dims) elements = hostcheck::Product(elements, size_t(d.second), caller);
    const size_t bytes = hostcheck::Product(elements, sizeof(float), caller + " bytes");
    (void)hostcheck::Product(bytes, 2, caller + " total K/V bytes");

    Reset();  // the old buffers go back before the new ones are taken
    CudaCache fresh;
    fresh.k_.Reset(bytes, device_id);
    fresh.v_.Reset(bytes, device_id);
    fresh.n_layers_ = n_layers;
    fresh.max_seq_len_ = max_seq_len;
    fresh.n_kv_heads_ = n_kv_heads;
    fresh.head_dim_ = head_dim;
    fresh.device_id_ = device_id;
    fresh.Clear();
    *this = std::move(fresh);
}

size_t CudaCache::SlotOffsetBytes(int layer, int pos) const {
    return Locate(*this, "CudaCache::SlotOffsetBytes", layer, pos);
}

size_t CudaCache::SlotOffsetBytes(int layer, int pos, int head) const {
    return Locate(*this, "CudaCache::SlotOffsetBytes", layer, pos, &head);
}

void CudaCache::WriteHost(int layer, int pos, const Tensor& k, const Tensor& v) const {
    const std::string caller = "CudaCache::WriteHost";
    const size_t offset = Locate(*this, caller, layer, pos);
    CheckRowShape(*this, k.shape, caller + " k");
    CheckRowShape(*this, v.shape, caller + " v");
    CheckRowCounts(*this, k.GetDataSize(), v.GetDataSize(), caller.c_str());
    SetCudaService(device_id_);
    const size_t bytes = k.GetDataSize() * sizeof(float);
    CudaMemcpy(At(k_, offset), k.data.data(), bytes, CudaMemoryKind::kHostDevice);
    CudaMemcpy(At(v_, offset), v.data.data(), bytes, CudaMemoryKind::kHostDevice);
}

void CudaCache::WriteDevice(int layer, int pos, const CudaTensor& k, const CudaTensor& v) const {
    const std::string caller = "CudaCache::WriteDevice";
    (void)Locate(*this, caller, layer, pos);
    CheckRowShape(*this, k.shape(), caller + " k");
    CheckRowShape(*this, v.shape(), caller + " v");
    if (k.DeviceId() != device_id_ || v.DeviceId() != device_id_) {
        Raise(caller, "K and V must be on cache device " + std::to_string(device_id_) +
                          ", got K device " + std::to_string(k.DeviceId()) + " and V device " +
                          std::to_string(v.DeviceId()));
    }
    CheckRowCounts(*this, k.NumEle(), v.NumEle(), caller.c_str());
    const int64_t row = static_cast<int64_t>(k.NumEle());
    SetCudaService(device_id_);
    Launched(mlk_kv_write_f32(At(k_, 0), At(v_, 0), n_layers_, max_seq_len_, n_kv_heads_,
                              head_dim_, layer, static_cast<const float*>(k.GetData()), row,
                              static_cast<const float*>(v.GetData()), row, nullptr, pos, 1,
                              nullptr, nullptr),
             caller);
}

Tensor CudaCache::ReadKey(int layer, int pos) const {
    return Fetch(k_, Locate(*this, "CudaCache::ReadKey", layer, pos), {n_kv_heads_, head_dim_},
                 device_id_);
}

Tensor CudaCache::ReadVal(int layer, int pos) const {
    return Fetch(v_, Locate(*this, "CudaCache::ReadVal", layer, pos), {n_kv_heads_, head_dim_},
                 device_id_);
}

Tensor CudaCache::ReadHeadKey(int layer, int pos, int head) const {
    return Fetch(k_, Locate(*this, "CudaCache::ReadHeadKey", layer, pos, &head), {head_dim_},
                 device_id_);
}

Tensor CudaCache::ReadHeadVal(int layer, int pos, int head) const {
    return Fetch(v_, Locate(*this, "CudaCache::ReadHeadVal", layer, pos, &head), {head_dim_},
                 device_id_);
}

const void* CudaCache::KData() const {
    if (k_.IsEmpty()) Raise("CudaCache::KData", "key cache is empty");
    return k_.GetData();
}

const void* CudaCache::vData() const {
    if (v_.IsEmpty()) Raise("CudaCache::vData", "value cache is empty");
    return v_.GetData();
}

size_t CudaCache::Bytes_() const { return k_.GetByteSize() + v_.GetByteSize(); }

void CudaKvWriteBatchDevice(const CudaCache& cache, int layer, int pos0, const CudaTensor& k,
                            const CudaTensor& v) {
    const std::string caller = "CudaKvWriteBatchDevice";
    float* kc = static_cast<float*>(const_cast<void*>(cache.KData()));
    float* vc = static_cast<float*>(const_cast<void*>(cache.vData()));
    InRange(layer, cache.n_layers(), caller + " layer", "index");
    const size_t row = static_cast<size_t>(cache.n_kv_heads()) * cache.head_dim();
    if (k.IsEmpty() || v.IsEmpty() || k.shape() != v.shape() || k.shape().empty()) {
        Raise(caller, "k and v must be non-empty tensors of the same shape");
    }
    const int T = k.shape()[0];
    if (k.NumEle() != static_cast<size_t>(T) * row) {
        Raise(caller, "expected k, v of shape [T, " + std::to_string(cache.n_kv_heads()) + ", " +
                          std::to_string(cache.head_dim()) + "], got " + ShapeText(k.shape()));
    }
    if (pos0 < 0 || static_cast<int64_t>(pos0) + T > cache.max_seq_len()) {
        Raise(caller, "positions " + std::to_string(pos0) + ".." +
                          std::to_string(static_cast<int64_t>(pos0) + T - 1) + " out of range [0, " +
                          std::to_string(cache.max_seq_len()) + ")");
    }
    if (k.DeviceId() != cache.device_id() || v.DeviceId() != cache.device_id()) {
        Raise(caller, "k and v must be on the cache's device " + std::to_string(cache.device_id()));
    }
    SetCudaService(cache.device_id());
    Launched(mlk_kv_write_f32(kc, vc, cache.n_layers(), cache.max_seq_len(), cache.n_kv_heads(),
                              cache.head_dim(), layer, static_cast<const float*>(k.GetData()),
                              static_cast<int64_t>(row), static_cast<const float*>(v.GetData()),
                              static_cast<int64_t>(row), nullptr, pos0, T, nullptr, nullptr),
             caller);
}

}  // namespace yan_lamma
