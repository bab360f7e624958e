// cuda_runtime.cc -- device runtime of the op surface (include/cuda_runtime.h)
// over the C ABI of libminilamma_hip.so.  No HIP header is included here.
//
// Behaviour callers rely on (the reference's src/cuda_runtime.cc): errors
// throw std::runtime_error "<what>: <message>", zero-byte allocations are
// nullptr, copies of zero bytes are no-ops, and every host <-> device copy
// is counted.  The counts go to two places: the CudaModelWeights that the
// reference's internal::CudaStatsScope (src/internal/cuda_stats.h) makes
// active through internal::active_cuda_stats, which this library defines
// in place of the reference's runtime, and this library's own
// CudaTransferStats scope.
//
// Allocation goes through a per-device caching allocator instead of one
// hipMalloc/hipFree per tensor (the reference allocates every op result
// with cudaMalloc): freed blocks are kept in size classes and handed out
// again.  Reuse is stream-ordered because every op of this surface runs on
// the null stream, and synchronous copies on it wait for earlier kernels.
#include "include/cuda_runtime.h"
#include "include/minilamma_hip.h"
#include "include/model.h"

#include <algorithm>
#include <map>
#include <mutex>
#include <sstream>
#include <stdexcept>
#include <unordered_map>
#include <utility>
#include <vector>

namespace yan_lamma {
namespace internal {
// Declared by the reference in src/internal/cuda_stats.h; its
// CudaStatsScope points this at the model whose forward pass is running.
thread_local CudaModelWeights* active_cuda_stats = nullptr;
}  // namespace internal

namespace {

thread_local std::shared_ptr<CudaAllocationStats> g_active_allocations;
thread_local CudaTransferStats* g_active_transfers = nullptr;

[[noreturn]] void Throw(const std::string& what) {
    throw std::runtime_error(what + ": " + mlk_last_error());
}

void Check(mlk_status st, const char* what) {
    if (st != MLK_OK) Throw(what);
}

// Size classes: 512-byte steps up to 1 MiB, 2 MiB steps above.
size_t SizeClass(size_t n) {
    constexpr size_t kSmall = size_t{1} << 20;
    constexpr size_t kLarge = size_t{2} << 20;
    return n <= kSmall ? (n + 511) / 512 * 512 : (n + kLarge - 1) / kLarge * kLarge;
}

class BlockCache {
 public:
    void* Take(int device, size_t bytes) {
        const size_t cls = SizeClass(bytes);
        {
            std::lock_guard<std::mutex> lock(mu_);
            auto it = free_.find({device, cls});
            if (it != free_.end() && !it->second.empty()) {
                void* p = it->second.back();
                it->second.pop_back();
                cached_ -= cls;
                live_[p] = {device, cls};
                return p;
            }
        }
        void* p = nullptr;
        if (mlk_malloc(&p, cls) != MLK_OK) {
            Release(device);  // give cached blocks back and try once more
            if (mlk_malloc(&p, cls) != MLK_OK) Throw("hipMalloc");
        }
        std::lock_guard<std::mutex> lock(mu_);
        live_[p] = {device, cls};
        return p;
    }

    void Give(void* p) {
        std::unique_lock<std::mutex> lock(mu_);
        auto it = live_.find(p);
        if (it == live_.end()) {
            lock.unlock();
            Check(mlk_free(p), "hipFree");  // not ours: plain free
            return;
        }
        free_[it->second].push_back(p);
        cached_ += it->second.second;
        live_.erase(it);
    }

    void Release(int device) {
        std::vector<std::pair<int, void*>> drop;
        {
            std::lock_guard<std::mutex> lock(mu_);
            for (auto& kv : free_) {
                if (device >= 0 && kv.first.first != device) continue;
                for (void* p : kv.second) {
                    drop.emplace_back(kv.first.first, p);
                    cached_ -= kv.first.second;
                }
                kv.second.clear();
            }
        }
        int current = 0;
        const bool restore = mlk_get_device(&current) == MLK_OK;
        for (auto& d : drop) {
            mlk_set_device(d.first);
            mlk_free(d.second);
        }
        if (restore) mlk_set_device(current);
    }

    size_t Cached() {
        std::lock_guard<std::mutex> lock(mu_);
        return cached_;
    }

 private:
    std::mutex mu_;
    std::unordered_map<void*, std::pair<int, size_t>> live_;
    std::map<std::pair<int, size_t>, std::vector<void*>> free_;
    size_t cached_ = 0;
};

// Never destroyed: blocks are returned to the driver by CudaEmptyCache or at
// process exit by the driver itself, never from a static destructor that may
// run after the HIP runtime is gone.
BlockCache& Cache() {
    static BlockCache* cache = new BlockCache;
    return *cache;
}

// One copy of `bytes` bytes added to a set of transfer counters (the same
// four fields in CudaTransferStats and in the model's CudaModelWeights);
// device-to-device copies are not transfers.
template <class Counters>
void Count(Counters* counters, CudaMemoryKind kind, size_t bytes) {
    if (counters == nullptr || kind == CudaMemoryKind::kDeviceDevice) return;
    const bool to_device = kind == CudaMemoryKind::kHostDevice;
    (to_device ? counters->host_to_device_copies : counters->device_to_host_copies) += 1;
    (to_device ? counters->host_to_device_bytes : counters->device_to_host_bytes) += bytes;
}

int32_t ToKind(CudaMemoryKind kind) {
    switch (kind) {
        case CudaMemoryKind::kHostDevice: return MLK_H2D;
        case CudaMemoryKind::kDeviceDevice: return MLK_D2D;
        case CudaMemoryKind::kDeviceHost: return MLK_D2H;
    }
    throw std::runtime_error("Invalid memory copy kind");
}

}  // namespace

// Scopes install their target for the thread and put the outer one back.
CudaAllocationScope::CudaAllocationScope(std::shared_ptr<CudaAllocationStats> stats)
    : previous_(std::exchange(g_active_allocations, std::move(stats))) {}

CudaAllocationScope::~CudaAllocationScope() { g_active_allocations.swap(previous_); }

CudaStatsScope::CudaStatsScope(CudaTransferStats* stats)
    : previous_(std::exchange(g_active_transfers, stats)) {}

CudaStatsScope::~CudaStatsScope() { g_active_transfers = previous_; }

bool CudaRuntimeBuilt() { return true; }

int DeviceCount() {
    int n = 0;
    Check(mlk_device_count(&n), "hipGetDeviceCount");
    return n;
}

void SetCudaService(int device_id) { Check(mlk_set_device(device_id), "cudaSetDevice"); }

struct CudaInfo GetCudaInfo(int device_id) {
    mlk_device_info raw{};
    Check(mlk_get_device_info(device_id, &raw), "GetCudaInfo");
    struct CudaInfo info;
    info.device_id = raw.device_id;
    info.name = raw.name[0] != '\0' ? raw.name : raw.arch;
    info.compute_major = raw.compute_major;
    info.compute_minor = raw.compute_minor;
    info.total_bytes = raw.total_bytes;
    info.runtime_version = raw.runtime_version;
    info.driver_version = raw.driver_version;
    return info;
}

std::string CudaInfo(const struct CudaInfo& info) {
    const std::pair<const char*, std::string> fields[] = {
        {"device_id", std::to_string(info.device_id)},
        {"name", '"' + info.name + '"'},
        {"compute", std::to_string(info.compute_major) + "." + std::to_string(info.compute_minor)},
        {"total_bytes", std::to_string(info.total_bytes)},
        {"runtime_version", std::to_string(info.runtime_version)},
        {"driver_version", std::to_string(info.driver_version)},
    };
    std::string line = "[HIP]";
    for (const auto& field : fields) line += std::string(" ") + field.first + "=" + field.second;
    return line;
}

void* CudaMemory(size_t byte_size) {
    if (byte_size == 0) return nullptr;
    int device = 0;
    Check(mlk_get_device(&device), "hipGetDevice");
    return Cache().Take(device, byte_size);
}

void CudaFreeMemory(void* ptr) {
    if (ptr == nullptr) return;
    Cache().Give(ptr);
}

void CudaEmptyCache(int device_id) { Cache().Release(device_id); }

size_t CudaCachedBytes() { return Cache().Cached(); }

void CudaMemcpy(void* des, const void* src, size_t bytes, CudaMemoryKind kind) {
    if (bytes == 0) return;
    if (des == nullptr || src == nullptr) {
        throw std::runtime_error("cudaMemcpy requires non-null src and dst for non-empty copies");
    }
    Check(mlk_memcpy(des, src, bytes, ToKind(kind)), "hipMemcpy");
    Count(internal::active_cuda_stats, kind, bytes);
    Count(g_active_transfers, kind, bytes);
}

// ---------------------------------------------------------- device buffer
//
// A buffer is empty or owns one block of the cache above.  Its fields
// change in three ways only: Reset claims a block (and charges the active
// allocation scope), ReSet returns it (and refunds the scope that was
// charged), and a move exchanges two buffers' states.  ReSet clears the
// fields before handing the block back, so a failure there never leaves a
// buffer pointing at memory it no longer owns.

namespace {

void Charge(CudaAllocationStats* scope, size_t bytes) {
    if (scope == nullptr) return;
    scope->current_bytes += bytes;
    scope->peak_bytes = std::max(scope->peak_bytes, scope->current_bytes);
}

void Refund(CudaAllocationStats* scope, size_t bytes) {
    if (scope != nullptr) scope->current_bytes -= bytes;
}

// The checks of a host transfer of `bytes` bytes with a buffer of
// `capacity` bytes (the reference's texts, which its tests match on).
void CheckHostTransfer(const char* verb, size_t bytes, size_t capacity, const void* host,
                       const void* device) {
    if (bytes > capacity) {
        throw std::runtime_error(std::string("CUDA ") + verb + " exceeds device buffer size");
    }
    if (host == nullptr || device == nullptr) {
        throw std::runtime_error(std::string("CUDA ") + verb +
                                 " requires non-null host and device pointers");
    }
}

}  // namespace

CudaDeviceBuffer::CudaDeviceBuffer(size_t byte_size, int device_id) { Reset(byte_size, device_id); }

CudaDeviceBuffer::CudaDeviceBuffer(CudaDeviceBuffer&& other) noexcept {
    // *this starts empty, so the exchange leaves `other` empty.
    std::swap(data_, other.data_);
    std::swap(byte_size_, other.byte_size_);
    std::swap(device_id_, other.device_id_);
    allocation_stats_.swap(other.allocation_stats_);
}

CudaDeviceBuffer& CudaDeviceBuffer::operator=(CudaDeviceBuffer&& other) noexcept {
    if (this != &other) {
        CudaDeviceBuffer previous(std::move(*this));  // returned when it goes out of scope
        std::swap(data_, other.data_);
        std::swap(byte_size_, other.byte_size_);
        std::swap(device_id_, other.device_id_);
        allocation_stats_.swap(other.allocation_stats_);
    }
    return *this;
}

void CudaDeviceBuffer::ReSet() {
    void* block = std::exchange(data_, nullptr);
    const size_t held = std::exchange(byte_size_, 0);
    const std::shared_ptr<CudaAllocationStats> scope = std::move(allocation_stats_);
    allocation_stats_.reset();
    device_id_ = 0;
    if (block == nullptr) return;
    Refund(scope.get(), held);
    Cache().Give(block);  // the cache knows the block's device
}

void CudaDeviceBuffer::Reset(size_t byte_size, int device_id) {
    ReSet();
    if (byte_size > 0) {
        SetCudaService(device_id);
        data_ = Cache().Take(device_id, byte_size);
        byte_size_ = byte_size;
        allocation_stats_ = g_active_allocations;
        Charge(allocation_stats_.get(), byte_size);
    }
    device_id_ = device_id;  // an empty buffer still records its device
}

void CudaDeviceBuffer::upload(const void* src, size_t byte_size) {
    if (byte_size == 0) return;
    CheckHostTransfer("upload", byte_size, byte_size_, src, data_);
    SetCudaService(device_id_);
    CudaMemcpy(data_, src, byte_size, CudaMemoryKind::kHostDevice);
}

void CudaDeviceBuffer::download(void* des, size_t byte_size) const {
    if (byte_size == 0) return;
    CheckHostTransfer("download", byte_size, byte_size_, des, data_);
    SetCudaService(device_id_);
    CudaMemcpy(des, data_, byte_size, CudaMemoryKind::kDeviceHost);
}

void CudaDeviceBuffer::ReleaseDevice() noexcept {
    try {
        ReSet();
    } catch (...) {
        // ReSet cleared the fields before it failed; nothing is left to undo
    }
}

CudaDeviceBuffer::~CudaDeviceBuffer() { ReleaseDevice(); }
}  // namespace yan_lamma
