// cuda_runtime.cc -- device runtime of the op surface (include/cuda_runtime.h)
// over the C ABI of libminilamma_hip.so.  No HIP header is included here.
//
// Semantics follow the reference runtime (src/cuda_runtime.cc of the
// reference tree): errors throw std::runtime_error "<what>: <message>",
// zero-byte allocations are nullptr, copies of zero bytes are no-ops, and
// host <-> device copies are counted for the thread's active stats.
//
// Allocation goes through a per-device caching allocator instead of one
// hipMalloc/hipFree per tensor (the reference allocates every op result
// with cudaMalloc): freed blocks are kept in size classes and handed out
// again.  Reuse is stream-ordered because every op of this surface runs on
// the null stream, and synchronous copies on it wait for earlier kernels.
#include "include/cuda_runtime.h"
#include "include/minilamma_hip.h"

#include <algorithm>
#include <map>
#include <mutex>
#include <sstream>
#include <stdexcept>
#include <unordered_map>
#include <utility>
#include <vector>

namespace yan_lamma {
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

int32_t ToKind(CudaMemoryKind kind) {
    switch (kind) {
        case CudaMemoryKind::kHostDevice: return MLK_H2D;
        case CudaMemoryKind::kDeviceDevice: return MLK_D2D;
        case CudaMemoryKind::kDeviceHost: return MLK_D2H;
    }
    throw std::runtime_error("Invalid memory copy kind");
}

}  // namespace

CudaAllocationScope::CudaAllocationScope(std::shared_ptr<CudaAllocationStats> stats)
    : previous_(std::move(g_active_allocations)) {
    g_active_allocations = std::move(stats);
}

CudaAllocationScope::~CudaAllocationScope() { g_active_allocations = std::move(previous_); }

CudaStatsScope::CudaStatsScope(CudaTransferStats* stats) : previous_(g_active_transfers) {
    g_active_transfers = stats;
}

CudaStatsScope::~CudaStatsScope() { g_active_transfers = previous_; }

bool CudaRuntimeBuilt() { return true; }

int DeviceCount() {
    int n = 0;
    Check(mlk_device_count(&n), "hipGetDeviceCount");
    return n;
}

void SetCudaService(int device_id) { Check(mlk_set_device(device_id), "hipSetDevice"); }

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
    std::ostringstream out;
    out << "[HIP] device_id=" << info.device_id << " name=\"" << info.name << "\""
        << " compute=" << info.compute_major << '.' << info.compute_minor
        << " total_bytes=" << info.total_bytes << " runtime_version=" << info.runtime_version
        << " driver_version=" << info.driver_version;
    return out.str();
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
    if (CudaTransferStats* s = g_active_transfers) {
        if (kind == CudaMemoryKind::kHostDevice) {
            ++s->host_to_device_copies;
            s->host_to_device_bytes += bytes;
        } else if (kind == CudaMemoryKind::kDeviceHost) {
            ++s->device_to_host_copies;
            s->device_to_host_bytes += bytes;
        }
    }
}

// ---------------------------------------------------------- device buffer

CudaDeviceBuffer::CudaDeviceBuffer(CudaDeviceBuffer&& other) noexcept
    : data_(std::exchange(other.data_, nullptr)),
      byte_size_(std::exchange(other.byte_size_, 0)),
      device_id_(std::exchange(other.device_id_, 0)),
      allocation_stats_(std::move(other.allocation_stats_)) {}

CudaDeviceBuffer& CudaDeviceBuffer::operator=(CudaDeviceBuffer&& other) noexcept {
    if (this != &other) {
        ReleaseDevice();
        data_ = std::exchange(other.data_, nullptr);
        byte_size_ = std::exchange(other.byte_size_, 0);
        device_id_ = std::exchange(other.device_id_, 0);
        allocation_stats_ = std::move(other.allocation_stats_);
    }
    return *this;
}

void CudaDeviceBuffer::ReSet() {
    if (data_ != nullptr) {
        SetCudaService(device_id_);
        CudaFreeMemory(data_);
        if (allocation_stats_) allocation_stats_->current_bytes -= byte_size_;
    }
    data_ = nullptr;
    byte_size_ = 0;
    device_id_ = 0;
    allocation_stats_.reset();
}

void CudaDeviceBuffer::Reset(size_t byte_size, int device_id) {
    ReSet();
    if (byte_size == 0) {
        device_id_ = device_id;
        return;
    }
    SetCudaService(device_id);
    data_ = CudaMemory(byte_size);
    byte_size_ = byte_size;
    device_id_ = device_id;
    allocation_stats_ = g_active_allocations;
    if (allocation_stats_) {
        allocation_stats_->current_bytes += byte_size;
        allocation_stats_->peak_bytes =
            std::max(allocation_stats_->peak_bytes, allocation_stats_->current_bytes);
    }
}

CudaDeviceBuffer::CudaDeviceBuffer(size_t byte_size, int device_id) { Reset(byte_size, device_id); }

void CudaDeviceBuffer::upload(const void* src, size_t byte_size) {
    if (byte_size == 0) return;
    if (byte_size > byte_size_) throw std::runtime_error("CUDA upload exceeds device buffer size");
    if (src == nullptr || data_ == nullptr) {
        throw std::runtime_error("CUDA upload requires non-null host and device pointers");
    }
    SetCudaService(device_id_);
    CudaMemcpy(data_, src, byte_size, CudaMemoryKind::kHostDevice);
}

void CudaDeviceBuffer::download(void* des, size_t byte_size) const {
    if (byte_size == 0) return;
    if (byte_size > byte_size_) {
        throw std::runtime_error("CUDA download exceeds device buffer size");
    }
    if (des == nullptr || data_ == nullptr) {
        throw std::runtime_error("CUDA download requires non-null host and device pointers");
    }
    SetCudaService(device_id_);
    CudaMemcpy(des, data_, byte_size, CudaMemoryKind::kDeviceHost);
}

void CudaDeviceBuffer::ReleaseDevice() noexcept {
    try {
        ReSet();
    } catch (...) {
        // a failed release must not escape a destructor or a move
    }
    data_ = nullptr;
    byte_size_ = 0;
    device_id_ = 0;
}

CudaDeviceBuffer::~CudaDeviceBuffer() { ReleaseDevice(); }
}  // namespace yan_lamma
