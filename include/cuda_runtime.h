// cuda_runtime.h -- device runtime of the op surface, on MI355X.
//
// Same declarations as the reference's device runtime
// (include/cuda_runtime.h:8-74 of the reference tree): device query and
// selection, raw allocation, counted copies, allocation-peak scopes and the
// move-only CudaDeviceBuffer (member layout unchanged).  The names keep the
// reference's "Cuda" prefix because forward.cc calls them by these names;
// the implementation (cpp-minilamma_amd/host/cuda_runtime.cc) runs on HIP
// through the C ABI in minilamma_hip.h.
//
// Differences a caller can see:
//   - CudaMemory / CudaFreeMemory go through a per-device caching allocator,
//     so releasing and re-creating an op result costs no hipMalloc/hipFree
//     (stream-ordered reuse: every op of this surface runs on the null
//     stream);  CudaEmptyCache() returns cached blocks to the driver;
//   - host <-> device copies are counted into the thread's active
//     CudaTransferStats (CudaStatsScope), the counters the reference keeps
//     in its model statistics.
#pragma once
#include <cstddef>
#include <memory>
#include <string>

namespace yan_lamma {
// True: this library is always built with the GPU backend.
bool CudaRuntimeBuilt();
struct CudaInfo {
    int device_id = 0;
    std::string name;
    int compute_major = 0;
    int compute_minor = 0;
    size_t total_bytes = 0;
    int runtime_version = 0;
    int driver_version = 0;
};
enum class CudaMemoryKind {
    kHostDevice,
    kDeviceDevice,
    kDeviceHost
};
CudaInfo GetCudaInfo(int device_id);
std::string CudaInfo(const struct CudaInfo& info);
int DeviceCount();
void SetCudaService(int device_id);
// Device allocation of byte_size bytes on the current device (nullptr for 0).
void* CudaMemory(size_t byte_size);
void CudaFreeMemory(void* ptr);
// Synchronous copy; H2D and D2H copies are counted (see CudaStatsScope).
void CudaMemcpy(void* des, const void* src, size_t bytes, CudaMemoryKind kind);

struct CudaAllocationStats {
    size_t current_bytes = 0;
    size_t peak_bytes = 0;
};
// Buffers created while a scope is active charge their bytes to its stats
// until they are released (the stats travel with moved buffers).
class CudaAllocationScope {
 public:
    explicit CudaAllocationScope(std::shared_ptr<CudaAllocationStats> stats);
    ~CudaAllocationScope();
    CudaAllocationScope(const CudaAllocationScope&) = delete;
    CudaAllocationScope& operator=(const CudaAllocationScope&) = delete;

 private:
    std::shared_ptr<CudaAllocationStats> previous_;
};

class CudaDeviceBuffer {
 public:
    CudaDeviceBuffer() = default;
    explicit CudaDeviceBuffer(size_t byte_size, int device_id = 0);
    void ReSet();
    void Reset(size_t byte_size, int device_id);
    ~CudaDeviceBuffer();
    CudaDeviceBuffer(const CudaDeviceBuffer&) = delete;
    CudaDeviceBuffer operator=(const CudaDeviceBuffer&) = delete;
    CudaDeviceBuffer(CudaDeviceBuffer&& other) noexcept;
    CudaDeviceBuffer& operator=(CudaDeviceBuffer&& other) noexcept;
    void upload(const void* src, size_t byte_size);
    void download(void* des, size_t byte_size) const;
    bool IsEmpty() const { return data_ == nullptr; }
    int GetDeviceId() const { return device_id_; }
    void* GetData() { return data_; }
    const void* GetData() const { return data_; }
    size_t GetByteSize() const { return byte_size_; }

 private:
    void ReleaseDevice() noexcept;

 private:
    void* data_ = nullptr;
    size_t byte_size_ = 0;
    int device_id_ = 0;
    std::shared_ptr<CudaAllocationStats> allocation_stats_;
};

// ---- additions (no reference counterpart) --------------------------------

// Host <-> device transfer counters, the four the reference keeps in its
// model statistics (host_to_device_copies ... device_to_host_bytes).
struct CudaTransferStats {
    size_t host_to_device_copies = 0;
    size_t device_to_host_copies = 0;
    size_t host_to_device_bytes = 0;
    size_t device_to_host_bytes = 0;
};
// Thread-local attribution of CudaMemcpy counts, nestable.
class CudaStatsScope {
 public:
    explicit CudaStatsScope(CudaTransferStats* stats);
    ~CudaStatsScope();
    CudaStatsScope(const CudaStatsScope&) = delete;
    CudaStatsScope& operator=(const CudaStatsScope&) = delete;

 private:
    CudaTransferStats* previous_;
};
// Returns every cached (free) block of device_id to the driver; -1 = all.
void CudaEmptyCache(int device_id = -1);
// Bytes currently held in the allocation cache (free blocks), all devices.
size_t CudaCachedBytes();
}  // namespace yan_lamma
