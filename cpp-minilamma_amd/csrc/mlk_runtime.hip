// mlk_runtime.hip -- error reporting and the thin HIP runtime layer of the
// C ABI (device selection, memory, copies, streams, events).
//
// Replaces the cudart calls of the reference runtime (src/cuda_runtime.cc:
// 57-161): device count / selection / properties, malloc, free and memcpy.
#include "mlk_common.h"

#include <cmath>

#include <cstring>
#include <mutex>

namespace mlk {
namespace {

thread_local char g_message[512] = "no error";

}  // namespace

mlk_status Fail(mlk_status status, const char* fmt, ...) {
    va_list args;
    va_start(args, fmt);
    std::vsnprintf(g_message, sizeof(g_message), fmt, args);
    va_end(args);
    return status;
}

mlk_status FromHip(hipError_t err, const char* what) {
    if (err == hipErrorNoDevice) {
        return Fail(MLK_ERR_NO_DEVICE, "%s: %s", what, hipGetErrorString(err));
    }
    return Fail(MLK_ERR_HIP, "%s: %s", what, hipGetErrorString(err));
}

RopeFreqs MakeRopeFreqs(float theta, int head_dim) {
    RopeFreqs f{};
    const int half = head_dim / 2 < kRopePairs ? head_dim / 2 : kRopePairs;
    for (int i = 0; i < half; ++i) {
        f.inv[i] = std::pow(static_cast<double>(theta), -2.0 * i / head_dim);
    }
    return f;
}

int ComputeUnits() {
    constexpr int kMaxDevices = 64;
    static int cache[kMaxDevices] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        return 256;
    }
    if (cache[dev] == 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cus <= 0) {
            cus = 256;
        }
        cache[dev] = cus;
    }
    return cache[dev];
}

namespace {

// Zero fill: 16-byte stores over the aligned body, bytes at the edges.
__global__ __launch_bounds__(256) void ZeroKernel(unsigned char* p, size_t head, size_t body16,
                                                  size_t tail) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    const size_t tid = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    uint4* body = reinterpret_cast<uint4*>(p + head);
    for (size_t i = tid; i < body16; i += stride) {
        body[i] = make_uint4(0, 0, 0, 0);
    }
    if (tid < head) {
        p[tid] = 0;
    }
    if (tid < tail) {
        p[head + body16 * 16 + tid] = 0;
    }
}

hipMemcpyKind ToKind(int32_t kind, bool* ok) {
    *ok = true;
    switch (kind) {
        case MLK_H2D: return hipMemcpyHostToDevice;
        case MLK_D2D: return hipMemcpyDeviceToDevice;
        case MLK_D2H: return hipMemcpyDeviceToHost;
        default: *ok = false; return hipMemcpyDefault;
    }
}

}  // namespace
}  // namespace mlk

using namespace mlk;

extern "C" {

const char* mlk_last_error(void) { return g_message; }

const char* mlk_status_string(int status) {
    switch (status) {
        case MLK_OK: return "success";
        case MLK_ERR_INVALID: return "invalid argument";
        case MLK_ERR_RANGE: return "value out of range";
        case MLK_ERR_HIP: return "HIP runtime error";
        case MLK_ERR_NO_DEVICE: return "no GPU device";
        default: return "unknown status";
    }
}

int mlk_abi_version(void) { return 2; }

mlk_status mlk_device_count(int* count) {
    if (count == nullptr) return Fail(MLK_ERR_INVALID, "mlk_device_count: null output");
    *count = 0;
    const hipError_t err = hipGetDeviceCount(count);
    if (err == hipErrorNoDevice) {
        *count = 0;
        return MLK_OK;
    }
    return err == hipSuccess ? MLK_OK : FromHip(err, "hipGetDeviceCount");
}

mlk_status mlk_set_device(int device_id) {
    const hipError_t err = hipSetDevice(device_id);
    return err == hipSuccess ? MLK_OK : FromHip(err, "hipSetDevice");
}

mlk_status mlk_get_device(int* device_id) {
    if (device_id == nullptr) return Fail(MLK_ERR_INVALID, "mlk_get_device: null output");
    const hipError_t err = hipGetDevice(device_id);
    return err == hipSuccess ? MLK_OK : FromHip(err, "hipGetDevice");
}

mlk_status mlk_get_device_info(int device_id, mlk_device_info* info) {
    if (info == nullptr) return Fail(MLK_ERR_INVALID, "mlk_get_device_info: null output");
    int count = 0;
    mlk_status st = mlk_device_count(&count);
    if (st != MLK_OK) return st;
    if (device_id < 0 || device_id >= count) {
        return Fail(MLK_ERR_NO_DEVICE, "GPU device %d is not available; detected %d device(s)",
                    device_id, count);
    }
    hipDeviceProp_t prop{};
    hipError_t err = hipGetDeviceProperties(&prop, device_id);
    if (err != hipSuccess) return FromHip(err, "hipGetDeviceProperties");
    std::memset(info, 0, sizeof(*info));
    info->device_id = device_id;
    std::snprintf(info->name, sizeof(info->name), "%s", prop.name);
    std::snprintf(info->arch, sizeof(info->arch), "%s", prop.gcnArchName);
    info->compute_major = prop.major;
    info->compute_minor = prop.minor;
    info->total_bytes = prop.totalGlobalMem;
    info->multiprocessors = prop.multiProcessorCount;
    info->clock_khz = prop.clockRate;
    info->memory_clock_khz = prop.memoryClockRate;
    info->memory_bus_bits = prop.memoryBusWidth;
    err = hipRuntimeGetVersion(&info->runtime_version);
    if (err != hipSuccess) return FromHip(err, "hipRuntimeGetVersion");
    err = hipDriverGetVersion(&info->driver_version);
    if (err != hipSuccess) return FromHip(err, "hipDriverGetVersion");
    return MLK_OK;
}

mlk_status mlk_malloc(void** ptr, size_t bytes) {
    if (ptr == nullptr) return Fail(MLK_ERR_INVALID, "mlk_malloc: null output");
    *ptr = nullptr;
    if (bytes == 0) return MLK_OK;
    const hipError_t err = hipMalloc(ptr, bytes);
    return err == hipSuccess ? MLK_OK : FromHip(err, "hipMalloc");
}

mlk_status mlk_free(void* ptr) {
    if (ptr == nullptr) return MLK_OK;
    const hipError_t err = hipFree(ptr);
    return err == hipSuccess ? MLK_OK : FromHip(err, "hipFree");
}

mlk_status mlk_memcpy(void* dst, const void* src, size_t bytes, int32_t kind) {
    if (bytes == 0) return MLK_OK;
    if (dst == nullptr || src == nullptr) {
        return Fail(MLK_ERR_INVALID, "memcpy requires non-null src and dst for non-empty copies");
    }
    bool ok = false;
    const hipMemcpyKind k = ToKind(kind, &ok);
    if (!ok) return Fail(MLK_ERR_INVALID, "Invalid memory copy kind %d", kind);
    const hipError_t err = hipMemcpy(dst, src, bytes, k);
    return err == hipSuccess ? MLK_OK : FromHip(err, "hipMemcpy");
}

mlk_status mlk_memcpy_async(void* dst, const void* src, size_t bytes, int32_t kind,
                            void* stream) {
    if (bytes == 0) return MLK_OK;
    if (dst == nullptr || src == nullptr) {
        return Fail(MLK_ERR_INVALID, "memcpy requires non-null src and dst for non-empty copies");
    }
    bool ok = false;
    const hipMemcpyKind k = ToKind(kind, &ok);
    if (!ok) return Fail(MLK_ERR_INVALID, "Invalid memory copy kind %d", kind);
    const hipError_t err = hipMemcpyAsync(dst, src, bytes, k, AsStream(stream));
    return err == hipSuccess ? MLK_OK : FromHip(err, "hipMemcpyAsync");
}

mlk_status mlk_zero_async(void* dst, size_t bytes, void* stream) {
    if (bytes == 0) return MLK_OK;
    if (dst == nullptr) return Fail(MLK_ERR_INVALID, "mlk_zero_async: null pointer");
    unsigned char* p = static_cast<unsigned char*>(dst);
    const size_t mis = reinterpret_cast<uintptr_t>(p) & 15u;
    size_t head = mis == 0 ? 0 : 16 - mis;
    if (head > bytes) head = bytes;
    const size_t body16 = (bytes - head) / 16;
    const size_t tail = bytes - head - body16 * 16;
    const unsigned grid = GridFor(static_cast<int64_t>(body16 > 16 ? body16 : 16), 256, 4);
    hipLaunchKernelGGL(ZeroKernel, dim3(grid), dim3(256), 0, AsStream(stream), p, head, body16,
                       tail);
    return CheckLaunch("ZeroKernel");
}

mlk_status mlk_device_synchronize(void) {
    const hipError_t err = hipDeviceSynchronize();
    return err == hipSuccess ? MLK_OK : FromHip(err, "hipDeviceSynchronize");
}

mlk_status mlk_stream_create(void** stream) {
    if (stream == nullptr) return Fail(MLK_ERR_INVALID, "mlk_stream_create: null output");
    hipStream_t s = nullptr;
    const hipError_t err = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    *stream = s;
    return err == hipSuccess ? MLK_OK : FromHip(err, "hipStreamCreate");
}

mlk_status mlk_stream_destroy(void* stream) {
    if (stream == nullptr) return MLK_OK;
    const hipError_t err = hipStreamDestroy(AsStream(stream));
    return err == hipSuccess ? MLK_OK : FromHip(err, "hipStreamDestroy");
}

mlk_status mlk_stream_synchronize(void* stream) {
    const hipError_t err = hipStreamSynchronize(AsStream(stream));
    return err == hipSuccess ? MLK_OK : FromHip(err, "hipStreamSynchronize");
}

mlk_status mlk_event_create(void** event) {
    if (event == nullptr) return Fail(MLK_ERR_INVALID, "mlk_event_create: null output");
    hipEvent_t e = nullptr;
    const hipError_t err = hipEventCreate(&e);
    *event = e;
    return err == hipSuccess ? MLK_OK : FromHip(err, "hipEventCreate");
}

mlk_status mlk_event_destroy(void* event) {
    if (event == nullptr) return MLK_OK;
    const hipError_t err = hipEventDestroy(static_cast<hipEvent_t>(event));
    return err == hipSuccess ? MLK_OK : FromHip(err, "hipEventDestroy");
}

mlk_status mlk_event_record(void* event, void* stream) {
    if (event == nullptr) return Fail(MLK_ERR_INVALID, "mlk_event_record: null event");
    const hipError_t err = hipEventRecord(static_cast<hipEvent_t>(event), AsStream(stream));
    return err == hipSuccess ? MLK_OK : FromHip(err, "hipEventRecord");
}

mlk_status mlk_event_synchronize(void* event) {
    if (event == nullptr) return Fail(MLK_ERR_INVALID, "mlk_event_synchronize: null event");
    const hipError_t err = hipEventSynchronize(static_cast<hipEvent_t>(event));
    return err == hipSuccess ? MLK_OK : FromHip(err, "hipEventSynchronize");
}

mlk_status mlk_event_elapsed_ms(float* ms, void* start, void* stop) {
    if (ms == nullptr || start == nullptr || stop == nullptr) {
        return Fail(MLK_ERR_INVALID, "mlk_event_elapsed_ms: null argument");
    }
    const hipError_t err = hipEventElapsedTime(ms, static_cast<hipEvent_t>(start),
                                               static_cast<hipEvent_t>(stop));
    return err == hipSuccess ? MLK_OK : FromHip(err, "hipEventElapsedTime");
}

mlk_status mlk_graph_begin_capture(void* stream) {
    if (stream == nullptr) {
        return Fail(MLK_ERR_INVALID, "mlk_graph_begin_capture: the null stream cannot be captured");
    }
    const hipError_t err =
        hipStreamBeginCapture(AsStream(stream), hipStreamCaptureModeThreadLocal);
    return err == hipSuccess ? MLK_OK : FromHip(err, "hipStreamBeginCapture");
}

mlk_status mlk_graph_end_capture(void* stream, void** graph_exec) {
    if (stream == nullptr || graph_exec == nullptr) {
        return Fail(MLK_ERR_INVALID, "mlk_graph_end_capture: null stream or output");
    }
    *graph_exec = nullptr;
    hipGraph_t graph = nullptr;
    hipError_t err = hipStreamEndCapture(AsStream(stream), &graph);
    if (err != hipSuccess) return FromHip(err, "hipStreamEndCapture");
    hipGraphExec_t exec = nullptr;
    err = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    const hipError_t destroy = hipGraphDestroy(graph);
    if (err != hipSuccess) return FromHip(err, "hipGraphInstantiate");
    if (destroy != hipSuccess) {
        (void)hipGraphExecDestroy(exec);
        return FromHip(destroy, "hipGraphDestroy");
    }
    *graph_exec = exec;
    return MLK_OK;
}

mlk_status mlk_graph_launch(void* graph_exec, void* stream) {
    if (graph_exec == nullptr) return Fail(MLK_ERR_INVALID, "mlk_graph_launch: null graph");
    const hipError_t err = hipGraphLaunch(static_cast<hipGraphExec_t>(graph_exec), AsStream(stream));
    return err == hipSuccess ? MLK_OK : FromHip(err, "hipGraphLaunch");
}

mlk_status mlk_graph_destroy(void* graph_exec) {
    if (graph_exec == nullptr) return MLK_OK;
    const hipError_t err = hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph_exec));
    return err == hipSuccess ? MLK_OK : FromHip(err, "hipGraphExecDestroy");
}

}  // extern "C"
