// mlk_elementwise.hip -- SwiGLU and the element-wise ops of the reference's
// op surface (SiLU, multiply, add), plus the synthetic-input generator.
//
// SwiGLU follows SwiGlu = ElementwiseMul(Silu(gate), up) (src/ops.cc:
// 135-151): s = g * (1 / (1 + exp(-g))) rounded to float, then y = s * up.
// The reference device path ran SiluKernel and ElementWiseMulKernel
// (src/cuda_ops.cu:165-179) with silu(gate) going to HBM and back (20 B per
// element); the fused kernel moves 12 B per element (read gate and up,
// write y), which is the whole roofline of the op.
//
// All kernels stream 16-byte vectors with non-temporal loads and stores:
// each thread owns kUnroll float4 slots spaced one workgroup apart, so a
// wave's loads of one slot cover 1 KiB of contiguous memory and all kUnroll
// loads are in flight before the first use; every workgroup gets its own
// 16 KiB chunk (a full grid, no grid-stride reuse), which measured fastest
// on MI355X.  The n % 4 tail is finished by the first workgroup.
#include "mlk_common.h"

#include <cmath>

namespace mlk {
namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 4;

struct SwiGluOp {
    __device__ float operator()(float g, float u) const { return SwiGluF(g, u); }
};
struct SiluOp {
    __device__ float operator()(float x, float) const {
        const float sig = 1.0f / (1.0f + expf(-x));
        return x * sig;
    }
};
struct MulOp {
    __device__ float operator()(float a, float b) const { return a * b; }
};
struct AddOp {
    __device__ float operator()(float a, float b) const { return a + b; }
};

template <typename Op, bool kBinary>
__global__ __launch_bounds__(kThreads) void StreamKernel(const float4* __restrict__ a,
                                                         const float4* __restrict__ b,
                                                         float4* __restrict__ y, int64_t n4,
                                                         const float* __restrict__ a_tail,
                                                         const float* __restrict__ b_tail,
                                                         float* __restrict__ y_tail, int tail) {
#pragma clang fp contract(off)
    const Op op;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads * kUnroll;
    for (int64_t base = static_cast<int64_t>(blockIdx.x) * kThreads * kUnroll + threadIdx.x;
         base < n4; base += stride) {
        float4 av[kUnroll];
        float4 bv[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int64_t i = base + static_cast<int64_t>(u) * kThreads;
            if (i < n4) av[u] = LoadNT(a + i);
        }
        if (kBinary) {
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                const int64_t i = base + static_cast<int64_t>(u) * kThreads;
                if (i < n4) bv[u] = LoadNT(b + i);
            }
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int64_t i = base + static_cast<int64_t>(u) * kThreads;
            if (i < n4) {
                const float4 bb = kBinary ? bv[u] : make_float4(0.f, 0.f, 0.f, 0.f);
                float4 o;
                o.x = op(av[u].x, bb.x);
                o.y = op(av[u].y, bb.y);
                o.z = op(av[u].z, bb.z);
                o.w = op(av[u].w, bb.w);
                StoreNT(y + i, o);
            }
        }
    }
    if (blockIdx.x == 0 && static_cast<int>(threadIdx.x) < tail) {
        const int j = threadIdx.x;
        y_tail[j] = op(a_tail[j], kBinary ? b_tail[j] : 0.0f);
    }
}

// Unaligned pointers: one element per thread.
template <typename Op, bool kBinary>
__global__ __launch_bounds__(kThreads) void ScalarKernel(const float* a, const float* b, float* y,
                                                         int64_t n) {
#pragma clang fp contract(off)
    const Op op;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
         i += stride) {
        y[i] = op(a[i], kBinary ? b[i] : 0.0f);
    }
}

template <typename Op, bool kBinary>
mlk_status LaunchStream(const char* caller, const float* a, const float* b, float* y, int64_t n,
                        hipStream_t stream) {
    if (a == nullptr || y == nullptr || (kBinary && b == nullptr)) {
        return Fail(MLK_ERR_INVALID, "%s: input and output pointers must not be null", caller);
    }
    if (n <= 0) {
        return Fail(MLK_ERR_INVALID, "%s: input tensor must not be empty", caller);
    }
    const bool vec = Aligned(a, 16) && Aligned(y, 16) && (!kBinary || Aligned(b, 16));
    if (vec) {
        const int64_t n4 = n / 4;
        const int tail = static_cast<int>(n - n4 * 4);
        const int64_t done = n4 * 4;
        const unsigned grid = FullGrid(n4, kThreads * kUnroll);
        hipLaunchKernelGGL((StreamKernel<Op, kBinary>), dim3(grid), dim3(kThreads), 0, stream,
                           reinterpret_cast<const float4*>(a),
                           reinterpret_cast<const float4*>(kBinary ? b : a),
                           reinterpret_cast<float4*>(y), n4, a + done, (kBinary ? b : a) + done,
                           y + done, tail);
        return CheckLaunch("StreamKernel");
    }
    const unsigned grid = GridFor(n, kThreads, 8);
    hipLaunchKernelGGL((ScalarKernel<Op, kBinary>), dim3(grid), dim3(kThreads), 0, stream, a,
                       kBinary ? b : a, y, n);
    return CheckLaunch("ScalarKernel");
}

// ------------------------------------------------------ synthetic inputs

__device__ inline uint64_t Mix64(uint64_t z) {
    // splitmix64 finalizer
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Box-Muller on two 32-bit uniforms drawn from the hash of (seed, i / 2);
// element 2j gets the cosine branch and 2j + 1 the sine branch.
__global__ __launch_bounds__(kThreads) void FillNormalKernel(float* x, int64_t n, float mean,
                                                             float std, uint64_t seed) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
         i += stride) {
        const uint64_t h = Mix64(seed * 0x9E3779B97F4A7C15ull + static_cast<uint64_t>(i >> 1));
        const float u1 = (static_cast<float>(static_cast<uint32_t>(h) >> 8) + 1.0f) * 0x1.0p-24f;
        const float u2 = static_cast<float>(static_cast<uint32_t>(h >> 32) >> 8) * 0x1.0p-24f;
        const float radius = sqrtf(-2.0f * logf(u1));
        const float angle = 6.28318530717958647692f * u2;
        const float z = (i & 1) ? radius * sinf(angle) : radius * cosf(angle);
        x[i] = mean + std * z;
    }
}

}  // namespace
}  // namespace mlk

using namespace mlk;

extern "C" {

mlk_status mlk_swiglu_f32(const float* gate, const float* up, float* y, int64_t n,
                          void* stream) {
    return LaunchStream<SwiGluOp, true>("mlk_swiglu_f32", gate, up, y, n, AsStream(stream));
}

mlk_status mlk_silu_f32(const float* x, float* y, int64_t n, void* stream) {
    return LaunchStream<SiluOp, false>("mlk_silu_f32", x, nullptr, y, n, AsStream(stream));
}

mlk_status mlk_mul_f32(const float* a, const float* b, float* y, int64_t n, void* stream) {
    return LaunchStream<MulOp, true>("mlk_mul_f32", a, b, y, n, AsStream(stream));
}

mlk_status mlk_add_f32(const float* a, const float* b, float* y, int64_t n, void* stream) {
    return LaunchStream<AddOp, true>("mlk_add_f32", a, b, y, n, AsStream(stream));
}

mlk_status mlk_fill_normal_f32(float* x, int64_t n, float mean, float std, uint64_t seed,
                               void* stream) {
    if (x == nullptr || n <= 0) {
        return Fail(MLK_ERR_INVALID, "mlk_fill_normal_f32: need a buffer and n > 0");
    }
    const unsigned grid = GridFor(n, kThreads, 8);
    hipLaunchKernelGGL(FillNormalKernel, dim3(grid), dim3(kThreads), 0, AsStream(stream), x, n,
                       mean, std, seed);
    return CheckLaunch("FillNormalKernel");
}

}  // extern "C"
