// mlk_softmax.hip -- row softmax, kept for the reference's op surface
// (CudaSoftmax, include/cuda_ops.h:29; CPU SoftMax src/ops.cc:113-134).
//
// One workgroup per row: block max, then the sum of exp(x - max) in float64
// (the CPU sums floats in order; a wider sum keeps the result within the
// reference's tolerance for any row length), then y = exp(x - max) / sum
// with the sum rounded to float as the CPU divides by a float.
#include "mlk_common.h"

namespace mlk {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;

__global__ __launch_bounds__(kThreads) void SoftmaxKernel(const float* __restrict__ x,
                                                          float* __restrict__ y, int64_t n_rows,
                                                          int64_t n) {
#pragma clang fp contract(off)
    __shared__ float max_scratch[2][kWaves];
    __shared__ double sum_scratch[2][kWaves];
    int parity = 0;
    for (int64_t r = blockIdx.x; r < n_rows; r += gridDim.x, parity ^= 1) {
        const float* xr = x + r * n;
        float* yr = y + r * n;
        float m = -3.402823466e+38F;
        for (int64_t i = threadIdx.x; i < n; i += kThreads) m = fmaxf(m, xr[i]);
        m = BlockMax<kWaves>(m, max_scratch[parity]);
        double s = 0.0;
        for (int64_t i = threadIdx.x; i < n; i += kThreads) s += static_cast<double>(expf(xr[i] - m));
        s = BlockSum<kWaves>(s, sum_scratch[parity]);
        const float sum = static_cast<float>(s);
        for (int64_t i = threadIdx.x; i < n; i += kThreads) yr[i] = expf(xr[i] - m) / sum;
    }
}

}  // namespace
}  // namespace mlk

using namespace mlk;

extern "C" {

mlk_status mlk_softmax_f32(const float* x, float* y, int64_t n_rows, int64_t n, void* stream) {
    if (x == nullptr || y == nullptr) {
        return Fail(MLK_ERR_INVALID, "mlk_softmax_f32: pointers must not be null");
    }
    if (n_rows <= 0 || n <= 0) {
        return Fail(MLK_ERR_INVALID, "mlk_softmax_f32: input tensor must not be empty");
    }
    if (x == y) {
        return Fail(MLK_ERR_INVALID, "mlk_softmax_f32: output must not alias the input");
    }
    const unsigned grid = GridFor(n_rows, 1, 8);
    hipLaunchKernelGGL(SoftmaxKernel, dim3(grid), dim3(kThreads), 0, AsStream(stream), x, y,
                       n_rows, n);
    return CheckLaunch("SoftmaxKernel");
}

}  // extern "C"
