// cuda_matmul.h -- F32 linear layers and matmul on MI355X.
//
// Same declarations as the reference (include/cuda_matmul.h:6-19 of the
// reference tree), which put them on cuBLAS (src/cuda_matmul.cc:122-275).
// Here they run the hand-written gfx950 kernels of libminilamma_hip.so
// (mlk_linear_f32 / mlk_matmul_f32) on the null stream.  Weights are
// row-major fp32 [out_features, in_features]; x is [in] or [rows, in] and
// y has the same rank.  Errors throw std::runtime_error "<Caller>: ..."
// before any launch.  Implemented in cpp-minilamma_amd/host/cuda_matmul.cc.
#pragma once
#include "include/cuda_runtime.h"
#include "include/cuda_tensor.h"
#include "include/tensor.h"

#include <vector>

namespace yan_lamma {
// True when the device kernels are built (always, in this build).
bool cuBLASBuilt();
// c = a @ b for host a [m, k] and b [k, n] (uploads both, downloads c).
Tensor CudaMatmul(const Tensor& a, const Tensor& b, int device_id);
// Host x and weight, host result; bias [out_features] is optional.
Tensor CudaLinear(const Tensor& x, const Tensor& weight, const Tensor* bias = nullptr,
                  int device_id = 0);
// Host x, weight already resident on device_id (borrowed), host result.
Tensor CudaLinearHostDevice(const Tensor& x, const void* w_data, const std::vector<int>& w_shape,
                            const Tensor* bias = nullptr, int device_id = 0);
// Device x and weight, new device result.
CudaTensor CudaLinearDevice(const CudaTensor& x, const void* w_data,
                            const std::vector<int>& w_shape, int device_id = 0);
}  // namespace yan_lamma
