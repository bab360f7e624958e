// cuda_quant.h -- linear layers with Q4_0 / Q4_1 / Q8_0 block-quantized
// weights on MI355X.
//
// Same declarations as the reference (include/cuda_quant.h:9-25 of the
// reference tree; kernels src/cuda_quant.cu:29-97).  Weights are out_features
// rows of ceil(in_features / 32) packed blocks; `shape` is the weight shape
// [out_features, in_features] and `block_size` the number of blocks the
// caller holds (validated against the shape).  x is [in] or [rows, in].
//   Cuda*Linear               host x, host blocks (uploaded), host result;
//   Cuda*DeviceLinear         host x, resident device blocks, host result;
//   Cuda*DeviceInputLinear    device x, resident device blocks, device result.
// Errors throw std::runtime_error before any launch.  Implemented in
// cpp-minilamma_amd/host/cuda_quant.cc over mlk_linear_quant.
#pragma once
#include "include/cuda_runtime.h"
#include "include/cuda_tensor.h"
#include "include/quantized_tensor.h"
#include "include/tensor.h"

#include <cstddef>
#include <vector>

namespace yan_lamma {
// True when the device kernels are built (always, in this build).
bool CudaQuantBuilt();
Tensor CudaQ40Linear(const Tensor& x, const std::vector<Block_Q40>& weight,
                     const std::vector<int>& shape, const Tensor* bias = nullptr,
                     int device_id = 0);
Tensor CudaQ40DeviceLinear(const Tensor& x, const void* device_weight,
                           const std::vector<int>& shape, const size_t block_size,
                           const Tensor* bias = nullptr, int device_id = 0);
CudaTensor CudaQ40DeviceInputLinear(const CudaTensor& x, const void* device_weight,
                                    const std::vector<int>& shape, const size_t block_size,
                                    int device_id = 0);
Tensor CudaQ41Linear(const Tensor& x, const std::vector<Block_Q41>& weight,
                     const std::vector<int>& shape, const Tensor* bias = nullptr,
                     int device_id = 0);
Tensor CudaQ41DeviceLinear(const Tensor& x, const void* device_weight,
                           const std::vector<int>& shape, const size_t block_size,
                           const Tensor* bias = nullptr, int device_id = 0);
CudaTensor CudaQ41DeviceInputLinear(const CudaTensor& x, const void* device_weight,
                                    const std::vector<int>& shape, const size_t block_size,
                                    int device_id = 0);
Tensor CudaQ80Linear(const Tensor& x, const std::vector<Block_Q80>& weight,
                     const std::vector<int>& shape, const Tensor* bias = nullptr,
                     int device_id = 0);
Tensor CudaQ80DeviceLinear(const Tensor& x, const void* device_weight,
                           const std::vector<int>& shape, const size_t block_size,
                           const Tensor* bias = nullptr, int device_id = 0);
CudaTensor CudaQ80DeviceInputLinear(const CudaTensor& x, const void* device_weight,
                                    const std::vector<int>& shape, const size_t block_size,
                                    int device_id = 0);
}  // namespace yan_lamma
