// cuda_quant.cc -- quantized linear layers (include/cuda_quant.h) over the C
// ABI of libminilamma_hip.so.  No HIP header is included here.
//
// Checks and messages follow the reference (src/cuda_quant.cu:99-316 of the
// reference tree): ValidateQuantLinearShape's shape / block-count rules, the
// null-weight and device-match checks, then the bias shape; all run before
// any allocation or launch.  The host variants add the bias on the host
// after the download, as the reference does.
#include "include/cuda_quant.h"
#include "include/minilamma_hip.h"
#include "linear_workspace.h"

#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

namespace yan_lamma {
namespace {

[[noreturn]] void Fail(const std::string& caller, const std::string& reason) {
    throw std::runtime_error(caller + ": " + reason);
}

void Launched(mlk_status st, const char* caller) {
    if (st != MLK_OK) Fail(caller, mlk_last_error());
}

std::string ShapeString(const std::vector<int>& shape) {
    std::string s = "[";
    for (size_t i = 0; i < shape.size(); ++i) s += (i ? ", " : "") + std::to_string(shape[i]);
    return s + "]";
}

// src/cuda_quant.cu:112-140 (messages prefixed "Quant linear").
void ValidateQuantShape(const std::vector<int>& x_shape, size_t block_count,
                        const std::vector<int>& w_shape) {
    const std::string caller = "Quant linear";
    if (w_shape.size() != 2) Fail(caller, "expected weight shape [out_features, in_features]");
    if (x_shape.size() != 1 && x_shape.size() != 2) {
        Fail(caller, "expected 1D or 2D input, got " + ShapeString(x_shape));
    }
    const int in_features = x_shape.back();
    if (in_features <= 0 || (x_shape.size() == 2 && x_shape[0] <= 0) || w_shape[0] <= 0 ||
        w_shape[1] <= 0) {
        Fail(caller, "dimensions and block size must be positive");
    }
    if (in_features != w_shape[1]) Fail(caller, "input and weight in_features do not match");
    const size_t per_row = (static_cast<size_t>(in_features) + kQuantBlockSize - 1) /
                           kQuantBlockSize;
    if (per_row * static_cast<size_t>(w_shape[0]) != block_count) {
        Fail(caller, "weight block count does not match shape");
    }
}

void ValidateBias(const Tensor* bias, int out_features, const std::string& caller) {
    if (bias != nullptr && (bias->GetNumDims() != 1 || bias->shape[0] != out_features)) {
        Fail(caller, "expected bias shape [out_features]");
    }
}

std::vector<int> OutShape(const std::vector<int>& x_shape, int out_features) {
    return x_shape.size() == 1 ? std::vector<int>{out_features}
                               : std::vector<int>{x_shape[0], out_features};
}

// Host x, resident weight: the reference's CudaQ*Device (src/cuda_quant.cu:
// 155-183 and its Q8_0 / Q4_1 twins).
Tensor DeviceWeightHostX(int32_t qt, const std::string& caller, const Tensor& x,
                         const void* device_weight, const std::vector<int>& shape,
                         size_t block_count, const Tensor* bias, int device_id) {
    if (device_weight == nullptr) Fail(caller, "device weight is null");
    ValidateQuantShape(x.shape, block_count, shape);
    ValidateBias(bias, shape[0], caller);
    const int rows = x.GetNumDims() == 1 ? 1 : x.shape[0];
    const int out = shape[0];
    SetCudaService(device_id);
    CudaDeviceBuffer xb(x.GetDataSize() * sizeof(float), device_id);
    CudaDeviceBuffer yb(static_cast<size_t>(rows) * out * sizeof(float), device_id);
    xb.upload(x.data.data(), x.GetDataSize() * sizeof(float));
    CudaDeviceBuffer ws = LinearWorkspace(rows, shape[1], out, device_id);
    Launched(mlk_linear_quant(qt, static_cast<const float*>(xb.GetData()), device_weight, nullptr,
                              static_cast<float*>(yb.GetData()), rows, shape[1], out,
                              ws.GetData(), ws.GetByteSize(), nullptr),
             caller.c_str());
    Tensor y(OutShape(x.shape, out));
    yb.download(y.data.data(), y.GetDataSize() * sizeof(float));
    if (bias != nullptr) {
        for (int r = 0; r < rows; ++r) {
            for (int c = 0; c < out; ++c) y.data[static_cast<size_t>(r) * out + c] += bias->data[c];
        }
    }
    return y;
}

// Device x and weight: the reference's CudaQ*DeviceInput (src/cuda_quant.cu:
// 184-208 and twins).
CudaTensor DeviceWeightDeviceX(int32_t qt, const std::string& caller, const CudaTensor& x,
                               const void* device_weight, const std::vector<int>& shape,
                               size_t block_count, int device_id) {
    if (x.DeviceId() != device_id) Fail(caller, "input device does not match device_id");
    if (device_weight == nullptr) Fail(caller, "device weight is null");
    if (x.IsEmpty()) Fail(caller, "input tensor must not be empty");
    ValidateQuantShape(x.shape(), block_count, shape);
    const int rows = x.num_dims() == 1 ? 1 : x.shape()[0];
    SetCudaService(device_id);
    CudaTensor y(OutShape(x.shape(), shape[0]), device_id);
    CudaDeviceBuffer ws = LinearWorkspace(rows, shape[1], shape[0], device_id);
    Launched(mlk_linear_quant(qt, static_cast<const float*>(x.GetData()), device_weight, nullptr,
                              static_cast<float*>(y.GetData()), rows, shape[1], shape[0],
                              ws.GetData(), ws.GetByteSize(), nullptr),
             caller.c_str());
    return y;
}

template <typename Block>
Tensor UploadedWeight(int32_t qt, const std::string& caller, const Tensor& x,
                      const std::vector<Block>& weight, const std::vector<int>& shape,
                      const Tensor* bias, int device_id) {
    // validate before the upload so a bad call moves no data
    ValidateQuantShape(x.shape, weight.size(), shape);
    ValidateBias(bias, shape[0], caller);
    SetCudaService(device_id);
    CudaDeviceBuffer wb(weight.size() * sizeof(Block), device_id);
    wb.upload(weight.data(), weight.size() * sizeof(Block));
    return DeviceWeightHostX(qt, caller, x, wb.GetData(), shape, weight.size(), bias, device_id);
}

}  // namespace

bool CudaQuantBuilt() { return CudaRuntimeBuilt(); }

Tensor CudaQ40Linear(const Tensor& x, const std::vector<Block_Q40>& weight,
                     const std::vector<int>& shape, const Tensor* bias, int device_id) {
    return UploadedWeight(MLK_Q4_0, "CudaQ40Device", x, weight, shape, bias, device_id);
}
Tensor CudaQ40DeviceLinear(const Tensor& x, const void* device_weight,
                           const std::vector<int>& shape, const size_t block_size,
                           const Tensor* bias, int device_id) {
    return DeviceWeightHostX(MLK_Q4_0, "CudaQ40Device", x, device_weight, shape, block_size, bias,
                             device_id);
}
CudaTensor CudaQ40DeviceInputLinear(const CudaTensor& x, const void* device_weight,
                                    const std::vector<int>& shape, const size_t block_size,
                                    int device_id) {
    return DeviceWeightDeviceX(MLK_Q4_0, "CudaQ40DeviceInput", x, device_weight, shape,
                               block_size, device_id);
}

Tensor CudaQ41Linear(const Tensor& x, const std::vector<Block_Q41>& weight,
                     const std::vector<int>& shape, const Tensor* bias, int device_id) {
    return UploadedWeight(MLK_Q4_1, "CudaQ41Device", x, weight, shape, bias, device_id);
}
Tensor CudaQ41DeviceLinear(const Tensor& x, const void* device_weight,
                           const std::vector<int>& shape, const size_t block_size,
                           const Tensor* bias, int device_id) {
    return DeviceWeightHostX(MLK_Q4_1, "CudaQ41Device", x, device_weight, shape, block_size, bias,
                             device_id);
}
CudaTensor CudaQ41DeviceInputLinear(const CudaTensor& x, const void* device_weight,
                                    const std::vector<int>& shape, const size_t block_size,
                                    int device_id) {
    return DeviceWeightDeviceX(MLK_Q4_1, "CudaQ41DeviceInput", x, device_weight, shape,
                               block_size, device_id);
}

Tensor CudaQ80Linear(const Tensor& x, const std::vector<Block_Q80>& weight,
                     const std::vector<int>& shape, const Tensor* bias, int device_id) {
    return UploadedWeight(MLK_Q8_0, "CudaQ80Device", x, weight, shape, bias, device_id);
}
Tensor CudaQ80DeviceLinear(const Tensor& x, const void* device_weight,
                           const std::vector<int>& shape, const size_t block_size,
                           const Tensor* bias, int device_id) {
    return DeviceWeightHostX(MLK_Q8_0, "CudaQ80Device", x, device_weight, shape, block_size, bias,
                             device_id);
}
CudaTensor CudaQ80DeviceInputLinear(const CudaTensor& x, const void* device_weight,
                                    const std::vector<int>& shape, const size_t block_size,
                                    int device_id) {
    return DeviceWeightDeviceX(MLK_Q8_0, "CudaQ80DeviceInput", x, device_weight, shape,
                               block_size, device_id);
}

}  // namespace yan_lamma
