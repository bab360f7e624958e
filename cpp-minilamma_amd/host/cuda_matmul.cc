// cuda_matmul.cc -- F32 linear and matmul (include/cuda_matmul.h) over the C
// ABI of libminilamma_hip.so.  No HIP header is included here.
//
// Checks and messages follow the reference's cuBLAS path
// (src/cuda_matmul.cc:70-189 of the reference tree); every check runs before
// any allocation or launch.  As there, the host variants upload x, run the
// kernel, download y and add the bias on the host.
#include "include/cuda_matmul.h"
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

// src/cuda_matmul.cc:92-117: x is [in] or [rows, in], weight [out, in].
void ValidateLinear(const std::vector<int>& x_shape, const std::vector<int>& w_shape,
                    const char* caller) {
    if (w_shape.size() != 2) Fail(caller, "expected weight shape [out_features, in_features]");
    if (x_shape.size() != 1 && x_shape.size() != 2) {
        Fail(caller, "expected x shape [in_features] or [batch, in_features], got " +
                         ShapeString(x_shape));
    }
    if (x_shape.back() != w_shape[1]) Fail(caller, "input features do not match weight");
    for (int d : x_shape) {
        if (d <= 0) Fail(caller, "dimensions must be positive");
    }
    if (w_shape[0] <= 0 || w_shape[1] <= 0) Fail(caller, "dimensions must be positive");
}

void ValidateBias(const Tensor* bias, int out_features, const char* caller) {
    if (bias != nullptr && (bias->GetNumDims() != 1 || bias->shape[0] != out_features)) {
        Fail(caller, "expected bias shape [out_features]");
    }
}

void AddBias(Tensor& y, const Tensor& bias, int rows, int cols) {
    for (int r = 0; r < rows; ++r) {
        for (int c = 0; c < cols; ++c) {
            y.data[static_cast<size_t>(r) * cols + c] += bias.data[c];
        }
    }
}

std::vector<int> OutShape(const std::vector<int>& x_shape, int out_features) {
    return x_shape.size() == 1 ? std::vector<int>{out_features}
                               : std::vector<int>{x_shape[0], out_features};
}

Tensor LinearHostX(const Tensor& x, const void* w_data, const std::vector<int>& w_shape,
                   const Tensor* bias, int device_id, const char* caller) {
    const int rows = x.GetNumDims() == 1 ? 1 : x.shape[0];
    const int in = w_shape[1], out = w_shape[0];
    SetCudaService(device_id);
    CudaDeviceBuffer xb(x.GetDataSize() * sizeof(float), device_id);
    CudaDeviceBuffer yb(static_cast<size_t>(rows) * out * sizeof(float), device_id);
    xb.upload(x.data.data(), x.GetDataSize() * sizeof(float));
    CudaDeviceBuffer ws = LinearWorkspace(rows, in, out, device_id);
    Launched(mlk_linear_f32(static_cast<const float*>(xb.GetData()),
                            static_cast<const float*>(w_data), nullptr,
                            static_cast<float*>(yb.GetData()), rows, in, out, ws.GetData(),
                            ws.GetByteSize(), nullptr),
             caller);
    Tensor y(OutShape(x.shape, out));
    yb.download(y.data.data(), y.GetDataSize() * sizeof(float));
    if (bias != nullptr) AddBias(y, *bias, rows, out);
    return y;
}

}  // namespace

bool cuBLASBuilt() { return CudaRuntimeBuilt(); }

Tensor CudaMatmul(const Tensor& a, const Tensor& b, int device_id) {
    const char* caller = "CudaMatmul";
    if (a.GetNumDims() != 2 || b.GetNumDims() != 2) Fail(caller, "expected two 2D tensors");
    if (a.shape[1] != b.shape[0]) Fail(caller, "expected a.shape[1] == b.shape[0]");
    if (a.shape[0] <= 0 || a.shape[1] <= 0 || b.shape[1] <= 0) {
        Fail(caller, "dimensions must be positive");
    }
    const int m = a.shape[0], k = a.shape[1], n = b.shape[1];
    SetCudaService(device_id);
    CudaDeviceBuffer ab(a.GetDataSize() * sizeof(float), device_id);
    CudaDeviceBuffer bb(b.GetDataSize() * sizeof(float), device_id);
    CudaDeviceBuffer cb(static_cast<size_t>(m) * n * sizeof(float), device_id);
    ab.upload(a.data.data(), a.GetDataSize() * sizeof(float));
    bb.upload(b.data.data(), b.GetDataSize() * sizeof(float));
    Launched(mlk_matmul_f32(static_cast<const float*>(ab.GetData()),
                            static_cast<const float*>(bb.GetData()),
                            static_cast<float*>(cb.GetData()), m, k, n, nullptr),
             caller);
    Tensor c({m, n});
    cb.download(c.data.data(), c.GetDataSize() * sizeof(float));
    return c;
}

Tensor CudaLinear(const Tensor& x, const Tensor& weight, const Tensor* bias, int device_id) {
    const char* caller = "CudaLinear";
    ValidateLinear(x.shape, weight.shape, caller);
    ValidateBias(bias, weight.shape[0], caller);
    SetCudaService(device_id);
    CudaDeviceBuffer wb(weight.GetDataSize() * sizeof(float), device_id);
    wb.upload(weight.data.data(), weight.GetDataSize() * sizeof(float));
    return LinearHostX(x, wb.GetData(), weight.shape, bias, device_id, caller);
}

Tensor CudaLinearHostDevice(const Tensor& x, const void* w_data, const std::vector<int>& w_shape,
                            const Tensor* bias, int device_id) {
    const char* caller = "CudaLinear";
    if (w_data == nullptr) Fail(caller, "device weight pointer is null");
    ValidateLinear(x.shape, w_shape, caller);
    ValidateBias(bias, w_shape[0], caller);
    return LinearHostX(x, w_data, w_shape, bias, device_id, caller);
}

CudaTensor CudaLinearDevice(const CudaTensor& x, const void* w_data,
                            const std::vector<int>& w_shape, int device_id) {
    const char* caller = "CudaLinearDevice";
    if (x.IsEmpty() || w_data == nullptr) Fail(caller, "device input or weight pointer is null");
    if (x.DeviceId() != device_id) Fail(caller, "input tensor is on a different CUDA device");
    ValidateLinear(x.shape(), w_shape, caller);
    const int rows = x.num_dims() == 1 ? 1 : x.shape()[0];
    SetCudaService(device_id);
    CudaTensor y(OutShape(x.shape(), w_shape[0]), device_id);
    CudaDeviceBuffer ws = LinearWorkspace(rows, w_shape[1], w_shape[0], device_id);
    Launched(mlk_linear_f32(static_cast<const float*>(x.GetData()),
                            static_cast<const float*>(w_data), nullptr,
                            static_cast<float*>(y.GetData()), rows, w_shape[1], w_shape[0],
                            ws.GetData(), ws.GetByteSize(), nullptr),
             caller);
    return y;
}

}  // namespace yan_lamma
