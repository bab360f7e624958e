// cuda_ops.cc -- the per-layer op surface (include/cuda_ops.h) over the C ABI
// of libminilamma_hip.so.  No HIP header is included here.
//
// Every entry validates its arguments first and throws std::runtime_error
// "<Caller>: <reason>" without launching anything, with the checks and
// messages of the reference's device ops (src/cuda_ops.cu:23-149 of the
// reference tree), then selects the device, allocates the result through
// the caching allocator and issues one kernel on the null stream.
// Differences from the reference that a caller can see:
//   - no 2^31 element limit (the kernels index with 64-bit offsets);
//   - CudaRmsNromDevice does not synchronize (it needs no temporary buffer);
//   - the *Host variants allocate from the cache instead of cudaMalloc.
#include "include/cuda_ops.h"
#include "include/minilamma_hip.h"

#include <cmath>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

namespace yan_lamma {
namespace {

[[noreturn]] void Fail(const std::string& caller, const std::string& reason) {
    throw std::runtime_error(caller + ": " + reason);
}

// Turns a C ABI status into the caller-prefixed exception.
void Launched(mlk_status st, const char* caller) {
    if (st != MLK_OK) Fail(caller, mlk_last_error());
}

void RequireElementwise(const CudaTensor& x, int device_id, const char* caller) {
    if (x.IsEmpty() || x.NumEle() == 0) Fail(caller, "input tensor must not be empty");
    if (x.DeviceId() != device_id) Fail(caller, "input tensor is on a different CUDA device");
}

void RequireSameShape(const Tensor& a, const Tensor& b, const char* caller) {
    if (a.shape != b.shape) Fail(caller, "input shapes must match");
}

void RequireSameShape(const CudaTensor& a, const CudaTensor& b, const char* caller) {
    if (a.shape() != b.shape()) Fail(caller, "input shapes must match");
    if (a.DeviceId() != b.DeviceId()) Fail(caller, "inputs must be on the same CUDA device");
}

void Require1d(const Tensor& x, const char* caller) {
    if (x.GetNumDims() != 1) Fail(caller, "expected a 1D input tensor");
    if (x.GetDataSize() == 0) Fail(caller, "input tensor must not be empty");
}

void Require1d(const CudaTensor& x, const char* caller) {
    if (x.num_dims() != 1) Fail(caller, "expected a 1D input tensor");
    if (x.NumEle() == 0 || x.IsEmpty()) Fail(caller, "input tensor must not be empty");
}

void RequireEps(float eps, const char* caller) {
    if (!std::isfinite(eps) || eps <= 0) Fail(caller, "eps must be finite and positive");
}

void RequireTheta(float theta, const char* caller) {
    if (!std::isfinite(theta) || theta <= 0) Fail(caller, "theta must be finite and positive");
}

void RequireHeads(int n_heads, int n_kv_heads, int head_dim, const char* caller) {
    if (n_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0 || head_dim % 2 != 0) {
        Fail(caller, "head counts must be positive and head_dim must be positive and even");
    }
}

float* F(CudaTensor& t) { return static_cast<float*>(t.GetData()); }
const float* F(const CudaTensor& t) { return static_cast<const float*>(t.GetData()); }

int32_t RopeCode(RopeType t) { return t == RopeType::kNormal ? MLK_ROPE_NORMAL : MLK_ROPE_NEOX; }

int32_t QuantCode(QuantType t, const char* caller) {
    switch (t) {
        case QuantType::kQ80: return MLK_Q8_0;
        case QuantType::kQ40: return MLK_Q4_0;
        case QuantType::kQ41: return MLK_Q4_1;
        default: Fail(caller, "unsupported quantization type (expected Q8_0, Q4_0 or Q4_1)");
    }
}

// [vocab, dim] table shape as (vocab, dim); token ids in range.
void RequireTable(const void* data, const std::vector<int>& shape, const char* caller) {
    if (data == nullptr) Fail(caller, "embedding weight pointer must not be null");
    if (shape.size() != 2) Fail(caller, "expected weight shape [vocab_size, dim]");
    if (shape[0] <= 0 || shape[1] <= 0) Fail(caller, "weight dimensions must be positive");
}

void RequireIds(const std::vector<int>& ids, int vocab, const char* caller) {
    if (ids.empty()) Fail(caller, "token_ids must not be empty");
    for (int id : ids) {
        if (id < 0 || id >= vocab) Fail(caller, "token_id must be in [0, vocab_size)");
    }
}

// Last-dimension width of a row-wise op and its weight checks.
int64_t RowWidth(const CudaTensor& x, const void* weight, const std::vector<int>& weight_shape,
                 int device_id, const char* caller) {
    if (x.IsEmpty() || x.NumEle() == 0) Fail(caller, "input tensor must not be empty");
    if (weight == nullptr) Fail(caller, "weight pointer must not be null");
    if (weight_shape.size() != 1 || weight_shape[0] != x.shape().back()) {
        Fail(caller, "weight shape must be [dim] with dim the input's last dimension");
    }
    if (x.DeviceId() != device_id) Fail(caller, "input device must match device_id");
    return x.shape().back();
}

// A device copy of host ids / positions (one counted host-to-device copy).
CudaDeviceBuffer UploadInts(const std::vector<int>& v, int device_id) {
    CudaDeviceBuffer buf(v.size() * sizeof(int32_t), device_id);
    buf.upload(v.data(), v.size() * sizeof(int32_t));
    return buf;
}

}  // namespace

bool CudaopsBuild() { return CudaRuntimeBuilt(); }

// ------------------------------------------------------ reference surface

CudaTensor CudaEmbeddingDevice(const void* embedding_data, const std::vector<int>& shape,
                               int token_id, int device_id) {
    const char* caller = "CudaEmbeddingDevice";
    RequireTable(embedding_data, shape, caller);
    if (token_id < 0 || token_id >= shape[0]) Fail(caller, "token_id must be in [0, vocab_size)");
    SetCudaService(device_id);
    CudaTensor y({shape[1]}, device_id);
    Launched(mlk_gather_f32(static_cast<const float*>(embedding_data), shape[0], shape[1], nullptr,
                            token_id, 1, F(y), nullptr, nullptr),
             caller);
    return y;
}

Tensor CudaRmsNormHost(const Tensor& x, const Tensor& weight, float eps, int device_id) {
    const char* caller = "CudaRmsNormHost";
    Require1d(x, caller);
    Require1d(weight, caller);
    RequireSameShape(x, weight, caller);
    RequireEps(eps, caller);
    SetCudaService(device_id);
    const size_t bytes = x.GetDataSize() * sizeof(float);
    CudaDeviceBuffer xb(bytes, device_id), wb(bytes, device_id), yb(bytes, device_id);
    xb.upload(x.data.data(), bytes);
    wb.upload(weight.data.data(), bytes);
    Launched(mlk_rmsnorm_f32(static_cast<const float*>(xb.GetData()),
                             static_cast<const float*>(wb.GetData()),
                             static_cast<float*>(yb.GetData()), 1,
                             static_cast<int64_t>(x.GetDataSize()), eps, nullptr),
             caller);
    Tensor y(x.shape);
    yb.download(y.data.data(), bytes);
    return y;
}

CudaTensor CudaRmsNromDevice(const CudaTensor& x, const void* weight_data,
                             const std::vector<int>& shape, float eps, int device_id) {
    const char* caller = "CudaRmsNromDevice";
    Require1d(x, caller);
    if (weight_data == nullptr) Fail(caller, "weight pointer must not be null");
    if (x.shape() != shape) Fail(caller, "weight shape must match input shape");
    if (x.DeviceId() != device_id) Fail(caller, "input device must match device_id");
    RequireEps(eps, caller);
    SetCudaService(device_id);
    CudaTensor y(x.shape(), device_id);
    Launched(mlk_rmsnorm_f32(F(x), static_cast<const float*>(weight_data), F(y), 1,
                             static_cast<int64_t>(x.NumEle()), eps, nullptr),
             caller);
    return y;
}

Tensor CudaSilu(const Tensor& a, int device_id) {
    const char* caller = "CudaSilu";
    if (a.GetDataSize() == 0) Fail(caller, "input tensor must not be empty");
    SetCudaService(device_id);
    const size_t bytes = a.GetDataSize() * sizeof(float);
    CudaDeviceBuffer ab(bytes, device_id), yb(bytes, device_id);
    ab.upload(a.data.data(), bytes);
    Launched(mlk_silu_f32(static_cast<const float*>(ab.GetData()), static_cast<float*>(yb.GetData()),
                          static_cast<int64_t>(a.GetDataSize()), nullptr),
             caller);
    Tensor y(a.shape);
    yb.download(y.data.data(), bytes);
    return y;
}

Tensor CudaElementwiseMul(const Tensor& a, const Tensor& b, int device_id) {
    const char* caller = "CudaElementwiseMul";
    RequireSameShape(a, b, caller);
    if (a.GetDataSize() == 0) Fail(caller, "input tensor must not be empty");
    SetCudaService(device_id);
    const size_t bytes = a.GetDataSize() * sizeof(float);
    CudaDeviceBuffer ab(bytes, device_id), bb(bytes, device_id), yb(bytes, device_id);
    ab.upload(a.data.data(), bytes);
    bb.upload(b.data.data(), bytes);
    Launched(mlk_mul_f32(static_cast<const float*>(ab.GetData()),
                         static_cast<const float*>(bb.GetData()), static_cast<float*>(yb.GetData()),
                         static_cast<int64_t>(a.GetDataSize()), nullptr),
             caller);
    Tensor y(a.shape);
    yb.download(y.data.data(), bytes);
    return y;
}

CudaTensor CudaSiluDevice(const CudaTensor& a, int device_id) {
    const char* caller = "CudaSiluDevice";
    RequireElementwise(a, device_id, caller);
    SetCudaService(device_id);
    CudaTensor y(a.shape(), device_id);
    Launched(mlk_silu_f32(F(a), F(y), static_cast<int64_t>(a.NumEle()), nullptr), caller);
    return y;
}

CudaTensor CudaElementwiseMulDevice(const CudaTensor& a, const CudaTensor& b, int device_id) {
    const char* caller = "CudaElementwiseMulDevice";
    RequireElementwise(a, device_id, caller);
    RequireElementwise(b, device_id, caller);
    RequireSameShape(a, b, caller);
    SetCudaService(device_id);
    CudaTensor y(a.shape(), device_id);
    Launched(mlk_mul_f32(F(a), F(b), F(y), static_cast<int64_t>(a.NumEle()), nullptr), caller);
    return y;
}

CudaTensor CudaElementAddDevice(const CudaTensor& a, const CudaTensor& b, int device_id) {
    RequireSameShape(a, b, "CudaElementAddDevice");
    return OCudaElementAddDevice(a, b.GetData(), b.shape(), device_id);
}

CudaTensor OCudaElementAddDevice(const CudaTensor& a, const void* b, const std::vector<int>& shape,
                                 int device_id) {
    const char* caller = "OCudaElementAddDevice";
    if (a.DeviceId() != device_id) Fail(caller, "input device must match device_id");
    if (b == nullptr) Fail(caller, "weight pointer must not be null");
    if (a.shape() != shape) Fail(caller, "weight shape must match input shape");
    if (a.IsEmpty()) Fail(caller, "input tensor must not be empty");
    SetCudaService(device_id);
    CudaTensor y(a.shape(), device_id);
    Launched(mlk_add_f32(F(a), static_cast<const float*>(b), F(y),
                         static_cast<int64_t>(a.NumEle()), nullptr),
             caller);
    return y;
}

Tensor CudaSoftmax(Tensor& x, int device_id) {
    const char* caller = "CudaSoftmax";
    Require1d(x, caller);
    SetCudaService(device_id);
    const size_t bytes = x.GetDataSize() * sizeof(float);
    CudaDeviceBuffer xb(bytes, device_id), yb(bytes, device_id);
    xb.upload(x.data.data(), bytes);
    Launched(mlk_softmax_f32(static_cast<const float*>(xb.GetData()),
                             static_cast<float*>(yb.GetData()), 1,
                             static_cast<int64_t>(x.GetDataSize()), nullptr),
             caller);
    Tensor y(x.shape);
    yb.download(y.data.data(), bytes);
    return y;
}

void CudaRopeHost(Tensor& q, Tensor& k, int pos, float theta, RopeType rope_type, int device_id) {
    const char* caller = "CudaRopeHost";
    if (q.GetNumDims() != 2 || k.GetNumDims() != 2) Fail(caller, "expected 2D q and k tensors");
    if (pos < 0) Fail(caller, "pos must be non-negative");
    RequireTheta(theta, caller);
    if (q.shape[1] != k.shape[1]) Fail(caller, "q and k head dimensions must match");
    if (q.shape[1] % 2 != 0) Fail(caller, "head dimension must be even");
    SetCudaService(device_id);
    const size_t qb = q.GetDataSize() * sizeof(float), kb = k.GetDataSize() * sizeof(float);
    CudaDeviceBuffer dq(qb, device_id), dk(kb, device_id);
    dq.upload(q.data.data(), qb);
    dk.upload(k.data.data(), kb);
    const int hd = q.shape[1];
    Launched(mlk_rope_f32(static_cast<float*>(dq.GetData()), static_cast<float*>(dk.GetData()), 1,
                          q.shape[0], k.shape[0], hd, static_cast<int64_t>(q.shape[0]) * hd,
                          static_cast<int64_t>(k.shape[0]) * hd, nullptr, pos, theta,
                          RopeCode(rope_type), nullptr, nullptr),
             caller);
    dq.download(q.data.data(), qb);
    dk.download(k.data.data(), kb);
}

void CudaRopeDevice(CudaTensor& q, CudaTensor& k, int pos, int n_heads, int n_kv_heads,
                    int head_dim, float theta, RopeType rope_type, int device_id) {
    const char* caller = "CudaRopeDevice";
    if (q.DeviceId() != device_id || k.DeviceId() != device_id) {
        Fail(caller, "q and k devices must match device_id");
    }
    if (pos < 0) Fail(caller, "pos must be non-negative");
    RequireTheta(theta, caller);
    RequireHeads(n_heads, n_kv_heads, head_dim, caller);
    if (q.NumEle() != static_cast<size_t>(n_heads) * static_cast<size_t>(head_dim)) {
        Fail(caller, "q element count must equal n_heads * head_dim");
    }
    if (k.NumEle() != static_cast<size_t>(n_kv_heads) * static_cast<size_t>(head_dim)) {
        Fail(caller, "k element count must equal n_kv_heads * head_dim");
    }
    SetCudaService(device_id);
    Launched(mlk_rope_f32(F(q), F(k), 1, n_heads, n_kv_heads, head_dim,
                          static_cast<int64_t>(n_heads) * head_dim,
                          static_cast<int64_t>(n_kv_heads) * head_dim, nullptr, pos, theta,
                          RopeCode(rope_type), nullptr, nullptr),
             caller);
}

// ------------------------------------------------ batched and fused entries

CudaTensor CudaAddRmsNormDevice(CudaTensor& residual, const CudaTensor* delta,
                                const void* weight_data, const std::vector<int>& weight_shape,
                                float eps, int device_id) {
    const char* caller = "CudaAddRmsNormDevice";
    const int64_t dim = RowWidth(residual, weight_data, weight_shape, device_id, caller);
    if (delta != nullptr) RequireSameShape(residual, *delta, caller);
    RequireEps(eps, caller);
    SetCudaService(device_id);
    CudaTensor y(residual.shape(), device_id);
    const int64_t rows = static_cast<int64_t>(residual.NumEle()) / dim;
    Launched(mlk_add_rmsnorm_f32(F(residual), delta != nullptr ? F(*delta) : nullptr,
                                 static_cast<const float*>(weight_data), F(y), rows, dim, eps,
                                 nullptr),
             caller);
    return y;
}

CudaTensor CudaRmsNormRowsDevice(const CudaTensor& x, const void* weight_data,
                                 const std::vector<int>& weight_shape, float eps, int device_id) {
    const char* caller = "CudaRmsNormRowsDevice";
    const int64_t dim = RowWidth(x, weight_data, weight_shape, device_id, caller);
    RequireEps(eps, caller);
    SetCudaService(device_id);
    CudaTensor y(x.shape(), device_id);
    Launched(mlk_rmsnorm_f32(F(x), static_cast<const float*>(weight_data), F(y),
                             static_cast<int64_t>(x.NumEle()) / dim, dim, eps, nullptr),
             caller);
    return y;
}

CudaTensor CudaSwiGluDevice(const CudaTensor& gate, const CudaTensor& up, int device_id) {
    const char* caller = "CudaSwiGluDevice";
    RequireElementwise(gate, device_id, caller);
    RequireElementwise(up, device_id, caller);
    RequireSameShape(gate, up, caller);
    SetCudaService(device_id);
    CudaTensor y(gate.shape(), device_id);
    Launched(mlk_swiglu_f32(F(gate), F(up), F(y), static_cast<int64_t>(gate.NumEle()), nullptr),
             caller);
    return y;
}

namespace {

void RopeBatch(const char* caller, CudaTensor& q, CudaTensor& k, int64_t n_tokens,
               const int32_t* positions, int pos0, int n_heads, int n_kv_heads, int head_dim,
               float theta, RopeType rope_type, int device_id) {
    if (q.DeviceId() != device_id || k.DeviceId() != device_id) {
        Fail(caller, "q and k devices must match device_id");
    }
    RequireTheta(theta, caller);
    RequireHeads(n_heads, n_kv_heads, head_dim, caller);
    const int64_t qw = static_cast<int64_t>(n_heads) * head_dim;
    const int64_t kw = static_cast<int64_t>(n_kv_heads) * head_dim;
    if (q.IsEmpty() || static_cast<int64_t>(q.NumEle()) != n_tokens * qw) {
        Fail(caller, "q element count must equal n_tokens * n_heads * head_dim");
    }
    if (k.IsEmpty() || static_cast<int64_t>(k.NumEle()) != n_tokens * kw) {
        Fail(caller, "k element count must equal n_tokens * n_kv_heads * head_dim");
    }
    SetCudaService(device_id);
    Launched(mlk_rope_f32(F(q), F(k), n_tokens, n_heads, n_kv_heads, head_dim, qw, kw, positions,
                          pos0, theta, RopeCode(rope_type), nullptr, nullptr),
             caller);
}

}  // namespace

void CudaRopeBatchDevice(CudaTensor& q, CudaTensor& k, const std::vector<int>& positions,
                         int n_heads, int n_kv_heads, int head_dim, float theta,
                         RopeType rope_type, int device_id) {
    const char* caller = "CudaRopeBatchDevice";
    if (positions.empty()) Fail(caller, "positions must not be empty");
    for (int p : positions) {
        if (p < 0) Fail(caller, "pos must be non-negative");
    }
    if (q.DeviceId() != device_id || k.DeviceId() != device_id) {
        Fail(caller, "q and k devices must match device_id");
    }
    SetCudaService(device_id);
    CudaDeviceBuffer dpos = UploadInts(positions, device_id);
    RopeBatch(caller, q, k, static_cast<int64_t>(positions.size()),
              static_cast<const int32_t*>(dpos.GetData()), 0, n_heads, n_kv_heads, head_dim, theta,
              rope_type, device_id);
}

void CudaRopeRangeDevice(CudaTensor& q, CudaTensor& k, int pos0, int n_heads, int n_kv_heads,
                         int head_dim, float theta, RopeType rope_type, int device_id) {
    const char* caller = "CudaRopeRangeDevice";
    if (pos0 < 0) Fail(caller, "pos must be non-negative");
    RequireHeads(n_heads, n_kv_heads, head_dim, caller);
    const int64_t qw = static_cast<int64_t>(n_heads) * head_dim;
    if (q.NumEle() == 0 || static_cast<int64_t>(q.NumEle()) % qw != 0) {
        Fail(caller, "q element count must be a positive multiple of n_heads * head_dim");
    }
    RopeBatch(caller, q, k, static_cast<int64_t>(q.NumEle()) / qw, nullptr, pos0, n_heads,
              n_kv_heads, head_dim, theta, rope_type, device_id);
}

CudaTensor CudaEmbeddingBatchDevice(const void* embedding_data, const std::vector<int>& shape,
                                    const std::vector<int>& token_ids, int device_id) {
    const char* caller = "CudaEmbeddingBatchDevice";
    RequireTable(embedding_data, shape, caller);
    RequireIds(token_ids, shape[0], caller);
    SetCudaService(device_id);
    // one id travels as a kernel argument (no copy, as CudaEmbeddingDevice);
    // more are copied to the device once
    const int n = static_cast<int>(token_ids.size());
    CudaDeviceBuffer ids = n > 1 ? UploadInts(token_ids, device_id) : CudaDeviceBuffer();
    CudaTensor y({n, shape[1]}, device_id);
    Launched(mlk_gather_f32(static_cast<const float*>(embedding_data), shape[0], shape[1],
                            static_cast<const int32_t*>(ids.GetData()), token_ids[0], n, F(y),
                            nullptr, nullptr),
             caller);
    return y;
}

CudaTensor CudaEmbeddingQuantDevice(const void* blocks, QuantType type,
                                    const std::vector<int>& shape,
                                    const std::vector<int>& token_ids, int device_id) {
    const char* caller = "CudaEmbeddingQuantDevice";
    const int32_t code = QuantCode(type, caller);
    RequireTable(blocks, shape, caller);
    RequireIds(token_ids, shape[0], caller);
    SetCudaService(device_id);
    const int n = static_cast<int>(token_ids.size());
    CudaDeviceBuffer ids = n > 1 ? UploadInts(token_ids, device_id) : CudaDeviceBuffer();
    CudaTensor y({n, shape[1]}, device_id);
    Launched(mlk_gather_quant(code, blocks, shape[0], shape[1],
                              static_cast<const int32_t*>(ids.GetData()), token_ids[0], n, F(y),
                              nullptr, nullptr),
             caller);
    return y;
}

CudaDeviceBuffer CudaQuantizeDevice(const CudaTensor& x, QuantType type, int device_id) {
    const char* caller = "CudaQuantizeDevice";
    const int32_t code = QuantCode(type, caller);
    if (x.IsEmpty() || x.NumEle() == 0) Fail(caller, "input tensor must not be empty");
    if (x.DeviceId() != device_id) Fail(caller, "input device must match device_id");
    const int64_t cols = x.shape().back();
    const int64_t rows = static_cast<int64_t>(x.NumEle()) / cols;
    SetCudaService(device_id);
    CudaDeviceBuffer out(static_cast<size_t>(mlk_quant_bytes(code, rows, cols)), device_id);
    Launched(mlk_quantize(code, F(x), rows, cols, out.GetData(), nullptr), caller);
    return out;
}
}  // namespace yan_lamma
