// cuda_tensor.cc -- move-only fp32 device tensor (include/cuda_tensor.h).
//
// A CudaTensor is a shape, a device id, an element count and one device
// buffer; all four change together or not at all.  Behaviour callers rely
// on (the reference's src/cuda_tensor.cc): shapes are non-empty with
// positive dimensions, a failed Reset leaves the tensor as it was, Reshape
// keeps the allocation and the element count, uploads and downloads need a
// non-empty tensor and a host tensor of exactly its shape.  Messages keep
// the reference's caller names and phrases, which its tests match on.
#include "include/cuda_tensor.h"

#include "host_checks.h"

#include <stdexcept>
#include <string>
#include <utility>

namespace yan_lamma {
namespace {
using hostcheck::Raise;
using hostcheck::ShapeText;

// The checks shared by UploadFromHost and DownloadToHost: a device tensor to
// copy with, and a host tensor of the same shape and length.
void CheckHostPeer(const CudaTensor& dev, const Tensor& host, const char* caller,
                   const char* verb) {
    if (dev.IsEmpty()) Raise(caller, std::string("cannot ") + verb + " an empty tensor");
    if (host.shape != dev.shape()) {
        Raise(caller, "expected host shape " + ShapeText(dev.shape()) + ", got " +
                          ShapeText(host.shape));
    }
    if (host.data.size() != dev.NumEle()) {
        Raise(caller, "expected " + std::to_string(dev.NumEle()) + " host elements, got " +
                          std::to_string(host.data.size()));
    }
}

}  // namespace

CudaTensor::CudaTensor(const std::vector<int>& shape, int device_id) { Reset(shape, device_id); }

CudaTensor::CudaTensor(CudaTensor&& other) noexcept {
    // *this starts as a default tensor; exchanging leaves `other` as one.
    shape_.swap(other.shape_);
    std::swap(device_id_, other.device_id_);
    std::swap(numel_, other.numel_);
    std::swap(cuda_buffer_, other.cuda_buffer_);
}

CudaTensor& CudaTensor::operator=(CudaTensor&& other) noexcept {
    if (this != &other) {
        CudaTensor previous(std::move(*this));  // released when it goes out of scope
        CudaTensor incoming(std::move(other));
        shape_.swap(incoming.shape_);
        std::swap(device_id_, incoming.device_id_);
        std::swap(numel_, incoming.numel_);
        std::swap(cuda_buffer_, incoming.cuda_buffer_);
    }
    return *this;
}

void CudaTensor::Reset() {
    CudaTensor previous(std::move(*this));
    previous.cuda_buffer_.ReSet();  // release now, so a failure is reported
}

void CudaTensor::Reset(const std::vector<int>& shape, int device_id) {
    // Build the new state completely (this may throw), then take it over.
    CudaTensor fresh;
    fresh.numel_ = hostcheck::ElementCount(shape, "CudaTensor::Reset", /*scalar_ok=*/false);
    fresh.cuda_buffer_.Reset(fresh.numel_ * sizeof(float), device_id);
    fresh.shape_ = shape;
    fresh.device_id_ = device_id;
    *this = std::move(fresh);
}

void CudaTensor::Reshape(const std::vector<int>& shape) {
    const size_t count =
        hostcheck::ElementCount(shape, "CudaTensor::Reshape", /*scalar_ok=*/false);
    if (IsEmpty() || count != numel_) {
        Raise("CudaTensor::Reshape", "element count must remain unchanged on a non-empty tensor");
    }
    shape_ = shape;
}

void CudaTensor::UploadFromHost(const Tensor& src) {
    CheckHostPeer(*this, src, "CudaTensor::UploadFromHost", "upload to");
    cuda_buffer_.upload(src.data.data(), Bytes());
}

void CudaTensor::DownloadToHost(Tensor& dst) const {
    CheckHostPeer(*this, dst, "CudaTensor::DownloadToHost", "download");
    cuda_buffer_.download(dst.data.data(), Bytes());
}

Tensor CudaTensor::Download() const {
    if (IsEmpty()) Raise("CudaTensor::Download", "cannot download an empty tensor");
    Tensor host(shape_);
    cuda_buffer_.download(host.data.data(), Bytes());
    return host;
}

void* CudaTensor::GetData() { return cuda_buffer_.GetData(); }
const void* CudaTensor::GetData() const { return cuda_buffer_.GetData(); }
bool CudaTensor::IsEmpty() const { return cuda_buffer_.IsEmpty(); }
size_t CudaTensor::NumEle() const { return numel_; }
int CudaTensor::num_dims() const { return static_cast<int>(shape_.size()); }
size_t CudaTensor::Bytes() const { return cuda_buffer_.GetByteSize(); }
int CudaTensor::DeviceId() const { return device_id_; }
std::string CudaTensor::ShapeStringShort() const { return ShapeText(shape_); }
const CudaDeviceBuffer& CudaTensor::buffer() const { return cuda_buffer_; }
const std::vector<int>& CudaTensor::shape() const { return shape_; }

CudaTensor TensorHostToDevice(const Tensor& src, int device_id) {
    CudaTensor dev(src.shape, device_id);
    dev.UploadFromHost(src);
    return dev;
}
}  // namespace yan_lamma
