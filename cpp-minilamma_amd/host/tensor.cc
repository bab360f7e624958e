// tensor.cc -- host fp32 tensor (include/tensor.h).
//
// Shapes must have positive dimensions and element counts that fit size_t;
// element accessors validate rank and every index and throw
// std::out_of_range / std::runtime_error with the caller's name, as the
// reference's host tensor does (src/tensor.cc of the reference tree).
#include "include/tensor.h"

#include <iomanip>
#include <iostream>
#include <limits>
#include <stdexcept>
#include <string>

namespace yan_lamma {
namespace {

std::string Join(const std::vector<int>& shape) {
    std::string s = "[";
    for (size_t i = 0; i < shape.size(); ++i) {
        if (i) s += ", ";
        s += std::to_string(shape[i]);
    }
    return s + "]";
}

std::string Who(const char* call) { return call == nullptr ? "Tensor" : call; }

size_t Numel(const std::vector<int>& shape, const char* call) {
    size_t total = 1;
    for (size_t axis = 0; axis < shape.size(); ++axis) {
        const int d = shape[axis];
        if (d <= 0) {
            throw std::runtime_error(Who(call) + ": dimension at axis " + std::to_string(axis) +
                                     " must be positive, got " + std::to_string(d) +
                                     " in shape " + Join(shape));
        }
        if (total > std::numeric_limits<size_t>::max() / static_cast<size_t>(d)) {
            throw std::runtime_error(Who(call) + ": shape element count overflow for " +
                                     Join(shape));
        }
        total *= static_cast<size_t>(d);
    }
    return total;
}

void Rank(const Tensor& t, size_t rank, const char* call) {
    if (t.GetNumDims() != rank) {
        throw std::runtime_error(Who(call) + ": expected " + std::to_string(rank) +
                                 "D tensor, got " + t.ShapeToString());
    }
}

void Index(const Tensor& t, int index, size_t axis, const char* call) {
    if (axis >= t.GetNumDims()) {
        throw std::out_of_range(Who(call) + ": axis " + std::to_string(axis) +
                                " out of range for tensor " + t.ShapeToString());
    }
    const int size = t.shape[axis];
    if (index < 0 || index >= size) {
        throw std::out_of_range(Who(call) + ": index " + std::to_string(index) +
                                " out of range for axis " + std::to_string(axis) + " with size " +
                                std::to_string(size) + " in tensor " + t.ShapeToString());
    }
}

size_t Flat(const Tensor& t, std::initializer_list<int> idx, const char* call) {
    Rank(t, idx.size(), call);
    size_t flat = 0;
    size_t axis = 0;
    for (int i : idx) {
        Index(t, i, axis, call);
        flat = flat * static_cast<size_t>(t.shape[axis]) + static_cast<size_t>(i);
        ++axis;
    }
    return flat;
}

}  // namespace

Tensor::Tensor(const std::vector<int>& data_shape, float default_data) : shape(data_shape) {
    data.assign(Numel(shape, "Tensor::Tensor"), default_data);
}

std::size_t Tensor::SwitchIdex(const std::vector<int>& indices) const {
    if (indices.size() != GetNumDims()) {
        throw std::invalid_argument("Tensor::SwitchIdex expected " +
                                    std::to_string(shape.size()) + " indices for tensor " +
                                    ShapeToString() + ", got " + std::to_string(indices.size()));
    }
    size_t flat = 0;
    for (size_t axis = 0; axis < shape.size(); ++axis) {
        Index(*this, indices[axis], axis, "Tensor::SwitchIdex");
        flat = flat * static_cast<size_t>(shape[axis]) + static_cast<size_t>(indices[axis]);
    }
    return flat;
}

float Tensor::At1(int i) const { return data[Flat(*this, {i}, "Tensor::At1")]; }
float& Tensor::At1(int i) { return data[Flat(*this, {i}, "Tensor::At1")]; }
float Tensor::At2(int i, int j) const { return data[Flat(*this, {i, j}, "Tensor::At2")]; }
float& Tensor::At2(int i, int j) { return data[Flat(*this, {i, j}, "Tensor::At2")]; }
float Tensor::At3(int i, int j, int k) const {
    return data[Flat(*this, {i, j, k}, "Tensor::At3")];
}
float& Tensor::At3(int i, int j, int k) { return data[Flat(*this, {i, j, k}, "Tensor::At3")]; }
float Tensor::At4(int i, int j, int k, int m) const {
    return data[Flat(*this, {i, j, k, m}, "Tensor::At4")];
}
float& Tensor::At4(int i, int j, int k, int m) {
    return data[Flat(*this, {i, j, k, m}, "Tensor::At4")];
}

float* Tensor::RowPtr(int row) {
    Rank(*this, 2, "Tensor::RowPtr");
    Index(*this, row, 0, "Tensor::RowPtr");
    return data.data() + static_cast<size_t>(row) * static_cast<size_t>(shape[1]);
}

const float* Tensor::RowPtr(int row) const {
    Rank(*this, 2, "Tensor::RowPtr");
    Index(*this, row, 0, "Tensor::RowPtr");
    return data.data() + static_cast<size_t>(row) * static_cast<size_t>(shape[1]);
}

void Tensor::AssertShape(const std::vector<int>& expected, const char* call) {
    if (shape != expected) {
        throw std::runtime_error(Who(call) + ": expected " + Join(expected) + ", got " +
                                 ShapeToString());
    }
}

Tensor Tensor::Reshape(const std::vector<int>& new_shape, const char* call) {
    const size_t total = Numel(new_shape, call);
    if (total != data.size()) {
        throw std::runtime_error(Who(call) + ": cannot reshape " + ShapeToString() + " with " +
                                 std::to_string(data.size()) + " elements to " +
                                 Join(new_shape) + " with " + std::to_string(total) +
                                 " elements");
    }
    Tensor r = *this;
    r.shape = new_shape;
    return r;
}

std::string Tensor::ShapeToString() const { return Join(shape); }

void Tensor::Print(const std::string& name, bool print_data) const {
    std::cout << name << ShapeToString() << " " << GetNumDims() << "\n";
    if (print_data) {
        for (size_t i = 0; i < data.size(); ++i) {
            std::cout << std::fixed << std::setprecision(6) << data[i]
                      << (i + 1 < data.size() ? " " : "");
        }
    }
    std::cout << std::endl;
}

Tensor Tensor::MakeOneD(int i, float v) { return Tensor({i}, v); }
Tensor Tensor::MakeSecondD(int i, int j, float v) { return Tensor({i, j}, v); }
Tensor Tensor::MakeThirdD(int i, int j, int k, float v) { return Tensor({i, j, k}, v); }
Tensor Tensor::MakeFouthD(int i, int j, int k, int m, float v) { return Tensor({i, j, k, m}, v); }
}  // namespace yan_lamma
