// tensor.cc -- the host fp32 tensor (include/tensor.h), for builds of this
// library without the reference tree.  Inside the reference's build its own
// src/tensor.cc is linked instead; the op surface only constructs tensors.
//
// Behaviour callers rely on (the reference's src/tensor.cc): dimensions
// must be positive and their product must fit size_t (an empty shape is a
// scalar); element accessors check the rank (std::runtime_error) and every
// index (std::out_of_range); SwitchIdex rejects an index vector of the
// wrong length with std::invalid_argument.  Every element access goes
// through one offset routine here.
#include "include/tensor.h"

#include "host_checks.h"

#include <initializer_list>
#include <iomanip>
#include <iostream>
#include <sstream>
#include <stdexcept>
#include <string>

namespace yan_lamma {
namespace {
using hostcheck::Raise;
using hostcheck::ShapeText;

std::string NameOf(const char* call) { return call != nullptr ? call : "Tensor"; }

// Row-major offset of one index per axis, after checking the index count
// against the rank and each index against its axis.
template <class Indices>
size_t Offset(const Tensor& t, const Indices& idx, const std::string& caller) {
    size_t flat = 0;
    size_t axis = 0;
    for (const int i : idx) {
        const int extent = t.shape[axis];
        if (i < 0 || i >= extent) {
            Raise<std::out_of_range>(caller, "index " + std::to_string(i) + " out of range for axis " +
                                                 std::to_string(axis) + " with size " +
                                                 std::to_string(extent) + " in tensor " +
                                                 t.ShapeToString());
        }
        flat = flat * static_cast<size_t>(extent) + static_cast<size_t>(i);
        ++axis;
    }
    return flat;
}

// The AtN accessors: the rank must be exactly N.
size_t Element(const Tensor& t, std::initializer_list<int> idx, const char* caller) {
    if (t.shape.size() != idx.size()) {
        Raise(caller, "expected " + std::to_string(idx.size()) + "D tensor, got " +
                          t.ShapeToString());
    }
    return Offset(t, idx, caller);
}

size_t RowStart(const Tensor& t, int row) {
    const char* caller = "Tensor::RowPtr";
    if (t.shape.size() != 2) Raise(caller, "expected 2D tensor, got " + t.ShapeToString());
    return Offset(t, std::initializer_list<int>{row}, caller) * static_cast<size_t>(t.shape[1]);
}

}  // namespace

Tensor::Tensor(const std::vector<int>& data_shape, float default_data) : shape(data_shape) {
    data.assign(hostcheck::ElementCount(shape, "Tensor::Tensor", /*scalar_ok=*/true),
                default_data);
}

size_t Tensor::SwitchIdex(const std::vector<int>& indices) const {
    if (indices.size() != shape.size()) {
        throw std::invalid_argument("Tensor::SwitchIdex expected " +
                                    std::to_string(shape.size()) + " indices for tensor " +
                                    ShapeToString() + ", got " + std::to_string(indices.size()));
    }
    return Offset(*this, indices, "Tensor::SwitchIdex");
}

float Tensor::At1(int i) const { return data[Element(*this, {i}, "Tensor::At1")]; }
float& Tensor::At1(int i) { return data[Element(*this, {i}, "Tensor::At1")]; }
float Tensor::At2(int i, int j) const { return data[Element(*this, {i, j}, "Tensor::At2")]; }
float& Tensor::At2(int i, int j) { return data[Element(*this, {i, j}, "Tensor::At2")]; }
float Tensor::At3(int i, int j, int k) const {
    return data[Element(*this, {i, j, k}, "Tensor::At3")];
}
float& Tensor::At3(int i, int j, int k) { return data[Element(*this, {i, j, k}, "Tensor::At3")]; }
float Tensor::At4(int i, int j, int k, int m) const {
    return data[Element(*this, {i, j, k, m}, "Tensor::At4")];
}
float& Tensor::At4(int i, int j, int k, int m) {
    return data[Element(*this, {i, j, k, m}, "Tensor::At4")];
}

float* Tensor::RowPtr(int row) { return data.data() + RowStart(*this, row); }
const float* Tensor::RowPtr(int row) const { return data.data() + RowStart(*this, row); }

void Tensor::AssertShape(const std::vector<int>& expected, const char* call) {
    if (shape == expected) return;
    Raise(NameOf(call), "expected " + ShapeText(expected) + ", got " + ShapeToString());
}

Tensor Tensor::Reshape(const std::vector<int>& new_shape, const char* call) {
    const std::string caller = NameOf(call);
    const size_t count = hostcheck::ElementCount(new_shape, caller, /*scalar_ok=*/true);
    if (count != data.size()) {
        Raise(caller, "cannot reshape " + ShapeToString() + " with " + std::to_string(data.size()) +
                          " elements to " + ShapeText(new_shape) + " with " +
                          std::to_string(count) + " elements");
    }
    Tensor view;
    view.shape = new_shape;
    view.data = data;
    return view;
}

std::string Tensor::ShapeToString() const { return ShapeText(shape); }

void Tensor::Print(const std::string& name, bool print_data) const {
    std::ostringstream line;
    line << name << ShapeToString() << ' ' << shape.size() << '\n';
    if (print_data) {
        line << std::fixed << std::setprecision(6);
        const char* sep = "";
        for (float v : data) {
            line << sep << v;
            sep = " ";
        }
    }
    std::cout << line.str() << std::endl;
}

Tensor Tensor::MakeOneD(int i, float default_data) { return Tensor({i}, default_data); }
Tensor Tensor::MakeSecondD(int i, int j, float default_data) {
    return Tensor({i, j}, default_data);
}
Tensor Tensor::MakeThirdD(int i, int j, int k, float default_data) {
    return Tensor({i, j, k}, default_data);
}
Tensor Tensor::MakeFouthD(int i, int j, int k, int m, float default_data) {
    return Tensor({i, j, k, m}, default_data);
}
}  // namespace yan_lamma
