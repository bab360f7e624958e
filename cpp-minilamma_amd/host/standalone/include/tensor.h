// tensor.h -- stand-in for the reference's host tensor header, used only when
// this library is built on its own (this directory comes after the
// repository root on the include path, so inside the reference tree its own
// include/tensor.h is found instead).  Same declarations and member layout
// as the reference (include/tensor.h:6-41 of the reference tree), so the
// op-surface library links against either cpp-minilamma_amd/host/tensor.cc
// or the reference's own src/tensor.cc.
#pragma once
#include <cstddef>
#include <string>
#include <vector>

namespace yan_lamma {
struct Tensor {
    std::vector<float> data;
    std::vector<int> shape;
    Tensor() = default;
    // Every dimension must be positive; storage is filled with default_data.
    explicit Tensor(const std::vector<int>& data_shape, float default_data = 0.0f);
    std::size_t GetDataSize() const { return data.size(); }
    std::size_t GetNumDims() const { return shape.size(); }
    // Checked element access (rank and every index are validated).
    float At1(int i) const;
    float& At1(int i);
    float At2(int i, int j) const;
    float& At2(int i, int j);
    float At3(int i, int j, int k) const;
    float& At3(int i, int j, int k);
    float At4(int i, int j, int k, int m) const;
    float& At4(int i, int j, int k, int m);
    float* RowPtr(int row);
    const float* RowPtr(int row) const;
    // Row-major flat index of a full index vector.
    std::size_t SwitchIdex(const std::vector<int>& indices) const;
    float& operator[](std::size_t i) { return data[i]; }
    float operator[](std::size_t i) const { return data[i]; }
    void AssertShape(const std::vector<int>& expected, const char* call);
    Tensor Reshape(const std::vector<int>& new_shape, const char* call);
    std::string ShapeToString() const;
    void Print(const std::string& name = "", bool print_data = true) const;
    Tensor MakeOneD(int i, float default_data = 0.0f);
    Tensor MakeSecondD(int i, int j, float default_data = 0.0f);
    Tensor MakeThirdD(int i, int j, int k, float default_data = 0.0f);
    Tensor MakeFouthD(int i, int j, int k, int m, float default_data = 0.0f);
};
}  // namespace yan_lamma
