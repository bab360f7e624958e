// host_checks.h -- the argument checks the host types share (Tensor,
// CudaTensor, CudaDeviceBuffer, CudaCache).
//
// A failed check throws std::runtime_error (std::out_of_range for element
// indices, std::invalid_argument for an index vector of the wrong length)
// whose text is "<caller>: <reason>".  The reasons are the phrases callers
// and tests of the reference match on ("must be positive", "out of range",
// "overflow", "shape must not be empty", ...), so they are kept word for
// word; everything else about how a check runs is this library's own.
#pragma once
#include <cstddef>
#include <limits>
#include <stdexcept>
#include <string>
#include <vector>

namespace yan_lamma::hostcheck {

template <class Error = std::runtime_error>
[[noreturn]] inline void Raise(const std::string& caller, const std::string& reason) {
    throw Error(caller + ": " + reason);
}

// "[d0, d1, ...]", the shape notation of every message.
inline std::string ShapeText(const std::vector<int>& shape) {
    std::string text;
    for (int d : shape) text += (text.empty() ? "[" : ", ") + std::to_string(d);
    return text.empty() ? "[]" : text + "]";
}

// a * b for positive sizes, or a failure naming the operands.
inline size_t Product(size_t a, size_t b, const std::string& caller) {
    if (a == 0 || b == 0) {
        Raise(caller, "multiplication dimensions must be positive, got " + std::to_string(a) +
                          " and " + std::to_string(b));
    }
    if (a > std::numeric_limits<size_t>::max() / b) {
        Raise(caller, "size multiplication overflow for " + std::to_string(a) + " * " +
                          std::to_string(b));
    }
    return a * b;
}

// Element count of a shape whose every dimension must be positive.  An
// empty shape is a one-element scalar when `scalar_ok`, an error otherwise.
inline size_t ElementCount(const std::vector<int>& shape, const std::string& caller,
                           bool scalar_ok) {
    if (shape.empty() && !scalar_ok) Raise(caller, "shape must not be empty");
    size_t count = 1;
    for (size_t axis = 0; axis < shape.size(); ++axis) {
        const int d = shape[axis];
        if (d <= 0) {
            Raise(caller, "dimension at axis " + std::to_string(axis) +
                              " must be positive, got " + std::to_string(d) + " in shape " +
                              ShapeText(shape));
        }
        if (count > std::numeric_limits<size_t>::max() / static_cast<size_t>(d)) {
            Raise(caller, "shape element count overflow for " + ShapeText(shape));
        }
        count *= static_cast<size_t>(d);
    }
    return count;
}

// `index` in [0, limit), reported as "<noun> <index> out of range [0, limit)".
inline void InRange(int index, int limit, const std::string& caller, const char* noun) {
    if (index >= 0 && index < limit) return;
    Raise(caller, std::string(noun) + " " + std::to_string(index) + " out of range [0, " +
                      std::to_string(limit) + ")");
}

}  // namespace yan_lamma::hostcheck
