// test_support.h -- a tiny harness for the C++ op-surface tests.
//
// Same style as the reference's standalone CUDA validation tests
// (tests/test_utils.h, tests/cuda_test_support.h of the reference tree): a
// binary runs named cases, "PASS <case>" per success, "FAIL <case>: <why>"
// and exit status 1 on the first failure.  Expected values come from the CPU
// oracle (oracle/oracle.h), never from the code under test.
#pragma once
#include "include/cuda_attention.h"
#include "include/cuda_forward.h"
#include "include/cuda_kvcache.h"
#include "include/cuda_ops.h"
#include "oracle/oracle.h"

#include <cmath>
#include <cstring>
#include <cstdint>
#include <functional>
#include <iomanip>
#include <iostream>
#include <limits>
#include <sstream>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace mlk_test {
using yan_lamma::Tensor;

inline void Require(bool ok, const std::string& message) {
    if (!ok) throw std::runtime_error(message);
}

// |a - e| <= tol * max(1, |e|) for every element (tol 1e-5 is the north
// star's bar for RMSNorm / RoPE / SwiGLU; 0 means bit-exact).
inline void RequireClose(const std::vector<float>& actual, const std::vector<float>& expected,
                         const std::string& label, double tol = 1e-5) {
    Require(actual.size() == expected.size(), label + ": size mismatch");
    for (size_t i = 0; i < actual.size(); ++i) {
        const double a = actual[i], e = expected[i];
        const bool ok = tol == 0.0 ? (std::memcmp(&actual[i], &expected[i], sizeof(float)) == 0)
                                   : (std::isfinite(a) &&
                                      std::abs(a - e) <= tol * std::max(1.0, std::abs(e)));
        if (!ok) {
            std::ostringstream m;
            m << std::setprecision(std::numeric_limits<float>::max_digits10) << label
              << ": index=" << i << " actual=" << a << " expected=" << e;
            throw std::runtime_error(m.str());
        }
    }
}

inline void RequireTensor(const Tensor& actual, const Tensor& expected, const std::string& label,
                          double tol = 1e-5) {
    Require(actual.shape == expected.shape, label + ": shape " + actual.ShapeToString() + " vs " +
                                                expected.ShapeToString());
    RequireClose(actual.data, expected.data, label, tol);
}

// The operation must throw std::runtime_error whose text contains `text`.
template <class F>
void RequireError(F operation, const std::string& text) {
    bool caught = false;
    try {
        operation();
    } catch (const std::runtime_error& e) {
        caught = true;
        Require(std::string(e.what()).find(text) != std::string::npos,
                "wrong error: \"" + std::string(e.what()) + "\", expected \"" + text + "\"");
    }
    Require(caught, "expected an error containing: " + text);
}

// test/cuda_ops_test.cc:70-76 input pattern of the reference tests.
inline Tensor Values(const std::vector<int>& shape) {
    Tensor t(shape);
    for (size_t i = 0; i < t.data.size(); ++i) {
        t.data[i] = static_cast<float>(static_cast<int>(i % 29) - 14) / 7.0f;
    }
    return t;
}

// tests/test_cuda_ops.cc input pattern of the reference tests.
inline Tensor Waves(const std::vector<int>& shape, float phase = 0.0f) {
    Tensor t(shape);
    for (size_t i = 0; i < t.data.size(); ++i) {
        t.data[i] = std::sin(static_cast<float>(i) * 0.19f + phase) * 0.3f;
    }
    return t;
}

// Deterministic N(mean, std) values (xorshift + Box-Muller), for shapes
// where a smooth pattern would hide indexing mistakes.
inline Tensor Random(const std::vector<int>& shape, uint64_t seed, float mean = 0.0f,
                     float std = 1.0f) {
    Tensor t(shape);
    uint64_t s = seed * 0x9E3779B97F4A7C15ull + 1;
    auto next = [&s]() {
        s ^= s << 13;
        s ^= s >> 7;
        s ^= s << 17;
        return (static_cast<double>(s >> 11) + 0.5) / 9007199254740992.0;
    };
    for (size_t i = 0; i < t.data.size(); ++i) {
        const double u1 = next(), u2 = next();
        t.data[i] = static_cast<float>(mean + std * std::sqrt(-2.0 * std::log(u1)) *
                                                  std::cos(6.283185307179586 * u2));
    }
    return t;
}

using Case = std::pair<const char*, std::function<void()>>;

// Runs the cases named by argv[1] ("all" or one case name, or a group
// prefix such as "cpu" / "gpu").
inline int Run(int argc, char** argv, const std::vector<Case>& cases) {
    const std::string mode = argc > 1 ? argv[1] : "all";
    int ran = 0;
    for (const auto& c : cases) {
        const std::string name = c.first;
        if (mode != "all" && name != mode && name.rfind(mode + ".", 0) != 0) continue;
        try {
            std::cout << "RUN  " << name << std::endl;
            c.second();
            std::cout << "PASS " << name << std::endl;
            ++ran;
        } catch (const std::exception& e) {
            std::cout << "FAIL " << name << ": " << e.what() << std::endl;
            return 1;
        }
    }
    if (ran == 0) {
        std::cout << "FAIL no case matches " << mode << std::endl;
        return 1;
    }
    std::cout << "OK " << ran << " cases" << std::endl;
    return 0;
}
}  // namespace mlk_test
