// test_cuda_ops.cc -- the C++ op surface (include/cuda_ops.h) against the
// CPU oracle, in the shape of the reference's own tests
// (test/cuda_ops_test.cc and tests/test_cuda_ops.cc of the reference tree).
//
//   test_cuda_ops cpu   argument checks that fail before any device work
//                       (runs without a GPU)
//   test_cuda_ops gpu   everything else, on device 0
#include "tests/cpp/test_support.h"

#include <algorithm>
#include <cstring>
#include <memory>

using namespace yan_lamma;
using namespace mlk_test;

namespace {

// ------------------------------------------------------ oracle wrappers

Tensor OracleRms(const Tensor& x, const Tensor& w, float eps) {
    Tensor y(x.shape);
    const int64_t dim = w.data.size();
    Require(orc_rmsnorm_row(x.data.data(), w.data.data(), y.data.data(), dim, eps) == ORC_OK,
            "oracle rmsnorm rejected its input");
    return y;
}

Tensor OracleSilu(const Tensor& x) {
    Tensor y(x.shape);
    orc_silu(x.data.data(), y.data.data(), x.data.size());
    return y;
}

Tensor OracleBinary(void (*f)(const float*, const float*, float*, int64_t), const Tensor& a,
                    const Tensor& b) {
    Tensor y(a.shape);
    f(a.data.data(), b.data.data(), y.data.data(), a.data.size());
    return y;
}

Tensor OracleSoftmax(const Tensor& x) {
    Tensor y(x.shape);
    Require(orc_softmax(x.data.data(), y.data.data(), x.data.size()) == ORC_OK, "oracle softmax");
    return y;
}

// q [T, H * hd], k [T, KV * hd] rotated per token.
std::pair<Tensor, Tensor> OracleRope(Tensor q, Tensor k, int H, int KV, int hd,
                                     const std::vector<int>& pos, float theta, RopeType type) {
    Require(orc_rope(q.data.data(), k.data.data(), static_cast<int64_t>(pos.size()), H, KV, hd,
                     pos.data(), 0, theta, type == kNormal ? ORC_ROPE_NORMAL : ORC_ROPE_NEOX) ==
                ORC_OK,
            "oracle rope");
    return {q, k};
}

int QuantIndex(QuantType t) { return t == QuantType::kQ80 ? 0 : (t == QuantType::kQ40 ? 1 : 2); }

std::vector<uint8_t> OracleQuantize(QuantType t, const Tensor& x) {
    const int64_t cols = x.shape.back(), rows = x.data.size() / cols;
    const int64_t bb = t == QuantType::kQ80 ? 34 : (t == QuantType::kQ40 ? 18 : 20);
    std::vector<uint8_t> out(rows * ((cols + 31) / 32) * bb);
    int rc = t == QuantType::kQ80   ? orc_quantize_q8_0(x.data.data(), rows, cols, out.data())
             : t == QuantType::kQ40 ? orc_quantize_q4_0(x.data.data(), rows, cols, out.data())
                                    : orc_quantize_q4_1(x.data.data(), rows, cols, out.data());
    Require(rc == ORC_OK, "oracle quantize");
    return out;
}

std::vector<uint8_t> Bytes(const CudaDeviceBuffer& b) {
    std::vector<uint8_t> out(b.GetByteSize());
    b.download(out.data(), out.size());
    return out;
}

// ------------------------------------------------------------- cpu cases

void CpuBuildPredicate() { Require(CudaopsBuild() == CudaRuntimeBuilt(), "build predicates"); }

// test/cuda_ops_test.cc:212-295: the checks that run before any device work.
void CpuRejectsInvalidInputs() {
    const Tensor x = Values({4}), weight = Values({4}), other = Values({3});
    const Tensor matrix = Values({2, 2});
    Tensor empty;
    empty.shape = {0};
    int host_word = 0;
    const void* fake = &host_word;  // never dereferenced: validation fails first
    RequireError([&] { (void)CudaEmbeddingDevice(nullptr, {3, 4}, 0); }, "must not be null");
    RequireError([&] { (void)CudaEmbeddingDevice(fake, {12}, 0); }, "expected weight shape");
    RequireError([&] { (void)CudaEmbeddingDevice(fake, {0, 4}, 0); }, "must be positive");
    RequireError([&] { (void)CudaEmbeddingDevice(fake, {3, 0}, 0); }, "must be positive");
    RequireError([&] { (void)CudaEmbeddingDevice(fake, {3, 4}, -1); }, "token_id must be in");
    RequireError([&] { (void)CudaEmbeddingDevice(fake, {3, 4}, 3); }, "token_id must be in");
    for (float eps : {0.0f, -1.0f, std::numeric_limits<float>::infinity(),
                      std::numeric_limits<float>::quiet_NaN()}) {
        RequireError([&] { (void)CudaRmsNormHost(x, weight, eps); }, "eps must be finite");
    }
    RequireError([&] { (void)CudaRmsNormHost(matrix, weight, 1e-5f); }, "expected a 1D");
    RequireError([&] { (void)CudaRmsNormHost(x, matrix, 1e-5f); }, "expected a 1D");
    RequireError([&] { (void)CudaRmsNormHost(x, other, 1e-5f); }, "shapes must match");
    RequireError([&] { (void)CudaRmsNormHost(empty, empty, 1e-5f); }, "must not be empty");
    const CudaTensor empty_device;
    RequireError([&] { (void)CudaRmsNromDevice(empty_device, fake, {4}, 1e-5f); },
                 "expected a 1D");
    Tensor m = matrix;
    RequireError([&] { (void)CudaSoftmax(m); }, "expected a 1D");
    RequireError([&] { (void)CudaSoftmax(empty); }, "must not be empty");
    RequireError([&] { (void)CudaElementwiseMul(x, matrix); }, "shapes must match");
    Tensor q = Values({2, 4}), k = Values({1, 4}), v = Values({4}), odd = Values({1, 3});
    Tensor mismatch = Values({1, 6});
    for (RopeType t : {kNormal, kNeoX}) {
        RequireError([&] { CudaRopeHost(v, k, 0, 10000.0f, t); }, "expected 2D");
        RequireError([&] { CudaRopeHost(q, v, 0, 10000.0f, t); }, "expected 2D");
        RequireError([&] { CudaRopeHost(odd, odd, 0, 10000.0f, t); }, "must be even");
        RequireError([&] { CudaRopeHost(q, mismatch, 0, 10000.0f, t); }, "must match");
        RequireError([&] { CudaRopeHost(q, k, -1, 10000.0f, t); }, "non-negative");
        for (float theta : {0.0f, -1.0f, std::numeric_limits<float>::infinity(),
                            std::numeric_limits<float>::quiet_NaN()}) {
            RequireError([&] { CudaRopeHost(q, k, 0, theta, t); }, "theta must be finite");
        }
    }
    CudaTensor dq, dk;
    RequireError([&] { CudaRopeDevice(dq, dk, 0, 1, 1, 4, 10000.0f, kNormal, 1); },
                 "devices must match");
    RequireError([&] { CudaRopeDevice(dq, dk, -1, 1, 1, 4, 10000.0f); }, "non-negative");
    RequireError([&] { CudaRopeDevice(dq, dk, 0, 0, 1, 4, 10000.0f); }, "head_dim must be");
    RequireError([&] { CudaRopeDevice(dq, dk, 0, 1, 1, 3, 10000.0f); }, "head_dim must be");
    RequireError([&] { CudaRopeDevice(dq, dk, 0, 1, 1, 4, 10000.0f); }, "element count");
    RequireError([&] { (void)CudaEmbeddingBatchDevice(fake, {3, 4}, {0, 3}); },
                 "token_id must be in");
    RequireError([&] { (void)CudaEmbeddingBatchDevice(fake, {3, 4}, {}); }, "must not be empty");
    RequireError([&] { (void)CudaEmbeddingQuantDevice(fake, QuantType::kF32, {3, 32}, {0}); },
                 "unsupported quantization type");
    RequireError([&] { CudaRopeBatchDevice(dq, dk, {0, -2}, 1, 1, 4, 1e4f); }, "non-negative");
    RequireError([&] { (void)CudaAddRmsNormDevice(dq, nullptr, fake, {4}, 1e-5f); },
                 "must not be empty");
    RequireError([&] { (void)CudaQuantizeDevice(dq, QuantType::kQ80); }, "must not be empty");
}

void CpuTensorChecks() {
    RequireError([] { Tensor t({2, 0}); }, "must be positive");
    Tensor t = Values({2, 3});
    Require(t.At2(1, 2) == t.data[5], "At2 indexing");
    bool threw = false;
    try {
        (void)t.At2(2, 0);
    } catch (const std::out_of_range&) {
        threw = true;
    }
    Require(threw, "At2 bounds");
    RequireError([&] { (void)t.Reshape({4, 2}, "Reshape"); }, "cannot reshape");
    Require(t.Reshape({3, 2}, "Reshape").shape == std::vector<int>({3, 2}), "reshape shape");
    Require(t.SwitchIdex({1, 1}) == 4, "flat index");
    RequireError([] { CudaTensor c({3, -1}); }, "must be positive");
}

// ------------------------------------------------------------- gpu cases

void GpuDeviceInfo() {
    Require(DeviceCount() > 0, "a GPU is required for the gpu cases");
    const struct CudaInfo info = GetCudaInfo(0);
    std::cout << "  " << CudaInfo(info) << std::endl;
    Require(info.total_bytes > 0, "device memory size");
    bool threw = false;
    try {
        (void)GetCudaInfo(DeviceCount());
    } catch (const std::runtime_error&) {
        threw = true;
    }
    Require(threw, "an absent device is rejected");
}

// test/cuda_ops_test.cc:91-103 and tests/test_cuda_ops.cc:27-30.
void GpuEmbedding() {
    const Tensor weight = Values({3, 259});
    CudaDeviceBuffer buffer(weight.data.size() * sizeof(float));
    buffer.upload(weight.data.data(), weight.data.size() * sizeof(float));
    for (int token : {0, 2}) {
        Tensor expected({259});
        std::copy_n(weight.data.begin() + token * 259, 259, expected.data.begin());
        const CudaTensor y = CudaEmbeddingDevice(buffer.GetData(), weight.shape, token);
        Require(y.DeviceId() == 0, "device id");
        RequireTensor(y.Download(), expected, "embedding", 0.0);
    }
    const Tensor table = Random({131, 64}, 7, 0.0f, 0.02f);
    const CudaTensor d = TensorHostToDevice(table);
    const std::vector<int> ids{0, 1, 130, 128, 104, 101, 108};
    const CudaTensor rows = CudaEmbeddingBatchDevice(d.GetData(), table.shape, ids);
    Tensor expected({static_cast<int>(ids.size()), 64});
    Require(orc_gather_f32(table.data.data(), 131, 64, ids.data(), ids.size(),
                           expected.data.data()) == ORC_OK,
            "oracle gather");
    RequireTensor(rows.Download(), expected, "batched embedding", 0.0);
    // one id goes to the kernel as an argument: no host-to-device copy; more
    // ids take one copy of 4 T bytes
    for (const std::vector<int>& few : {std::vector<int>{130}, std::vector<int>{5, 9}}) {
        CudaTransferStats stats;
        CudaTensor got;
        {
            CudaStatsScope scope(&stats);
            got = CudaEmbeddingBatchDevice(d.GetData(), table.shape, few);
        }
        const bool one = few.size() == 1;
        Require(stats.host_to_device_copies == (one ? 0u : 1u) &&
                    stats.host_to_device_bytes == (one ? 0u : 4 * few.size()),
                "batched embedding host-to-device copies");
        Tensor want({static_cast<int>(few.size()), 64});
        Require(orc_gather_f32(table.data.data(), 131, 64, few.data(), few.size(),
                               want.data.data()) == ORC_OK, "oracle gather");
        RequireTensor(got.Download(), want, "batched embedding of few ids", 0.0);
    }
}

// test/cuda_ops_test.cc:105-126.
void GpuRmsNorm() {
    for (int n : {1, 7, 259, 1025}) {
        for (bool zero : {false, true}) {
            Tensor x = Values({n});
            if (zero) std::fill(x.data.begin(), x.data.end(), 0.0f);
            const Tensor weight = Values({n});
            const auto original = x.data;
            const Tensor expected = OracleRms(x, weight, 1e-5f);
            RequireTensor(CudaRmsNormHost(x, weight, 1e-5f), expected, "host rmsnorm");
            const CudaTensor dx = TensorHostToDevice(x);
            const CudaTensor dw = TensorHostToDevice(weight);
            const CudaTensor y = CudaRmsNromDevice(dx, dw.GetData(), weight.shape, 1e-5f);
            Require(y.DeviceId() == 0, "device id");
            RequireTensor(y.Download(), expected, "device rmsnorm");
            Require(x.data == original, "host input unchanged");
            RequireTensor(dx.Download(), x, "device input unchanged", 0.0);
        }
    }
}

// test/cuda_ops_test.cc:128-153 and tests/test_cuda_ops.cc:5-23.
void GpuElementwise() {
    for (const auto& shape :
         {std::vector<int>{1}, std::vector<int>{86}, std::vector<int>{259}, std::vector<int>{3, 173}}) {
        Tensor a = Values(shape), b = Values(shape);
        for (float& v : b.data) v = 0.5f - v;
        const auto oa = a.data, ob = b.data;
        RequireTensor(CudaSilu(a), OracleSilu(a), "host silu");
        RequireTensor(CudaElementwiseMul(a, b), OracleBinary(orc_mul, a, b), "host mul", 0.0);
        const CudaTensor da = TensorHostToDevice(a), db = TensorHostToDevice(b);
        RequireTensor(CudaSiluDevice(da).Download(), OracleSilu(a), "device silu");
        RequireTensor(CudaElementwiseMulDevice(da, db).Download(), OracleBinary(orc_mul, a, b),
                      "device mul", 0.0);
        const Tensor sum = OracleBinary(orc_add, a, b);
        RequireTensor(CudaElementAddDevice(da, db).Download(), sum, "add", 0.0);
        RequireTensor(OCudaElementAddDevice(da, db.GetData(), shape).Download(), sum, "bias add",
                      0.0);
        RequireTensor(CudaSwiGluDevice(da, db).Download(), OracleBinary(orc_swiglu, a, b),
                      "fused swiglu");
        RequireTensor(da.Download(), a, "a unchanged", 0.0);
        RequireTensor(db.Download(), b, "b unchanged", 0.0);
        Require(a.data == oa && b.data == ob, "host inputs unchanged");
    }
    const CudaTensor a = TensorHostToDevice(Values({4})), b = TensorHostToDevice(Values({2, 2}));
    RequireError([&] { (void)CudaElementAddDevice(a, b); }, "shapes must match");
    RequireError([&] { (void)OCudaElementAddDevice(a, nullptr, {4}); }, "must not be null");
    RequireError([&] { (void)OCudaElementAddDevice(a, b.GetData(), {2, 2}); }, "must match");
    RequireError([&] { (void)CudaElementAddDevice(a, a, 1); }, "device must match");
    RequireError([&] { (void)CudaSwiGluDevice(a, b); }, "shapes must match");
}

// test/cuda_ops_test.cc:155-183.
void GpuSoftmax() {
    std::vector<Tensor> cases;
    for (const auto& v : {std::vector<float>{3.0f}, std::vector<float>{2.0f, 2.0f, 2.0f},
                          std::vector<float>{-5.0f, -2.0f, -9.0f},
                          std::vector<float>{10000.0f, 10001.0f, -10000.0f},
                          std::vector<float>{-1000, 0, 1000, 999, -999}}) {
        Tensor x({static_cast<int>(v.size())});
        x.data = v;
        cases.push_back(x);
    }
    cases.push_back(Values({259}));
    cases.push_back(Values({1025}));
    for (Tensor& x : cases) {
        const auto original = x.data;
        const Tensor y = CudaSoftmax(x);
        RequireTensor(y, OracleSoftmax(x), "softmax");
        double total = 0.0;
        for (float v : y.data) {
            Require(v >= 0.0f, "non-negative");
            total += v;
        }
        Require(std::abs(total - 1.0) <= 1e-5, "sums to one");
        Require(x.data == original, "input unchanged");
    }
}

// test/cuda_ops_test.cc:185-210 and tests/test_cuda_ops.cc:32-49.
void GpuRope() {
    for (RopeType type : {kNormal, kNeoX}) {
        for (int head_dim : {2, 8, 130}) {
            for (int pos : {0, 7, 63}) {
                Tensor q = Values({5, head_dim}), k = Waves({2, head_dim}, 0.3f);
                const auto expected = OracleRope(q, k, 5, 2, head_dim, {pos}, 10000.0f, type);
                CudaTensor dq = TensorHostToDevice(q), dk = TensorHostToDevice(k);
                CudaRopeHost(q, k, pos, 10000.0f, type);
                RequireTensor(q, expected.first, "host q");
                RequireTensor(k, expected.second, "host k");
                CudaRopeDevice(dq, dk, pos, 5, 2, head_dim, 10000.0f, type);
                RequireTensor(dq.Download(), expected.first, "device q");
                RequireTensor(dk.Download(), expected.second, "device k");
            }
        }
    }
    CudaTensor dq = TensorHostToDevice(Values({2, 4})), dk = TensorHostToDevice(Values({1, 4}));
    RequireError([&] { CudaRopeDevice(dq, dk, 0, 3, 1, 4, 1e4f); }, "q element count");
    RequireError([&] { CudaRopeDevice(dq, dk, 0, 2, 2, 4, 1e4f); }, "k element count");
    RequireError([&] { CudaRopeDevice(dq, dk, 0, 2, 1, 4, 1e4f, kNormal, 1); }, "devices must");
}

// Batched RoPE over T tokens equals T one-token calls and the oracle.
void GpuRopeBatched() {
    const int T = 9, H = 8, KV = 2, hd = 64;
    const std::vector<int> pos{0, 1, 5, 100, 4095, 8191, 17, 3, 2047};
    for (RopeType type : {kNormal, kNeoX}) {
        const Tensor q = Random({T, H * hd}, 11, 0.0f, 0.02f), k = Random({T, KV * hd}, 12, 0.0f, 0.02f);
        const auto expected = OracleRope(q, k, H, KV, hd, pos, 500000.0f, type);
        CudaTensor dq = TensorHostToDevice(q), dk = TensorHostToDevice(k);
        CudaRopeBatchDevice(dq, dk, pos, H, KV, hd, 500000.0f, type);
        RequireTensor(dq.Download(), expected.first, "batched q");
        RequireTensor(dk.Download(), expected.second, "batched k");
        // the same tokens one at a time through the reference signature
        Tensor one_q({H * hd}), one_k({KV * hd});
        for (int t = 0; t < T; ++t) {
            std::copy_n(q.data.begin() + t * H * hd, H * hd, one_q.data.begin());
            std::copy_n(k.data.begin() + t * KV * hd, KV * hd, one_k.data.begin());
            CudaTensor tq = TensorHostToDevice(one_q), tk = TensorHostToDevice(one_k);
            CudaRopeDevice(tq, tk, pos[t], H, KV, hd, 500000.0f, type);
            const Tensor gq = tq.Download();
            const Tensor bq = dq.Download();
            Require(std::memcmp(gq.data.data(), bq.data.data() + t * H * hd,
                                H * hd * sizeof(float)) == 0,
                    "one-token and batched RoPE agree bit for bit");
        }
        CudaTensor rq = TensorHostToDevice(q), rk = TensorHostToDevice(k);
        CudaRopeRangeDevice(rq, rk, 40, H, KV, hd, 500000.0f, type);
        std::vector<int> range(T);
        for (int t = 0; t < T; ++t) range[t] = 40 + t;
        const auto er = OracleRope(q, k, H, KV, hd, range, 500000.0f, type);
        RequireTensor(rq.Download(), er.first, "range q");
        RequireTensor(rk.Download(), er.second, "range k");
    }
}

// Fused residual add + RMSNorm over [T, D] equals ForwardAdd then RmsNorm.
void GpuAddRmsNorm() {
    for (auto shape : {std::vector<int>{1, 64}, std::vector<int>{6, 64}, std::vector<int>{3, 4096},
                       std::vector<int>{2, 4, 130}, std::vector<int>{2, 8192}}) {
        const int D = shape.back();
        const Tensor x = Random(shape, 21, 0.0f, 0.02f), d = Random(shape, 22, 0.0f, 0.02f);
        const Tensor w = Random({D}, 23, 1.0f, 0.1f);
        Tensor r = x, y(shape);
        Require(orc_add_rmsnorm(r.data.data(), d.data.data(), w.data.data(), y.data.data(),
                                x.data.size() / D, D, 1e-5f) == ORC_OK,
                "oracle add_rmsnorm");
        CudaTensor dx = TensorHostToDevice(x);
        const CudaTensor dd = TensorHostToDevice(d), dw = TensorHostToDevice(w);
        const CudaTensor dy = CudaAddRmsNormDevice(dx, &dd, dw.GetData(), {D}, 1e-5f);
        RequireTensor(dx.Download(), r, "residual", 0.0);
        RequireTensor(dy.Download(), y, "norm");
        const CudaTensor plain = CudaRmsNormRowsDevice(dx, dw.GetData(), {D}, 1e-5f);
        RequireTensor(plain.Download(), y, "rows norm");
        const CudaTensor untouched = CudaAddRmsNormDevice(dx, nullptr, dw.GetData(), {D}, 1e-5f);
        RequireTensor(untouched.Download(), y, "no-delta norm");
        RequireTensor(dx.Download(), r, "residual unchanged without delta", 0.0);
        RequireError([&] { (void)CudaAddRmsNormDevice(dx, &dd, dw.GetData(), {D + 1}, 1e-5f); },
                     "weight shape");
        RequireError([&] { (void)CudaAddRmsNormDevice(dx, &dd, dw.GetData(), {D}, 0.0f); },
                     "eps must be finite");
    }
}

void GpuQuantized() {
    for (QuantType t : {QuantType::kQ80, QuantType::kQ40, QuantType::kQ41}) {
        for (auto shape : {std::vector<int>{17, 64}, std::vector<int>{9, 100}, std::vector<int>{5, 4096}}) {
            const Tensor table = Random(shape, 31 + QuantIndex(t), 0.0f, 0.02f);
            const CudaTensor dt = TensorHostToDevice(table);
            const CudaDeviceBuffer blocks = CudaQuantizeDevice(dt, t);
            const std::vector<uint8_t> want = OracleQuantize(t, table);
            Require(Bytes(blocks) == want, "device quantizer equals TensorToQ* bytes");
            const std::vector<int> ids{0, shape[0] - 1, 1, 3, 0};
            const CudaTensor rows = CudaEmbeddingQuantDevice(blocks.GetData(), t, shape, ids);
            Tensor expected({static_cast<int>(ids.size()), shape[1]});
            Require(orc_gather_quant(QuantIndex(t), want.data(), shape[0], shape[1], ids.data(),
                                     ids.size(), expected.data.data()) == ORC_OK,
                    "oracle quant gather");
            RequireTensor(rows.Download(), expected, "quantized gather", 0.0);
            CudaTransferStats stats;
            CudaTensor one;
            {
                CudaStatsScope scope(&stats);
                one = CudaEmbeddingQuantDevice(blocks.GetData(), t, shape, {shape[0] - 1});
            }
            Require(stats.host_to_device_copies == 0, "one id: no host-to-device copy");
            Tensor last({1, shape[1]});
            std::copy_n(expected.data.begin() + shape[1], shape[1], last.data.begin());
            RequireTensor(one.Download(), last, "quantized gather of one id", 0.0);
        }
    }
}

// The reference's forward path issues these ops with every input already
// on the device: none of them may copy between host and device.
void GpuNoHostTransfersInDeviceChain() {
    const int D = 64, H = 4, KV = 2, hd = 16, F = 172;
    const Tensor table = Random({131, D}, 41, 0.0f, 0.02f);
    const CudaTensor dt = TensorHostToDevice(table), dw = TensorHostToDevice(Random({D}, 42, 1.0f, 0.1f));
    CudaTensor delta = TensorHostToDevice(Random({D}, 43, 0.0f, 0.02f));
    CudaTensor q = TensorHostToDevice(Random({H * hd}, 44)), k = TensorHostToDevice(Random({KV * hd}, 45));
    const CudaTensor gate = TensorHostToDevice(Random({F}, 46)), up = TensorHostToDevice(Random({F}, 47));
    CudaTransferStats stats;
    {
        CudaStatsScope scope(&stats);
        for (int pos = 0; pos < 6; ++pos) {
            CudaTensor h = CudaEmbeddingDevice(dt.GetData(), table.shape, 100 + pos);
            const CudaTensor y = CudaAddRmsNormDevice(h, &delta, dw.GetData(), {D}, 1e-5f);
            CudaRopeDevice(q, k, pos, H, KV, hd, 10000.0f);
            const CudaTensor ff = CudaSwiGluDevice(gate, up);
            (void)y;
            (void)ff;
        }
    }
    Require(stats.host_to_device_copies == 0 && stats.host_to_device_bytes == 0, "no H2D");
    Require(stats.device_to_host_copies == 0 && stats.device_to_host_bytes == 0, "no D2H");
    {
        CudaStatsScope scope(&stats);
        (void)q.Download();
    }
    Require(stats.device_to_host_copies == 1 && stats.device_to_host_bytes == H * hd * 4,
            "one counted download");
}

void GpuAllocator() {
    CudaEmptyCache();
    Require(CudaCachedBytes() == 0, "cache empty");
    auto stats = std::make_shared<CudaAllocationStats>();
    const void* first = nullptr;
    {
        CudaAllocationScope scope(stats);
        CudaTensor a({1000});
        CudaTensor b({2000});
        first = a.GetData();
        Require(stats->current_bytes == 12000 && stats->peak_bytes == 12000, "peak counting");
        a.Reset();
        Require(stats->current_bytes == 8000, "release counting");
        CudaTensor c({1000});  // same size class: the freed block comes back
        Require(c.GetData() == first, "cached block reused");
    }
    Require(stats->peak_bytes == 12000, "peak kept");
    Require(stats->current_bytes == 0, "all released");
    Require(CudaCachedBytes() > 0, "freed blocks cached");
    CudaEmptyCache();
    Require(CudaCachedBytes() == 0, "cache returned to the driver");
    CudaTensor moved({8});
    CudaTensor target = std::move(moved);
    Require(moved.IsEmpty() && moved.shape().empty() && !target.IsEmpty(), "move semantics");
    target.Reshape({2, 4});
    Require(target.num_dims() == 2 && target.NumEle() == 8, "reshape keeps the buffer");
    RequireError([&] { target.Reshape({3, 3}); }, "element count must remain unchanged");
}

// ----------------------------------------------- KV cache and attention

// Argument checks that throw before any device allocation.
void CpuCacheAndAttentionChecks() {
    Require(CudaCacheBuild() == CudaRuntimeBuilt(), "cache build predicate");
    Require(CudaAttentionBuilt() == CudaRuntimeBuilt(), "attention build predicate");
    RequireError([] { CudaCache c(0, 2, 1, 4); }, "value must be positive");
    RequireError([] { CudaCache c(1, 2, 1, 4, -1); }, "device_id must be non-negative");
    const CudaCache empty;
    Require(empty.Bytes_() == 0 && empty.n_layers() == 0, "empty cache");
    RequireError([&] { (void)empty.KData(); }, "key cache is empty");
    RequireError([&] { (void)empty.ReadKey(0, 0); }, "must both be initialized");
    const Tensor q({2, 3});
    RequireError([&] { (void)CudaAttentionDecode(q, empty, 0, 0, 2, 1, 3); }, "key cache is empty");
}

// tests/test_cuda_kv_cache.cc:5-47 of the reference tree: host and device
// slot writes (checked against the oracle's KvCache::Write), slot / head
// reads, byte offsets, move, Clear, Reset.
void GpuKvCache() {
    const int L = 2, S = 6, KV = 2, hd = 8;
    std::vector<float> kc(L * S * KV * hd, 0.0f), vc(kc.size(), 0.0f);
    CudaCache gpu(L, S, KV, hd);
    Require(gpu.Bytes_() == 2ull * L * S * KV * hd * sizeof(float), "KV allocation bytes");
    for (int layer : {0, 1}) {
        for (int pos : {0, 2, 5}) {
            const Tensor k = Random({KV, hd}, 100 + layer * 7 + pos);
            const Tensor v = Random({KV, hd}, 200 + layer + pos, 0.7f);
            const int32_t p = pos;
            Require(orc_kv_write(kc.data(), vc.data(), L, S, KV, hd, layer, &p, 1, k.data.data(),
                                 v.data.data()) == ORC_OK,
                    "oracle kv write");
            if (pos == 2) {
                gpu.WriteDevice(layer, pos, TensorHostToDevice(k), TensorHostToDevice(v));
            } else {
                gpu.WriteHost(layer, pos, k, v);
            }
        }
    }
    for (int layer : {0, 1}) {
        for (int pos : {0, 2, 5}) {
            const size_t slot = (static_cast<size_t>(layer) * S + pos) * KV * hd;
            Tensor k({KV, hd}), v({KV, hd}), kh({hd}), vh({hd});
            std::copy_n(kc.begin() + slot, KV * hd, k.data.begin());
            std::copy_n(vc.begin() + slot, KV * hd, v.data.begin());
            std::copy_n(kc.begin() + slot + hd, hd, kh.data.begin());
            std::copy_n(vc.begin() + slot + hd, hd, vh.data.begin());
            RequireTensor(gpu.ReadKey(layer, pos), k, "KV key slot", 0.0);
            RequireTensor(gpu.ReadVal(layer, pos), v, "KV value slot", 0.0);
            RequireTensor(gpu.ReadHeadKey(layer, pos, 1), kh, "KV head key", 0.0);
            RequireTensor(gpu.ReadHeadVal(layer, pos, 1), vh, "KV head value", 0.0);
            Require(gpu.SlotOffsetBytes(layer, pos, 1) == ((layer * S + pos) * 16 + 8) * 4ull,
                    "KV byte offset");
        }
    }
    RequireError([&] { (void)gpu.ReadKey(2, 0); }, "out of range");
    RequireError([&] { (void)gpu.ReadVal(0, 6); }, "out of range");
    RequireError([&] { (void)gpu.ReadHeadKey(0, 0, 2); }, "KV head 2 out of range");
    RequireError([&] { gpu.WriteHost(0, 0, Tensor({KV, hd + 1}), Tensor({KV, hd + 1})); },
                 "expected shape [2, 8]");
    RequireError([&] { gpu.WriteDevice(0, 0, TensorHostToDevice(Tensor({hd})),
                                       TensorHostToDevice(Tensor({hd}))); },
                 "expected 2D KV tensor");
    CudaCache moved(std::move(gpu));
    Require(gpu.Bytes_() == 0 && moved.Bytes_() > 0, "KV move ownership");
    moved.Clear();
    RequireTensor(moved.ReadKey(1, 5), Tensor({KV, hd}, 0.0f), "KV clear", 0.0);
    RequireTensor(moved.ReadVal(1, 5), Tensor({KV, hd}, 0.0f), "KV value clear", 0.0);
    moved.Reset();
    Require(moved.Bytes_() == 0 && moved.n_layers() == 0, "KV release");
    moved.Reset(1, 2, 1, 8);
    RequireTensor(moved.ReadKey(0, 1), Tensor({1, 8}, 0.0f), "KV reinitialize", 0.0);
}

Tensor AttentionFloat64(const Tensor& q, const std::vector<Tensor>& keys,
                        const std::vector<Tensor>& values, int pos) {
    // test/cuda_attention_test.cc:50-80 of the reference tree
    const int heads = q.shape[0], dim = q.shape[1];
    const int group = heads / keys[0].shape[0];
    Tensor out(q.shape);
    for (int h = 0; h < heads; ++h) {
        std::vector<double> scores(pos + 1);
        for (int t = 0; t <= pos; ++t) {
            double dot = 0.0;
            for (int d = 0; d < dim; ++d) {
                dot += static_cast<double>(q.data[h * dim + d]) * keys[t].data[(h / group) * dim + d];
            }
            scores[t] = dot / std::sqrt(static_cast<double>(dim));
        }
        const double mx = *std::max_element(scores.begin(), scores.end());
        double denom = 0.0;
        for (double& s : scores) {
            s = std::exp(s - mx);
            denom += s;
        }
        for (int d = 0; d < dim; ++d) {
            double value = 0.0;
            for (int t = 0; t <= pos; ++t) {
                value += scores[t] / denom * values[t].data[(h / group) * dim + d];
            }
            out.data[h * dim + d] = static_cast<float>(value);
        }
    }
    return out;
}

// test/cuda_attention_test.cc:82-158 of the reference tree: host and device
// attention within 2e-5 of float64 (a populated future slot must not count),
// then the argument checks.
void GpuAttention() {
    struct Case {
        int heads, kv_heads, dim, pos, layer;
    };
    for (const Case c : {Case{2, 2, 7, 0, 0}, Case{4, 2, 9, 5, 1}, Case{4, 1, 133, 130, 1}}) {
        CudaCache cache(2, c.pos + 2, c.kv_heads, c.dim);
        Tensor q({c.heads, c.dim});
        for (size_t i = 0; i < q.data.size(); ++i) q.data[i] = std::sin(static_cast<float>(i) * 0.17f);
        std::vector<Tensor> keys, values;
        for (int t = 0; t < cache.max_seq_len(); ++t) {
            Tensor k({c.kv_heads, c.dim}), v({c.kv_heads, c.dim});
            for (size_t i = 0; i < k.data.size(); ++i) {
                k.data[i] = std::cos(static_cast<float>(i) * 0.13f + t * 0.1f);
                v.data[i] = std::sin(static_cast<float>(i) * 0.11f - t * 0.2f);
            }
            cache.WriteHost(c.layer, t, k, v);
            keys.push_back(k);
            values.push_back(v);
        }
        const Tensor expected = AttentionFloat64(q, keys, values, c.pos);
        const Tensor host = CudaAttentionDecode(q, cache, c.layer, c.pos, c.heads, c.kv_heads, c.dim);
        const CudaTensor dev = CudaAttentionDevice(TensorHostToDevice(q), cache, c.layer, c.pos,
                                                   c.heads, c.kv_heads, c.dim);
        Require(dev.DeviceId() == 0, "attention device id");
        RequireTensor(host, expected, "attention host", 2e-5);
        RequireTensor(dev.Download(), expected, "attention device", 2e-5);
    }
    const CudaCache cache(2, 3, 2, 5);
    Tensor q({4, 5});
    auto invalid = [&](int layer, int pos, int heads, int kv, int dim, int device, const char* text) {
        RequireError([&] { (void)CudaAttentionDecode(q, cache, layer, pos, heads, kv, dim, device); },
                     text);
    };
    invalid(-1, 0, 4, 2, 5, 0, "out of range");
    invalid(2, 0, 4, 2, 5, 0, "out of range");
    invalid(0, -1, 4, 2, 5, 0, "out of range");
    invalid(0, 3, 4, 2, 5, 0, "out of range");
    invalid(0, 0, 0, 2, 5, 0, "value must be positive");
    invalid(0, 0, 4, 0, 5, 0, "value must be positive");
    invalid(0, 0, 4, -2, 5, 0, "value must be positive");
    invalid(0, 0, 4, 2, 0, 0, "value must be positive");
    invalid(0, 0, 3, 2, 5, 0, "divide n_heads");
    invalid(0, 0, 4, 1, 5, 0, "cache n_kv_heads mismatch");
    invalid(0, 0, 4, 2, 6, 0, "cache head_dim mismatch");
    invalid(0, 0, 4, 2, 5, -1, "cache device_id mismatch");
    q.shape = {20};
    invalid(0, 0, 4, 2, 5, 0, "q shape and element count");
    q.shape = {4, 5};
    q.data.pop_back();
    invalid(0, 0, 4, 2, 5, 0, "q shape and element count");
    const CudaTensor empty;
    RequireError([&] { (void)CudaAttentionDevice(empty, cache, 0, 0, 4, 2, 5); }, "q shape");
}

// The batched additions: a prefill chunk of T rows written in one launch and
// attended causally over the cache, against the oracle row by row.
void GpuAttentionBatched() {
    const int L = 2, S = 300, H = 8, KV = 2, hd = 128, layer = 1, pos0 = 150, T = 37;
    CudaCache cache(L, S, KV, hd);
    std::vector<float> kc(static_cast<size_t>(L) * S * KV * hd, 0.0f), vc(kc.size(), 0.0f);
    const Tensor k0 = Random({pos0, KV, hd}, 31), v0 = Random({pos0, KV, hd}, 32);
    std::vector<int32_t> first(pos0);
    for (int i = 0; i < pos0; ++i) first[i] = i;
    CudaKvWriteBatchDevice(cache, layer, 0, TensorHostToDevice(k0), TensorHostToDevice(v0));
    Require(orc_kv_write(kc.data(), vc.data(), L, S, KV, hd, layer, first.data(), pos0,
                         k0.data.data(), v0.data.data()) == ORC_OK, "oracle kv write");
    const Tensor k = Random({T, KV, hd}, 33), v = Random({T, KV, hd}, 34);
    const Tensor q = Random({T, H, hd}, 35);
    CudaKvWriteBatchDevice(cache, layer, pos0, TensorHostToDevice(k), TensorHostToDevice(v));
    std::vector<int32_t> pos(T);
    for (int t = 0; t < T; ++t) pos[t] = pos0 + t;
    Require(orc_kv_write(kc.data(), vc.data(), L, S, KV, hd, layer, pos.data(), T, k.data.data(),
                         v.data.data()) == ORC_OK, "oracle kv write");
    RequireTensor(cache.ReadKey(layer, pos0 + 5), [&] {
        Tensor r({KV, hd});
        std::copy_n(k.data.begin() + 5 * KV * hd, KV * hd, r.data.begin());
        return r;
    }(), "batched write slot", 0.0);
    const CudaTensor out = CudaAttentionBatchDevice(TensorHostToDevice(q), cache, layer, pos0, H,
                                                    KV, hd);
    Tensor want({T, H, hd});
    Require(orc_attention(q.data.data(), kc.data(), vc.data(), L, S, H, KV, hd, layer, pos.data(),
                          T, want.data.data()) == ORC_OK, "oracle attention");
    RequireTensor(out.Download(), want, "batched attention", 2e-5);
    RequireError([&] { CudaKvWriteBatchDevice(cache, layer, S - 2, TensorHostToDevice(k),
                                              TensorHostToDevice(v)); }, "out of range");
    RequireError([&] { (void)CudaAttentionBatchDevice(TensorHostToDevice(q), cache, layer, S - 2,
                                                      H, KV, hd); }, "out of range");
}

// The batched layer (include/cuda_forward.h): one call over T tokens equals
// T single-token calls at the same positions (the reference's own batch
// test, test/forward_test.cc:118-183), for the decode (head_dim 32) and the
// prefill (head_dim 64) attention kernels, fp32 and Q8_0 weights with a q
// bias, within the reference's device-forward tolerance 1e-5 + 1e-4 |x|
// (test/forward_test.cc:276-285).
void GpuForwardLayerBatched() {
    for (const int hd : {32, 64}) {
        for (QuantType t : {QuantType::kF32, QuantType::kQ80}) {
            CudaLayerConfig c;
            c.dim = 128;
            c.hidden_dim = 200;
            c.n_heads = 4;
            c.n_kv_heads = 2;
            c.head_dim = hd;
            c.rope_theta = 10000.0f;
            const int T = 20, S = 32, QD = c.n_heads * hd, KD = c.n_kv_heads * hd;
            std::vector<CudaTensor> keep;
            std::vector<CudaDeviceBuffer> blocks;
            auto weight = [&](int out, int in, uint64_t seed) {
                CudaLinearWeight w;
                w.type = t;
                keep.push_back(TensorHostToDevice(Random({out, in}, seed, 0.0f, 0.05f)));
                if (t == QuantType::kF32) {
                    w.data = keep.back().GetData();
                } else {
                    blocks.push_back(CudaQuantizeDevice(keep.back(), t));
                    w.data = blocks.back().GetData();
                }
                return w;
            };
            blocks.reserve(8);
            keep.reserve(16);
            CudaLayerWeights w;
            w.wq = weight(QD, c.dim, 1);
            w.wk = weight(KD, c.dim, 2);
            w.wv = weight(KD, c.dim, 3);
            w.wo = weight(c.dim, QD, 4);
            w.w_gate = weight(c.hidden_dim, c.dim, 5);
            w.w_up = weight(c.hidden_dim, c.dim, 6);
            w.w_down = weight(c.dim, c.hidden_dim, 7);
            keep.push_back(TensorHostToDevice(Random({QD}, 8, 0.0f, 0.1f)));
            w.wq.bias = static_cast<const float*>(keep.back().GetData());
            keep.push_back(TensorHostToDevice(Random({c.dim}, 9, 1.0f, 0.1f)));
            w.attention_norm = static_cast<const float*>(keep.back().GetData());
            keep.push_back(TensorHostToDevice(Random({c.dim}, 10, 1.0f, 0.1f)));
            w.ffn_norm = static_cast<const float*>(keep.back().GetData());
            const Tensor x0 = Random({T, c.dim}, 11);
            CudaCache batched(2, S, c.n_kv_heads, hd), single(2, S, c.n_kv_heads, hd);
            batched.Clear();
            single.Clear();
            CudaTensor xb = TensorHostToDevice(x0);
            CudaForwardLayerBatchDevice(c, w, xb, batched, 1, 0);
            const Tensor got = xb.Download();
            Tensor want({T, c.dim});
            for (int i = 0; i < T; ++i) {
                Tensor row({1, c.dim});
                std::copy_n(x0.data.begin() + static_cast<size_t>(i) * c.dim, c.dim,
                            row.data.begin());
                CudaTensor xr = TensorHostToDevice(row);
                CudaForwardLayerBatchDevice(c, w, xr, single, 1, i);
                const Tensor r = xr.Download();
                std::copy_n(r.data.begin(), c.dim, want.data.begin() + static_cast<size_t>(i) * c.dim);
            }
            for (size_t i = 0; i < want.data.size(); ++i) {
                Require(std::isfinite(got.data[i]), "batched layer output finite");
                Require(std::abs(got.data[i] - want.data[i]) <= 1e-5f + 1e-4f * std::abs(want.data[i]),
                        "batched layer equals the token loop (hd " + std::to_string(hd) + ")");
            }
            RequireTensor(batched.ReadKey(1, T - 1), single.ReadKey(1, T - 1), "cache slot", 1e-5);
            RequireError([&] { CudaForwardLayerBatchDevice(c, w, xb, batched, 1, S - 5); },
                         "out of range");
            RequireError([&] { CudaForwardLayerBatchDevice(c, w, xb, batched, 2, 0); },
                         "layer 2 out of range");
        }
    }
}

}  // namespace

int main(int argc, char** argv) {
    const std::vector<Case> cases = {
        {"cpu.build_predicate", CpuBuildPredicate},
        {"cpu.rejects_invalid_inputs", CpuRejectsInvalidInputs},
        {"cpu.tensor_checks", CpuTensorChecks},
        {"cpu.cache_and_attention_checks", CpuCacheAndAttentionChecks},
        {"gpu.device_info", GpuDeviceInfo},
        {"gpu.embedding", GpuEmbedding},
        {"gpu.rmsnorm", GpuRmsNorm},
        {"gpu.elementwise", GpuElementwise},
        {"gpu.softmax", GpuSoftmax},
        {"gpu.rope", GpuRope},
        {"gpu.rope_batched", GpuRopeBatched},
        {"gpu.add_rmsnorm", GpuAddRmsNorm},
        {"gpu.quantized", GpuQuantized},
        {"gpu.no_host_transfers", GpuNoHostTransfersInDeviceChain},
        {"gpu.allocator", GpuAllocator},
        {"gpu.kv_cache", GpuKvCache},
        {"gpu.attention", GpuAttention},
        {"gpu.attention_batched", GpuAttentionBatched},
        {"gpu.forward_layer_batched", GpuForwardLayerBatched},
    };
    return Run(argc, argv, cases);
}
