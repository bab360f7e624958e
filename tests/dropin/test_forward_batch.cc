// test_forward_batch.cc -- the reference-side binding (forward_batch_device.cc)
// held to the reference's own device-forward bar: the reference's tiny model
// (models/tiny, tests/cuda_test_support.h:44), uploaded by the reference's
// UploadModelWeightToCuda, runs its 9-token prompt as one batch through
// ForwardBatchDevice, and the logits are compared with the reference's CPU
// ForwardBatch on a second copy of the model; then the transfer counters the
// reference keeps in its model statistics (tests/cuda_test_support.h:88-125).
// The comparison bar is the reference's device-forward tolerance
// |got - want| <= 1e-5 + 1e-4 |want| (test/forward_test.cc:276-285), and the
// reference's own RequireCloseTensor on top.
//
// Modes (one per line of tests/test_gpu_dropin.py):
//   f32 / q8_0 / q4_0   linears of that type, F32 token table: the prompt as
//                       one batch; a prefill of 6 then 3 one-token batches;
//                       the prompt at positions with gaps
//   table_q8_0 / table_q4_0 / table_q4_1
//                       Q8_0 linears, the token table kept on the device as
//                       blocks (UploadTokenTableBlocks); the CPU model's table
//                       is the same blocks dequantized, as the GGUF load gives
//                       (src/gguf_load.cc:370-404)
//   fallback            positions that do not increase: ForwardBatch itself
//   rejects             the checks and messages of ForwardBatch / ForwardToken
#include "tests/cuda_test_support.h"
#include "tests/dropin/forward_batch_device.h"

#include "include/quant.h"

#include <algorithm>
#include <cmath>
#include <sstream>
#include <string>
#include <vector>

using namespace yan_lamma;
using namespace yan_lamma::test;

namespace {

const std::vector<int> kPrompt{128, 104, 101, 108, 108, 111, 32, 119, 111};  // "<bos>hello wo"

void RequireForwardClose(const Tensor& got, const Tensor& want, const std::string& what) {
    Require(got.shape == want.shape, what + ": shape");
    for (size_t i = 0; i < want.data.size(); ++i) {
        const double g = got.data[i], w = want.data[i];
        if (!(std::abs(g - w) <= 1e-5 + 1e-4 * std::abs(w))) {
            std::ostringstream m;
            m.precision(9);
            m << what << ": logit " << i << " got " << g << " want " << w;
            throw std::runtime_error(m.str());
        }
    }
    RequireCloseTensor(got, want, what);
}

struct Counts {
    size_t h2d, h2d_bytes, d2h, d2h_bytes;
};

void RequireCounts(const Model& gpu, const Counts& c, const std::string& what) {
    const Counts got{ModelCudaHostToDeviceCopies(gpu), ModelCudaHostToDeviceBytes(gpu),
                     ModelCudaDeviceToHostCopies(gpu), ModelCudaDeviceToHostBytes(gpu)};
    std::ostringstream m;
    m << what << ": transfers H2D " << got.h2d << " (" << got.h2d_bytes << " B), D2H " << got.d2h
      << " (" << got.d2h_bytes << " B); want H2D " << c.h2d << " (" << c.h2d_bytes << " B), D2H "
      << c.d2h << " (" << c.d2h_bytes << " B)";
    Require(got.h2d == c.h2d && got.h2d_bytes == c.h2d_bytes && got.d2h == c.d2h &&
                got.d2h_bytes == c.d2h_bytes,
            m.str());
    std::cout << m.str() << '\n';
}

Batch Of(const std::vector<int>& tokens, const std::vector<int>& poss) {
    Batch b;
    b.tokens = tokens;
    b.poss = poss;
    return b;
}

std::vector<int> Range(int first, int n) {
    std::vector<int> v(n);
    for (int i = 0; i < n; ++i) v[i] = first + i;
    return v;
}

// One batch on both models, compared; the GPU side's transfers counted.
void Step(Model& cpu, Context& cpu_ctx, Model& gpu, Context& gpu_ctx, const Batch& b,
          const std::string& what, bool gapped) {
    const Tensor want = ForwardBatch(cpu, cpu_ctx, b);
    ResetModelCudaRuntimeStats(gpu);
    const Tensor got = ForwardBatchDevice(gpu, gpu_ctx, b);
    RequireForwardClose(got, want, what);
    const size_t T = b.tokens.size();
    const size_t ids = T > 1 ? 1 : 0;
    const size_t pos = gapped ? size_t(gpu.config.layers) : 0;
    RequireCounts(gpu, {ids + pos, 4 * T * (ids + pos), 1, 4 * size_t(gpu.config.vocab_size)},
                  what);
    Require(gpu_ctx.pos == size_t(b.poss.back()) && gpu_ctx.token_id_ == cpu_ctx.token_id_,
            what + ": context as ForwardBatch leaves it");
}

// The device cache's rows at the batch's positions against the CPU cache.
void RequireCachesAgree(const Model& cpu, Context& cpu_ctx, Context& gpu_ctx,
                        const std::vector<int>& poss, const std::string& what) {
    for (int layer = 0; layer < cpu.config.layers; ++layer) {
        for (int p : poss) {
            const Tensor gk = gpu_ctx.cuda_cache_.ReadKey(layer, p);
            const Tensor gv = gpu_ctx.cuda_cache_.ReadVal(layer, p);
            Tensor ck(gk.shape), cv(gv.shape);  // [n_kv_heads, head_dim], one slot
            const float* k = cpu_ctx.cpu_cache_.KeyPtr(layer, p, 0);
            const float* v = cpu_ctx.cpu_cache_.ValPtr(layer, p, 0);
            std::copy(k, k + ck.data.size(), ck.data.begin());
            std::copy(v, v + cv.data.size(), cv.data.begin());
            RequireForwardClose(gk, ck, what + " K layer " + std::to_string(layer) + " pos " +
                                            std::to_string(p));
            RequireForwardClose(gv, cv, what + " V layer " + std::to_string(layer) + " pos " +
                                            std::to_string(p));
        }
    }
}

void Linears(QuantType type) {
    Model cpu = Tiny(), gpu = Tiny();
    Quantize(cpu, type);
    Quantize(gpu, type);
    UploadModelWeightToCuda(gpu, 0);
    {  // the prompt as one batch
        Context cc(&cpu), gc(&gpu);
        Step(cpu, cc, gpu, gc, Of(kPrompt, Range(0, 9)), "prompt of 9 as one batch", false);
        RequireCachesAgree(cpu, cc, gc, Range(0, 9), "prompt");
    }
    {  // a prefill of 6, then one token at a time
        Context cc(&cpu), gc(&gpu);
        Step(cpu, cc, gpu, gc, Of({kPrompt.begin(), kPrompt.begin() + 6}, Range(0, 6)),
             "prefill of 6", false);
        for (int t = 6; t < 9; ++t) {
            Step(cpu, cc, gpu, gc, Batch::Single(kPrompt[t], t), "decode token " + std::to_string(t),
                 false);
        }
    }
    {  // positions with gaps
        Context cc(&cpu), gc(&gpu);
        const std::vector<int> poss{0, 1, 2, 5, 6, 9, 10, 11, 14};
        Step(cpu, cc, gpu, gc, Of(kPrompt, poss), "prompt at gapped positions", true);
        RequireCachesAgree(cpu, cc, gc, poss, "gapped");
    }
}

void TokenTable(QuantType table_type) {
    Model cpu = Tiny(), gpu = Tiny();
    Quantize(cpu, QuantType::kQ80);
    Quantize(gpu, QuantType::kQ80);
    QuanTensor blocks;
    blocks.type = table_type;
    blocks.shape = cpu.embedding_data_.shape;
    Tensor dequantized;
    if (table_type == QuantType::kQ80) {
        blocks.kQ80_data = TensorToQ80(cpu.embedding_data_);
        dequantized = Q80ToTensor(blocks);
    } else if (table_type == QuantType::kQ40) {
        blocks.kQ40_data = TensorToQ40(cpu.embedding_data_);
        dequantized = Q40ToTensor(blocks);
    } else {
        blocks.kQ41_data = TensorToQ41(cpu.embedding_data_);
        dequantized = Q41ToTensor(blocks);
    }
    cpu.embedding_data_ = dequantized;  // what the load leaves on the host
    UploadModelWeightToCuda(gpu, 0);
    const size_t count = gpu.cuda_weights->uploaded_weight_count;
    UploadTokenTableBlocks(gpu, blocks);
    const CudaloadWeight* t = DeviceTokenTable(gpu);
    Require(t != nullptr && t->type == table_type && !t->linear &&
                gpu.cuda_weights->uploaded_weight_count == count,
            "the token table is replaced by its blocks");
    Context cc(&cpu), gc(&gpu);
    Step(cpu, cc, gpu, gc, Of(kPrompt, Range(0, 9)), "prompt, token table as blocks", false);
    Step(cpu, cc, gpu, gc, Batch::Single(kPrompt[2], 9), "one token, token table as blocks",
         false);
}

void Fallback() {
    Model cpu = Tiny(), gpu = Tiny();
    UploadModelWeightToCuda(gpu, 0);
    Context cc(&cpu), gc(&gpu);
    const Batch b = Of({128, 104, 101}, {4, 2, 0});
    const Tensor want = ForwardBatch(cpu, cc, b);
    ResetModelCudaRuntimeStats(gpu);
    const Tensor got = ForwardBatchDevice(gpu, gc, b);
    RequireForwardClose(got, want, "decreasing positions");
    // the reference's own token loop ran: its per-token counters
    Require(ModelCudaLinearCalls(gpu) == 45 && ModelCudaAttentionCalls(gpu) == 6,
            "decreasing positions run ForwardBatch's token loop");
}

void Rejects() {
    Model gpu = Tiny();
    UploadModelWeightToCuda(gpu, 0);
    Context gc(&gpu);
    RequireError([&] { (void)ForwardBatchDevice(gpu, gc, Batch{}); }, "Empty Batch");
    RequireError([&] { (void)ForwardBatchDevice(gpu, gc, Of({1, 2}, {0})); },
                 "Tokens Pos Not Matched");
    bool caught = false;
    try {
        (void)ForwardBatchDevice(gpu, gc, Of({1, 131}, {0, 1}));
    } catch (const std::out_of_range& e) {
        caught = std::string(e.what()).find("token out of range") != std::string::npos;
    }
    Require(caught, "token out of range");
    caught = false;
    try {
        (void)ForwardBatchDevice(gpu, gc, Of({1, 2}, {0, gpu.config.max_seq_len}));
    } catch (const std::out_of_range& e) {
        caught = std::string(e.what()).find("position out of range") != std::string::npos;
    }
    Require(caught, "position out of range");
    QuanTensor wrong;
    wrong.type = QuantType::kQ80;
    wrong.shape = {gpu.config.vocab_size, gpu.config.dim};
    RequireError([&] { UploadTokenTableBlocks(gpu, wrong); }, "expected");
}

}  // namespace

int main(int argc, char** argv) {
    return Run(argc, argv,
               {{"f32", [] { Linears(QuantType::kF32); }},
                {"q8_0", [] { Linears(QuantType::kQ80); }},
                {"q4_0", [] { Linears(QuantType::kQ40); }},
                {"table_q8_0", [] { TokenTable(QuantType::kQ80); }},
                {"table_q4_0", [] { TokenTable(QuantType::kQ40); }},
                {"table_q4_1", [] { TokenTable(QuantType::kQ41); }},
                {"fallback", Fallback},
                {"rejects", Rejects}});
}
