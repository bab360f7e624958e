// ref_shim.cc -- C entry points over the reference's own CPU sources.
//
// TEST INFRASTRUCTURE ONLY.  oracle/Makefile compiles this file together
// with the reference's CPU sources (the ops, the quantizers, the KV cache,
// the forward pass and the CPU builds of its device-layer files, which only
// throw), straight from where they lie under the reference tree, into
// oracle/_ref/libref*.so.  Tests use
// it to pin the C restatement (oracle.c) and tests/golden/make_golden.py
// writes the golden fixtures from it; bench.py times ref_chain as the
// "reference" CPU baseline.  Nothing here is reference source: it only
// converts between raw buffers and the reference's Tensor / block types.
#include "include/context.h"
#include "include/forward.h"
#include "include/kvcache.h"
#include "include/model.h"
#include "include/ops.h"
#include "include/quant.h"
#include "include/quantized_tensor.h"
#include "include/tensor.h"
#include "src/internal/forward.h"
#include "thread_pool/thread_pool.h"

#include <cmath>
#include <cstdint>
#include <cstring>
#include <exception>
#include <stdexcept>
#include <vector>

using yan_lamma::Block_Q40;
using yan_lamma::Block_Q41;
using yan_lamma::Block_Q80;
using yan_lamma::QuanTensor;
using yan_lamma::QuantType;
using yan_lamma::RopeType;
using yan_lamma::Tensor;

namespace {

Tensor Wrap(const float* p, std::vector<int> shape) {
    Tensor t(shape);
    std::memcpy(t.data.data(), p, t.data.size() * sizeof(float));
    return t;
}

void Unwrap(const Tensor& t, float* out) {
    std::memcpy(out, t.data.data(), t.data.size() * sizeof(float));
}

template <typename F>
int Guard(F&& f) {
    try {
        f();
        return 0;
    } catch (const std::exception&) {
        return 1;
    }
}

template <typename Block>
std::vector<Block> ToBlocks(const uint8_t* raw, size_t count) {
    std::vector<Block> blocks(count);
    std::memcpy(blocks.data(), raw, count * sizeof(Block));
    return blocks;
}

size_t RowBlocks(int cols) { return (static_cast<size_t>(cols) + 31) / 32; }

// A linear weight [out, in] of type t (-1 F32, 0 Q8_0, 1 Q4_0, 2 Q4_1) as
// the reference's QuanTensor.
QuanTensor MakeWeight(int t, const void* data, int out, int in) {
    QuanTensor w;
    w.shape = {out, in};
    const size_t n = static_cast<size_t>(out) * RowBlocks(in);
    const uint8_t* raw = static_cast<const uint8_t*>(data);
    if (t < 0) {
        w.type = QuantType::kF32;
        const float* f = static_cast<const float*>(data);
        w.kF32_data.assign(f, f + static_cast<size_t>(out) * in);
    } else if (t == 0) {
        w.type = QuantType::kQ80;
        w.kQ80_data = ToBlocks<Block_Q80>(raw, n);
    } else if (t == 1) {
        w.type = QuantType::kQ40;
        w.kQ40_data = ToBlocks<Block_Q40>(raw, n);
    } else {
        w.type = QuantType::kQ41;
        w.kQ41_data = ToBlocks<Block_Q41>(raw, n);
    }
    return w;
}

}  // namespace

extern "C" {

int ref_rmsnorm_row(const float* x, const float* w, float* y, int dim, float eps) {
    return Guard([&] { Unwrap(yan_lamma::RmsNorm(Wrap(x, {dim}), Wrap(w, {dim}), eps), y); });
}

int ref_rope_token(float* q, float* k, int n_heads, int n_kv_heads, int head_dim, int pos,
                   float theta, int rope_type) {
    return Guard([&] {
        Tensor tq = Wrap(q, {n_heads, head_dim});
        Tensor tk = Wrap(k, {n_kv_heads, head_dim});
        yan_lamma::Rope(tq, tk, pos, theta,
                        rope_type == 0 ? RopeType::kNormal : RopeType::kNeoX);
        Unwrap(tq, q);
        Unwrap(tk, k);
    });
}

int ref_silu(const float* x, float* y, int n) {
    return Guard([&] { Unwrap(yan_lamma::Silu(Wrap(x, {n})), y); });
}

int ref_mul(const float* a, const float* b, float* y, int n) {
    return Guard([&] { Unwrap(yan_lamma::ElementwiseMul(Wrap(a, {n}), Wrap(b, {n})), y); });
}

int ref_swiglu(const float* g, const float* u, float* y, int n) {
    return Guard([&] { Unwrap(yan_lamma::SwiGlu(Wrap(g, {n}), Wrap(u, {n})), y); });
}

int ref_softmax(const float* x, float* y, int n) {
    return Guard([&] { Unwrap(yan_lamma::SoftMax(Wrap(x, {n})), y); });
}

// Row-wise block quantizers and dequantizers (std::vector<Block> overloads).
int ref_quantize(int type, const float* x, int rows, int cols, uint8_t* out) {
    return Guard([&] {
        const Tensor t = Wrap(x, {rows, cols});
        if (type == 0) {
            const auto b = yan_lamma::TensorToQ80(t);
            std::memcpy(out, b.data(), b.size() * sizeof(Block_Q80));
        } else if (type == 1) {
            const auto b = yan_lamma::TensorToQ40(t);
            std::memcpy(out, b.data(), b.size() * sizeof(Block_Q40));
        } else {
            const auto b = yan_lamma::TensorToQ41(t);
            std::memcpy(out, b.data(), b.size() * sizeof(Block_Q41));
        }
    });
}

int ref_dequantize(int type, const uint8_t* raw, int rows, int cols, float* out) {
    return Guard([&] {
        const size_t n = static_cast<size_t>(rows) * RowBlocks(cols);
        const std::vector<int> shape{rows, cols};
        if (type == 0) {
            Unwrap(yan_lamma::Q80ToTensor(ToBlocks<Block_Q80>(raw, n), shape), out);
        } else if (type == 1) {
            Unwrap(yan_lamma::Q40ToTensor(ToBlocks<Block_Q40>(raw, n), shape), out);
        } else {
            Unwrap(yan_lamma::Q41ToTensor(ToBlocks<Block_Q41>(raw, n), shape), out);
        }
    });
}

// QuanTensor overloads (src/quantiezd_tensor.cc), the ones the GGUF loader
// uses on the embedding table; they need cols % 32 == 0.
int ref_dequantize_flat(int type, const uint8_t* raw, int rows, int cols, float* out) {
    return Guard([&] {
        QuanTensor q;
        q.shape = {rows, cols};
        const size_t n = static_cast<size_t>(rows) * static_cast<size_t>(cols) / 32;
        if (type == 0) {
            q.type = QuantType::kQ80;
            q.kQ80_data = ToBlocks<Block_Q80>(raw, n);
            Unwrap(yan_lamma::Q80ToTensor(q), out);
        } else if (type == 1) {
            q.type = QuantType::kQ40;
            q.kQ40_data = ToBlocks<Block_Q40>(raw, n);
            Unwrap(yan_lamma::Q40ToTensor(q), out);
        } else {
            q.type = QuantType::kQ41;
            q.kQ41_data = ToBlocks<Block_Q41>(raw, n);
            Unwrap(yan_lamma::Q41ToTensor(q), out);
        }
    });
}

// Quantized linear: LinearQ80/Q40/Q41 (src/quant.cc), y [rows, out].
// n_threads > 0 sets the reference thread pool's size for the call.
int ref_linear_quant(int type, const float* x, const uint8_t* raw, float* y, int rows, int in,
                     int out, int n_threads) {
    return Guard([&] {
        const Tensor tx = Wrap(x, {rows, in});
        const size_t n = static_cast<size_t>(out) * RowBlocks(in);
        const std::vector<int> shape{out, in};
        if (n_threads > 0) yan_lamma::SetThreadNum(n_threads);
        Tensor r;
        if (type == 0) {
            r = yan_lamma::LinearQ80(tx, ToBlocks<Block_Q80>(raw, n), shape);
        } else if (type == 1) {
            r = yan_lamma::LinearQ40(tx, ToBlocks<Block_Q40>(raw, n), shape);
        } else {
            r = yan_lamma::LinearQ41(tx, ToBlocks<Block_Q41>(raw, n), shape);
        }
        yan_lamma::SetThreadNum(0);
        Unwrap(r, y);
    });
}

// F32 linear: Linear(x, W) (src/ops.cc:152-154, the default LinearDispatch
// mode) on each row of x, since the reference's CPU Linear takes one row.
int ref_linear_f32(const float* x, const float* w, float* y, int rows, int in, int out) {
    return Guard([&] {
        const Tensor tw = Wrap(w, {out, in});
        for (int r = 0; r < rows; ++r) {
            Unwrap(yan_lamma::Linear(Wrap(x + static_cast<size_t>(r) * in, {in}), tw),
                   y + static_cast<size_t>(r) * out);
        }
    });
}

// Matmul(a, b) (src/ops.cc:76-80).
int ref_matmul_f32(const float* a, const float* b, float* c, int m, int k, int n) {
    return Guard([&] { Unwrap(yan_lamma::Matmul(Wrap(a, {m, k}), Wrap(b, {k, n})), c); });
}

// Decode attention for one query token: the K/V rows 0..pos-1 go into the
// reference's own KvCache (src/kvcache.cc) with KvCache::Write, then the
// reference's own ForwardAttention (src/forward.cc:265-298, exported through
// src/internal/forward.h) writes row pos and attends over 0..pos.
int ref_attention(const float* q, const float* k_rows, const float* v_rows, int n_layers,
                  int max_seq, int n_heads, int n_kv_heads, int head_dim, int layer, int pos,
                  float* out) {
    return Guard([&] {
        yan_lamma::KvCache cache(n_layers, max_seq, n_kv_heads, head_dim);
        const int row = n_kv_heads * head_dim;
        for (int j = 0; j < pos; ++j) {
            cache.Write(layer, j, Wrap(k_rows + j * row, {n_kv_heads, head_dim}),
                        Wrap(v_rows + j * row, {n_kv_heads, head_dim}));
        }
        const yan_lamma::Model unused;  // ForwardAttention's CPU path reads nothing from it
        Unwrap(yan_lamma::ForwardAttention(unused, Wrap(q, {n_heads, head_dim}),
                                           Wrap(k_rows + pos * row, {n_kv_heads, head_dim}),
                                           Wrap(v_rows + pos * row, {n_kv_heads, head_dim}),
                                           layer, pos, cache, n_heads, n_kv_heads, head_dim),
               out);
    });
}

// A Model holding only an F32 token table [vocab, dim] (copied once), for the
// reference's own Embedding (src/forward.cc:198-205) in ref_chain.
void* ref_embedding_model(const float* table, int64_t vocab, int64_t dim) {
    try {
        auto* model = new yan_lamma::Model();
        model->config.vocab_size = static_cast<int>(vocab);
        model->config.dim = static_cast<int>(dim);
        model->embedding_data_ = Wrap(table, {static_cast<int>(vocab), static_cast<int>(dim)});
        model->is_loaded = true;
        return model;
    } catch (const std::exception&) {
        return nullptr;
    }
}

void ref_model_free(void* model) { delete static_cast<yan_lamma::Model*>(model); }

// The per-token op chain as the reference's CPU forward runs it, every op the
// reference's own function on Tensor objects (one heap allocation per
// result): Embedding and ForwardAdd (src/forward.cc:198-222, exported through
// src/internal/forward.h), RmsNorm, Rope, SwiGlu (src/ops.cc).  With
// model == NULL there is no gather: row t of x_in is the residual input (the
// 70B chain).  n_threads > 1 spreads the tokens over the reference's own
// ParallelFor (thread_pool/thread_pool.cc).
int ref_chain(const void* model, const int32_t* ids, const float* x_in, float* x,
              const float* delta, const float* norm_w, float* y, float eps, float* q, float* k,
              int n_heads, int n_kv_heads, int head_dim, const int32_t* positions, float theta,
              const float* gate, const float* up, float* ffn_out, int64_t dim, int64_t ffn_dim,
              int64_t n_tokens, int n_threads) {
    return Guard([&] {
        const auto* m = static_cast<const yan_lamma::Model*>(model);
        const yan_lamma::Model unused;
        const int D = static_cast<int>(dim);
        const int F = static_cast<int>(ffn_dim);
        const Tensor w = Wrap(norm_w, {D});
        auto rows = [&](int begin, int end) {
            for (int t = begin; t < end; ++t) {
                Tensor e;
                if (m != nullptr) {
                    if (ids[t] < 0 || ids[t] >= m->config.vocab_size) {
                        throw std::runtime_error("token id out of range");
                    }
                    e = yan_lamma::Embedding(*m, ids[t]);
                } else {
                    e = Wrap(x_in + t * dim, {D});
                }
                const Tensor h = yan_lamma::ForwardAdd(m != nullptr ? *m : unused, e,
                                                       Wrap(delta + t * dim, {D}));
                Unwrap(h, x + t * dim);
                Unwrap(yan_lamma::RmsNorm(h, w, eps), y + t * dim);
                const int64_t qs = static_cast<int64_t>(n_heads) * head_dim;
                const int64_t ks = static_cast<int64_t>(n_kv_heads) * head_dim;
                Tensor tq = Wrap(q + t * qs, {n_heads, head_dim});
                Tensor tk = Wrap(k + t * ks, {n_kv_heads, head_dim});
                yan_lamma::Rope(tq, tk, positions[t], theta, RopeType::kNormal);
                Unwrap(tq, q + t * qs);
                Unwrap(tk, k + t * ks);
                Unwrap(yan_lamma::SwiGlu(Wrap(gate + t * ffn_dim, {F}), Wrap(up + t * ffn_dim, {F})),
                       ffn_out + t * ffn_dim);
            }
        };
        if (n_threads <= 1) {
            rows(0, static_cast<int>(n_tokens));
        } else {
            yan_lamma::SetThreadNum(n_threads);
            yan_lamma::ParallelFor(static_cast<int>(n_tokens), rows);
            yan_lamma::SetThreadNum(0);
        }
    });
}

// The quantized token gather on the CPU: each token's row of blocks through
// the reference's own dequantizer (Q80ToTensor / Q40ToTensor / Q41ToTensor,
// the std::vector<Block> overloads of src/quant.cc) into out [T, dim].  The
// reference has no quantized gather (it dequantizes the whole table at load,
// src/gguf_load.cc:370-404); this is its per-row equivalent, timed as the C4
// CPU baseline.  n_threads > 1 spreads the tokens over ParallelFor.
int ref_gather_quant(int type, const uint8_t* blocks, int64_t vocab, int64_t dim,
                     const int32_t* ids, int64_t n_tokens, float* out, int n_threads) {
    return Guard([&] {
        const size_t nb = RowBlocks(static_cast<int>(dim));
        const size_t row_bytes = nb * (type == 0 ? sizeof(Block_Q80)
                                                 : (type == 1 ? sizeof(Block_Q40) : sizeof(Block_Q41)));
        const std::vector<int> shape{1, static_cast<int>(dim)};
        auto rows = [&](int begin, int end) {
            for (int t = begin; t < end; ++t) {
                if (ids[t] < 0 || ids[t] >= vocab) throw std::runtime_error("token id out of range");
                const uint8_t* raw = blocks + static_cast<size_t>(ids[t]) * row_bytes;
                float* dst = out + t * dim;
                if (type == 0) {
                    Unwrap(yan_lamma::Q80ToTensor(ToBlocks<Block_Q80>(raw, nb), shape), dst);
                } else if (type == 1) {
                    Unwrap(yan_lamma::Q40ToTensor(ToBlocks<Block_Q40>(raw, nb), shape), dst);
                } else {
                    Unwrap(yan_lamma::Q41ToTensor(ToBlocks<Block_Q41>(raw, nb), shape), dst);
                }
            }
        };
        if (n_threads <= 1) {
            rows(0, static_cast<int>(n_tokens));
        } else {
            yan_lamma::SetThreadNum(n_threads);
            yan_lamma::ParallelFor(static_cast<int>(n_tokens), rows);
            yan_lamma::SetThreadNum(0);
        }
    });
}

// The reference's own CPU forward pass over an in-memory Model: ForwardToken
// (src/forward.cc) for tokens[t] at positions[t], t = 0..T-1, one at a time
// with one Context, exactly the loop of ForwardBatch; the logits of every
// step go to logits [T, vocab].
//   cfg      vocab, dim, hidden_dim, layers, n_heads, n_kv_heads, head_dim,
//            max_seq_len, rope_type
//   norms    per layer: attention_norm, ffn_norm
//   types    per layer: wq wk wv wo w_gate w_up w_down, then lm_head
//            (-1 F32, 0 Q8_0, 1 Q4_0, 2 Q4_1); weights the same order
//   biases   per layer: bq bk bv (NULL: none)
int ref_forward_tokens(const int32_t* cfg, float theta, float eps, const float* embedding,
                       const float* const* norms, const int32_t* types,
                       const void* const* weights, const float* const* biases,
                       const float* final_norm, const int32_t* tokens,
                       const int32_t* positions, int n_tokens, float* logits) {
    return Guard([&] {
        yan_lamma::Model model;
        yan_lamma::ModelConfig& c = model.config;
        c.vocab_size = cfg[0];
        c.dim = cfg[1];
        c.hidden_dim = cfg[2];
        c.layers = cfg[3];
        c.n_heads = cfg[4];
        c.n_kv_heads = cfg[5];
        c.head_dim = cfg[6];
        c.max_seq_len = cfg[7];
        c.rope_type = cfg[8] == 0 ? RopeType::kNormal : RopeType::kNeoX;
        c.rope_theta = theta;
        c.rms_norm_eps = eps;
        const int D = c.dim, F = c.hidden_dim, QD = c.n_heads * c.head_dim,
                  KD = c.n_kv_heads * c.head_dim;
        model.embedding_data_ = Wrap(embedding, {c.vocab_size, D});
        model.n_layers_.resize(c.layers);
        for (int l = 0; l < c.layers; ++l) {
            yan_lamma::Layer& L = model.n_layers_[l];
            const int32_t* t = types + 7 * l;
            const void* const* w = weights + 7 * l;
            L.attention_norm = Wrap(norms[2 * l], {D});
            L.ffn_norm = Wrap(norms[2 * l + 1], {D});
            L.wq = MakeWeight(t[0], w[0], QD, D);
            L.wk = MakeWeight(t[1], w[1], KD, D);
            L.wv = MakeWeight(t[2], w[2], KD, D);
            L.wo = MakeWeight(t[3], w[3], D, QD);
            L.w_gate = MakeWeight(t[4], w[4], F, D);
            L.w_up = MakeWeight(t[5], w[5], F, D);
            L.w_down = MakeWeight(t[6], w[6], D, F);
            if (biases[3 * l] != nullptr) L.bq = Wrap(biases[3 * l], {QD});
            if (biases[3 * l + 1] != nullptr) L.bk = Wrap(biases[3 * l + 1], {KD});
            if (biases[3 * l + 2] != nullptr) L.bv = Wrap(biases[3 * l + 2], {KD});
        }
        model.final_norm = Wrap(final_norm, {D});
        model.lm_head_ = MakeWeight(types[7 * c.layers], weights[7 * c.layers], c.vocab_size, D);
        model.is_loaded = true;
        yan_lamma::Context ctx(&model);
        for (int t = 0; t < n_tokens; ++t) {
            ctx.pos = static_cast<size_t>(positions[t]);
            Unwrap(yan_lamma::ForwardToken(model, ctx, tokens[t]),
                   logits + static_cast<size_t>(t) * c.vocab_size);
        }
    });
}

}  // extern "C"
