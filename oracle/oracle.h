/*
 * oracle.h -- CPU restatement of cpp-minilamma's per-layer ops.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product links, loads or calls
 * this library: it is used by tests/, by __graft_entry__.smoke() as the
 * checker, and by bench.py's cpu_baseline leg as the timed CPU port.
 *
 * Every function follows one reference function; the citation in front of
 * each declaration is the file:line under the reference tree it restates.
 * Floating point is evaluated in the same order and precision as the
 * reference and the file is compiled with -ffp-contract=off, so the results
 * equal the reference's own default (no -mfma) build bit for bit.
 *
 * Block layouts are the reference's packed structs
 * (include/quantized_tensor.h:10-35), little-endian:
 *   Q8_0  34 B: u16 d | i8 qs[32]
 *   Q4_0  18 B: u16 d | u8 qs[16]   (low nibble = element i, high = i+16)
 *   Q4_1  20 B: u16 d | u16 m | u8 qs[16]
 * Every row of the last dimension is cut into ceil(cols/32) blocks; the tail
 * block is padded with float zeros before quantization and only valid
 * elements are written by dequantization (src/quant.cc:136-368).
 *
 * Pinning (what checks each function; tests/test_oracle.py):
 *   fp16 decode/encode  exhaustive over all 65536 codes vs IEEE (numpy), the
 *                       reference KAT codes, and the compiled reference.
 *   quantizers          golden blocks written by the compiled reference
 *                       (tests/golden), reference tail/zero-block rules.
 *   dequantizers        reference KATs (test/quantized_tensor_test.cc
 *                       179-303), closed form fp16(d)*q in float64, golden.
 *   rmsnorm             reference KATs (test/ops_test.cc:158-188), float64
 *                       closed form, golden.
 *   rope                reference KATs (test/ops_test.cc:749-769), identity
 *                       at pos 0, composition, norm preservation, golden.
 *   silu/swiglu/mul     closed forms (test/ops_test.cc:713-725), golden.
 *   softmax             float64 closed form, sum to one, golden.
 *   gather/add          closed forms (row copy, IEEE add).
 *   linear / matmul     the compiled reference (bit for bit against its
 *                       default build), float64 closed form within the
 *                       fp32 summation bound, the reference's test vectors
 *                       (test/cuda_quant_test.cc:33-39, 99-127;
 *                       tests/test_cuda_linear.cc), bias and tail blocks.
 */
#ifndef MINILAMMA_ORACLE_H
#define MINILAMMA_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    ORC_OK = 0,
    ORC_EINVAL = 1,   /* the reference throws for this input */
};

enum { ORC_ROPE_NORMAL = 0, ORC_ROPE_NEOX = 1 };  /* include/model.h:37-40 */

enum { ORC_QK = 32, ORC_Q8_0_BYTES = 34, ORC_Q4_0_BYTES = 18, ORC_Q4_1_BYTES = 20 };

/* src/quant.cc:81-112 (and src/quantiezd_tensor.cc:16-42, same mapping). */
float orc_fp16_to_fp32(uint16_t bits);
/* src/quant.cc:31-79: round to nearest even, overflow -> inf, NaN -> quiet. */
uint16_t orc_fp32_to_fp16(float value);

/* Element-wise array forms of the two conversions above. */
void orc_fp16_to_fp32_array(const uint16_t* in, float* out, int64_t n);
void orc_fp32_to_fp16_array(const float* in, uint16_t* out, int64_t n);

/* src/quant.cc:136-174 TensorToQ80 over a [rows, cols] matrix. */
int orc_quantize_q8_0(const float* x, int64_t rows, int64_t cols, uint8_t* blocks);
/* src/quant.cc:205-249 TensorToQ40. */
int orc_quantize_q4_0(const float* x, int64_t rows, int64_t cols, uint8_t* blocks);
/* src/quant.cc:286-331 TensorToQ41. */
int orc_quantize_q4_1(const float* x, int64_t rows, int64_t cols, uint8_t* blocks);

/* src/quant.cc:175-204 Q80ToTensor, src/quant.cc:250-285 Q40ToTensor,
 * src/quant.cc:332-368 Q41ToTensor, row-wise with tail blocks. */
int orc_dequantize_q8_0(const uint8_t* blocks, int64_t rows, int64_t cols, float* out);
int orc_dequantize_q4_0(const uint8_t* blocks, int64_t rows, int64_t cols, float* out);
int orc_dequantize_q4_1(const uint8_t* blocks, int64_t rows, int64_t cols, float* out);

/* src/forward.cc:198-205 Embedding (one row copy per token) for a batch of
 * token ids; ids outside [0, vocab) return ORC_EINVAL before writing. */
int orc_gather_f32(const float* table, int64_t vocab, int64_t dim,
                   const int32_t* ids, int64_t n_tokens, float* out);
/* Quantized gather: the rows of Q*ToTensor(table) selected by ids, i.e. the
 * load-time dequantization (src/gguf_load.cc:370-404) followed by the F32
 * gather above. quant_type: 0 = Q8_0, 1 = Q4_0, 2 = Q4_1. */
int orc_gather_quant(int quant_type, const uint8_t* blocks, int64_t vocab, int64_t dim,
                     const int32_t* ids, int64_t n_tokens, float* out);

/* src/forward.cc:213-222 ForwardAdd. */
void orc_add(const float* a, const float* b, float* y, int64_t n);
/* src/ops.cc:50-60 ElementwiseMul. */
void orc_mul(const float* a, const float* b, float* y, int64_t n);
/* src/ops.cc:135-144 Silu. */
void orc_silu(const float* x, float* y, int64_t n);
/* src/ops.cc:145-151 SwiGlu = ElementwiseMul(Silu(gate), up). */
void orc_swiglu(const float* gate, const float* up, float* y, int64_t n);
/* src/ops.cc:113-134 SoftMax (1-D). */
int orc_softmax(const float* x, float* y, int64_t n);

/* src/ops.cc:82-112 RmsNorm over one row. */
int orc_rmsnorm_row(const float* x, const float* w, float* y, int64_t dim, float eps);
/* ForwardAdd then RmsNorm for each of n_rows rows (src/forward.cc:213-222,
 * src/ops.cc:82-112): residual <- residual + delta, y <- RmsNorm(residual).
 * delta may be NULL (plain RmsNorm of residual, residual left untouched). */
int orc_add_rmsnorm(float* residual, const float* delta, const float* w, float* y,
                    int64_t n_rows, int64_t dim, float eps);

/* src/ops.cc:177-224 Rope for one token: q [n_heads, head_dim],
 * k [n_kv_heads, head_dim], rotated in place. */
int orc_rope_token(float* q, float* k, int32_t n_heads, int32_t n_kv_heads,
                   int32_t head_dim, int32_t pos, float theta, int32_t rope_type);
/* Rope over n_tokens tokens: q [T, n_heads, head_dim], k [T, n_kv_heads,
 * head_dim]; token t uses positions[t], or pos0 + t when positions is NULL. */
int orc_rope(float* q, float* k, int64_t n_tokens, int32_t n_heads, int32_t n_kv_heads,
             int32_t head_dim, const int32_t* positions, int32_t pos0,
             float theta, int32_t rope_type);

/* ---- linear layers ----
 * Weights are [out_features, in_features] row-major (F32) or out_features
 * rows of ceil(in_features/32) packed blocks (quantized).  x is
 * [rows, in_features], y is [rows, out_features].  bias (may be NULL) is
 * added to the finished fp32 sum, as src/cuda_quant.cu:99-110 and
 * src/cuda_matmul.cc:79-90 add it on the host after the kernel.
 * n_threads: ParallelFor over the rows * out_features outputs as the
 * reference does (<= 0: hardware concurrency, 1: serial); the result does
 * not depend on it. */

/* src/quant.cc:393-463 LinearQuant, which is LinearQ80/Q40/Q41 of the
 * reference's default build (src/quant.cc:645-650, 865-870, 1089-1094):
 * sum += x[k] * Dequant(block, i) over k ascending, one fp32 accumulator per
 * output, dequantized weights as DequantQ80/Q40/Q41 (src/quant.cc:369-391). */
int orc_linear_quant(int quant_type, const float* x, const uint8_t* blocks, const float* bias,
                     float* y, int64_t rows, int64_t in_features, int64_t out_features,
                     int n_threads);
/* matumal/matuml_ops.cc:146-163 LinearNative applied to each row of x
 * (sum += x[k] * w[j, k], k ascending). */
int orc_linear_f32(const float* x, const float* w, const float* bias, float* y, int64_t rows,
                   int64_t in_features, int64_t out_features, int n_threads);
/* matumal/matuml_ops.cc:225-271 MatmulNative / MatmulThread:
 * c[i, j] = sum_k a[i, k] * b[k, j], k ascending; a [m, k], b [k, n]. */
int orc_matmul_f32(const float* a, const float* b, float* c, int64_t m, int64_t k, int64_t n,
                   int n_threads);

/* ---- decode attention and the KV cache ----
 * Caches are [n_layers, max_seq, n_kv_heads, head_dim] fp32 (the layout of
 * KvCache, include/kvcache.h:8-10, and of CudaCache, include/cuda_kvcache.h:5-6).
 *
 * src/kvcache.cc:19-50 KvCache::Write, for n_tokens rows: k and v rows t
 * ([n_kv_heads, head_dim] each) are copied to slot (layer, positions[t]). */
int orc_kv_write(float* k_cache, float* v_cache, int64_t n_layers, int64_t max_seq,
                 int32_t n_kv_heads, int32_t head_dim, int64_t layer, const int32_t* positions,
                 int64_t n_tokens, const float* k, const float* v);
/* src/forward.cc:265-298 ForwardAttention after its cache write, for
 * n_tokens query rows q [n_tokens, n_heads, head_dim] at positions[t]: query
 * head i reads KV head i / (n_heads / n_kv_heads); score j = (float sum of
 * q_d * k_d in d order) * (1 / sqrtf(head_dim)) for j = 0..pos; SoftMax
 * (src/ops.cc:113-134: max, expf(s - max), float sum in order, divide);
 * out_d = float sum of p_j * v_jd in j order. */
int orc_attention(const float* q, const float* k_cache, const float* v_cache, int64_t n_layers,
                  int64_t max_seq, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                  int64_t layer, const int32_t* positions, int64_t n_tokens, float* out);

/* ---- CPU baseline (bench.py cpu_baseline leg, kind "port") ----
 * thread_pool/thread_pool.cc:31-90 ParallelFor: static contiguous chunks,
 * serial when n/16 < threads.  n_threads <= 0 means hardware concurrency. */
int orc_parallel_threads(int n_threads);

/* One op chain per token, exactly as ForwardBatch drives it one token at a
 * time (src/forward.cc:482-486): gather -> residual add + RmsNorm -> RoPE on
 * q/k -> SwiGLU.  Buffers are [n_tokens, ...] and rows are independent, so
 * the ParallelFor variant splits tokens across threads. */
int orc_chain(const float* table, int64_t vocab, int64_t dim, const int32_t* ids,
              float* x, const float* delta, const float* norm_w, float* y, float eps,
              float* q, float* k, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
              const int32_t* positions, float theta,
              const float* gate, const float* up, float* ffn_out, int64_t ffn_dim,
              int64_t n_tokens, int n_threads);

#ifdef __cplusplus
}
#endif

#endif
