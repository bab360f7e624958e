/*
 * minilamma_hip.h -- C ABI of libminilamma_hip.so, the MI355X (gfx950) kernels
 * for cpp-minilamma's per-layer memory-bound ops.
 *
 * This is the only interface the HIP translation units export.  The C++17
 * op surface (include/cuda_ops.h, libminilamma_ops.so) and the Python
 * binding (cpp-minilamma_amd/__init__.py) sit on top of it.
 *
 * Conventions
 *   - every data pointer is a borrowed device pointer unless the name says
 *     "host"; the library never frees or keeps what it is handed;
 *   - sizes are int64_t, token ids and positions are int32_t;
 *   - `stream` is an opaque hipStream_t; NULL is the null stream;
 *   - kernels are asynchronous on `stream`; nothing synchronizes unless the
 *     entry point says so;
 *   - every entry returns an mlk_status; 0 is success, and
 *     mlk_last_error() gives a message for the calling thread's last failure;
 *   - validation happens before any launch, so a rejected call changes no
 *     memory; nothing throws or allocates device memory across this ABI
 *     except mlk_malloc.
 *
 * Reference interfaces replaced (paths are under the reference tree):
 *   include/cuda_ops.h:11-33        -> the op entries below (one-token
 *                                      signatures become n_tokens = 1)
 *   include/cuda_matmul.h:7-18      -> mlk_linear_f32, mlk_matmul_f32
 *   include/cuda_quant.h:12-25      -> mlk_linear_quant
 *   include/cuda_kvcache.h:23       -> mlk_kv_write_f32
 *   include/cuda_attention.h:9-13   -> mlk_attention_decode_f32, mlk_attention_prefill_f32
 *   include/cuda_runtime.h:8-42     -> the runtime entries at the end
 */
#ifndef MINILAMMA_HIP_H
#define MINILAMMA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    MLK_OK = 0,
    MLK_ERR_INVALID = 1,     /* bad pointer, shape, eps, theta, position ... */
    MLK_ERR_RANGE = 2,       /* a token id / position outside its range */
    MLK_ERR_HIP = 3,         /* the HIP runtime reported an error */
    MLK_ERR_NO_DEVICE = 4,   /* no usable GPU */
} mlk_status;

typedef enum { MLK_ROPE_NORMAL = 0, MLK_ROPE_NEOX = 1 } mlk_rope_type; /* include/model.h:37-40 */

typedef enum { MLK_Q8_0 = 0, MLK_Q4_0 = 1, MLK_Q4_1 = 2 } mlk_quant_type;

/* Thread-local message for the last failed call on this thread. */
const char* mlk_last_error(void);
/* Static text for a status code. */
const char* mlk_status_string(int status);
/* Version of this ABI (bumped on any signature change). */
int mlk_abi_version(void);

/* ------------------------------------------------------------------ ops */

/*
 * Residual add fused with RMSNorm over n_rows rows of width dim.
 *   residual[r] <- residual[r] + delta[r]            (when delta != NULL)
 *   y[r]        <- residual[r] * weight * 1/sqrt(mean(residual[r]^2) + eps)
 * The mean of squares, the scale and the per-element product are evaluated
 * in float64 and the product is rounded once to float, as the CPU RmsNorm
 * does.  eps must be finite and > 0.  y may not alias residual or delta.
 * Replaces CudaElementAddDevice + CudaRmsNromDevice (include/cuda_ops.h:16,
 * :25; src/cuda_ops.cu:335-355, :432-435), which ran as three kernels.
 */
mlk_status mlk_add_rmsnorm_f32(float* residual, const float* delta, const float* weight,
                               float* y, int64_t n_rows, int64_t dim, float eps, void* stream);

/* Plain RMSNorm of x into y (x read-only).  include/cuda_ops.h:15-16. */
mlk_status mlk_rmsnorm_f32(const float* x, const float* weight, float* y, int64_t n_rows,
                           int64_t dim, float eps, void* stream);

/* y = silu(gate) * up over n elements, silu(g) = g * (1 / (1 + exp(-g))).
 * Replaces CudaSiluDevice + CudaElementwiseMulDevice (include/cuda_ops.h:
 * 19-23, two kernels and an HBM round trip of silu(gate)). */
mlk_status mlk_swiglu_f32(const float* gate, const float* up, float* y, int64_t n,
                          void* stream);
/* y = silu(x).  include/cuda_ops.h:19-20. */
mlk_status mlk_silu_f32(const float* x, float* y, int64_t n, void* stream);
/* y = a * b.  include/cuda_ops.h:22-23. */
mlk_status mlk_mul_f32(const float* a, const float* b, float* y, int64_t n, void* stream);
/* y = a + b (residual or bias add).  include/cuda_ops.h:25-27. */
mlk_status mlk_add_f32(const float* a, const float* b, float* y, int64_t n, void* stream);

/* Softmax of each of n_rows rows of width n (max-subtracted, then
 * normalised).  include/cuda_ops.h:29 (one row there). */
mlk_status mlk_softmax_f32(const float* x, float* y, int64_t n_rows, int64_t n, void* stream);

/*
 * Rotary position embedding, in place, on q [n_tokens, n_heads, head_dim]
 * and k [n_tokens, n_kv_heads, head_dim]; row t of q starts at
 * q + t * q_row_stride (likewise k), so q and k may be column slices of a
 * fused QKV activation.  Token t is at position positions[t] (device array)
 * or, when positions is NULL, at pos0 + t.  For pair i < head_dim/2 the angle
 * is pos * theta^(-2i/head_dim), computed with cos and sin in float64 and the
 * rotation rounded once to float (src/ops.cc:177-224).  Normal rotates
 * (2i, 2i+1), NeoX rotates (i, i + head_dim/2).  A negative entry of
 * `positions` leaves that token unrotated and, when err != NULL, stores a
 * nonzero value in *err (the caller clears it).
 * Replaces CudaRopeDevice (include/cuda_ops.h:32-33, two launches per token).
 */
mlk_status mlk_rope_f32(float* q, float* k, int64_t n_tokens, int32_t n_heads,
                        int32_t n_kv_heads, int32_t head_dim, int64_t q_row_stride,
                        int64_t k_row_stride, const int32_t* positions, int32_t pos0,
                        float theta, int32_t rope_type, int32_t* err, void* stream);

/*
 * Token-embedding gather from an F32 table [vocab, dim]:
 *   out[t, :] = table[ids[t], :]   (bit-exact row copy)
 * ids is a device array of n_tokens ids; when ids is NULL the single host
 * id `token` is used (n_tokens must be 1), which is the reference's
 * one-token signature.  An id outside [0, vocab) writes a zero row and, when
 * err != NULL, a nonzero value to *err.
 * Replaces CudaEmbeddingDevice (include/cuda_ops.h:13).
 */
mlk_status mlk_gather_f32(const float* table, int64_t vocab, int64_t dim, const int32_t* ids,
                          int32_t token, int64_t n_tokens, float* out, int32_t* err,
                          void* stream);

/*
 * Token-embedding gather from a block-quantized table, dequantizing only the
 * gathered rows.  The table is vocab rows of ceil(dim/32) packed blocks
 * (Q8_0 34 B, Q4_0 18 B, Q4_1 20 B, little-endian fp16 scales, low nibble =
 * first 16 elements), exactly the layout TensorToQ80/Q40/Q41 produce
 * (src/quant.cc:136-331).  Outputs equal Q80ToTensor/Q40ToTensor/Q41ToTensor
 * (src/quant.cc:175-368) of those rows bit for bit.  ids/token/err as in
 * mlk_gather_f32.  No reference counterpart on the device: the reference
 * dequantizes the whole table on the host at load (src/gguf_load.cc:370-404).
 */
mlk_status mlk_gather_quant(int32_t quant_type, const void* blocks, int64_t vocab, int64_t dim,
                            const int32_t* ids, int32_t token, int64_t n_tokens, float* out,
                            int32_t* err, void* stream);

/* Block quantizer on the device: x [rows, cols] -> packed blocks, bit-identical
 * to TensorToQ80/Q40/Q41 (src/quant.cc:136-331), tail blocks zero padded. */
mlk_status mlk_quantize(int32_t quant_type, const float* x, int64_t rows, int64_t cols,
                        void* blocks, void* stream);
/* Bytes of the packed blocks of a [rows, cols] matrix (0 on bad input). */
int64_t mlk_quant_bytes(int32_t quant_type, int64_t rows, int64_t cols);

/*
 * Linear layer with a block-quantized weight:
 *   y[t, j] = sum_k x[t, k] * W[j, k] (+ bias[j])   t < rows, j < out_features
 * W is out_features rows of ceil(in_features / 32) packed blocks (the layout
 * above); x [rows, in_features] and y [rows, out_features] are row-major
 * fp32; bias may be NULL and is added to the finished sum.  The sum is fp32
 * in an order of the kernel's choosing: within gamma_K * sum_k |x w| of the
 * exact value, like the reference's serial loop.  y may not alias x or W.
 * workspace / workspace_bytes: optional scratch for splitting K (see
 * mlk_linear_workspace_bytes; NULL, 0 is always valid).
 * Replaces CudaQ40/Q41/Q80DeviceInputLinear (include/cuda_quant.h:12-25;
 * kernels src/cuda_quant.cu:29-97, one thread per output).
 */
mlk_status mlk_linear_quant(int32_t quant_type, const float* x, const void* w_blocks,
                            const float* bias, float* y, int64_t rows, int64_t in_features,
                            int64_t out_features, void* workspace, size_t workspace_bytes,
                            void* stream);

/* The same with an fp32 weight W [out_features, in_features] row-major.
 * Replaces CudaLinearDevice (include/cuda_matmul.h:16-18; cublasSgemm,
 * src/cuda_matmul.cc:155-189). */
mlk_status mlk_linear_f32(const float* x, const float* w, const float* bias, float* y,
                          int64_t rows, int64_t in_features, int64_t out_features,
                          void* workspace, size_t workspace_bytes, void* stream);

/* Device bytes of the optional workspace of mlk_linear_quant / mlk_linear_f32
 * for this shape on the current device (0: the call uses none).  Calls of
 * 32 rows or more run on the matrix cores in 128 x 128 output tiles; when
 * those tiles are fewer than two per compute unit, a workspace of this size
 * (16-byte aligned, not aliasing x, W or y) lets the call split K over
 * workgroups and add the partial sums in a fixed order.  Without it (NULL or
 * smaller) the call is still correct, only slower.  No counterpart in the
 * reference (cuBLAS keeps its own workspace). */
int64_t mlk_linear_workspace_bytes(int64_t rows, int64_t in_features, int64_t out_features);

/* Planar layout of Q8_0 / Q4_0 weights [out, in] (in % 256 == 0), made once
 * at upload from the block layout by mlk_quant_to_planar.  The values are
 * the blocks' (the same scale and codes per element); only their order
 * differs, so that the few-token linear layers load each row tile's bytes
 * 1 KB-contiguous per wave, already in matrix-core operand order:
 *   codes: rows in tiles of 16 (the last tile padded with rows of zero
 *     bytes, codes and scales alike); tile rt, lane l = 16 g + r (row
 *     16 rt + r, inputs 8g .. 8g + 7 of each
 *     block) holds 16 bytes per group of blocks: Q8_0 per block pair, bytes
 *     0..7 the first block's codes, 8..15 the second's; Q4_0 per 4 blocks,
 *     bytes 4j .. 4j + 3 block j, byte e holding input 8g + e in its low
 *     nibble and 8g + e + 4 in its high one, each as (code - 8) in 4-bit
 *     two's complement.  Order: [tile][group][lane][16 bytes];
 *   scales: after the codes, [tile][in / 256][16 rows][8 blocks] fp16.
 * No counterpart in the reference (its device weights keep the blocks,
 * include/quantized_tensor.h:10-35); for callers that upload weights once
 * and run few-token decode steps.  0: no planar layout for this shape (Q4_1,
 * or in % 256 != 0). */
int64_t mlk_quant_planar_bytes(int32_t quant_type, int64_t rows, int64_t cols);
mlk_status mlk_quant_to_planar(int32_t quant_type, const void* blocks, int64_t rows,
                               int64_t cols, void* planar, void* stream);

/* y = x W^T (+ bias) with W in the planar layout (quant_type MLK_Q8_0 or
 * MLK_Q4_0), the same sum bound as mlk_linear_quant.  One row with
 * in_features up to 14336 takes a streaming GEMV in fp32 (no workspace:
 * mlk_linear_planar_workspace_bytes is 0); up to 32 rows run on the bf16
 * matrix cores with exact products (codes are exact in bf16 and x is split
 * into three exact bf16 pieces), and need a workspace of
 * mlk_linear_planar_workspace_bytes (16-byte aligned); more rows take the
 * tiled matrix-core GEMM (from 65 rows with in_features a multiple of 256,
 * on the same exact bf16 products), with the optional workspace of
 * mlk_linear_workspace_bytes.  No counterpart in the reference. */
mlk_status mlk_linear_planar(int32_t quant_type, const float* x, const void* w_planar,
                             const float* bias, float* y, int64_t rows, int64_t in_features,
                             int64_t out_features, void* workspace, size_t workspace_bytes,
                             void* stream);
int64_t mlk_linear_planar_workspace_bytes(int64_t rows, int64_t in_features,
                                          int64_t out_features);

/* c = a @ b for row-major a [m, k], b [k, n], c [m, n].  Replaces CudaMatmul
 * (include/cuda_matmul.h:7; src/cuda_matmul.cc:199-232). */
mlk_status mlk_matmul_f32(const float* a, const float* b, float* c, int64_t m, int64_t k,
                          int64_t n, void* stream);

/*
 * KV cache write: rows t of k and v (n_kv_heads * head_dim floats each, row
 * t at k + t * k_row_stride) go to slot (layer, pos_t) of the caches
 * [n_layers, max_seq, n_kv_heads, head_dim], pos_t = positions[t] (device
 * array) or pos0 + t.  A position outside [0, max_seq) writes nothing and,
 * when err != NULL, stores a nonzero value in *err (the caller clears it).
 * Replaces CudaCache::WriteDevice (include/cuda_kvcache.h:23;
 * src/cuda_kvcache.cc:209-237, two device copies per token).
 */
mlk_status mlk_kv_write_f32(float* k_cache, float* v_cache, int64_t n_layers, int64_t max_seq,
                            int32_t n_kv_heads, int32_t head_dim, int64_t layer, const float* k,
                            int64_t k_row_stride, const float* v, int64_t v_row_stride,
                            const int32_t* positions, int32_t pos0, int64_t n_tokens,
                            int32_t* err, void* stream);

/* Bytes of workspace mlk_attention_decode_f32 needs for these sizes (0 when
 * one chunk covers max_ctx and no workspace is used; 0 on bad input). */
int64_t mlk_attention_workspace_bytes(int64_t n_tokens, int32_t n_heads, int32_t n_kv_heads,
                                      int32_t head_dim, int64_t max_ctx);

/*
 * Decode attention over the cache of `layer`: for query row t (q row t at
 * q + t * q_row_stride, [n_heads, head_dim]) at position pos_t
 * (positions[t] or pos0 + t), query head i reads KV head
 * i / (n_heads / n_kv_heads):
 *   s_j = (q_i . k_j) / sqrt(head_dim),  p = softmax(s_0..s_pos),
 *   out[t, i] = sum_j p_j v_j
 * (src/forward.cc:265-298).  Every pos_t must be < max_ctx <= max_seq (a
 * bound the caller knows, e.g. the cache length); a position outside
 * [0, max_ctx) gives a zero row and raises *err.  head_dim <= 256.  When
 * mlk_attention_workspace_bytes() is nonzero, `workspace` must hold that many
 * bytes (chunk partials); out must not alias q.  Sums are fp32 in the
 * kernel's order (the reference's tolerance: 2e-5 against float64,
 * test/cuda_attention_test.cc:108-109); with head_dim 128, batches of 5 or
 * more tokens and the prefill kernel form each q.k and p.v product from the
 * six bf16 piece products above 2^-21 relative, so each product is within
 * 2^-20 of its exact value (fp32 rounds at 2^-24).  With positions == NULL, 16 or more
 * tokens, head_dim 64 or 128 and 16-byte aligned q rows, out and caches, the
 * call runs mlk_attention_prefill_f32's kernel; from 1024 tokens at head_dim
 * 128, a 16-byte aligned workspace of at least 12 * KV * head_dim *
 * (pos0 + n_tokens rounded up to 32) bytes lets it split K and V into bf16
 * pieces once (one extra launch) instead of in every workgroup, with the
 * same results; otherwise it uses no workspace.
 * Replaces CudaAttentionDevice (include/cuda_attention.h:12-13;
 * src/cuda_attention.cu:77-176, 2 launches, one cudaMalloc and a device
 * synchronize per call).
 */
mlk_status mlk_attention_decode_f32(const float* q, int64_t q_row_stride, const float* k_cache,
                                    const float* v_cache, int64_t n_layers, int64_t max_seq,
                                    int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                                    int64_t layer, const int32_t* positions, int32_t pos0,
                                    int64_t n_tokens, int64_t max_ctx, float* out,
                                    void* workspace, size_t workspace_bytes, int32_t* err,
                                    void* stream);

/*
 * mlk_attention_decode_f32 for callers that cannot allocate device memory
 * (code under HIP graph capture, serving loops and harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  Same arguments, semantics
 * and results as mlk_attention_decode_f32 without the workspace: the chunk
 * partials go to a fixed device array of the library, one per GPU, of
 * mlk_attention_noalloc_scratch_bytes() bytes (64 MiB).  The array is part of
 * the library's code object, so it is reserved on a GPU as soon as any
 * kernel of the library loads there (for every user of the library, whether
 * or not it calls this entry) and is held until the process ends.  Calls
 * needing more than that
 * (mlk_attention_workspace_bytes() of the shape) are rejected with
 * MLK_ERR_INVALID before any launch; at max_ctx 8192 every batch up to 256
 * tokens of the 8B and 70B head shapes fits.  Nothing is allocated and no
 * allocating routine is called.  Every call on one GPU uses the same array:
 * calls that overlap on one GPU (other streams, other threads) race.
 */
mlk_status mlk_attention_decode_f32_noalloc(const float* q, int64_t q_row_stride,
                                            const float* k_cache, const float* v_cache,
                                            int64_t n_layers, int64_t max_seq, int32_t n_heads,
                                            int32_t n_kv_heads, int32_t head_dim, int64_t layer,
                                            const int32_t* positions, int32_t pos0,
                                            int64_t n_tokens, int64_t max_ctx, float* out,
                                            int32_t* err, void* stream);
/* Bytes of that fixed device array. */
size_t mlk_attention_noalloc_scratch_bytes(void);

/*
 * Causal attention of a prompt chunk: tokens t < n_tokens at positions
 * pos0 + t (their K/V rows already in the cache, e.g. by mlk_kv_write_f32),
 * token t attending to cache positions 0 .. pos0 + t -- the per-token
 * attention of ForwardBatch's token loop (src/forward.cc:482-486, each step
 * src/forward.cc:265-298) for the whole chunk in one launch, on the matrix
 * cores.  Same semantics, layout and error bound as mlk_attention_decode_f32
 * with positions == NULL; needs head_dim 64 or 128, q_row_stride % 4 == 0,
 * 16-byte aligned q, out and caches, pos0 + n_tokens <= max_seq.  No
 * workspace.  No counterpart in the reference's device code (it ran the
 * decode kernel once per token).
 */
mlk_status mlk_attention_prefill_f32(const float* q, int64_t q_row_stride, const float* k_cache,
                                     const float* v_cache, int64_t n_layers, int64_t max_seq,
                                     int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                                     int64_t layer, int32_t pos0, int64_t n_tokens, float* out,
                                     void* stream);

/* ------------------------------------------------------ batched forward
 * One transformer layer over a batch of tokens: the reference's
 * ForwardLayerDevice (src/forward.cc:337-384) for all tokens at once, i.e.
 * ForwardBatch (src/forward.cc:473-488) without its token loop, layer by
 * layer.  No counterpart in the reference (its batch runs one token at a
 * time through the whole model). */

enum { MLK_WEIGHT_F32 = -1 };  /* mlk_linear_weight.type of fp32 weights */

typedef struct {
    int32_t type;        /* MLK_WEIGHT_F32, MLK_Q8_0, MLK_Q4_0 or MLK_Q4_1 */
    const void* data;    /* [out, in]: fp32 row-major, or out rows of ceil(in / 32) blocks */
    const float* bias;   /* [out] or NULL */
    const void* planar;  /* NULL, or the same Q8_0 / Q4_0 weight in the planar layout
                            (mlk_quant_to_planar, 16-byte aligned): calls of 1..32 tokens
                            then run on it.  No counterpart in the reference. */
} mlk_linear_weight;

/* A layer's device weights (the reference's Layer, include/model.h:41-55). */
typedef struct {
    const float* attention_norm;          /* [dim] */
    mlk_linear_weight wq, wk, wv, wo;     /* [H*hd, dim], [KV*hd, dim] x2, [dim, H*hd] */
    const float* ffn_norm;                /* [dim] */
    mlk_linear_weight w_gate, w_up, w_down; /* [hidden, dim] x2, [dim, hidden] */
} mlk_layer_weights;

/* The ModelConfig fields a layer uses (include/model.h:57-81). */
typedef struct {
    int64_t dim, hidden_dim;
    int32_t n_heads, n_kv_heads, head_dim, rope_type;  /* rope_type: mlk_rope_type */
    float rope_theta, rms_norm_eps;
} mlk_layer_config;

/* Device bytes of the workspace of mlk_forward_layer_batch for n_tokens
 * tokens attending up to max_ctx positions; consecutive_positions != 0 when
 * the call passes positions == NULL (0 on bad input).  A prompt chunk of
 * 1024 or more tokens at head_dim 128 includes the attention's pre-split
 * K/V (12 bytes per cached K and V element of a layer up to max_ctx), and
 * more than 64 tokens the bf16 planes of the normed rows (6 * n_tokens *
 * dim bytes). */
int64_t mlk_forward_layer_workspace_bytes(const mlk_layer_config* cfg, int64_t n_tokens,
                                          int64_t max_ctx, int32_t consecutive_positions);

/*
 * x [n_tokens, dim] (the residual stream, updated in place) through layer
 * `layer`: RmsNorm -> q/k/v linears (+ bias) -> RoPE -> K/V rows written to
 * the caches -> attention -> wo, residual add -> RmsNorm -> SwiGLU FFN,
 * residual add, with the reference's op semantics (each op as its own entry
 * above documents).  Token t sits at positions[t] (device array) or
 * pos0 + t (positions == NULL); all tokens' K/V rows are written before
 * any token attends, so the result equals the reference's token loop when
 * the positions increase along the batch.  Every position is < max_ctx <=
 * max_seq.  The workspace (256-byte aligned, at least
 * mlk_forward_layer_workspace_bytes(cfg, n_tokens, max_ctx, positions ==
 * NULL)) holds every intermediate; the caches must be 16-byte aligned.  A device-side position error raises
 * *err as the op entries do.
 */
mlk_status mlk_forward_layer_batch(const mlk_layer_config* cfg, const mlk_layer_weights* w,
                                   float* x, int64_t n_tokens, const int32_t* positions,
                                   int32_t pos0, float* k_cache, float* v_cache,
                                   int64_t n_layers, int64_t max_seq, int64_t layer,
                                   int64_t max_ctx, void* workspace, size_t workspace_bytes,
                                   int32_t* err, void* stream);

/* Synthetic-input helper (not a reference op): fills x[i] with
 * mean + std * N(0,1) from a counter-based generator keyed by seed and i, so
 * the values do not depend on launch shape. */
mlk_status mlk_fill_normal_f32(float* x, int64_t n, float mean, float std, uint64_t seed,
                               void* stream);

/* -------------------------------------------------------------- runtime
 * A thin layer over the HIP runtime for hosts that do not link HIP
 * themselves (the C++ op surface, ctypes).  Replaces the cudart calls of
 * src/cuda_runtime.cc:57-161. */

typedef enum { MLK_H2D = 0, MLK_D2D = 1, MLK_D2H = 2 } mlk_copy_kind;

typedef struct {
    int device_id;
    char name[256];
    char arch[64];          /* gcnArchName, e.g. gfx950:sramecc+:xnack- */
    int compute_major;
    int compute_minor;
    size_t total_bytes;
    int multiprocessors;    /* compute units */
    int clock_khz;
    int memory_clock_khz;
    int memory_bus_bits;
    int runtime_version;
    int driver_version;
} mlk_device_info;

mlk_status mlk_device_count(int* count);
mlk_status mlk_set_device(int device_id);
mlk_status mlk_get_device(int* device_id);
mlk_status mlk_get_device_info(int device_id, mlk_device_info* info);
mlk_status mlk_malloc(void** ptr, size_t bytes);
mlk_status mlk_free(void* ptr);
/* Synchronous copy (hipMemcpy semantics). */
mlk_status mlk_memcpy(void* dst, const void* src, size_t bytes, int32_t kind);
mlk_status mlk_memcpy_async(void* dst, const void* src, size_t bytes, int32_t kind,
                            void* stream);
/* Fills bytes with zero through a kernel (safe under graph capture). */
mlk_status mlk_zero_async(void* dst, size_t bytes, void* stream);
mlk_status mlk_device_synchronize(void);
mlk_status mlk_stream_create(void** stream);
mlk_status mlk_stream_destroy(void* stream);
mlk_status mlk_stream_synchronize(void* stream);
mlk_status mlk_event_create(void** event);
mlk_status mlk_event_destroy(void* event);
mlk_status mlk_event_record(void* event, void* stream);
mlk_status mlk_event_synchronize(void* event);
mlk_status mlk_event_elapsed_ms(float* ms, void* start, void* stop);

/* HIP graphs for launch-bound sequences (decode steps issue a handful of
 * microsecond kernels): capture the ops issued on `stream` (not the null
 * stream) between begin and end into an executable graph, then replay it
 * with one launch.  The ops above record kernels only (no memset or copy
 * nodes), so a captured sequence replays exactly.  The kernels' pointer
 * and size arguments are frozen at capture time. */
mlk_status mlk_graph_begin_capture(void* stream);
mlk_status mlk_graph_end_capture(void* stream, void** graph_exec);
mlk_status mlk_graph_launch(void* graph_exec, void* stream);
mlk_status mlk_graph_destroy(void* graph_exec);

#ifdef __cplusplus
}
#endif

#endif
