// mlk_attention.h -- the causal prefill attention kernel (mlk_prefill.hip)
// as used by the attention entry points (mlk_attention.hip).
#pragma once

#include "mlk_common.h"

namespace mlk {

// The prefill kernel handles head_dim 64 and 128 with 16-byte aligned q
// rows (q_row_stride % 4 == 0), output and caches.
bool PrefillSupported(int32_t head_dim, const float* q, int64_t q_row_stride, const float* out,
                      const float* k_cache, const float* v_cache);

// Tokens t < T at positions pos0 + t, each attending to cache positions
// 0 .. pos0 + t; kc / vc point at the layer's [max_seq, KV, head_dim] slice,
// slot = KV * head_dim floats per position.  Arguments already validated.
// With a 16-byte aligned workspace of PrefillImageBytes(KV, head_dim,
// pos0 + T) bytes (head_dim 128, T >= kPrefillImageMinTokens), K and V of
// positions 0 .. pos0 + T - 1 are first split into bf16 piece images, one
// launch, which the tiles then copy instead of splitting each tile in every
// workgroup; the sums are the same.  Otherwise no workspace is used.  Below
// that many tokens a tile is staged by too few workgroups for the extra
// launch to pay (Llama-3-70B heads, T = 512: 44 -> 48 us with the images;
// T = 4096: 1569 -> 1443 us).  a_planes (16-byte aligned, H * head_dim a
// multiple of 32), when set, also receives the output rows as StorePlanes
// planes.
constexpr int64_t kPrefillImageMinTokens = 1024;
int64_t PrefillImageBytes(int32_t n_kv_heads, int32_t head_dim, int64_t n_pos);
mlk_status LaunchPrefill(const float* q, int64_t q_row_stride, const float* kc, const float* vc,
                         int64_t slot, int32_t H, int32_t KV, int32_t head_dim, int32_t pos0,
                         int64_t T, float* out, hipStream_t s, void* workspace = nullptr,
                         size_t workspace_bytes = 0, uint32_t* a_planes = nullptr);

// Decode tokens at any positions (positions[t], or pos0 + t) on the same
// matrix-core tiles: a workgroup holds 16 tokens and shares each K/V tile
// among them, over one chunk of TileChunk() cache positions.  With more than
// one chunk it writes (acc, m, l) partials to ws_acc / ws_ml ([T, H, n_chunks,
// hd] / [.., 2], n_chunks = ceil(max_ctx / chunk)) for AttnCombine; with one
// it writes out.  Invalid positions raise err (their rows are zeroed by the
// merge, or here with one chunk).  Arguments already validated.
int TileChunk(int64_t T, int32_t H, int32_t KV, int64_t max_ctx);
mlk_status LaunchDecodeTile(const float* q, int64_t q_row_stride, const float* kc,
                            const float* vc, int64_t slot, int32_t H, int32_t KV,
                            int32_t head_dim, const int32_t* positions, int32_t pos0, int64_t T,
                            int64_t max_ctx, float* out, float* ws_acc, float* ws_ml,
                            int32_t* err, hipStream_t s);

// mlk_attention_decode_f32 with one more output: when the chunk merge runs
// (more than one chunk of cache positions) and planes is not null, the merge
// also writes out's bf16 planes (StorePlanes1 over rows of n_heads * head_dim,
// which must be a multiple of 32) and sets *planes_written, and so does the
// prefill kernel (positions == NULL, 16 or more tokens); otherwise planes
// are untouched and *planes_written is false.
mlk_status AttentionDecode(const float* q, int64_t q_row_stride, const float* k_cache,
                           const float* v_cache, int64_t n_layers, int64_t max_seq,
                           int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, int64_t layer,
                           const int32_t* positions, int32_t pos0, int64_t n_tokens,
                           int64_t max_ctx, float* out, void* workspace, size_t workspace_bytes,
                           int32_t* err, void* stream, uint32_t* planes, bool* planes_written);

}  // namespace mlk
