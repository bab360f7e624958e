// mlk_forward.hip -- one transformer layer over a batch of tokens: the
// reference's ForwardLayerDevice (src/forward.cc:337-384; CPU twin
// ForwardLayer :385-414) for all T tokens at once, which replaces the token
// loop of ForwardBatch (:473-488) layer by layer.
//
// Per layer, on one stream (x [T, dim] is the residual stream, in place;
// for 1 and for 2..32 tokens with quantized weights q/k/v are one launch,
// gate/up carry the SwiGLU and the down projection adds into x; for many
// tokens over Q8_0 / Q4_0 blocks gate/up carry the SwiGLU, wo and down add
// into x and k, v may share one launch; with separate q/k/v launches at
// consecutive positions k and v are written to their cache rows and
// rotated there, with no copy; see below):
//   h = RmsNorm(x, attention_norm)                    mlk_rmsnorm_f32
//   q, k, v = h W^T (+ bias)                          mlk_linear_* (GEMM from 8 rows)
//   RoPE(q, k) at each token's position               mlk_rope_f32
//   write k, v to the cache; a = attention(q)         mlk_kv_write_f32, then
//                                                     mlk_attention_prefill_f32
//                                                     (consecutive positions)
//                                                     or mlk_attention_decode_f32
//   x += a Wo^T; h = RmsNorm(x, ffn_norm)             mlk_linear_*, mlk_add_rmsnorm_f32
//   g = h Wgate^T, u = h Wup^T; g = silu(g) * u       mlk_linear_*, mlk_swiglu_f32
//   x += g Wdown^T                                    mlk_linear_*, mlk_add_f32
// Every op keeps the reference's arithmetic (the fused residual add and
// RmsNorm computes r = x + delta in fp32 and then RmsNorm(r), as
// ForwardAdd + ForwardRmsForm do); the linear sums and the attention sums
// are fp32 in the kernels' orders.  All K/V rows of the batch are written
// before any token attends, so the batch equals the token loop when the
// positions increase from token to token (a later token never writes a slot
// an earlier one reads).
//
// The intermediates live in the caller's workspace (no allocation here):
// h, q, k, v, a, a Wo^T, gate, up, then the linear layers' split-K scratch
// and the decode attention's chunk scratch, each 256-byte aligned.
#include "mlk_attention.h"
#include "mlk_common.h"
#include "mlk_quant.h"

#include <algorithm>
#include <initializer_list>

namespace mlk {
namespace {

constexpr int kLinearF32 = MLK_WEIGHT_F32;

struct Plan {
    int64_t off[11];  // float offsets: h q k v a proj gate up | byte offsets: lin att planes
    int64_t lin_bytes = 0, att_bytes = 0, plane_bytes = 0, total = 0;
};

int64_t Align256(int64_t bytes) { return (bytes + 255) / 256 * 256; }

bool Contiguous(const int32_t* positions) { return positions == nullptr; }

// Token counts whose linear layers run the skinny GEMM (8..32 rows): with
// quantized weights the layer fuses them as the one-token path does, with
// the epilogues in the split-K reduction.
bool FusedRows(int64_t T) { return T >= 8 && T <= 32; }

// Token counts that take the planar weights when a layer has them (the
// bf16 kernel, fused as FusedRows; one token keeps the block-layout GEMVs).
bool PlanarRows(int64_t T) { return T >= 2 && T <= 32; }

Plan MakePlan(const mlk_layer_config& c, int64_t T, int64_t max_ctx, bool contiguous) {
    const int64_t D = c.dim, F = c.hidden_dim;
    const int64_t QD = static_cast<int64_t>(c.n_heads) * c.head_dim;
    const int64_t KD = static_cast<int64_t>(c.n_kv_heads) * c.head_dim;
    const int64_t sizes[8] = {T * D, T * QD, T * KD, T * KD, T * QD, T * D, T * F, T * F};
    Plan p;
    int64_t at = 0;
    for (int i = 0; i < 8; ++i) {
        p.off[i] = at;
        at += Align256(sizes[i] * 4);
    }
    const int64_t shapes[5][2] = {{D, QD}, {D, KD}, {QD, D}, {D, F}, {F, D}};  // (in, out)
    for (const auto& s : shapes) {
        const int64_t b = mlk_linear_workspace_bytes(T, s[0], s[1]);
        if (b > p.lin_bytes) p.lin_bytes = b;
    }
    if (FusedRows(T)) {  // q/k/v, gate/up and down as fused skinny launches
        const int64_t fused[3][2] = {{D, QD + 2 * KD}, {D, 2 * F}, {F, D}};  // (in, all outputs)
        for (const auto& s : fused) {
            const int64_t b = SkinnyFusedWorkspaceBytes(MLK_Q8_0, T, s[0], s[1]);
            if (b > p.lin_bytes) p.lin_bytes = b;
        }
    }
    if (PlanarRows(T)) {  // the same groups (and wo) on planar weights
        const int64_t groups[4][3] = {{D, QD + 2 * KD, 1}, {D, 2 * F, 1}, {F, D, 1}, {QD, D, 1}};
        for (const auto& g : groups) {
            if (g[0] % 256 != 0) continue;
            const int64_t b = PlanarWorkspaceBytes(T, g[0], g[1], g[2] != 0);
            if (b > p.lin_bytes) p.lin_bytes = b;
        }
    }
    p.off[8] = at;
    at += Align256(p.lin_bytes);
    // the decode kernel's chunk scratch, for the calls that take that path;
    // a prompt chunk's pre-split K/V tile images (positions up to max_ctx)
    const bool prefill = contiguous && T >= 16 && (c.head_dim == 64 || c.head_dim == 128);
    p.att_bytes = prefill ? (T >= kPrefillImageMinTokens
                                 ? PrefillImageBytes(c.n_kv_heads, c.head_dim, max_ctx)
                                 : 0)
                          : mlk_attention_workspace_bytes(T, c.n_heads, c.n_kv_heads, c.head_dim,
                                                          max_ctx);
    p.off[9] = at;
    at += Align256(p.att_bytes);
    // bf16 planes of the planar layers' x (h, attention's output, then
    // SwiGLU's output)
    const int64_t widest = std::max(D, std::max(F, QD));
    // (many tokens: h's planes for the tiled q, k/v and gate/up launches,
    // and the prefill attention's output planes for wo)
    p.plane_bytes = PlanarRows(T) ? T * widest * 6
                                  : (T > 64 && D % 32 == 0 ? T * std::max(D, QD) * 6 : 0);
    p.off[10] = at;
    at += Align256(p.plane_bytes);
    p.total = at;
    return p;
}

mlk_status Linear(const mlk_linear_weight& w, const float* x, float* y, int64_t T, int64_t in,
                  int64_t out, void* ws, size_t ws_bytes, void* stream) {
    if (w.type == kLinearF32) {
        return mlk_linear_f32(x, static_cast<const float*>(w.data), w.bias, y, T, in, out, ws,
                              ws_bytes, stream);
    }
    return mlk_linear_quant(w.type, x, w.data, w.bias, y, T, in, out, ws, ws_bytes, stream);
}

// A weight the one-row streaming GEMV takes (quantized, in_features a
// multiple of 64 that fits its LDS, 4-byte aligned blocks).
bool RowStreamable(const mlk_linear_weight& w, int64_t in) {
    return w.type != kLinearF32 && StreamFits(in) && Aligned(w.data, 4);
}

StreamSeg Seg(const mlk_linear_weight& w, float* y, int64_t rows, const float* res = nullptr) {
    return StreamSeg{static_cast<const uint8_t*>(w.data), w.bias, y, res, rows, 0};
}

// The weights of a group run planar: T in PlanarRows, all Q8_0 or all
// Q4_0 with planar copies, in_features a multiple of 256.
bool Planar(int64_t T, int64_t in, std::initializer_list<const mlk_linear_weight*> ws) {
    const int t = (*ws.begin())->type;
    if (!PlanarRows(T) || in % 256 != 0 || (t != MLK_Q8_0 && t != MLK_Q4_0)) return false;
    for (const mlk_linear_weight* w : ws) {
        if (w->type != t || w->planar == nullptr) return false;
    }
    return true;
}

// One token over planar copies (LinearRowPlanar): all Q8_0 or all Q4_0 with
// planar copies, in_features within the kernel's reach for `mode`.
bool PlanarRow(int64_t in, std::initializer_list<const mlk_linear_weight*> ws,
               int mode = kStreamPlain, bool norm = false) {
    const int t = (*ws.begin())->type;
    if ((t != MLK_Q8_0 && t != MLK_Q4_0) || !RowPlanarApplies(t, in, mode, norm)) return false;
    for (const mlk_linear_weight* w : ws) {
        if (w->type != t || w->planar == nullptr) return false;
    }
    return true;
}

StreamSeg PlanarSeg(const mlk_linear_weight& w, float* y, int64_t rows,
                    const float* res = nullptr) {
    return StreamSeg{static_cast<const uint8_t*>(w.planar), w.bias, y, res, rows, 0};
}

mlk_status CheckConfig(const char* fn, const mlk_layer_config* c) {
    if (c == nullptr) return Fail(MLK_ERR_INVALID, "%s: config must not be null", fn);
    if (c->dim <= 0 || c->hidden_dim <= 0 || c->n_heads <= 0 || c->n_kv_heads <= 0 ||
        c->head_dim <= 0 || c->n_heads % c->n_kv_heads != 0) {
        return Fail(MLK_ERR_INVALID,
                    "%s: dims and head counts must be positive and n_kv_heads must divide "
                    "n_heads (dim %lld, hidden %lld, heads %d / %d, head_dim %d)",
                    fn, static_cast<long long>(c->dim), static_cast<long long>(c->hidden_dim),
                    c->n_heads, c->n_kv_heads, c->head_dim);
    }
    return MLK_OK;
}

mlk_status CheckWeight(const char* fn, const char* name, const mlk_linear_weight& w) {
    if (w.data == nullptr) return Fail(MLK_ERR_INVALID, "%s: weight %s is null", fn, name);
    if (w.type != kLinearF32 && (w.type < MLK_Q8_0 || w.type > MLK_Q4_1)) {
        return Fail(MLK_ERR_INVALID, "%s: weight %s has unknown type %d", fn, name, w.type);
    }
    if (w.planar != nullptr &&
        ((w.type != MLK_Q8_0 && w.type != MLK_Q4_0) || !Aligned(w.planar, 16))) {
        return Fail(MLK_ERR_INVALID,
                    "%s: weight %s: a planar copy needs Q8_0 or Q4_0 and 16-byte alignment", fn,
                    name);
    }
    return MLK_OK;
}

}  // namespace
}  // namespace mlk

using namespace mlk;

extern "C" {

int64_t mlk_forward_layer_workspace_bytes(const mlk_layer_config* cfg, int64_t n_tokens,
                                          int64_t max_ctx, int32_t consecutive_positions) {
    if (cfg == nullptr || n_tokens <= 0 || max_ctx <= 0 ||
        CheckConfig("mlk_forward_layer_workspace_bytes", cfg) != MLK_OK) {
        return 0;
    }
    return MakePlan(*cfg, n_tokens, max_ctx, consecutive_positions != 0).total;
}

mlk_status mlk_forward_layer_batch(const mlk_layer_config* cfg, const mlk_layer_weights* w,
                                   float* x, int64_t n_tokens, const int32_t* positions,
                                   int32_t pos0, float* k_cache, float* v_cache,
                                   int64_t n_layers, int64_t max_seq, int64_t layer,
                                   int64_t max_ctx, void* workspace, size_t workspace_bytes,
                                   int32_t* err, void* stream) {
    const char* fn = "mlk_forward_layer_batch";
    mlk_status st = CheckConfig(fn, cfg);
    if (st != MLK_OK) return st;
    if (w == nullptr || x == nullptr) return Fail(MLK_ERR_INVALID, "%s: weights and x must not be null", fn);
    if (w->attention_norm == nullptr || w->ffn_norm == nullptr) {
        return Fail(MLK_ERR_INVALID, "%s: norm weights must not be null", fn);
    }
    const struct {
        const char* name;
        const mlk_linear_weight* w;
    } lins[] = {{"wq", &w->wq}, {"wk", &w->wk}, {"wv", &w->wv}, {"wo", &w->wo},
                {"w_gate", &w->w_gate}, {"w_up", &w->w_up}, {"w_down", &w->w_down}};
    for (const auto& l : lins) {
        st = CheckWeight(fn, l.name, *l.w);
        if (st != MLK_OK) return st;
    }
    if (n_tokens <= 0) return Fail(MLK_ERR_INVALID, "%s: n_tokens must be positive", fn);
    if (k_cache == nullptr || v_cache == nullptr || k_cache == v_cache) {
        return Fail(MLK_ERR_INVALID, "%s: key and value caches must be distinct buffers", fn);
    }
    if (!Aligned(k_cache, 16) || !Aligned(v_cache, 16)) {
        return Fail(MLK_ERR_INVALID, "%s: the caches must be 16-byte aligned", fn);
    }
    if (n_layers <= 0 || max_seq <= 0 || max_seq > 0x7FFFFFFF) {
        return Fail(MLK_ERR_INVALID, "%s: cache dimensions out of range (layers %lld, max_seq %lld)",
                    fn, static_cast<long long>(n_layers), static_cast<long long>(max_seq));
    }
    if (layer < 0 || layer >= n_layers) {
        return Fail(MLK_ERR_RANGE, "%s: layer %lld out of range [0, %lld)", fn,
                    static_cast<long long>(layer), static_cast<long long>(n_layers));
    }
    const bool contiguous = Contiguous(positions);
    if (contiguous && pos0 < 0) {
        return Fail(MLK_ERR_RANGE, "%s: positions %d..%lld out of range (pos must be "
                    "non-negative)", fn, pos0, static_cast<long long>(pos0 + n_tokens - 1));
    }
    if (max_ctx <= 0 || max_ctx > max_seq || (contiguous && pos0 + n_tokens > max_ctx)) {
        return Fail(MLK_ERR_RANGE, "%s: max_ctx %lld must cover the positions and be <= max_seq "
                    "%lld", fn, static_cast<long long>(max_ctx), static_cast<long long>(max_seq));
    }
    const Plan p = MakePlan(*cfg, n_tokens, max_ctx, contiguous);
    if (workspace == nullptr || static_cast<int64_t>(workspace_bytes) < p.total ||
        !Aligned(workspace, 256)) {
        return Fail(MLK_ERR_INVALID,
                    "%s: a 256-byte aligned workspace of %lld bytes is needed (got %zu)", fn,
                    static_cast<long long>(p.total), workspace_bytes);
    }
    const mlk_layer_config& c = *cfg;
    const int64_t T = n_tokens, D = c.dim, F = c.hidden_dim;
    const int64_t QD = static_cast<int64_t>(c.n_heads) * c.head_dim;
    const int64_t KD = static_cast<int64_t>(c.n_kv_heads) * c.head_dim;
    char* base = static_cast<char*>(workspace);
    auto buf = [&](int i) { return reinterpret_cast<float*>(base + p.off[i]); };
    float *h = buf(0), *q = buf(1), *k = buf(2), *v = buf(3), *a = buf(4), *proj = buf(5),
          *gate = buf(6), *up = buf(7);
    void* lin_ws = p.lin_bytes > 0 ? base + p.off[8] : nullptr;
    void* att_ws = p.att_bytes > 0 ? base + p.off[9] : nullptr;
    uint32_t* planes = p.plane_bytes > 0 ? reinterpret_cast<uint32_t*>(base + p.off[10]) : nullptr;
    const size_t lin_b = static_cast<size_t>(p.lin_bytes);
    const float eps = c.rms_norm_eps;

#define MLK_TRY(call)              \
    do {                           \
        const mlk_status s_ = (call); \
        if (s_ != MLK_OK) return s_;  \
    } while (0)
    // One token (the decode step) with quantized weights: q, k and v in one
    // launch, gate and up with SwiGLU in the epilogue, and the down
    // projection adding into x (the same per-element arithmetic as the
    // separate kernels), over the planar copies where a group has them
    // (contiguous loads), else over the blocks.  8..32 tokens: the same
    // groups as skinny GEMM launches, with the epilogues in their split-K
    // reductions.
    const hipStream_t hs = AsStream(stream);
    const bool row = T == 1;
    // one token on planar copies: the same launches over the planar layout
    const bool qkv1p = row && PlanarRow(D, {&w->wq, &w->wk, &w->wv}, kStreamQkvRope);
    const bool ffn1p = row && PlanarRow(D, {&w->w_gate, &w->w_up}, kStreamSwiGlu);
    const bool down1p = row && PlanarRow(F, {&w->w_down}, kStreamAdd);
    const bool wo1p = row && PlanarRow(QD, {&w->wo});
    const bool qkv1 = qkv1p || (row && w->wq.type == w->wk.type && w->wq.type == w->wv.type &&
                                RowStreamable(w->wq, D) && RowStreamable(w->wk, D) &&
                                RowStreamable(w->wv, D));
    const bool ffn1 = ffn1p || (row && w->w_gate.type == w->w_up.type &&
                                RowStreamable(w->w_gate, D) && RowStreamable(w->w_up, D));
    const bool down1 = down1p || (row && RowStreamable(w->w_down, F));
    // 2..32 tokens on planar copies: the same three groups, plus wo
    const bool qkvp = Planar(T, D, {&w->wq, &w->wk, &w->wv});
    const bool ffnp = Planar(T, D, {&w->w_gate, &w->w_up});
    const bool downp = Planar(T, F, {&w->w_down});
    const bool wop = Planar(T, QD, {&w->wo});
    const bool mid = FusedRows(T);
    const bool qkvm = qkvp || (mid && w->wq.type == w->wk.type && w->wq.type == w->wv.type &&
                               w->wq.type != kLinearF32 && SkinnyFusedApplies(w->wq.type, T, D));
    const bool ffnm = ffnp || (mid && w->w_gate.type == w->w_up.type &&
                               w->w_gate.type != kLinearF32 &&
                               SkinnyFusedApplies(w->w_gate.type, T, D));
    const bool downm = downp || (mid && w->w_down.type != kLinearF32 &&
                                 SkinnyFusedApplies(w->w_down.type, T, F));
    // The separate q/k/v launches at consecutive positions (pos0 + T <=
    // max_ctx <= max_seq, checked above): k and v go straight to their cache
    // rows, which RoPE then rotates in place, so no copy launch; for many
    // tokens k and v run as one launch where that fills the GPU without a K
    // split (each split alone)
    const bool kv_direct = !(qkv1 || qkvm) && contiguous;
    float* const k_rows = kv_direct ? k_cache + (layer * max_seq + pos0) * KD : k;
    float* const v_rows = kv_direct ? v_cache + (layer * max_seq + pos0) * KD : v;
    const bool kv_pair = !(qkv1 || qkvm) && w->wk.type == w->wv.type &&
                         TiledFusedApplies(w->wk.type, T, D, KD, kStreamPlain) &&
                         Aligned(w->wk.data, 2) && Aligned(w->wv.data, 2);
    // q alone on the tiled launch when h's planes are at hand (below)
    const bool q_tiled = !(qkv1 || qkvm) && TiledFusedApplies(w->wq.type, T, D, QD, kStreamAdd) &&
                         Aligned(w->wq.data, 2);
    // Many tokens (128-row tiles, K in one pass): the same groups' epilogues
    // in the GEMM itself, gate/up as one launch with SwiGLU, wo and down
    // adding into x (the plain GEMM's sums, so the separate kernels' values)
    const bool wo_add = !wop && !wo1p && TiledFusedApplies(w->wo.type, T, QD, D, kStreamAdd) &&
                        Aligned(w->wo.data, 2);
    const bool ffn_tiled = !ffn1 && !ffnp && !ffnm && w->w_gate.type == w->w_up.type &&
                           TiledFusedApplies(w->w_gate.type, T, D, F, kStreamSwiGlu) &&
                           Aligned(w->w_gate.data, 2) && Aligned(w->w_up.data, 2);
    const bool down_tiled = !down1 && !downp && !downm &&
                            TiledFusedApplies(w->w_down.type, T, F, D, kStreamAdd) &&
                            Aligned(w->w_down.data, 2);
    // The fused q/k/v launches also rotate q and k (normal-layout pairs) and
    // write k and v into the cache rows, in place of mlk_rope_f32 and
    // mlk_kv_write_f32; the NeoX layout keeps the separate launches.
    const bool rope_fused = (qkvm || qkv1p || (qkv1 && StreamRopeFits(D, c.head_dim))) &&
                            c.rope_type == MLK_ROPE_NORMAL && c.head_dim % 2 == 0 &&
                            c.head_dim <= 2 * kRopePairs;
    if (rope_fused && positions == nullptr && (pos0 < 0 || pos0 + T > max_seq)) {
        return Fail(MLK_ERR_RANGE, "%s: positions %d..%lld out of range [0, %lld)", fn, pos0,
                    static_cast<long long>(pos0 + T - 1), static_cast<long long>(max_seq));
    }
    // one token: each norm folded into the streaming GEMV that reads its
    // output (the same sums in the same order), where the norm kernel's
    // block shape allows it; the ffn norm's residual x + proj then goes to
    // h's buffer and the down projection adds into x from there
    int nw = 0, nvpt = 0;
    const bool norm_fold = NormShape(x, proj, w->attention_norm, h, D, &nw, &nvpt) &&
                           Aligned(w->ffn_norm, 16) && (nw == 8 || nw == 16) && nvpt <= 2;
    const bool attn_fold =
        qkv1 && norm_fold &&
        (!qkv1p || RowPlanarApplies(w->wq.type, D, rope_fused ? kStreamQkvRope : kStreamPlain,
                                    true));
    const bool ffn_fold = ffn1 && down1 && norm_fold &&
                          (!ffn1p || RowPlanarApplies(w->w_gate.type, D, kStreamSwiGlu, true));
    // planar q/k/v: the norm also writes h's bf16 planes (no split launch)
    const uint32_t* h_planes = nullptr;
    if (attn_fold) {
        // in the q/k/v launch below
    } else if ((qkvp || q_tiled || kv_pair) && planes != nullptr &&
               NormPlanesApplies(x, nullptr, w->attention_norm, h, D)) {
        MLK_TRY(AddRmsNormPlanes(x, nullptr, w->attention_norm, h, planes, T, D, eps, hs));
        h_planes = planes;
    } else {
        MLK_TRY(mlk_rmsnorm_f32(x, w->attention_norm, h, T, D, eps, stream));
    }
    if (qkv1 || qkvm) {
        const int64_t slot = KD;
        float* ky = rope_fused ? k_cache + layer * max_seq * slot : k;
        float* vy = rope_fused ? v_cache + layer * max_seq * slot : v;
        StreamArgs a{};
        const bool pl = qkvp || qkv1p;
        a.seg[0] = pl ? PlanarSeg(w->wq, q, QD) : Seg(w->wq, q, QD);
        a.seg[1] = pl ? PlanarSeg(w->wk, ky, KD) : Seg(w->wk, ky, KD);
        a.seg[2] = pl ? PlanarSeg(w->wv, vy, KD) : Seg(w->wv, vy, KD);
        a.n_seg = 3;
        a.rope = RopeArgs{positions, pos0, c.head_dim, slot, max_seq, err,
                          MakeRopeFreqs(c.rope_theta, c.head_dim)};
        const int mode = rope_fused ? kStreamQkvRope : kStreamPlain;
        if (qkv1 && attn_fold) {
            a.norm = StreamNorm{w->attention_norm, nullptr, nullptr, eps, nw, nvpt};
            MLK_TRY(qkv1p ? LinearRowPlanar(w->wq.type, x, D, a, mode, hs)
                          : LinearRowStream(w->wq.type, x, D, a, mode, hs));
        } else if (qkv1) {
            MLK_TRY(qkv1p ? LinearRowPlanar(w->wq.type, h, D, a, mode, hs)
                          : LinearRowStream(w->wq.type, h, D, a, mode, hs));
        } else if (qkvp) {
            MLK_TRY(LinearPlanarFused(w->wq.type, h, T, D, a, mode, lin_ws, lin_b, hs, h_planes));
        } else {
            MLK_TRY(LinearSkinnyFused(w->wq.type, h, T, D, a, mode, lin_ws, lin_b, hs));
        }
    } else {
        if (q_tiled && h_planes != nullptr) {  // h's planes instead of splitting h per tile
            StreamArgs a{};
            a.seg[0] = Seg(w->wq, q, QD);
            a.n_seg = 1;
            a.x_planes = h_planes;
            MLK_TRY(LinearTiledFused(w->wq.type, h, T, D, a, kStreamPlain, hs));
        } else {
            MLK_TRY(Linear(w->wq, h, q, T, D, QD, lin_ws, lin_b, stream));
        }
        if (kv_pair) {
            StreamArgs a{};
            a.seg[0] = Seg(w->wk, k_rows, KD);
            a.seg[1] = Seg(w->wv, v_rows, KD);
            a.n_seg = 2;
            a.x_planes = h_planes;
            MLK_TRY(LinearTiledFused(w->wk.type, h, T, D, a, kStreamPlain, hs));
        } else {
            MLK_TRY(Linear(w->wk, h, k_rows, T, D, KD, lin_ws, lin_b, stream));
            MLK_TRY(Linear(w->wv, h, v_rows, T, D, KD, lin_ws, lin_b, stream));
        }
    }
    if (!rope_fused) {
        MLK_TRY(mlk_rope_f32(q, k_rows, T, c.n_heads, c.n_kv_heads, c.head_dim, QD, KD, positions,
                             pos0, c.rope_theta, c.rope_type, err, stream));
        if (!kv_direct) {
            MLK_TRY(mlk_kv_write_f32(k_cache, v_cache, n_layers, max_seq, c.n_kv_heads,
                                     c.head_dim, layer, k, KD, v, KD, positions, pos0, T, err,
                                     stream));
        }
    }
    // the chunk merge also writes a's planes for a planar wo (over h's: the
    // q/k/v GEMM has read them)
    bool a_planes = false;
    MLK_TRY(AttentionDecode(q, QD, k_cache, v_cache, n_layers, max_seq, c.n_heads, c.n_kv_heads,
                            c.head_dim, layer, positions, pos0, T, max_ctx, a, att_ws,
                            static_cast<size_t>(p.att_bytes), err, stream,
                            (wop || (wo_add && TiledTakesPlanes(T, D))) && QD % 32 == 0
                                ? planes
                                : nullptr,
                            &a_planes));
    h_planes = nullptr;
    const bool wo_norm = wop && ffnp && planes != nullptr && lin_ws != nullptr &&
                         NormPlanesApplies(x, static_cast<const float*>(lin_ws), w->ffn_norm, h,
                                           D) &&
                         (w->wo.bias == nullptr || Aligned(w->wo.bias, 16));
    if (wo_norm) {
        // wo's split-K partial sums reduced by the residual add + RMSNorm,
        // which also writes h's planes for gate/up
        float* partial = nullptr;
        int splits = 1;
        MLK_TRY(LinearPlanarPartials(w->wo.type, a, w->wo.planar, T, QD, D, lin_ws, lin_b, hs,
                                     a_planes ? planes : nullptr, &partial, &splits));
        MLK_TRY(AddRmsNormPlanes(x, partial, w->ffn_norm, h, planes, T, D, eps, hs, splits,
                                 w->wo.bias));
        h_planes = planes;
    } else {
        if (wop) {
            MLK_TRY(LinearPlanar(w->wo.type, a, w->wo.planar, w->wo.bias, proj, T, QD, D, lin_ws,
                                 lin_b, hs, a_planes ? planes : nullptr));
        } else if (wo1p) {
            StreamArgs sa{};
            sa.seg[0] = PlanarSeg(w->wo, proj, D);
            sa.n_seg = 1;
            MLK_TRY(LinearRowPlanar(w->wo.type, a, QD, sa, kStreamPlain, hs));
        } else if (wo_add) {
            StreamArgs sa{};
            sa.seg[0] = Seg(w->wo, x, D, x);
            sa.n_seg = 1;
            sa.x_planes = a_planes ? planes : nullptr;  // written by the prefill attention
            MLK_TRY(LinearTiledFused(w->wo.type, a, T, QD, sa, kStreamAdd, hs));
        } else {
            MLK_TRY(Linear(w->wo, a, proj, T, QD, D, lin_ws, lin_b, stream));
        }
        if (wo_add && ffn_tiled && planes != nullptr &&
            NormPlanesApplies(x, nullptr, w->ffn_norm, h, D)) {
            // x already holds x + proj; h's planes for the gate/up launch
            MLK_TRY(AddRmsNormPlanes(x, nullptr, w->ffn_norm, h, planes, T, D, eps, hs));
            h_planes = planes;
        } else if (wo_add) {  // x already holds x + proj
            MLK_TRY(mlk_rmsnorm_f32(x, w->ffn_norm, h, T, D, eps, stream));
        } else if ((ffnp || ffn_tiled) && planes != nullptr &&
                   NormPlanesApplies(x, proj, w->ffn_norm, h, D)) {
            MLK_TRY(AddRmsNormPlanes(x, proj, w->ffn_norm, h, planes, T, D, eps, hs));
            h_planes = planes;
        } else if (!ffn_fold) {
            MLK_TRY(mlk_add_rmsnorm_f32(x, proj, w->ffn_norm, h, T, D, eps, stream));
        }
    }
    const uint32_t* g_planes = nullptr;
    if (ffn1) {
        StreamArgs a{};
        a.seg[0] = ffn1p ? PlanarSeg(w->w_gate, gate, F) : Seg(w->w_gate, gate, F);
        a.seg[1] = ffn1p ? PlanarSeg(w->w_up, gate, F) : Seg(w->w_up, gate, F);
        a.n_seg = 2;
        const float* in = h;
        if (ffn_fold) {  // RMSNorm(x + proj) staged in the launch; x + proj into h's buffer
            a.norm = StreamNorm{w->ffn_norm, proj, h, eps, nw, nvpt};
            in = x;
        }
        MLK_TRY(ffn1p ? LinearRowPlanar(w->w_gate.type, in, D, a, kStreamSwiGlu, hs)
                      : LinearRowStream(w->w_gate.type, in, D, a, kStreamSwiGlu, hs));
    } else if (ffnp) {
        // the SwiGLU epilogue also writes the planes of its output for a
        // planar down projection (over h's planes: the GEMM has read them)
        StreamArgs a{};
        a.seg[0] = PlanarSeg(w->w_gate, gate, F);
        a.seg[1] = PlanarSeg(w->w_up, gate, F);
        a.n_seg = 2;
        a.planes = downp && planes != nullptr && F % 32 == 0 ? planes : nullptr;
        MLK_TRY(LinearPlanarFused(w->w_gate.type, h, T, D, a, kStreamSwiGlu, lin_ws, lin_b, hs,
                                  h_planes));
        g_planes = a.planes;
    } else if (ffnm) {
        StreamArgs a{};
        a.seg[0] = Seg(w->w_gate, gate, F);
        a.seg[1] = Seg(w->w_up, gate, F);
        a.n_seg = 2;
        MLK_TRY(LinearSkinnyFused(w->w_gate.type, h, T, D, a, kStreamSwiGlu, lin_ws, lin_b, hs));
    } else if (ffn_tiled) {
        StreamArgs a{};
        a.seg[0] = Seg(w->w_gate, gate, F);
        a.seg[1] = Seg(w->w_up, gate, F);
        a.n_seg = 2;
        a.x_planes = h_planes;
        MLK_TRY(LinearTiledFused(w->w_gate.type, h, T, D, a, kStreamSwiGlu, hs));
    } else {
        MLK_TRY(Linear(w->w_gate, h, gate, T, D, F, lin_ws, lin_b, stream));
        MLK_TRY(Linear(w->w_up, h, up, T, D, F, lin_ws, lin_b, stream));
        MLK_TRY(mlk_swiglu_f32(gate, up, gate, T * F, stream));
    }
    if (down1) {
        StreamArgs a{};
        const float* res = ffn_fold ? h : x;  // x = (x + proj) + down
        a.seg[0] = down1p ? PlanarSeg(w->w_down, x, D, res) : Seg(w->w_down, x, D, res);
        a.n_seg = 1;
        MLK_TRY(down1p ? LinearRowPlanar(w->w_down.type, gate, F, a, kStreamAdd, hs)
                       : LinearRowStream(w->w_down.type, gate, F, a, kStreamAdd, hs));
    } else if (downp) {
        StreamArgs a{};
        a.seg[0] = PlanarSeg(w->w_down, x, D, x);
        a.n_seg = 1;
        MLK_TRY(LinearPlanarFused(w->w_down.type, gate, T, F, a, kStreamAdd, lin_ws, lin_b, hs,
                                  g_planes));
    } else if (downm) {
        StreamArgs a{};
        a.seg[0] = Seg(w->w_down, x, D, x);
        a.n_seg = 1;
        MLK_TRY(LinearSkinnyFused(w->w_down.type, gate, T, F, a, kStreamAdd, lin_ws, lin_b, hs));
    } else if (down_tiled) {
        StreamArgs a{};
        a.seg[0] = Seg(w->w_down, x, D, x);
        a.n_seg = 1;
        MLK_TRY(LinearTiledFused(w->w_down.type, gate, T, F, a, kStreamAdd, hs));
    } else {
        MLK_TRY(Linear(w->w_down, gate, proj, T, F, D, lin_ws, lin_b, stream));
        MLK_TRY(mlk_add_f32(x, proj, x, T * D, stream));
    }
#undef MLK_TRY
    return MLK_OK;
}

}  // extern "C"
