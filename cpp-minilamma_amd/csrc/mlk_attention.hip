// mlk_attention.hip -- decode attention over the device KV cache, and the
// cache write.
//
// Semantics (the reference, paths under its tree):
//   cache       keys / values [n_layers, max_seq, n_kv_heads, head_dim] fp32
//               (include/cuda_kvcache.h:5-6, include/kvcache.h:8-10);
//   write       slot (layer, pos) <- k, v [n_kv_heads, head_dim]
//               (CudaCache::WriteDevice, src/cuda_kvcache.cc:209-237; CPU
//               KvCache::Write, src/kvcache.cc:19-50);
//   attention   query head i reads KV head i / (n_heads / n_kv_heads);
//               s_j = (q . k_j) * (1 / sqrt(head_dim)) for j = 0..pos,
//               p = softmax(s), out = sum_j p_j v_j
//               (ForwardAttention, src/forward.cc:265-298; device
//               ScoresKernel + AttentionReduceKernel, src/cuda_attention.cu:77-176).
// The sums here run in another order than the reference's serial loops
// (and the softmax is normalized once at the end); the parity tests hold
// both to the float64 value.
//
// The path is HBM-bound: every attended K and V row is read once per
// (token, KV head), 8 * head_dim bytes per position, and the arithmetic per
// byte is a few flops.  Layout of the work (flash-decoding):
//   - a workgroup (4 waves) owns one token, one KV head, a block of up to
//     GB query heads of that KV head's group, and a chunk of positions; it
//     reads each K and V row of the chunk once for all GB heads (the
//     reference re-reads them for every query head);
//   - scores: a half-wave per position, lane l holding head dims
//     l, l + 32, ... (coalesced 128-byte row segments); the 32 lanes' partial
//     dot products of P positions x GB heads are summed with one
//     transpose-reduce (P * GB = 32 values, one result per lane);
//   - the chunk's softmax (max, exp, sum) in LDS, then the value rows, again a
//     half-wave per position, with the probabilities broadcast from LDS;
//   - one chunk covers all positions: the workgroup divides by the sum and
//     writes out; otherwise it writes (acc, max, sum) to the workspace and
//     AttnCombine rescales and adds the chunks (max-shifted, like the
//     reference's softmax).
#include "mlk_common.h"

#include <math.h>

namespace mlk {
namespace {

constexpr int kAttnThreads = 256;
constexpr int kAttnWaves = kAttnThreads / kWave;
constexpr int kHalf = kWave / 2;  // lanes per position
constexpr int kMaxHeadDim = 256;

struct AttnParams {
    const float* q;
    int64_t q_stride;  // floats between token rows of q
    const float* kc;   // key cache at `layer`
    const float* vc;   // value cache at `layer`
    int64_t slot;      // floats per cache slot: n_kv_heads * head_dim
    const int32_t* positions;
    int32_t pos0;
    int64_t max_ctx;   // positions are < max_ctx (<= max_seq)
    int H, hd, group, n_hblk;
    int chunk, n_chunks;
    float scale;
    float* out;        // [T, H, hd]
    float* ws_acc;     // [T, H, n_chunks, hd]
    float* ws_ml;      // [T, H, n_chunks, 2]
    int32_t* err;
};

__device__ inline int32_t TokenPos(const AttnParams& p, int64_t t) {
    return p.positions != nullptr ? p.positions[t] : p.pos0 + static_cast<int32_t>(t);
}

__device__ inline float MaskF(float v, bool keep) {
    return __uint_as_float(__float_as_uint(v) & (keep ? ~0u : 0u));
}

__device__ inline float WaveSumF(float v) {
#pragma unroll
    for (int o = kWave / 2; o > 0; o /= 2) v += __shfl_xor(v, o, kWave);
    return v;
}

// Sums 32 values per lane over the 32 lanes of each half-wave: every step
// halves the values a lane holds (lanes with bit o clear keep the lower
// half and add the partner's lower half); after five steps lane l holds the
// total of value index HalfIdx(l).
__device__ inline float HalfTransposeReduce(float (&v)[kHalf], int hl) {
#pragma unroll
    for (int h = kHalf / 2, o = kHalf / 2; h >= 1; h /= 2, o /= 2) {
        const bool upper = (hl & o) != 0;
#pragma unroll
        for (int i = 0; i < h; ++i) {
            const float send = upper ? v[i] : v[i + h];
            const float keep = upper ? v[i + h] : v[i];
            v[i] = keep + __shfl_xor(send, o, kWave);
        }
    }
    return v[0];
}

__device__ inline int HalfIdx(int hl) {
    int idx = 0;
#pragma unroll
    for (int h = kHalf / 2, o = kHalf / 2; h >= 1; h /= 2, o /= 2) idx += (hl & o) ? h : 0;
    return idx;
}

// NQ: head dims per lane (head_dim <= 32 * NQ); GB: query heads per
// workgroup.  Dynamic LDS: GB * chunk scores + kAttnWaves * GB * 32 * NQ
// value partials.
template <int NQ, int GB>
__global__ __launch_bounds__(kAttnThreads) void AttnChunk(AttnParams p) {
    constexpr int P = kHalf / GB;  // position steps per transpose-reduce
    constexpr int W = kHalf * NQ;  // value partials per head
    extern __shared__ float smem[];
    float* sc = smem;
    float* red = smem + GB * p.chunk;
    __shared__ float ml[GB][2];

    const int c = static_cast<int>(blockIdx.x % p.n_chunks);
    const int64_t t = blockIdx.x / p.n_chunks;
    const int kvh = static_cast<int>(blockIdx.y) / p.n_hblk;
    const int hb = static_cast<int>(blockIdx.y) % p.n_hblk;
    const int h0 = kvh * p.group + hb * GB;
    const int nh = min(GB, p.group - hb * GB);
    const int32_t pos = TokenPos(p, t);
    const int64_t j0 = static_cast<int64_t>(c) * p.chunk;
    if (pos < 0 || pos >= p.max_ctx) {
        // out-of-range position: a zero row (written here when no combine
        // pass follows) and the error flag
        if (c == 0) {
            if (threadIdx.x == 0) RaiseFlag(p.err, 1);
            if (p.n_chunks == 1) {
                for (int e = threadIdx.x; e < nh * p.hd; e += kAttnThreads) {
                    p.out[(t * p.H + h0 + e / p.hd) * p.hd + e % p.hd] = 0.0f;
                }
            }
        }
        return;
    }
    if (j0 > pos) return;  // chunk past the token's last position
    const int cl = static_cast<int>(min(static_cast<int64_t>(p.chunk), pos + 1 - j0));
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int half = lane / kHalf;
    const int hl = lane % kHalf;
    const int per_wave = p.chunk / kAttnWaves;
    const float* kbase = p.kc + j0 * p.slot + static_cast<int64_t>(kvh) * p.hd;
    const float* vbase = p.vc + j0 * p.slot + static_cast<int64_t>(kvh) * p.hd;

    // ---- scores
    float qr[GB][NQ];
#pragma unroll
    for (int h = 0; h < GB; ++h) {
#pragma unroll
        for (int i = 0; i < NQ; ++i) {
            const int d = hl + kHalf * i;
            const bool ok = h < nh && d < p.hd;
            qr[h][i] = MaskF(p.q[t * p.q_stride + static_cast<int64_t>(h0 + (ok ? h : 0)) * p.hd +
                                 (ok ? d : 0)],
                             ok);
        }
    }
    for (int b = 0; b < per_wave; b += 2 * P) {
        float part[kHalf];
#pragma unroll
        for (int s = 0; s < P; ++s) {
            const int jl = wave * per_wave + b + 2 * s + half;
            // rows past the chunk's end read row 0 of the chunk (in bounds);
            // their scores are replaced below
            const bool ok = b + 2 * s + half < per_wave && jl < cl;
            const float* kr = kbase + static_cast<int64_t>(ok ? jl : 0) * p.slot;
            float kv[NQ];
#pragma unroll
            for (int i = 0; i < NQ; ++i) {
                const int d = hl + kHalf * i;
                kv[i] = MaskF(kr[d < p.hd ? d : 0], d < p.hd);
            }
#pragma unroll
            for (int h = 0; h < GB; ++h) {
                float a = 0.0f;
#pragma unroll
                for (int i = 0; i < NQ; ++i) a = fmaf(qr[h][i], kv[i], a);
                part[s * GB + h] = a;
            }
        }
        const float tot = HalfTransposeReduce(part, hl);
        const int idx = HalfIdx(hl);
        const int s_ = idx / GB, h_ = idx % GB;
        if (b + 2 * s_ + half < per_wave) {
            const int jl = wave * per_wave + b + 2 * s_ + half;
            sc[h_ * p.chunk + jl] = jl < cl ? tot * p.scale : -INFINITY;
        }
    }
    __syncthreads();

    // ---- softmax of the chunk: e_j = exp(s_j - max), sum
    for (int h = wave; h < GB; h += kAttnWaves) {
        if (h >= nh) break;
        float* sh = sc + h * p.chunk;
        float m = -INFINITY;
        for (int i = lane; i < cl; i += kWave) m = fmaxf(m, sh[i]);
        m = WaveMax(m);
        float l = 0.0f;
        for (int i = lane; i < p.chunk; i += kWave) {
            const float e = i < cl ? expf(sh[i] - m) : 0.0f;
            sh[i] = e;
            l += e;
        }
        l = WaveSumF(l);
        if (lane == 0) {
            ml[h][0] = m;
            ml[h][1] = l;
        }
    }
    __syncthreads();

    // ---- values
    float acc[GB][NQ];
#pragma unroll
    for (int h = 0; h < GB; ++h)
#pragma unroll
        for (int i = 0; i < NQ; ++i) acc[h][i] = 0.0f;
    const int jend = min((wave + 1) * per_wave, cl);
#pragma unroll 4
    for (int jl = wave * per_wave + half; jl < jend; jl += 2) {
        const float* vr = vbase + static_cast<int64_t>(jl) * p.slot;
        float vv[NQ];
#pragma unroll
        for (int i = 0; i < NQ; ++i) {
            const int d = hl + kHalf * i;
            vv[i] = MaskF(vr[d < p.hd ? d : 0], d < p.hd);
        }
#pragma unroll
        for (int h = 0; h < GB; ++h) {
            const float e = sc[h * p.chunk + jl];
#pragma unroll
            for (int i = 0; i < NQ; ++i) acc[h][i] = fmaf(e, vv[i], acc[h][i]);
        }
    }
#pragma unroll
    for (int h = 0; h < GB; ++h) {
#pragma unroll
        for (int i = 0; i < NQ; ++i) {
            const float a = acc[h][i] + __shfl_xor(acc[h][i], kHalf, kWave);
            if (half == 0) red[(wave * GB + h) * W + hl + kHalf * i] = a;
        }
    }
    __syncthreads();
    for (int e = threadIdx.x; e < GB * W; e += kAttnThreads) {
        const int h = e / W, d = e % W;
        if (h >= nh || d >= p.hd) continue;
        float a = red[h * W + d];
#pragma unroll
        for (int w = 1; w < kAttnWaves; ++w) a += red[(w * GB + h) * W + d];
        const int64_t row = t * p.H + h0 + h;
        if (p.n_chunks == 1) {
            p.out[row * p.hd + d] = a / ml[h][1];
        } else {
            p.ws_acc[(row * p.n_chunks + c) * p.hd + d] = a;
        }
    }
    if (p.n_chunks > 1 && static_cast<int>(threadIdx.x) < nh) {
        const int64_t row = t * p.H + h0 + threadIdx.x;
        p.ws_ml[(row * p.n_chunks + c) * 2] = ml[threadIdx.x][0];
        p.ws_ml[(row * p.n_chunks + c) * 2 + 1] = ml[threadIdx.x][1];
    }
}

// out = sum_c acc_c exp(m_c - M) / sum_c l_c exp(m_c - M), M = max_c m_c,
// over the chunks that hold positions 0..pos; one workgroup per (token,
// query head).
__global__ __launch_bounds__(kAttnThreads) void AttnCombine(AttnParams p) {
    const int64_t row = blockIdx.x;  // t * H + h
    const int64_t t = row / p.H;
    const int32_t pos = TokenPos(p, t);
    float* o = p.out + row * p.hd;
    if (pos < 0 || pos >= p.max_ctx) {
        for (int d = threadIdx.x; d < p.hd; d += kAttnThreads) o[d] = 0.0f;
        return;
    }
    const int nc = pos / p.chunk + 1;
    const float* mlr = p.ws_ml + row * p.n_chunks * 2;
    float M = -INFINITY;
    for (int c = 0; c < nc; ++c) M = fmaxf(M, mlr[2 * c]);
    float L = 0.0f;
    for (int c = 0; c < nc; ++c) L += mlr[2 * c + 1] * expf(mlr[2 * c] - M);
    const float* acc = p.ws_acc + row * p.n_chunks * p.hd;
    for (int d = threadIdx.x; d < p.hd; d += kAttnThreads) {
        float a = 0.0f;
        for (int c = 0; c < nc; ++c) a = fmaf(acc[c * p.hd + d], expf(mlr[2 * c] - M), a);
        o[d] = a / L;
    }
}

template <int NQ>
hipError_t LaunchChunk(int gb, dim3 grid, size_t lds, hipStream_t s, const AttnParams& p) {
    switch (gb) {
        case 1: hipLaunchKernelGGL((AttnChunk<NQ, 1>), grid, dim3(kAttnThreads), lds, s, p); break;
        case 2: hipLaunchKernelGGL((AttnChunk<NQ, 2>), grid, dim3(kAttnThreads), lds, s, p); break;
        case 4: hipLaunchKernelGGL((AttnChunk<NQ, 4>), grid, dim3(kAttnThreads), lds, s, p); break;
        default: hipLaunchKernelGGL((AttnChunk<NQ, 8>), grid, dim3(kAttnThreads), lds, s, p); break;
    }
    return hipGetLastError();
}

int HeadsPerBlock(int group) {
    int gb = 1;
    while (gb < group && gb < 8) gb *= 2;
    return gb;
}

int DimsPerLane(int hd) {
    int nq = 1;
    while (kHalf * nq < hd) nq *= 2;
    return nq;
}

// Positions per workgroup: the largest of 64..512 that still gives at least
// 512 workgroups (two per compute unit), else 64.  (512 keeps the dynamic LDS
// under 64 KiB: 8 heads x 512 scores + the value partials of head_dim 256.)
int ChunkFor(int64_t max_ctx, int64_t base_blocks) {
    int chunk = 512;
    while (chunk > 64 && base_blocks * ((max_ctx + chunk - 1) / chunk) < 512) chunk /= 2;
    return chunk;
}

// Copies n_tokens rows of k and v into their cache slots.
__global__ __launch_bounds__(kAttnThreads) void KvWriteKernel(
    float* __restrict__ kc, float* __restrict__ vc, int64_t slot, int64_t max_seq,
    const float* __restrict__ k, const float* __restrict__ v, int64_t k_stride, int64_t v_stride,
    const int32_t* __restrict__ positions, int32_t pos0, int32_t* err, int vec) {
    const int64_t t = blockIdx.x;
    const int32_t pos = positions != nullptr ? positions[t] : pos0 + static_cast<int32_t>(t);
    if (pos < 0 || pos >= max_seq) {
        if (threadIdx.x == 0) RaiseFlag(err, 1);
        return;
    }
    float* kd = kc + static_cast<int64_t>(pos) * slot;
    float* vd = vc + static_cast<int64_t>(pos) * slot;
    const float* ks = k + t * k_stride;
    const float* vs = v + t * v_stride;
    if (vec) {
        for (int64_t e = threadIdx.x; e < slot / 4; e += kAttnThreads) {
            reinterpret_cast<float4*>(kd)[e] = reinterpret_cast<const float4*>(ks)[e];
            reinterpret_cast<float4*>(vd)[e] = reinterpret_cast<const float4*>(vs)[e];
        }
    } else {
        for (int64_t e = threadIdx.x; e < slot; e += kAttnThreads) {
            kd[e] = ks[e];
            vd[e] = vs[e];
        }
    }
}

mlk_status CheckCache(const char* fn, const void* kc, const void* vc, int64_t n_layers,
                      int64_t max_seq, int32_t n_kv_heads, int32_t head_dim, int64_t layer) {
    if (kc == nullptr || vc == nullptr) {
        return Fail(MLK_ERR_INVALID, "%s: key and value cache buffers must both be initialized",
                    fn);
    }
    if (n_layers <= 0 || max_seq <= 0 || n_kv_heads <= 0 || head_dim <= 0) {
        return Fail(MLK_ERR_INVALID, "%s: cache dimensions must be positive", fn);
    }
    if (max_seq > 0x7FFFFFFF) {
        return Fail(MLK_ERR_INVALID, "%s: max_seq %lld exceeds 2^31 - 1", fn,
                    static_cast<long long>(max_seq));
    }
    if (layer < 0 || layer >= n_layers) {
        return Fail(MLK_ERR_RANGE, "%s: layer %lld out of range [0, %lld)", fn,
                    static_cast<long long>(layer), static_cast<long long>(n_layers));
    }
    if (kc == vc) {
        return Fail(MLK_ERR_INVALID, "%s: key and value caches must be distinct", fn);
    }
    return MLK_OK;
}

}  // namespace
}  // namespace mlk

using namespace mlk;

extern "C" {

mlk_status mlk_kv_write_f32(float* k_cache, float* v_cache, int64_t n_layers, int64_t max_seq,
                            int32_t n_kv_heads, int32_t head_dim, int64_t layer, const float* k,
                            int64_t k_row_stride, const float* v, int64_t v_row_stride,
                            const int32_t* positions, int32_t pos0, int64_t n_tokens,
                            int32_t* err, void* stream) {
    const char* fn = "mlk_kv_write_f32";
    mlk_status st = CheckCache(fn, k_cache, v_cache, n_layers, max_seq, n_kv_heads, head_dim,
                               layer);
    if (st != MLK_OK) return st;
    const int64_t slot = static_cast<int64_t>(n_kv_heads) * head_dim;
    if (k == nullptr || v == nullptr) return Fail(MLK_ERR_INVALID, "%s: k and v must not be null", fn);
    if (n_tokens < 0 || n_tokens > 0x7FFFFFFF) {
        return Fail(MLK_ERR_INVALID, "%s: n_tokens %lld out of range", fn,
                    static_cast<long long>(n_tokens));
    }
    if (k_row_stride < slot || v_row_stride < slot) {
        return Fail(MLK_ERR_INVALID, "%s: row strides must be at least n_kv_heads * head_dim", fn);
    }
    if (positions == nullptr && (pos0 < 0 || pos0 + n_tokens > max_seq)) {
        return Fail(MLK_ERR_RANGE, "%s: positions %d..%lld out of range [0, %lld)", fn, pos0,
                    static_cast<long long>(pos0 + n_tokens - 1), static_cast<long long>(max_seq));
    }
    if (n_tokens == 0) return MLK_OK;
    float* kc = k_cache + layer * max_seq * slot;
    float* vc = v_cache + layer * max_seq * slot;
    const int vec = slot % 4 == 0 && k_row_stride % 4 == 0 && v_row_stride % 4 == 0 &&
                    Aligned(k_cache, 16) && Aligned(v_cache, 16) && Aligned(k, 16) &&
                    Aligned(v, 16);
    hipLaunchKernelGGL(KvWriteKernel, dim3(static_cast<unsigned>(n_tokens)), dim3(kAttnThreads),
                       0, AsStream(stream), kc, vc, slot, max_seq, k, v, k_row_stride,
                       v_row_stride, positions, pos0, err, vec);
    return CheckLaunch("KvWriteKernel");
}

int64_t mlk_attention_workspace_bytes(int64_t n_tokens, int32_t n_heads, int32_t n_kv_heads,
                                      int32_t head_dim, int64_t max_ctx) {
    if (n_tokens <= 0 || n_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0 || max_ctx <= 0 ||
        n_heads % n_kv_heads != 0) {
        return 0;
    }
    const int group = n_heads / n_kv_heads;
    const int64_t base = n_tokens * n_kv_heads * ((group + HeadsPerBlock(group) - 1) / HeadsPerBlock(group));
    const int chunk = ChunkFor(max_ctx, base);
    const int64_t nc = (max_ctx + chunk - 1) / chunk;
    if (nc == 1) return 0;
    return n_tokens * n_heads * nc * (head_dim + 2) * static_cast<int64_t>(sizeof(float));
}

mlk_status mlk_attention_decode_f32(const float* q, int64_t q_row_stride, const float* k_cache,
                                    const float* v_cache, int64_t n_layers, int64_t max_seq,
                                    int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                                    int64_t layer, const int32_t* positions, int32_t pos0,
                                    int64_t n_tokens, int64_t max_ctx, float* out,
                                    void* workspace, size_t workspace_bytes, int32_t* err,
                                    void* stream) {
    const char* fn = "mlk_attention_decode_f32";
    mlk_status st = CheckCache(fn, k_cache, v_cache, n_layers, max_seq, n_kv_heads, head_dim,
                               layer);
    if (st != MLK_OK) return st;
    if (q == nullptr || out == nullptr) return Fail(MLK_ERR_INVALID, "%s: q and out must not be null", fn);
    if (n_heads <= 0 || n_heads % n_kv_heads != 0) {
        return Fail(MLK_ERR_INVALID,
                    "%s: n_kv_heads must be non-zero and divide n_heads, got n_heads=%d, "
                    "n_kv_heads=%d", fn, n_heads, n_kv_heads);
    }
    if (head_dim > kMaxHeadDim) {
        return Fail(MLK_ERR_INVALID, "%s: head_dim %d above %d is not supported", fn, head_dim,
                    kMaxHeadDim);
    }
    if (n_tokens <= 0 || n_tokens > 0x7FFFFFFF) {
        return Fail(MLK_ERR_INVALID, "%s: n_tokens %lld out of range", fn,
                    static_cast<long long>(n_tokens));
    }
    if (q_row_stride < static_cast<int64_t>(n_heads) * head_dim) {
        return Fail(MLK_ERR_INVALID, "%s: q_row_stride must be at least n_heads * head_dim", fn);
    }
    if (max_ctx <= 0 || max_ctx > max_seq) {
        return Fail(MLK_ERR_INVALID, "%s: max_ctx %lld out of range [1, max_seq=%lld]", fn,
                    static_cast<long long>(max_ctx), static_cast<long long>(max_seq));
    }
    if (positions == nullptr && (pos0 < 0 || pos0 + n_tokens > max_ctx)) {
        return Fail(MLK_ERR_RANGE, "%s: positions %d..%lld out of range [0, %lld)", fn, pos0,
                    static_cast<long long>(pos0 + n_tokens - 1), static_cast<long long>(max_ctx));
    }
    if (out >= q && out < q + (n_tokens - 1) * q_row_stride + static_cast<int64_t>(n_heads) * head_dim) {
        return Fail(MLK_ERR_INVALID, "%s: out must not alias q", fn);
    }
    const int group = n_heads / n_kv_heads;
    const int gb = HeadsPerBlock(group);
    const int n_hblk = (group + gb - 1) / gb;
    const int64_t base = n_tokens * n_kv_heads * n_hblk;
    const int chunk = ChunkFor(max_ctx, base);
    const int64_t nc = (max_ctx + chunk - 1) / chunk;
    const int64_t need = mlk_attention_workspace_bytes(n_tokens, n_heads, n_kv_heads, head_dim,
                                                       max_ctx);
    if (nc > 1 && (workspace == nullptr || static_cast<int64_t>(workspace_bytes) < need ||
                   !Aligned(workspace, 4))) {
        return Fail(MLK_ERR_INVALID, "%s: workspace of %lld bytes needed (got %zu)", fn,
                    static_cast<long long>(need), workspace_bytes);
    }
    if (n_tokens * nc > 0x7FFFFFFF || static_cast<int64_t>(n_kv_heads) * n_hblk > 65535) {
        return Fail(MLK_ERR_INVALID, "%s: launch too large", fn);
    }
    AttnParams p;
    const int64_t slot = static_cast<int64_t>(n_kv_heads) * head_dim;
    p.q = q;
    p.q_stride = q_row_stride;
    p.kc = k_cache + layer * max_seq * slot;
    p.vc = v_cache + layer * max_seq * slot;
    p.slot = slot;
    p.positions = positions;
    p.pos0 = pos0;
    p.max_ctx = max_ctx;
    p.H = n_heads;
    p.hd = head_dim;
    p.group = group;
    p.n_hblk = n_hblk;
    p.chunk = chunk;
    p.n_chunks = static_cast<int>(nc);
    p.scale = 1.0f / sqrtf(static_cast<float>(head_dim));
    p.out = out;
    p.ws_acc = nc > 1 ? static_cast<float*>(workspace) : nullptr;
    p.ws_ml = nc > 1 ? static_cast<float*>(workspace) + n_tokens * n_heads * nc * head_dim : nullptr;
    p.err = err;
    const int nq = DimsPerLane(head_dim);
    const size_t lds = (static_cast<size_t>(gb) * chunk + static_cast<size_t>(kAttnWaves) * gb * kHalf * nq) *
                       sizeof(float);
    const dim3 grid(static_cast<unsigned>(n_tokens * nc), static_cast<unsigned>(n_kv_heads * n_hblk));
    const hipStream_t s = AsStream(stream);
    hipError_t e;
    switch (nq) {
        case 1: e = LaunchChunk<1>(gb, grid, lds, s, p); break;
        case 2: e = LaunchChunk<2>(gb, grid, lds, s, p); break;
        case 4: e = LaunchChunk<4>(gb, grid, lds, s, p); break;
        default: e = LaunchChunk<8>(gb, grid, lds, s, p); break;
    }
    if (e != hipSuccess) return FromHip(e, "AttnChunk");
    if (nc > 1) {
        hipLaunchKernelGGL(AttnCombine, dim3(static_cast<unsigned>(n_tokens * n_heads)),
                           dim3(kAttnThreads), 0, s, p);
        return CheckLaunch("AttnCombine");
    }
    return MLK_OK;
}

}  // extern "C"
