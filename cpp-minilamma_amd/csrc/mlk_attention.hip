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
// byte is a few flops.  head_dim 64 and 128 with a 16-byte aligned key cache
// take AttnDecodeMf (matrix cores, described at the kernel); other head
// dims take AttnSplit.  Layout of AttnSplit's work (flash-decoding):
//   - a workgroup (4 waves) owns one token, one KV head, a block of up to
//     GB query heads of that KV head's group, and a chunk of positions; it
//     reads each K and V row of the chunk once for all GB heads (the
//     reference re-reads them for every query head);
//   - each wave owns two positions per step (one per half-wave), lane l
//     holding head dims l, l + 32, ... of K and V (coalesced 128-byte row
//     segments); it keeps the rows of its next positions loading while it
//     computes the current ones;
//   - scores: the 32 lanes' partial dot products of all its positions and
//     heads are summed with one transpose-reduce;
//   - a running softmax per head (max, sum, weighted value sum) is updated
//     with lane shuffles, no LDS round trip or barrier inside the loop;
//   - the four waves merge their (max, sum, acc) through LDS at the end;
//   - one chunk covers all positions: the workgroup divides by the sum and
//     writes out; otherwise it writes (acc, max, sum) to the workspace and
//     AttnCombine rescales and adds the chunks (max-shifted, like the
//     reference's softmax).
#include "mlk_attention.h"

#include <math.h>

#include <mutex>
#include <utility>

namespace mlk {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kAttnThreads = 256;
constexpr int kAttnWaves = kAttnThreads / kWave;
constexpr int kHalf = kWave / 2;  // lanes per position
constexpr int kMaxHeadDim = 256;
constexpr int64_t kPrefillMinTokens = 16;  // consecutive positions from here: AttnPrefill
constexpr int64_t kTileMinTokens = 5;      // other batches from here: AttnPrefill's chunked form

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
    uint32_t* planes;  // AttnCombine: also out's bf16 planes (the [T, H * hd] rows)
};

__device__ inline int32_t TokenPos(const AttnParams& p, int64_t t) {
    return p.positions != nullptr ? p.positions[t] : p.pos0 + static_cast<int32_t>(t);
}

__device__ inline float MaskF(float v, bool keep) {
    return __uint_as_float(__float_as_uint(v) & (keep ? ~0u : 0u));
}

// Sums N (a power of two <= 32) values per lane over the 32 lanes of each
// half-wave.  Each of the log2(N) steps halves the values a lane holds
// (lanes with bit o clear keep the lower half and add the partner's lower
// half, the others the upper half); a butterfly over the remaining lane
// bits completes the sums.  Lane l then holds the total of value index
// l >> (5 - log2 N), and the 32 / N lanes of a group hold the same total.
template <int N>
__device__ inline float HalfTransposeReduce(float (&v)[N], int hl) {
    // all sends of a step first, then all shuffles, then the adds: the
    // step's shuffles are independent and wait on the LDS pipe once
#pragma unroll
    for (int h = N / 2, o = kHalf / 2; h >= 1; h /= 2, o /= 2) {
        const bool upper = (hl & o) != 0;
        float send[N / 2 > 0 ? N / 2 : 1], recv[N / 2 > 0 ? N / 2 : 1];
#pragma unroll
        for (int i = 0; i < h; ++i) send[i] = upper ? v[i] : v[i + h];
#pragma unroll
        for (int i = 0; i < h; ++i) recv[i] = __shfl_xor(send[i], o, kWave);
#pragma unroll
        for (int i = 0; i < h; ++i) v[i] = (upper ? v[i + h] : v[i]) + recv[i];
    }
    float r = v[0];
    constexpr int rest = kHalf / N;
#pragma unroll
    for (int o = rest / 2; o >= 1; o /= 2) r += __shfl_xor(r, o, kWave);
    return r;
}

constexpr int Log2(int n) { return n <= 1 ? 0 : 1 + Log2(n / 2); }
constexpr int MinI(int a, int b) { return a < b ? a : b; }

// One workgroup: one token, one KV head, a block of GB of its query heads,
// and the positions [j0, j0 + chunk) (cut at pos).  The positions go in
// sub-chunks of 8 * NPOS: wave w, half h takes positions
// w * 2 * NPOS + 2 s + h (s < NPOS) of each sub-chunk.  A lane keeps the K
// and V values of its NPOS positions and head dims l, l + 32, ... in
// registers (NPOS * NQ <= 16 and NPOS * GB <= 16, which bounds the
// registers of the loads in flight and of the score partials), and a
// running softmax per head:
//   scores   NPOS * GB partial dot products per lane, one transpose-reduce
//            (lane l then holds the score of (s, h) with
//            s * GB + h = l >> (5 - log2(NPOS * GB)));
//   softmax  per-head max and sum over the wave's 2 * NPOS positions by
//            butterflies over the lane bits of s and of the half; the
//            running (m, l, acc) is rescaled by exp(m_old - m_new);
//   values   acc[h] += p(s, h) * v_s, p(s, h) shuffled from its lane.
// The four waves' (m, l, acc) are merged through LDS at the end.
// kFull: head_dim == 32 * NQ, so no lane's head dims need masking.
template <int NQ, int GB, bool kFull>
__global__ __launch_bounds__(kAttnThreads) void AttnSplit(AttnParams p) {
    constexpr int NPOS = MinI(16 / GB > 0 ? 16 / GB : 1, 16 / NQ > 0 ? 16 / NQ : 1);
    constexpr int N = NPOS * GB;
    constexpr int SHIFT = 5 - Log2(N);        // lane l holds value l >> SHIFT
    constexpr int OMIN = kHalf / NPOS;        // lowest lane bit of s
    constexpr int SUB = 2 * kAttnWaves * NPOS;  // positions per sub-chunk
    constexpr int W = kHalf * NQ;             // head dims per half-wave
    __shared__ float wm[kAttnWaves][GB];
    __shared__ float wl[kAttnWaves][GB];
    __shared__ float wacc[kAttnWaves][GB][W];

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
    const int n_it = (cl + SUB - 1) / SUB;
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int half = lane / kHalf;
    const int hl = lane % kHalf;
    const float* kbase = p.kc + j0 * p.slot + static_cast<int64_t>(kvh) * p.hd;
    const float* vbase = p.vc + j0 * p.slot + static_cast<int64_t>(kvh) * p.hd;
    const int jw = wave * 2 * NPOS + half;  // the lane's first position in a sub-chunk

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

    // rows past cl read row 0 of the chunk (in bounds); their scores are
    // replaced by -inf and their weights are zero.  Offsets are 32-bit (a
    // chunk spans at most 2048 slots of <= 64 KiB), added to the uniform
    // chunk base.
    // unsigned offsets from the uniform bases, so the loads take the
    // scalar-base + 32-bit vector-offset form (immediate offsets for i)
    const char* kb8 = reinterpret_cast<const char*>(kbase);
    const char* vb8 = reinterpret_cast<const char*>(vbase);
    auto at = [](const char* b, uint32_t byte_off) {
        return *reinterpret_cast<const float*>(b + byte_off);
    };
    auto load = [&](int it, float (&kk)[NPOS][NQ], float (&vv)[NPOS][NQ]) {
#pragma unroll
        for (int s = 0; s < NPOS; ++s) {
            const int jl = it * SUB + jw + 2 * s;
            const uint32_t off = (static_cast<uint32_t>(jl < cl ? jl : 0) *
                                  static_cast<uint32_t>(p.slot) + static_cast<uint32_t>(hl)) * 4u;
#pragma unroll
            for (int i = 0; i < NQ; ++i) {
                if constexpr (kFull) {
                    kk[s][i] = at(kb8, off + 4u * kHalf * i);
                    vv[s][i] = at(vb8, off + 4u * kHalf * i);
                } else {
                    const bool dok = hl + kHalf * i < p.hd;
                    const uint32_t o = dok ? off + 4u * kHalf * i : off - 4u * hl;
                    kk[s][i] = MaskF(at(kb8, o), dok);
                    vv[s][i] = MaskF(at(vb8, o), dok);
                }
            }
        }
    };

    float m[GB], l[GB], acc[GB][NQ];
#pragma unroll
    for (int h = 0; h < GB; ++h) {
        m[h] = -INFINITY;
        l[h] = 0.0f;
#pragma unroll
        for (int i = 0; i < NQ; ++i) acc[h][i] = 0.0f;
    }
    const int my_idx = hl >> SHIFT;
    const int my_s = my_idx / GB, my_h = my_idx % GB;

    // One sub-chunk: scores, running-softmax update, values.  A sub-chunk
    // past cl (the odd trip of the unrolled loop) is all -inf and changes
    // nothing.
    auto step = [&](int it, const float (&kr)[NPOS][NQ], const float (&vr)[NPOS][NQ]) {
        float part[N];
#pragma unroll
        for (int s = 0; s < NPOS; ++s) {
#pragma unroll
            for (int h = 0; h < GB; ++h) {
                float a = 0.0f;
#pragma unroll
                for (int i = 0; i < NQ; ++i) a = fmaf(qr[h][i], kr[s][i], a);
                part[s * GB + h] = a;
            }
        }
        const float tot = HalfTransposeReduce<N>(part, hl);
        const bool valid = it * SUB + jw + 2 * my_s < cl;
        const float score = valid ? tot * p.scale : -INFINITY;
        // per-head max over the wave's positions of this sub-chunk
        float mx = score;
#pragma unroll
        for (int o = OMIN; o <= kHalf; o *= 2) mx = fmaxf(mx, __shfl_xor(mx, o, kWave));
        float mh[GB];
#pragma unroll
        for (int h = 0; h < GB; ++h) mh[h] = __shfl(mx, h << SHIFT, kWave);
        float mine = -INFINITY;
#pragma unroll
        for (int h = 0; h < GB; ++h) {
            const float mnew = fmaxf(m[h], mh[h]);
            const float corr = m[h] == -INFINITY ? 0.0f : expf(m[h] - mnew);
            m[h] = mnew;
            l[h] *= corr;
#pragma unroll
            for (int i = 0; i < NQ; ++i) acc[h][i] *= corr;
            mine = my_h == h ? mnew : mine;
        }
        const float e = valid ? expf(score - mine) : 0.0f;
        float ps[NPOS * GB];
#pragma unroll
        for (int v = 0; v < NPOS * GB; ++v) ps[v] = __shfl(e, (v << SHIFT) + kHalf * half, kWave);
        float es = e;
#pragma unroll
        for (int o = OMIN; o <= kHalf; o *= 2) es += __shfl_xor(es, o, kWave);
        float eh[GB];
#pragma unroll
        for (int h = 0; h < GB; ++h) eh[h] = __shfl(es, h << SHIFT, kWave);
#pragma unroll
        for (int h = 0; h < GB; ++h) l[h] += eh[h];
#pragma unroll
        for (int s = 0; s < NPOS; ++s) {
#pragma unroll
            for (int h = 0; h < GB; ++h) {
#pragma unroll
                for (int i = 0; i < NQ; ++i) acc[h][i] = fmaf(ps[s * GB + h], vr[s][i], acc[h][i]);
            }
        }
    };

    // two register sets, loop unrolled by two: each set is reloaded as soon
    // as its sub-chunk is done, so one sub-chunk loads while the other
    // computes, with no copies between the sets
    float ka[NPOS][NQ], va[NPOS][NQ], kb[NPOS][NQ], vb[NPOS][NQ];
    load(0, ka, va);
    for (int it = 0; it < n_it; it += 2) {
        load(it + 1, kb, vb);
        step(it, ka, va);
        load(it + 2, ka, va);
        step(it + 1, kb, vb);
    }

    // merge the halves (same m and l), then the waves through LDS
#pragma unroll
    for (int h = 0; h < GB; ++h) {
#pragma unroll
        for (int i = 0; i < NQ; ++i) {
            const float a = acc[h][i] + __shfl_xor(acc[h][i], kHalf, kWave);
            if (half == 0) wacc[wave][h][hl + kHalf * i] = a;
        }
        if (lane == 0) {
            wm[wave][h] = m[h];
            wl[wave][h] = l[h];
        }
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < GB * W; idx += kAttnThreads) {
        const int h = idx / W, d = idx % W;
        if (h >= nh || d >= p.hd) continue;
        float M = wm[0][h];
#pragma unroll
        for (int w = 1; w < kAttnWaves; ++w) M = fmaxf(M, wm[w][h]);
        float L = 0.0f, A = 0.0f;
#pragma unroll
        for (int w = 0; w < kAttnWaves; ++w) {
            const float f = wm[w][h] == -INFINITY ? 0.0f : expf(wm[w][h] - M);
            L = fmaf(wl[w][h], f, L);
            A = fmaf(wacc[w][h][d], f, A);
        }
        const int64_t row = t * p.H + h0 + h;
        if (p.n_chunks == 1) {
            p.out[row * p.hd + d] = A / L;
        } else {
            p.ws_acc[(row * p.n_chunks + c) * p.hd + d] = A;
            if (d == 0) {
                p.ws_ml[(row * p.n_chunks + c) * 2] = M;
                p.ws_ml[(row * p.n_chunks + c) * 2 + 1] = L;
            }
        }
    }
}

// ------------------------------------------------------------ MFMA decode
// head_dim 64 / 128: v_mfma_f32_4x4x1_16b_f32 (16 blocks of a 4 x 4 outer
// product per instruction; block b's A values come from lanes 4b + i, or
// with CBSZ = 4 from lanes 4 ABID + i for every block, B from lanes 4b + j,
// and D[b][i][j] lands in lane 4b + j, register i).  A workgroup owns one
// token, one KV head, a group of up to 4 of its query heads (the A rows) and
// a chunk of positions; each wave takes tiles of 64 positions:
//   scores   lane l = position p0 + l, register i = head i: for each head
//            dim d one MFMA with A = q broadcast from the block of d (a
//            register holds q of 4 heads x 16 dims, lane 4b + i = q[i][16k
//            + b], selected by ABID = b) and B = the lane's own K[p][d].  No
//            cross-lane sum: each lane streams its own K row.
//   softmax  per head, the tile maximum by DPP row operations (no LDS), the
//            running (m, l) rescaled by exp(m_old - m_new); l stays a per-lane
//            partial sum until the end.
//   values   p goes through 1 KB of the wave's LDS to lanes 4b + i = p_i(16R
//            + b); then per position one MFMA per 64 head dims with A = p
//            broadcast (ABID = position within the 16) and B = V[p][64 hh +
//            lane] (coalesced 256-byte row segments): lane l, register i
//            accumulates out[head i][64 hh + l].
// The 4 waves' (m, l, out) are merged through LDS; chunks are combined by
// AttnCombine as for AttnSplit.
constexpr int kMfTile = 64;   // positions per tile: one per lane
constexpr int kMfHeads = 4;   // query heads per workgroup: the MFMA's A rows

template <int CTRL, int ROW_MASK>
__device__ inline float Dpp(float old, float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), CTRL,
                                                      ROW_MASK, 0xF, false));
}

// Maximum / sum over the 64 lanes (uniform result): xor 1 and 2 within
// quads, mirrors within half-rows and rows, then row broadcasts into lane 63.
__device__ inline float WaveMaxDpp(float v) {
    v = fmaxf(v, Dpp<0xB1, 0xF>(v, v));
    v = fmaxf(v, Dpp<0x4E, 0xF>(v, v));
    v = fmaxf(v, Dpp<0x141, 0xF>(v, v));
    v = fmaxf(v, Dpp<0x140, 0xF>(v, v));
    v = fmaxf(v, Dpp<0x142, 0xA>(v, v));
    v = fmaxf(v, Dpp<0x143, 0xC>(v, v));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ inline float WaveSumDpp(float v) {
    v += Dpp<0xB1, 0xF>(0.0f, v);
    v += Dpp<0x4E, 0xF>(0.0f, v);
    v += Dpp<0x141, 0xF>(0.0f, v);
    v += Dpp<0x140, 0xF>(0.0f, v);
    v += Dpp<0x142, 0xA>(0.0f, v);
    v += Dpp<0x143, 0xC>(0.0f, v);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ inline float Comp(const float4& v, int e) {
    return e == 0 ? v.x : (e == 1 ? v.y : (e == 2 ? v.z : v.w));
}

// sc += q (4 heads x 16 dims, broadcast from block b for dim 16k + b) times
// the lane's K at those dims, k4 = its float4 16k / 4 .. + 3.  ABID must be
// a constant: the 16 instructions come from a parameter pack.
template <int... Bs>
__device__ inline f32x4 QkDims(float q, const float4* k4, f32x4 sc,
                               std::integer_sequence<int, Bs...>) {
    ((sc = __builtin_amdgcn_mfma_f32_4x4x1f32(q, Comp(k4[Bs / 4], Bs % 4), sc, 4, Bs, 0)), ...);
    return sc;
}

// acc[hh] += p (4 heads, broadcast from block S = the position within the
// 16) times V[position][64 hh + lane].
template <int NH, int S>
__device__ inline void PvOne(float pr, const float (&v)[NH], f32x4 (&acc)[NH]) {
#pragma unroll
    for (int hh = 0; hh < NH; ++hh) {
        acc[hh] = __builtin_amdgcn_mfma_f32_4x4x1f32(pr, v[hh], acc[hh], 4, S, 0);
    }
}

template <int NH, int... Ss>
__device__ inline void PvPositions(float pr, const float (&v)[16][NH], f32x4 (&acc)[NH],
                                   std::integer_sequence<int, Ss...>) {
    (PvOne<NH, Ss>(pr, v[Ss], acc), ...);
}

// V[ps][64 hh + lane] of the 16 positions from ps0 (rows past pos read row
// pos; their weights are zero).
template <int NH>
__device__ inline void LoadMfV(const float* vbase, int64_t slot, int64_t ps0, int64_t pos,
                               int lane, float (&v)[16][NH]) {
#pragma unroll
    for (int s2 = 0; s2 < 16; ++s2) {
        const int64_t ps = ps0 + s2;
        const int64_t pr = ps <= pos ? ps : pos;
#pragma unroll
        for (int hh = 0; hh < NH; ++hh) v[s2][hh] = vbase[pr * slot + 64 * hh + lane];
    }
}

template <int HD>
__global__ __launch_bounds__(kAttnThreads) void AttnDecodeMf(AttnParams p, int tpw) {
    constexpr int NK = HD / 4;   // float4 per K row
    constexpr int NQ = HD / 16;  // q registers
    constexpr int NH = HD / 64;  // 64-dim parts of the output
    __shared__ __align__(16) float ptile[kAttnWaves][kMfTile * kMfHeads];
    __shared__ float wm[kAttnWaves][kMfHeads], wl[kAttnWaves][kMfHeads];
    __shared__ float wo[kAttnWaves][kMfHeads][HD];

    const int c = static_cast<int>(blockIdx.x % p.n_chunks);
    const int64_t t = blockIdx.x / p.n_chunks;
    const int kvh = static_cast<int>(blockIdx.y) / p.n_hblk;
    const int hb = static_cast<int>(blockIdx.y) % p.n_hblk;
    const int h0 = kvh * p.group + hb * kMfHeads;
    const int nh = min(kMfHeads, p.group - hb * kMfHeads);
    const int32_t pos = TokenPos(p, t);
    const int64_t j0 = static_cast<int64_t>(c) * p.chunk;
    if (pos < 0 || pos >= p.max_ctx) {
        if (c == 0) {
            if (threadIdx.x == 0) RaiseFlag(p.err, 1);
            if (p.n_chunks == 1) {
                for (int e = threadIdx.x; e < nh * HD; e += kAttnThreads) {
                    p.out[(t * p.H + h0 + e / HD) * HD + e % HD] = 0.0f;
                }
            }
        }
        return;
    }
    if (j0 > pos) return;  // chunk past the token's last position
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int bq = lane / 4, iq = lane % 4;

    float qr[NQ];  // lane 4b + i: q[h0 + i][16k + b]
#pragma unroll
    for (int k = 0; k < NQ; ++k) {
        const bool ok = iq < nh;
        qr[k] = MaskF(p.q[t * p.q_stride + static_cast<int64_t>(h0 + (ok ? iq : 0)) * HD + 16 * k +
                          bq],
                      ok);
    }
    const float* kbase = p.kc + static_cast<int64_t>(kvh) * HD;
    const float* vbase = p.vc + static_cast<int64_t>(kvh) * HD;
    float m[kMfHeads], lsum[kMfHeads];
    f32x4 acc[NH];
#pragma unroll
    for (int r = 0; r < kMfHeads; ++r) {
        m[r] = -INFINITY;
        lsum[r] = 0.0f;
    }
#pragma unroll
    for (int hh = 0; hh < NH; ++hh) acc[hh] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int tt = 0; tt < tpw; ++tt) {
        const int64_t p0 = j0 + static_cast<int64_t>(tt * kAttnWaves + wave) * kMfTile;
        if (p0 > pos) break;
        const int64_t mine = p0 + lane;
        const bool valid = mine <= pos;
        const int64_t row = valid ? mine : pos;
        // the lane's K row, then the first 16 positions' V values
        float4 kr[NK];
#pragma unroll
        for (int e = 0; e < NK; ++e) {
            kr[e] = *reinterpret_cast<const float4*>(kbase + row * p.slot + 4 * e);
        }
        float vr[4][16][NH];
        LoadMfV<NH>(vbase, p.slot, p0 + 0, pos, lane, vr[0]);
        LoadMfV<NH>(vbase, p.slot, p0 + 16, pos, lane, vr[1]);
        __builtin_amdgcn_sched_barrier(0);
        f32x4 sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < NQ; ++k) {
            sc = QkDims(qr[k], kr + 4 * k, sc, std::make_integer_sequence<int, 16>{});
        }
        LoadMfV<NH>(vbase, p.slot, p0 + 32, pos, lane, vr[2]);
        LoadMfV<NH>(vbase, p.slot, p0 + 48, pos, lane, vr[3]);
        float pv[kMfHeads];
#pragma unroll
        for (int r = 0; r < kMfHeads; ++r) {
            const float sv = valid ? sc[r] * p.scale : -INFINITY;
            const float mnew = fmaxf(m[r], WaveMaxDpp(sv));  // finite: lane 0 is valid
            const float corr = m[r] == -INFINITY ? 0.0f : expf(m[r] - mnew);
            pv[r] = valid ? expf(sv - mnew) : 0.0f;
            lsum[r] = lsum[r] * corr + pv[r];
#pragma unroll
            for (int hh = 0; hh < NH; ++hh) acc[hh][r] *= corr;
            m[r] = mnew;
        }
        // p to lanes 4b + i = p_i(16 R + b) through the wave's LDS
        float* pt = ptile[wave];
        *reinterpret_cast<float4*>(pt + 4 * lane) = make_float4(pv[0], pv[1], pv[2], pv[3]);
        float pr[4];
#pragma unroll
        for (int R = 0; R < 4; ++R) pr[R] = pt[kMfTile * R + lane];
#pragma unroll
        for (int R = 0; R < 4; ++R) {
            PvPositions<NH>(pr[R], vr[R], acc, std::make_integer_sequence<int, 16>{});
        }
    }
    // merge: l over lanes, then the 4 waves through LDS
#pragma unroll
    for (int r = 0; r < kMfHeads; ++r) {
        const float L = WaveSumDpp(lsum[r]);
        if (lane == 0) {
            wm[wave][r] = m[r];
            wl[wave][r] = L;
        }
#pragma unroll
        for (int hh = 0; hh < NH; ++hh) wo[wave][r][64 * hh + lane] = acc[hh][r];
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < nh * HD; idx += kAttnThreads) {
        const int r = idx / HD, d = idx % HD;
        float M = wm[0][r];
#pragma unroll
        for (int w = 1; w < kAttnWaves; ++w) M = fmaxf(M, wm[w][r]);
        float L = 0.0f, A = 0.0f;
#pragma unroll
        for (int w = 0; w < kAttnWaves; ++w) {
            const float f = wm[w][r] == -INFINITY ? 0.0f : expf(wm[w][r] - M);
            L = fmaf(wl[w][r], f, L);
            A = fmaf(wo[w][r][d], f, A);
        }
        const int64_t orow = t * p.H + h0 + r;
        if (p.n_chunks == 1) {
            p.out[orow * HD + d] = A / L;
        } else {
            p.ws_acc[(orow * p.n_chunks + c) * HD + d] = A;
            if (d == 0) {
                p.ws_ml[(orow * p.n_chunks + c) * 2] = M;
                p.ws_ml[(orow * p.n_chunks + c) * 2 + 1] = L;
            }
        }
    }
}

// out = sum_c acc_c exp(m_c - M) / sum_c l_c exp(m_c - M), M = max_c m_c,
// over the chunks that hold positions 0..pos; one workgroup per (token,
// query head).  The chunk weights exp(m_c - M) are computed once into LDS
// (in tiles of kCombineTile chunks).
constexpr int kCombineTile = 1024;
constexpr int kCombinePre = 32;  // partials per thread requested before the reductions

__global__ __launch_bounds__(kAttnThreads) void AttnCombine(AttnParams p) {
    __shared__ float wgt[kCombineTile];
    __shared__ double red[kAttnWaves];
    __shared__ float redf[kAttnWaves];
    const int64_t row = blockIdx.x;  // t * H + h
    const int64_t t = row / p.H;
    const int32_t pos = TokenPos(p, t);
    float* o = p.out + row * p.hd;
    const int64_t k0 = (row - t * p.H) * p.hd;  // h * hd: the row's place in [H * hd]
    const int64_t T = gridDim.x / p.H;
    if (pos < 0 || pos >= p.max_ctx) {
        for (int d = threadIdx.x; d < p.hd; d += kAttnThreads) {
            o[d] = 0.0f;
            if (p.planes != nullptr) StorePlanes1(p.planes, T, t, k0 + d, 0.0f);
        }
        return;
    }
    const int nc = pos / p.chunk + 1;
    const float* mlr = p.ws_ml + row * p.n_chunks * 2;
    const float* acc = p.ws_acc + row * p.n_chunks * p.hd;
    const int d = threadIdx.x;
    // the first kCombinePre chunks' partials of this thread's dim, requested
    // before the reductions below (clamped rows past nc are never used)
    float pre[kCombinePre];
#pragma unroll
    for (int c = 0; c < kCombinePre; ++c) {
        const int cc = c < nc ? c : nc - 1;
        pre[c] = acc[static_cast<int64_t>(cc) * p.hd + (d < p.hd ? d : 0)];
    }
    // at most one chunk per thread (every context up to kAttnThreads chunks):
    // its (m, l) stay in registers for the max, the sum and the weight, in
    // place of two more dependent reads after each reduction
    const bool one = nc <= kAttnThreads;
    const int c1 = one && static_cast<int>(threadIdx.x) < nc ? static_cast<int>(threadIdx.x) : 0;
    const float m1 = mlr[2 * c1], l1 = mlr[2 * c1 + 1];
    float mloc = -INFINITY;
    if (one) {
        if (static_cast<int>(threadIdx.x) < nc) mloc = fmaxf(mloc, m1);
    } else {
        for (int c = threadIdx.x; c < nc; c += kAttnThreads) mloc = fmaxf(mloc, mlr[2 * c]);
    }
    const float M = BlockMax<kAttnWaves>(mloc, redf);
    float lloc = 0.0f;
    float w1 = 0.0f;  // this thread's chunk weight exp(m - M) (one chunk per thread)
    if (one) {
        if (static_cast<int>(threadIdx.x) < nc) {
            w1 = expf(m1 - M);
            lloc += l1 * w1;
        }
    } else {
        for (int c = threadIdx.x; c < nc; c += kAttnThreads) lloc += mlr[2 * c + 1] * expf(mlr[2 * c] - M);
    }
    const float L = static_cast<float>(BlockSum<kAttnWaves>(static_cast<double>(lloc), red));
    float a = 0.0f;
    for (int c0 = 0; c0 < nc; c0 += kCombineTile) {
        const int n = min(kCombineTile, nc - c0);
        __syncthreads();
        if (one) {
            if (static_cast<int>(threadIdx.x) < n) wgt[threadIdx.x] = w1;
        } else {
            for (int c = threadIdx.x; c < n; c += kAttnThreads) wgt[c] = expf(mlr[2 * (c0 + c)] - M);
        }
        __syncthreads();
        if (d < p.hd) {
            int c = 0;
            if (c0 == 0) {
#pragma unroll
                for (int cp = 0; cp < kCombinePre; ++cp) {
                    if (cp < n) a = fmaf(pre[cp], wgt[cp], a);
                }
                c = n < kCombinePre ? n : kCombinePre;
            }
            const float* ac = acc + static_cast<int64_t>(c0) * p.hd + d;
#pragma unroll 8
            for (; c < n; ++c) a = fmaf(ac[static_cast<int64_t>(c) * p.hd], wgt[c], a);
        }
    }
    if (d < p.hd) {
        const float v = a / L;
        o[d] = v;
        if (p.planes != nullptr) StorePlanes1(p.planes, T, t, k0 + d, v);
    }
}

template <int NQ, bool kFull>
hipError_t LaunchSplit(int gb, dim3 grid, hipStream_t s, const AttnParams& p) {
    switch (gb) {
        case 1: hipLaunchKernelGGL((AttnSplit<NQ, 1, kFull>), grid, dim3(kAttnThreads), 0, s, p); break;
        case 2: hipLaunchKernelGGL((AttnSplit<NQ, 2, kFull>), grid, dim3(kAttnThreads), 0, s, p); break;
        case 4: hipLaunchKernelGGL((AttnSplit<NQ, 4, kFull>), grid, dim3(kAttnThreads), 0, s, p); break;
        default: hipLaunchKernelGGL((AttnSplit<NQ, 8, kFull>), grid, dim3(kAttnThreads), 0, s, p); break;
    }
    return hipGetLastError();
}

template <int NQ>
hipError_t LaunchSplit(int gb, int hd, dim3 grid, hipStream_t s, const AttnParams& p) {
    return hd == kHalf * NQ ? LaunchSplit<NQ, true>(gb, grid, s, p)
                            : LaunchSplit<NQ, false>(gb, grid, s, p);
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

// Positions per workgroup: the largest power of two in 64..2048 that still
// gives at least 512 workgroups (two per compute unit at the kernel's
// occupancy), else 64.  Larger chunks mean fewer partials to combine and
// more sub-chunks per workgroup to overlap loads with arithmetic.
int ChunkFor(int64_t max_ctx, int64_t base_blocks) {
    int chunk = 2048;
    while (chunk > 64 && base_blocks * ((max_ctx + chunk - 1) / chunk) < 512) chunk /= 2;
    return chunk;
}

// The MFMA kernel's launch: query heads in groups of 4; a workgroup's chunk
// is 4 waves x tpw tiles of 64 positions, tpw 1 unless that makes more than
// 16384 workgroups (then fewer partial results to combine).
struct MfPlan {
    int n_hblk, tpw, chunk;
    int64_t nc;
};

bool MfSupported(int32_t head_dim) { return head_dim == 64 || head_dim == 128; }

MfPlan PlanMf(int64_t n_tokens, int32_t n_kv_heads, int group, int64_t max_ctx) {
    MfPlan m;
    m.n_hblk = (group + kMfHeads - 1) / kMfHeads;
    const int64_t base = n_tokens * n_kv_heads * m.n_hblk;
    const int64_t per_tile = static_cast<int64_t>(kAttnWaves) * kMfTile;
    int tpw = 1;
    while (tpw < 32 && base * ((max_ctx + per_tile * tpw - 1) / (per_tile * tpw)) > 16384) tpw *= 2;
    m.tpw = tpw;
    m.chunk = static_cast<int>(per_tile * tpw);
    m.nc = (max_ctx + m.chunk - 1) / m.chunk;
    return m;
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
    int64_t nc = (max_ctx + chunk - 1) / chunk;
    if (MfSupported(head_dim)) {
        // either kernel may run (the MFMA one needs a 16-byte aligned key cache)
        const int64_t nmf = PlanMf(n_tokens, n_kv_heads, group, max_ctx).nc;
        if (nmf > nc) nc = nmf;
        if (n_tokens >= kTileMinTokens) {  // or the shared-tile kernel (aligned buffers)
            const int tchunk = TileChunk(n_tokens, n_heads, n_kv_heads, max_ctx);
            const int64_t ntl = (max_ctx + tchunk - 1) / tchunk;
            if (ntl > nc) nc = ntl;
        }
    }
    if (nc == 1) return 0;
    return n_tokens * n_heads * nc * (head_dim + 2) * static_cast<int64_t>(sizeof(float));
}

}  // extern "C"

namespace mlk {

mlk_status AttentionDecode(const float* q, int64_t q_row_stride, const float* k_cache,
                           const float* v_cache, int64_t n_layers, int64_t max_seq,
                           int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, int64_t layer,
                           const int32_t* positions, int32_t pos0, int64_t n_tokens,
                           int64_t max_ctx, float* out, void* workspace, size_t workspace_bytes,
                           int32_t* err, void* stream, uint32_t* planes, bool* planes_written) {
    const char* fn = "mlk_attention_decode_f32";
    if (planes_written != nullptr) *planes_written = false;
    if (planes != nullptr &&
        ((static_cast<int64_t>(n_heads) * head_dim) % 32 != 0 || !Aligned(planes, 16))) {
        return Fail(MLK_ERR_INVALID, "%s: planes need n_heads * head_dim %% 32 == 0", fn);
    }
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
    const int64_t slot = static_cast<int64_t>(n_kv_heads) * head_dim;
    if (positions == nullptr && n_tokens >= kPrefillMinTokens &&
        PrefillSupported(head_dim, q, q_row_stride, out, k_cache, v_cache)) {
        // a prompt chunk at consecutive positions: the matrix-core prefill
        // kernel (a workspace of PrefillImageBytes holds the pre-split tiles)
        // (and a's planes, when asked, for a tiled wo)
        if (planes != nullptr && planes_written != nullptr) *planes_written = true;
        return LaunchPrefill(q, q_row_stride, k_cache + layer * max_seq * slot,
                             v_cache + layer * max_seq * slot, slot, n_heads, n_kv_heads,
                             head_dim, pos0, n_tokens, out, AsStream(stream), workspace,
                             workspace_bytes, planes);
    }
    if (n_tokens >= kTileMinTokens && PrefillSupported(head_dim, q, q_row_stride, out, k_cache, v_cache) &&
        Aligned(workspace, 16)) {
        // several decode tokens: 16 per workgroup share each K/V tile of a
        // chunk of positions (the prefill kernel's matrix-core tiles), then
        // AttnCombine merges the chunks
        const int tchunk = TileChunk(n_tokens, n_heads, n_kv_heads, max_ctx);
        const int64_t tnc = (max_ctx + tchunk - 1) / tchunk;
        const int64_t need = tnc > 1 ? n_tokens * n_heads * tnc * (head_dim + 2) *
                                           static_cast<int64_t>(sizeof(float))
                                     : 0;
        if (tnc > 1 && (workspace == nullptr || static_cast<int64_t>(workspace_bytes) < need)) {
            return Fail(MLK_ERR_INVALID, "%s: workspace of %lld bytes needed (got %zu)", fn,
                        static_cast<long long>(need), workspace_bytes);
        }
        if (n_tokens * n_heads > 0x7FFFFFFF) return Fail(MLK_ERR_INVALID, "%s: launch too large", fn);
        float* ws_acc = tnc > 1 ? static_cast<float*>(workspace) : nullptr;
        float* ws_ml = tnc > 1 ? ws_acc + n_tokens * n_heads * tnc * head_dim : nullptr;
        const hipStream_t s = AsStream(stream);
        st = LaunchDecodeTile(q, q_row_stride, k_cache + layer * max_seq * slot,
                              v_cache + layer * max_seq * slot, slot, n_heads, n_kv_heads,
                              head_dim, positions, pos0, n_tokens, max_ctx, out, ws_acc, ws_ml,
                              err, s);
        if (st != MLK_OK || tnc == 1) return st;
        AttnParams p{};
        p.positions = positions;
        p.pos0 = pos0;
        p.max_ctx = max_ctx;
        p.H = n_heads;
        p.hd = head_dim;
        p.chunk = tchunk;
        p.n_chunks = static_cast<int>(tnc);
        p.out = out;
        p.ws_acc = ws_acc;
        p.ws_ml = ws_ml;
        p.err = err;
        p.planes = planes;
        hipLaunchKernelGGL(AttnCombine, dim3(static_cast<unsigned>(n_tokens * n_heads)),
                           dim3(kAttnThreads), 0, s, p);
        st = CheckLaunch("AttnCombine");
        if (st == MLK_OK && planes_written != nullptr) *planes_written = planes != nullptr;
        return st;
    }
    const int group = n_heads / n_kv_heads;
    const bool mf = MfSupported(head_dim) && Aligned(k_cache, 16);
    const MfPlan mp = PlanMf(n_tokens, n_kv_heads, group, max_ctx);
    const int gb = mf ? kMfHeads : HeadsPerBlock(group);
    const int n_hblk = (group + gb - 1) / gb;
    const int64_t base = n_tokens * n_kv_heads * n_hblk;
    const int chunk = mf ? mp.chunk : ChunkFor(max_ctx, base);
    const int64_t nc = (max_ctx + chunk - 1) / chunk;
    const int64_t need = nc > 1 ? n_tokens * n_heads * nc * (head_dim + 2) *
                                      static_cast<int64_t>(sizeof(float))
                                : 0;
    if (nc > 1 && (workspace == nullptr || static_cast<int64_t>(workspace_bytes) < need ||
                   !Aligned(workspace, 4))) {
        return Fail(MLK_ERR_INVALID, "%s: workspace of %lld bytes needed (got %zu)", fn,
                    static_cast<long long>(need), workspace_bytes);
    }
    if (n_tokens * nc > 0x7FFFFFFF || static_cast<int64_t>(n_kv_heads) * n_hblk > 65535) {
        return Fail(MLK_ERR_INVALID, "%s: launch too large", fn);
    }
    AttnParams p{};
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
    const dim3 grid(static_cast<unsigned>(n_tokens * nc), static_cast<unsigned>(n_kv_heads * n_hblk));
    const hipStream_t s = AsStream(stream);
    hipError_t e;
    if (mf) {
        if (head_dim == 64) {
            hipLaunchKernelGGL(AttnDecodeMf<64>, grid, dim3(kAttnThreads), 0, s, p, mp.tpw);
        } else {
            hipLaunchKernelGGL(AttnDecodeMf<128>, grid, dim3(kAttnThreads), 0, s, p, mp.tpw);
        }
        e = hipGetLastError();
    } else {
    switch (nq) {
        case 1: e = LaunchSplit<1>(gb, head_dim, grid, s, p); break;
        case 2: e = LaunchSplit<2>(gb, head_dim, grid, s, p); break;
        case 4: e = LaunchSplit<4>(gb, head_dim, grid, s, p); break;
        default: e = LaunchSplit<8>(gb, head_dim, grid, s, p); break;
    }
    }
    if (e != hipSuccess) return FromHip(e, mf ? "AttnDecodeMf" : "AttnSplit");
    if (nc > 1) {
        p.planes = planes;
        hipLaunchKernelGGL(AttnCombine, dim3(static_cast<unsigned>(n_tokens * n_heads)),
                           dim3(kAttnThreads), 0, s, p);
        st = CheckLaunch("AttnCombine");
        if (st == MLK_OK && planes_written != nullptr) *planes_written = planes != nullptr;
        return st;
    }
    return MLK_OK;
}

}  // namespace mlk

extern "C" {

mlk_status mlk_attention_decode_f32(const float* q, int64_t q_row_stride, const float* k_cache,
                                    const float* v_cache, int64_t n_layers, int64_t max_seq,
                                    int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                                    int64_t layer, const int32_t* positions, int32_t pos0,
                                    int64_t n_tokens, int64_t max_ctx, float* out,
                                    void* workspace, size_t workspace_bytes, int32_t* err,
                                    void* stream) {
    return AttentionDecode(q, q_row_stride, k_cache, v_cache, n_layers, max_seq, n_heads,
                           n_kv_heads, head_dim, layer, positions, pos0, n_tokens, max_ctx, out,
                           workspace, workspace_bytes, err, stream, nullptr, nullptr);
}

}  // extern "C"

// ------------------------------------------- no-allocation decode attention
//
// mlk_attention_decode_f32_noalloc keeps its chunk partials (per token, head
// and chunk: head_dim weighted sums, the running max and the sum) in this
// file-scope device array instead of a caller workspace.  Every GPU the
// library runs on holds its own copy, at its own address, until the process
// ends.  In host code `scratch` names a host-side stand-in, never the
// device memory: the address each device uses comes from
// hipGetSymbolAddress, taken once per device with that device current, and
// only that address reaches a kernel.  The kernels write every partial the
// combine step reads in the same call, so nothing needs clearing between
// calls; calls that overlap on one GPU share the array and race.
namespace mlk {
namespace {
constexpr size_t kScratchBytes = size_t{64} << 20;
constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kScratchDevices] = {};
}  // namespace
}  // namespace mlk

static __device__ __align__(256) unsigned char scratch[mlk::kScratchBytes];

namespace mlk {
namespace {
// The device address of `scratch` on the current device, looked up on the
// first call there.
mlk_status ScratchOnCurrentDevice(const char* fn, void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return FromHip(e, "hipGetDevice");
    if (dev < 0 || dev >= kScratchDevices) {
        return Fail(MLK_ERR_INVALID, "%s: device %d beyond the %d devices this entry supports", fn,
                    dev, kScratchDevices);
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return FromHip(e, "hipGetSymbolAddress(scratch)");
        if (ptr == nullptr) return Fail(MLK_ERR_HIP, "%s: no device address for the scratch", fn);
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return MLK_OK;
}
}  // namespace
}  // namespace mlk

extern "C" {

size_t mlk_attention_noalloc_scratch_bytes(void) { return mlk::kScratchBytes; }

mlk_status mlk_attention_decode_f32_noalloc(const float* q, int64_t q_row_stride,
                                            const float* k_cache, const float* v_cache,
                                            int64_t n_layers, int64_t max_seq, int32_t n_heads,
                                            int32_t n_kv_heads, int32_t head_dim, int64_t layer,
                                            const int32_t* positions, int32_t pos0,
                                            int64_t n_tokens, int64_t max_ctx, float* out,
                                            int32_t* err, void* stream) {
    const char* fn = "mlk_attention_decode_f32_noalloc";
    const int64_t need =
        mlk_attention_workspace_bytes(n_tokens, n_heads, n_kv_heads, head_dim, max_ctx);
    if (need > static_cast<int64_t>(mlk::kScratchBytes)) {
        return Fail(MLK_ERR_INVALID,
                    "%s: %lld bytes of chunk partials exceed the %zu-byte scratch of this entry "
                    "(fewer tokens or a smaller max_ctx, or mlk_attention_decode_f32 with a "
                    "workspace)", fn, static_cast<long long>(need), mlk::kScratchBytes);
    }
    void* ws = nullptr;
    const mlk_status st = mlk::ScratchOnCurrentDevice(fn, &ws);
    if (st != MLK_OK) return st;
    return mlk_attention_decode_f32(q, q_row_stride, k_cache, v_cache, n_layers, max_seq, n_heads,
                                    n_kv_heads, head_dim, layer, positions, pos0, n_tokens,
                                    max_ctx, out, ws, mlk::kScratchBytes, err, stream);
}

mlk_status mlk_attention_prefill_f32(const float* q, int64_t q_row_stride, const float* k_cache,
                                     const float* v_cache, int64_t n_layers, int64_t max_seq,
                                     int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                                     int64_t layer, int32_t pos0, int64_t n_tokens, float* out,
                                     void* stream) {
    const char* fn = "mlk_attention_prefill_f32";
    mlk_status st = CheckCache(fn, k_cache, v_cache, n_layers, max_seq, n_kv_heads, head_dim,
                               layer);
    if (st != MLK_OK) return st;
    if (q == nullptr || out == nullptr) return Fail(MLK_ERR_INVALID, "%s: q and out must not be null", fn);
    if (n_heads <= 0 || n_heads % n_kv_heads != 0) {
        return Fail(MLK_ERR_INVALID,
                    "%s: n_kv_heads must be non-zero and divide n_heads, got n_heads=%d, "
                    "n_kv_heads=%d", fn, n_heads, n_kv_heads);
    }
    if (n_tokens <= 0 || n_tokens > 0x7FFFFFFF) {
        return Fail(MLK_ERR_INVALID, "%s: n_tokens %lld out of range", fn,
                    static_cast<long long>(n_tokens));
    }
    if (q_row_stride < static_cast<int64_t>(n_heads) * head_dim) {
        return Fail(MLK_ERR_INVALID, "%s: q_row_stride must be at least n_heads * head_dim", fn);
    }
    if (pos0 < 0 || pos0 + n_tokens > max_seq) {
        return Fail(MLK_ERR_RANGE, "%s: positions %d..%lld out of range [0, %lld)", fn, pos0,
                    static_cast<long long>(pos0 + n_tokens - 1), static_cast<long long>(max_seq));
    }
    if (!PrefillSupported(head_dim, q, q_row_stride, out, k_cache, v_cache)) {
        return Fail(MLK_ERR_INVALID,
                    "%s: needs head_dim 64 or 128, q_row_stride %% 4 == 0 and 16-byte aligned q, "
                    "out and caches (mlk_attention_decode_f32 takes any shape)", fn);
    }
    if (out >= q && out < q + (n_tokens - 1) * q_row_stride + static_cast<int64_t>(n_heads) * head_dim) {
        return Fail(MLK_ERR_INVALID, "%s: out must not alias q", fn);
    }
    const int64_t slot = static_cast<int64_t>(n_kv_heads) * head_dim;
    return LaunchPrefill(q, q_row_stride, k_cache + layer * max_seq * slot,
                         v_cache + layer * max_seq * slot, slot, n_heads, n_kv_heads, head_dim,
                         pos0, n_tokens, out, AsStream(stream));
}

}  // extern "C"
