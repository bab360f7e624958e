// mlk_prefill.hip -- causal attention of a prompt chunk on the matrix cores.
//
// Tokens t < T sit at positions pos0 + t; token t's head h attends to cache
// positions 0 .. pos0 + t of its KV head g = h / (H / KV) (the reference's
// ForwardAttention per token, src/forward.cc:265-298, with the chunk's own
// K/V rows already written to the cache):
//   s_j = (q . k_j) * (1 / sqrt(hd)),  p = softmax(s),  out = sum_j p_j v_j
// in fp32.  The dot products and the weighted sum run on
// v_mfma_f32_16x16x4_f32, so their fp32 summation order differs from the
// reference's serial loops; the result is held to the same float64 error
// bound as the decode kernel's (every order of the fp32 sums meets it).
//
// Work layout: a workgroup of 4 waves owns 16 consecutive tokens and 4 query
// heads of one KV head (wave w: head 4 * head_block + w of the group), so
// the 4 waves share each K/V tile.  Workgroups run in reverse token order,
// the longest prefixes first.  Per tile of 32 cache positions (staged
// through two LDS buffers, rows hd + 4 floats apart; the next tile's global
// loads are issued before the current tile's MFMAs):
//   - S^T = K Q^T (16 positions x 16 queries per instruction block): K rows
//     come from LDS, each lane's q row (query l % 16, dims 16c + 4(l / 16)
//     .. + 3) lives in registers for the whole kernel.  S^T rather than S,
//     because the MFMA output layout of S^T (lane l, register r: position
//     4(l / 16) + r, query l % 16) is exactly the B-operand layout of
//     O^T = V^T P^T, so p never goes through LDS or a transpose.
//   - Online softmax per query: the running max needs 2 cross-lane
//     shuffles per tile (the 4 lane groups of a query); the running sum
//     stays per lane and is reduced once at the end.
//   - O^T += V^T P^T: V read from LDS one float per lane and step (16
//     consecutive dims per 16 lanes), 32 accumulators per lane at hd = 128.
// Positions past the workgroup's last token are clamped on load and masked
// (-inf score) per query.  A wave whose head is past its group (head counts
// per KV head that are not a multiple of 4) computes on head 0's query and
// stores nothing: no branch around the loop body.  FLOPs: 4 * hd * H * sum_t (pos0 + t + 1).
//
// bf16 products (kBf: every launch at head_dim 128; head_dim 64 keeps the
// fp32 instruction above): K, V, q and p are each the exact sum of three
// bf16 pieces (x with its low 16 bits cleared, the same of the rest, the
// rest: at most 8 significant bits each), staged once per tile by the
// thread that loaded them.  Two tile buffers (111 KB) when the grid has at
// most one workgroup per compute unit (16-token decode blocks of the 8B
// shape); otherwise one (56.8 KB, a barrier before each restage), so two
// workgroups share a unit and one's softmax and staging overlap the other's
// matrix work: 8B prefill of 4096 tokens 1339 -> 1107 us, 64 decode tokens
// 100 -> 79 us.  v_mfma_f32_16x16x32_bf16 takes 32 dims (scores)
// or the tile's 32 positions (values) per instruction in half the cycles of
// the fp32 instruction's 4.  Scores and values each keep the 6 piece
// products above 2^-21 relative: with pieces below 2^-7 and 2^-14 of the
// value, the dropped three are below 2^-20 |a b| (16 u) a product; for
// scores within the gamma_{hd+1} score bound with the fp32 sums, for values
// 16 u of sum_j p_j |v_jd| on top of the fp32 sums' (n + 6) u (the
// (n + 22) u the tests hold the tiles to).  The value MFMA's k index is the
// lane's own 8 probabilities: slot 8 kq + j is position 16 (j / 4) + 4 kq +
// j % 4 of the tile, the order V^T is staged in.
#include "mlk_attention.h"

#include <cmath>
#include <type_traits>

namespace mlk {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kPfThreads = 256;
constexpr int kPfTokens = 16;  // tokens per workgroup: the MFMA's 16 query columns
constexpr int kPfTile = 32;    // cache positions per K/V tile
constexpr int kPfHeads = 4;    // query heads per workgroup, one per wave

template <int HD>
struct __align__(16) PrefillSmem {
    float k[2][kPfTile * (HD + 4)];
    float v[2][kPfTile * (HD + 4)];
};

// The next K and V tiles in registers: thread tid holds float4 tid + 256 i
// of the [32][HD] tiles (positions past max_pos read max_pos's row).  The
// registers are native 4-vectors: with HIP's float4 struct, each copy is an
// aggregate memcpy, and the optimizer fuses load and LDS store into one
// global-to-LDS copy at the store, so the prefetch would not happen.
template <int HD>
struct KvTile {
    static constexpr int NL = kPfTile * HD / 4 / kPfThreads;
    f32x4 k[NL], v[NL];  // vectors, not float4 structs (see Load)
    const float* kb;
    const float* vb;
    int64_t slot, max_pos;
    __device__ void Load(int64_t p0) {
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const int idx = static_cast<int>(threadIdx.x) + kPfThreads * i;
            const int64_t p = p0 + idx / (HD / 4);
            const int64_t pos = p <= max_pos ? p : max_pos;
            const int c4 = idx % (HD / 4);
            k[i] = *reinterpret_cast<const f32x4*>(kb + pos * slot + 4 * c4);
            v[i] = *reinterpret_cast<const f32x4*>(vb + pos * slot + 4 * c4);
        }
    }
    __device__ void Store(float* ks, float* vs) const {
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const int idx = static_cast<int>(threadIdx.x) + kPfThreads * i;
            const int o = (idx / (HD / 4)) * (HD + 4) + 4 * (idx % (HD / 4));
            *reinterpret_cast<f32x4*>(ks + o) = k[i];
            *reinterpret_cast<f32x4*>(vs + o) = v[i];
        }
    }
};

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
constexpr int kBfKLd = 8;  // bf16 padding per K plane row (rows 16 bytes apart in bank terms)
constexpr int kBfVLd = kPfTile + 8;  // V^T plane row: 32 slots + 8 padding

// K planes [piece][32 positions][HD + 8] and V^T planes [piece][HD][40] of
// a tile, bf16: NBUF buffers (one: 56.8 KB, two workgroups per compute unit).
template <int HD, int NBUF>
struct __align__(16) PrefillSmemBf {
    uint16_t k[NBUF][3 * kPfTile * (HD + kBfKLd)];
    uint16_t v[NBUF][3 * HD * kBfVLd];
};

// The three bf16 pieces of 4 floats, 4 per dword pair (low half first).
__device__ inline void SplitPieces4(f32x4 x, uint2 (&o)[3]) {
    uint32_t h[4], m[4], l[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t u = __float_as_uint(x[i]);
        const float r = x[i] - __uint_as_float(u & 0xFFFF0000u);
        const uint32_t ru = __float_as_uint(r);
        h[i] = u;
        m[i] = ru;
        l[i] = __float_as_uint(r - __uint_as_float(ru & 0xFFFF0000u));
    }
    o[0] = make_uint2(__builtin_amdgcn_perm(h[1], h[0], 0x07060302u),
                      __builtin_amdgcn_perm(h[3], h[2], 0x07060302u));
    o[1] = make_uint2(__builtin_amdgcn_perm(m[1], m[0], 0x07060302u),
                      __builtin_amdgcn_perm(m[3], m[2], 0x07060302u));
    o[2] = make_uint2(__builtin_amdgcn_perm(l[1], l[0], 0x07060302u),
                      __builtin_amdgcn_perm(l[3], l[2], 0x07060302u));
}

// The three pieces of 8 floats as bf16x8 operands.
__device__ inline void SplitPieces8(f32x4 a, f32x4 b, bf16x8 (&o)[3]) {
    uint2 pa[3], pb[3];
    SplitPieces4(a, pa);
    SplitPieces4(b, pb);
#pragma unroll
    for (int p = 0; p < 3; ++p) {
        const uint4 w = make_uint4(pa[p].x, pa[p].y, pb[p].x, pb[p].y);
        o[p] = __builtin_bit_cast(bf16x8, w);
    }
}

// The next tile for the bf16 kernel: thread tid holds one 4 x 4 block of K
// and one of V, at positions 4 a .. 4 a + 3 and dims 4 c4 .. 4 c4 + 3
// (head_dim 128), positions past max_pos reading max_pos's row.  K takes
// a = tid / 32, c4 = tid % 32 (a 16-lane group writes 128 contiguous bytes
// of a plane row); V takes a = tid % 8, c4 = tid / 8, so a group's V^T
// writes (8 position groups x 2 dim rows, 80 bytes apart) meet each LDS
// bank once.
struct KvBlockBf {
    f32x4 k[4], v[4];
    const float* kb;
    const float* vb;
    int64_t slot, max_pos;
    __device__ void Load(int64_t p0) {
        const int tid = static_cast<int>(threadIdx.x);
        const int ak = tid / 32, ck = tid % 32, av = tid % 8, cv = tid / 8;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t p = p0 + 4 * ak + r;
            const int64_t pos = p <= max_pos ? p : max_pos;
            k[r] = *reinterpret_cast<const f32x4*>(kb + pos * slot + 4 * ck);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t p = p0 + 4 * av + r;
            const int64_t pos = p <= max_pos ? p : max_pos;
            v[r] = *reinterpret_cast<const f32x4*>(vb + pos * slot + 4 * cv);
        }
    }
    // K rows 4 a + r; V^T rows 4 c4 + e at slots s0 .. s0 + 3, where
    // positions 4 a .. 4 a + 3 sit (slot 8 kq + j: position 16 (j / 4) +
    // 4 kq + j % 4)
    // KL / VLD: the K and V^T plane row strides (the LDS layout's, or the
    // unpadded images of KvPieces)
    template <int KL = 128 + kBfKLd, int VLD = kBfVLd>
    __device__ void Store(uint16_t* ks, uint16_t* vs) const {
        constexpr int HD = 128;
        const int tid = static_cast<int>(threadIdx.x);
        const int a = tid / 32, c4 = tid % 32, av = tid % 8, cv = tid / 8;
        const int s0 = av < 4 ? 8 * av : 8 * (av - 4) + 4;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            uint2 pc[3];
            SplitPieces4(k[r], pc);
#pragma unroll
            for (int p = 0; p < 3; ++p) {
                *reinterpret_cast<uint2*>(ks + (p * kPfTile + 4 * a + r) * KL + 4 * c4) = pc[p];
            }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            uint2 pc[3];
            SplitPieces4(f32x4{v[0][e], v[1][e], v[2][e], v[3][e]}, pc);
#pragma unroll
            for (int p = 0; p < 3; ++p) {
                *reinterpret_cast<uint2*>(vs + (p * HD + 4 * cv + e) * VLD + s0) = pc[p];
            }
        }
    }
};

// Pre-split tiles (head_dim 128): per KV head g and tile t of 32 cache
// positions, the K planes [3][32][128] and the V^T planes [3][128][32] in
// bf16, exactly what KvBlockBf::Store writes to LDS, without the row
// padding: one 48 KB image a tile, images of head g at g * n_tiles + t.
// A prompt chunk's workgroups each stage every tile of their prefix, so
// the split (most of the VALU work of a tile) is done once here instead of
// once per 16 tokens.
constexpr int kPieceHalves = 3 * kPfTile * 128;        // bf16 of a K (or V^T) image
constexpr int kPieceTileU4 = 2 * kPieceHalves * 2 / 16;  // uint4 of a tile's two images

__global__ __launch_bounds__(kPfThreads) void KvPieces(const float* __restrict__ kc,
                                                       const float* __restrict__ vc,
                                                       int64_t slot, int KV, int64_t max_pos,
                                                       int64_t n_tiles,
                                                       uint16_t* __restrict__ images) {
    const int64_t t = blockIdx.x / KV;
    const int g = static_cast<int>(blockIdx.x % KV);
    KvBlockBf tile;
    tile.kb = kc + static_cast<int64_t>(g) * 128;
    tile.vb = vc + static_cast<int64_t>(g) * 128;
    tile.slot = slot;
    tile.max_pos = max_pos;  // positions past it read its row
    tile.Load(t * kPfTile);
    uint16_t* ks = images + (static_cast<int64_t>(g) * n_tiles + t) * (2 * kPieceHalves);
    tile.Store<128, kPfTile>(ks, ks + kPieceHalves);
}

// The next tile from KvPieces' images: thread tid copies uint4 tid + 256 i
// (i < 6) of the K image and of the V^T image.  K image uint4 u: piece
// u / 512, row (u / 16) % 32, dims 8 (u % 16) ..; V^T image: piece u / 512,
// dim (u / 4) % 128, slots 8 (u % 4) ...  In the workgroup's last tile, V
// at positions past its last token's is zeroed (their probabilities are 0;
// KvBlockBf reads the last token's row there, so finite values give the
// same sums), and K there needs nothing (those scores are replaced by -inf).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct KvBlockPre {
    u32x4 k[6], v[6];   // native vectors, not uint4 structs (see KvTile::Load)
    const u32x4* base;  // head g's first image
    int64_t max_pos;
    __device__ void Load(int64_t p0) {
        const u32x4* src = base + (p0 / kPfTile) * kPieceTileU4;
        const int tid = static_cast<int>(threadIdx.x);
#pragma unroll
        for (int i = 0; i < 6; ++i) {
            k[i] = src[tid + kPfThreads * i];
            v[i] = src[kPieceTileU4 / 2 + tid + kPfThreads * i];
        }
        const int64_t mp = max_pos - p0;  // the last position kept, within the tile
        if (mp < kPfTile - 1) {
#pragma unroll
            for (int i = 0; i < 6; ++i) {
                // slots 8 q4 + 2d, + 1 (dword d): positions 16 (d / 2) + 4 q4 +
                // 2 (d % 2), + 1
                const int64_t b = 4 * ((tid + kPfThreads * i) % 4);
                const auto keep = [&](int64_t pl) {
                    return (pl <= mp ? 0x0000FFFFu : 0u) | (pl + 1 <= mp ? 0xFFFF0000u : 0u);
                };
                v[i].x &= keep(b);
                v[i].y &= keep(b + 2);
                v[i].z &= keep(b + 16);
                v[i].w &= keep(b + 18);
            }
        }
    }
    __device__ void Store(uint16_t* ks, uint16_t* vs) const {
        constexpr int KL = 128 + kBfKLd;
        const int tid = static_cast<int>(threadIdx.x);
#pragma unroll
        for (int i = 0; i < 6; ++i) {
            const int u = tid + kPfThreads * i;
            *reinterpret_cast<u32x4*>(ks + ((u / 512) * kPfTile + (u / 16) % kPfTile) * KL +
                                      8 * (u % 16)) = k[i];
            *reinterpret_cast<u32x4*>(vs + ((u / 512) * 128 + (u / 4) % 128) * kBfVLd +
                                      8 * (u % 4)) = v[i];
        }
    }
};

// kChunked (decode tokens at any positions, AttnDecodeTile below): the
// token's position comes from `positions`, and the workgroup covers one
// chunk of cache positions, writing partials for AttnCombine.
struct TileChunks {
    const int32_t* positions;  // per token, or null: pos0 + t
    int64_t max_ctx;
    int chunk, n_chunks;
    float* ws_acc;  // [T, H, n_chunks, hd]
    float* ws_ml;   // [T, H, n_chunks, 2]
    int32_t* err;
};

template <int HD, bool kChunked, bool kBf, int NBUF = 2, bool kPre = false>
__global__ __launch_bounds__(kPfThreads) void AttnPrefill(
    const float* __restrict__ q, int64_t q_stride, const float* __restrict__ kc,
    const float* __restrict__ vc, int64_t slot, int KV, int H, int32_t pos0, int64_t T,
    float scale, float* __restrict__ out, int head_blocks, TileChunks tc,
    const uint16_t* __restrict__ images, int64_t n_image_tiles, uint32_t* __restrict__ a_planes) {
#pragma clang fp contract(off)
    static_assert(!kBf || HD == 128, "bf16 products: head_dim 128");
    static_assert(!kPre || (kBf && !kChunked), "pre-split tiles: prompt chunks, bf16 products");
    static_assert(NBUF == 2 || (NBUF == 1 && kBf), "one tile buffer: bf16 products only");
    constexpr int LD = HD + 4;
    constexpr int NC = HD / 16;                          // 16-dim chunks
    constexpr int KL = HD + kBfKLd;                      // K plane row (bf16)
    __shared__ typename std::conditional<kBf, PrefillSmemBf<HD, NBUF>, PrefillSmem<HD>>::type sm;
    const int group = H / KV;
    const int64_t n_tb = (T + kPfTokens - 1) / kPfTokens;
    int64_t bid = blockIdx.x;
    const int hb = static_cast<int>(bid % head_blocks);
    bid /= head_blocks;
    const int g = static_cast<int>(bid % KV);
    bid /= KV;
    int ck = 0;  // the chunk (kChunked)
    if constexpr (kChunked) {
        ck = static_cast<int>(bid / n_tb);
        bid %= n_tb;
    }
    const int64_t t0 = (n_tb - 1 - bid) * kPfTokens;
    const int wave = threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    const int i16 = lane & 15, kq = lane >> 4;
    const int hq = hb * kPfHeads + wave;  // query head within the group
    const bool active = hq < group;
    const int h = g * group + (active ? hq : 0);
    const int64_t last_t = (t0 + kPfTokens < T ? t0 + kPfTokens : T) - 1;
    const int64_t t = t0 + i16 <= last_t ? t0 + i16 : last_t;  // this lane's query token
    int64_t my_pos = pos0 + t;
    int64_t max_pos = pos0 + last_t;
    int64_t p_begin = 0, p_end = max_pos + 1;  // cache positions of this workgroup
    bool valid = true;
    if constexpr (kChunked) {
        const int32_t pt = tc.positions != nullptr ? tc.positions[t] : pos0 + static_cast<int32_t>(t);
        valid = pt >= 0 && pt < tc.max_ctx;
        if (!valid && ck == 0 && hb == 0 && g == 0 && t0 + i16 <= last_t) RaiseFlag(tc.err, 1);
        my_pos = valid ? pt : -1;  // an invalid token attends nothing
        // the block's last position: the maximum over its 16 tokens
        int32_t mx = static_cast<int32_t>(my_pos);
#pragma unroll
        for (int o = 1; o < 16; o *= 2) mx = max(mx, __shfl_xor(mx, o, kWave));
        max_pos = mx;
        p_begin = static_cast<int64_t>(ck) * tc.chunk;
        p_end = p_begin + tc.chunk < max_pos + 1 ? p_begin + tc.chunk : max_pos + 1;
        if (p_begin >= p_end) {  // no token of the block reaches this chunk
            if (tc.n_chunks == 1 && active && t0 + i16 <= last_t) {
                // every token invalid, and no merge follows: zero rows
                float* orow = out + (t * H + h) * static_cast<int64_t>(HD) + 4 * kq;
#pragma unroll
                for (int cc = 0; cc < NC; ++cc) {
                    *reinterpret_cast<float4*>(orow + 16 * cc) = make_float4(0.f, 0.f, 0.f, 0.f);
                }
            }
            return;
        }
    }

    f32x4 qv[NC];         // fp32: dims 16 c + 4 kq .. + 3
    bf16x8 qp[3][HD / 32];  // bf16: pieces of dims 32 c + 8 kq .. + 7
    if constexpr (kBf) {
        const float* qrow = q + t * q_stride + static_cast<int64_t>(h) * HD + 8 * kq;
#pragma unroll
        for (int c = 0; c < HD / 32; ++c) {
            bf16x8 pc[3];
            SplitPieces8(*reinterpret_cast<const f32x4*>(qrow + 32 * c),
                         *reinterpret_cast<const f32x4*>(qrow + 32 * c + 4), pc);
#pragma unroll
            for (int p = 0; p < 3; ++p) qp[p][c] = pc[p];
        }
    } else {
        const float* qrow = q + t * q_stride + static_cast<int64_t>(h) * HD + 4 * kq;
#pragma unroll
        for (int c = 0; c < NC; ++c) qv[c] = *reinterpret_cast<const f32x4*>(qrow + 16 * c);
    }

    typename std::conditional<kPre, KvBlockPre,
                              typename std::conditional<kBf, KvBlockBf, KvTile<HD>>::type>::type
        tile;
    if constexpr (kPre) {
        tile.base = reinterpret_cast<const u32x4*>(images) +
                    static_cast<int64_t>(g) * n_image_tiles * kPieceTileU4;
    } else {
        tile.kb = kc + static_cast<int64_t>(g) * HD;
        tile.vb = vc + static_cast<int64_t>(g) * HD;
        tile.slot = slot;
    }
    tile.max_pos = max_pos;
    auto load = [&](int64_t p0) { tile.Load(p0); };
    auto store = [&](int buf) { tile.Store(sm.k[buf], sm.v[buf]); };

    f32x4 acc[NC];  // O^T: acc[c][r] = dim 16c + 4 kq + r of query i16
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY;  // running max of query i16 (equal in its 4 lane groups)
    float l = 0.0f;       // this lane's part of the running sum

    const int64_t n_tiles = (p_end - p_begin + kPfTile - 1) / kPfTile;
    load(p_begin);
    store(0);
    __syncthreads();
    // positions fit in 32 bits (below max_seq); log2-unit score scale
    const int32_t my_pos_32 = static_cast<int32_t>(my_pos);
    const float scale2 = scale * 1.44269504088896340736f;
    for (int64_t it = 0; it < n_tiles; ++it) {
        const int buf = NBUF == 2 ? static_cast<int>(it & 1) : 0;
        const int32_t p0_32 = static_cast<int32_t>(p_begin + it * kPfTile);
        load(p_begin + (it + 1 < n_tiles ? it + 1 : it) * kPfTile);
        // Nothing crosses this point: without it the scheduler sinks the
        // next tile's global loads to their LDS stores at the bottom of the
        // loop, and every tile then waits out a full HBM round trip.
        __builtin_amdgcn_sched_barrier(0);
        {  // idle waves (a head block past the group) compute too, unstored
            f32x4 s[2];
#pragma unroll
            for (int pt = 0; pt < 2; ++pt) {
                s[pt] = f32x4{0.f, 0.f, 0.f, 0.f};
                if constexpr (kBf) {
                    const uint16_t* krow = &sm.k[buf][(pt * 16 + i16) * KL + 8 * kq];
#pragma unroll
                    for (int c = 0; c < HD / 32; ++c) {
                        bf16x8 kp[3];
#pragma unroll
                        for (int p = 0; p < 3; ++p) {
                            kp[p] = *reinterpret_cast<const bf16x8*>(krow + p * kPfTile * KL + 32 * c);
                        }
                        // the 6 largest piece products, smallest first
                        s[pt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kp[2], qp[0][c], s[pt], 0, 0, 0);
                        s[pt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kp[0], qp[2][c], s[pt], 0, 0, 0);
                        s[pt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kp[1], qp[1][c], s[pt], 0, 0, 0);
                        s[pt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kp[1], qp[0][c], s[pt], 0, 0, 0);
                        s[pt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kp[0], qp[1][c], s[pt], 0, 0, 0);
                        s[pt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kp[0], qp[0][c], s[pt], 0, 0, 0);
                    }
                } else {
                    const float* krow = &sm.k[buf][(pt * 16 + i16) * LD + 4 * kq];
#pragma unroll
                    for (int c = 0; c < NC; ++c) {
                        const f32x4 kk = *reinterpret_cast<const f32x4*>(krow + 16 * c);
#pragma unroll
                        for (int st = 0; st < 4; ++st) {
                            s[pt] = __builtin_amdgcn_mfma_f32_16x16x4f32(kk[st], qv[c][st], s[pt],
                                                                         0, 0, 0);
                        }
                    }
                }
            }
            float sv[8];
            float tmax = -INFINITY;
#pragma unroll
            for (int pt = 0; pt < 2; ++pt) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    // scores in log2 units (scale * log2(e)), for exp2 below
                    const int32_t pos = p0_32 + pt * 16 + 4 * kq + r;
                    const float x = pos <= my_pos_32 ? s[pt][r] * scale2 : -INFINITY;
                    sv[pt * 4 + r] = x;
                    tmax = fmaxf(tmax, x);
                }
            }
            tmax = fmaxf(tmax, __shfl_xor(tmax, 16, kWave));
            tmax = fmaxf(tmax, __shfl_xor(tmax, 32, kWave));
            // finite: position 0 is in every query's range.  In a chunk, a
            // token before the chunk (or invalid) sees only -inf: it is
            // referenced to 0 and keeps m = -inf, l = 0 (AttnCombine never
            // reads that partial).
            const float mnew = fmaxf(m, tmax);
            const float mref = kChunked && mnew == -INFINITY ? 0.0f : mnew;
            // rescale only when some query's max moved (the factor is then
            // exactly 1 for the others: skipping it changes nothing)
            if (__builtin_amdgcn_ballot_w64(mnew != m) != 0) {
                const float corr = __builtin_amdgcn_exp2f(m - mref);
                l *= corr;
#pragma unroll
                for (int c = 0; c < NC; ++c) acc[c] *= corr;
            }
            float pv[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                pv[i] = __builtin_amdgcn_exp2f(sv[i] - mref);
                l += pv[i];
            }
            m = mnew;
            if constexpr (kBf) {
                // B: this lane's probabilities, slot j = position 16 (j / 4) + 4 kq + j % 4
                bf16x8 pp[3];
                SplitPieces8(f32x4{pv[0], pv[1], pv[2], pv[3]}, f32x4{pv[4], pv[5], pv[6], pv[7]}, pp);
#pragma unroll
                for (int c = 0; c < NC; ++c) {
                    const uint16_t* vrow = &sm.v[buf][(16 * c + i16) * kBfVLd + 8 * kq];
                    bf16x8 vp[3];
#pragma unroll
                    for (int p = 0; p < 3; ++p) {
                        vp[p] = *reinterpret_cast<const bf16x8*>(vrow + p * HD * kBfVLd);
                    }
                    // the 6 piece products above 2^-21 relative, smallest first
                    acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vp[2], pp[0], acc[c], 0, 0, 0);
                    acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vp[0], pp[2], acc[c], 0, 0, 0);
                    acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vp[1], pp[1], acc[c], 0, 0, 0);
                    acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vp[1], pp[0], acc[c], 0, 0, 0);
                    acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vp[0], pp[1], acc[c], 0, 0, 0);
                    acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vp[0], pp[0], acc[c], 0, 0, 0);
                }
            } else {
#pragma unroll
                for (int c = 0; c < NC; ++c) {
#pragma unroll
                    for (int pt = 0; pt < 2; ++pt) {
#pragma unroll
                        for (int st = 0; st < 4; ++st) {
                            const float vv = sm.v[buf][(pt * 16 + 4 * kq + st) * LD + 16 * c + i16];
                            acc[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv, pv[pt * 4 + st],
                                                                          acc[c], 0, 0, 0);
                        }
                    }
                }
            }
        }
        if constexpr (NBUF == 1) {
            __syncthreads();  // every wave is done with the tile before it is replaced
            store(0);
        } else {
            store(buf ^ 1);
        }
        __syncthreads();
    }
    l += __shfl_xor(l, 16, kWave);
    l += __shfl_xor(l, 32, kWave);
    if (!active || t0 + i16 > last_t) return;
    if constexpr (kChunked) {
        const int64_t row = t * H + h;
        if (tc.n_chunks > 1) {  // unnormalized partials, merged by AttnCombine
            float* arow = tc.ws_acc + (row * tc.n_chunks + ck) * HD + 4 * kq;
#pragma unroll
            for (int cc = 0; cc < NC; ++cc) {
                *reinterpret_cast<float4*>(arow + 16 * cc) =
                    make_float4(acc[cc][0], acc[cc][1], acc[cc][2], acc[cc][3]);
            }
            if (kq == 0) {  // the max back in natural-log units, as AttnCombine takes it
                tc.ws_ml[(row * tc.n_chunks + ck) * 2] = m * 0.69314718055994530942f;
                tc.ws_ml[(row * tc.n_chunks + ck) * 2 + 1] = l;
            }
            return;
        }
        if (!valid) {  // one chunk: the row is final here
            float* orow = out + row * HD + 4 * kq;
#pragma unroll
            for (int cc = 0; cc < NC; ++cc) {
                *reinterpret_cast<float4*>(orow + 16 * cc) = make_float4(0.f, 0.f, 0.f, 0.f);
            }
            return;
        }
    }
    float* orow = out + (t * H + h) * static_cast<int64_t>(HD) + 4 * kq;
    const float inv = 1.0f / l;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const float4 o = make_float4(acc[c][0] * inv, acc[c][1] * inv, acc[c][2] * inv,
                                     acc[c][3] * inv);
        *reinterpret_cast<float4*>(orow + 16 * c) = o;
        // the output rows [T, H * HD] also as StorePlanes planes (wo's x)
        if (a_planes != nullptr) {
            StorePlanes4(a_planes, T, t, static_cast<int64_t>(h) * HD + 16 * c + 4 * kq, o.x, o.y,
                         o.z, o.w);
        }
    }
}

}  // namespace

bool PrefillSupported(int32_t head_dim, const float* q, int64_t q_row_stride, const float* out,
                      const float* k_cache, const float* v_cache) {
    return (head_dim == 64 || head_dim == 128) && q_row_stride % 4 == 0 && Aligned(q, 16) &&
           Aligned(out, 16) && Aligned(k_cache, 16) && Aligned(v_cache, 16);
}

int64_t PrefillImageBytes(int32_t n_kv_heads, int32_t head_dim, int64_t n_pos) {
    if (head_dim != 128 || n_kv_heads <= 0 || n_pos <= 0) return 0;
    return static_cast<int64_t>(n_kv_heads) * ((n_pos + kPfTile - 1) / kPfTile) * kPieceTileU4 *
           16;
}

mlk_status LaunchPrefill(const float* q, int64_t q_row_stride, const float* kc, const float* vc,
                         int64_t slot, int32_t H, int32_t KV, int32_t head_dim, int32_t pos0,
                         int64_t T, float* out, hipStream_t s, void* workspace,
                         size_t workspace_bytes, uint32_t* a_planes) {
    const int group = H / KV;
    const int head_blocks = (group + kPfHeads - 1) / kPfHeads;
    const int64_t n_tb = (T + kPfTokens - 1) / kPfTokens;
    const int64_t blocks = n_tb * KV * head_blocks;
    if (blocks > 0x7FFFFFFF) return Fail(MLK_ERR_INVALID, "attention prefill: launch too large");
    const float scale = 1.0f / sqrtf(static_cast<float>(head_dim));
    const dim3 grid(static_cast<unsigned>(blocks));
    const TileChunks none{};
    // head_dim 128 with room for the tile images: split K and V once
    // (positions 0 .. pos0 + T - 1), then stage the images
    const int64_t n_pos = pos0 + T;
    const int64_t image_bytes = PrefillImageBytes(KV, head_dim, n_pos);
    if (image_bytes > 0 && T >= kPrefillImageMinTokens && workspace != nullptr &&
        Aligned(workspace, 16) &&
        static_cast<int64_t>(workspace_bytes) >= image_bytes) {
        const int64_t n_tiles = (n_pos + kPfTile - 1) / kPfTile;
        if (n_tiles * KV > 0x7FFFFFFF) return Fail(MLK_ERR_INVALID, "attention prefill: launch too large");
        uint16_t* images = static_cast<uint16_t*>(workspace);
        hipLaunchKernelGGL(KvPieces, dim3(static_cast<unsigned>(n_tiles * KV)), dim3(kPfThreads), 0,
                           s, kc, vc, slot, KV, n_pos - 1, n_tiles, images);
        mlk_status st = CheckLaunch("KvPieces");
        if (st != MLK_OK) return st;
        hipLaunchKernelGGL((AttnPrefill<128, false, true, 1, true>), grid, dim3(kPfThreads), 0, s,
                           q, q_row_stride, kc, vc, slot, KV, H, pos0, T, scale, out, head_blocks,
                           none, images, n_tiles, a_planes);
        return CheckLaunch("AttnPrefill");
    }
    if (head_dim == 64) {
        hipLaunchKernelGGL((AttnPrefill<64, false, false>), grid, dim3(kPfThreads), 0, s, q,
                           q_row_stride, kc, vc, slot, KV, H, pos0, T, scale, out, head_blocks,
                           none, nullptr, 0, a_planes);
    } else {
        hipLaunchKernelGGL((AttnPrefill<128, false, true, 1>), grid, dim3(kPfThreads), 0, s, q,
                           q_row_stride, kc, vc, slot, KV, H, pos0, T, scale, out, head_blocks,
                           none, nullptr, 0, a_planes);
    }
    return CheckLaunch("AttnPrefill");
}

// Positions per chunk: a power of two from 256 up to the whole context,
// halved while the grid has fewer than 512 workgroups.  Large batches then
// take the context in one chunk (no partials, no merge).
int TileChunk(int64_t T, int32_t H, int32_t KV, int64_t max_ctx) {
    const int group = H / KV;
    const int64_t base = (T + kPfTokens - 1) / kPfTokens * KV * ((group + kPfHeads - 1) / kPfHeads);
    int64_t chunk = 256;
    while (chunk < max_ctx && chunk < (int64_t{1} << 30)) chunk *= 2;
    while (chunk > 256 && base * ((max_ctx + chunk - 1) / chunk) < 512) chunk /= 2;
    return static_cast<int>(chunk);
}

mlk_status LaunchDecodeTile(const float* q, int64_t q_row_stride, const float* kc,
                            const float* vc, int64_t slot, int32_t H, int32_t KV,
                            int32_t head_dim, const int32_t* positions, int32_t pos0, int64_t T,
                            int64_t max_ctx, float* out, float* ws_acc, float* ws_ml,
                            int32_t* err, hipStream_t s) {
    const int group = H / KV;
    const int head_blocks = (group + kPfHeads - 1) / kPfHeads;
    const int64_t n_tb = (T + kPfTokens - 1) / kPfTokens;
    const int chunk = TileChunk(T, H, KV, max_ctx);
    const int64_t nc = (max_ctx + chunk - 1) / chunk;
    const int64_t blocks = n_tb * KV * head_blocks * nc;
    if (blocks > 0x7FFFFFFF) return Fail(MLK_ERR_INVALID, "attention decode: launch too large");
    TileChunks tc{positions, max_ctx, chunk, static_cast<int>(nc), ws_acc, ws_ml, err};
    const float scale = 1.0f / sqrtf(static_cast<float>(head_dim));
    const dim3 grid(static_cast<unsigned>(blocks));
    if (head_dim == 64) {
        hipLaunchKernelGGL((AttnPrefill<64, true, false>), grid, dim3(kPfThreads), 0, s, q,
                           q_row_stride, kc, vc, slot, KV, H, pos0, T, scale, out, head_blocks,
                           tc, nullptr, 0, nullptr);
    } else if (blocks <= ComputeUnits()) {
        // bf16 products: their 111 KB of LDS leave one workgroup per unit,
        // which a grid this small uses anyway
        hipLaunchKernelGGL((AttnPrefill<128, true, true>), grid, dim3(kPfThreads), 0, s, q,
                           q_row_stride, kc, vc, slot, KV, H, pos0, T, scale, out, head_blocks,
                           tc, nullptr, 0, nullptr);
    } else {
        hipLaunchKernelGGL((AttnPrefill<128, true, true, 1>), grid, dim3(kPfThreads), 0, s, q,
                           q_row_stride, kc, vc, slot, KV, H, pos0, T, scale, out, head_blocks,
                           tc, nullptr, 0, nullptr);
    }
    return CheckLaunch("AttnPrefill (decode tokens)");
}

}  // namespace mlk
