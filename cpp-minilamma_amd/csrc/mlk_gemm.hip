// mlk_gemm.hip -- prefill-shaped linear layers on the matrix cores:
// y[T, O] = x[T, K] W[O, K]^T (+ bias), W fp32 or Q8_0 / Q4_0 / Q4_1 blocks.
//
// Semantics are those of the GEMV kernels (mlk_linear.hip; the reference's
// LinearQ80/Q40/Q41, src/quant.cc:393-463, and cublasSgemm for F32,
// src/cuda_matmul.cc:142-186): every product is x * dequant(w) in fp32 and
// the sum is fp32, in an order of this kernel's choosing, within
// gamma_K * sum_k |x w| of the exact value.  Dequantized weights are the
// reference's element values: Q8_0 d * q and Q4_0 d * (code - 8) are exact
// in fp32 (an 11-bit scale times a small integer); Q4_1 is d * code + m
// rounded once per product and once per sum, as the reference's
// DequantQ41 (src/quant.cc:369-391).
//
// Work layout (one workgroup = 256 threads = 4 waves per BM x 128 tile of
// y, BM = 128 token rows, or 64 / 32 when T is that small; each wave owns
// a BM/2 x 64 quarter as BM/32 x 4 tiles of v_mfma_f32_16x16x4_f32, up to
// 64 accumulators per lane):
//   - K advances in stages of 32 (one quantization block).  A stage's
//     x tile [BM tokens][32] and weight tile [128 outputs][32] are staged
//     through LDS as fp32, rows 36 floats apart (16-byte aligned rows, and
//     the b128 reads of 8 consecutive lanes fall on all 32 banks);
//     quantized weights are decoded on the way in, so the matrix cores only
//     ever see fp32.
//   - Two LDS buffers: stage s+1's global loads are issued before stage
//     s's MFMAs and written to the other buffer after them, with one
//     barrier per stage.
//   - MFMA operands: lane l supplies row l % 16 and k-slot l / 16.  The
//     four k-slots of one instruction are taken 4 apart (k = 4 * (l / 16) +
//     s for step s), so each lane's four consecutive k values come from one
//     16-byte LDS read and feed four instructions; x and W use the same
//     assignment, so every product x[t, k] * w[o, k] is formed exactly once.
//   - Output: lane l, register r of a 16 x 16 tile holds row 4 * (l / 16) +
//     r, column l % 16; bias is added to the finished sum.
// Tiles past T or O load zeros (clamped addresses, masked values) and store
// nothing.  When the tiles are fewer than two per CU (few token rows), K is
// split over up to 32 workgroups per tile (each split at least 8 stages);
// the splits write partial sums to a caller-provided workspace and a second
// kernel adds them in split order (deterministic) plus the bias.
// FLOPs per call: 2 T O K.
#include "mlk_quant.h"

#include <type_traits>

namespace mlk {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kBN = 128;         // outputs per tile (token rows per tile: BM = 32, 64 or 128)
constexpr int kBK = 32;          // K per stage: one quantization block
constexpr int kLd = kBK + 4;     // LDS row stride, floats
constexpr int kGemmThreads = 256;
constexpr int kWF32 = -1;        // weight type value of fp32 weights

template <int BM>
struct GemmSmem {
    float x[2][BM * kLd];
    float w[2][kBN * kLd];
};

__device__ inline float4 Mask4(float4 v, uint32_t m) {
    return make_float4(__uint_as_float(__float_as_uint(v.x) & m),
                       __uint_as_float(__float_as_uint(v.y) & m),
                       __uint_as_float(__float_as_uint(v.z) & m),
                       __uint_as_float(__float_as_uint(v.w) & m));
}

// An [R][32] fp32 tile of a row-major [rows, K] matrix (x, or fp32 W):
// thread tid loads float4 (tid + 256 i) for i < R / 32, 8 per row, so 8
// consecutive lanes read one row's 128 contiguous bytes.  Rows past `rows`
// read row 0 and are zeroed -- at Store, so that nothing consumes the
// loaded values before the MFMAs of the stage in between have been issued.
template <int R>
struct F32Tile {
    static constexpr int kN = R / 32;
    float4 v[kN];
    uint32_t keep;  // bit i: float4 i is in range
    __device__ void Load(const float* p, int64_t rows, int64_t K, int64_t r0, int64_t k0) {
        keep = 0;
#pragma unroll
        for (int i = 0; i < kN; ++i) {
            const int idx = static_cast<int>(threadIdx.x) + kGemmThreads * i;
            const int64_t r = r0 + (idx >> 3);
            const int64_t c = k0 + 4 * (idx & 7);
            const bool ok = r < rows && c < K;
            keep |= static_cast<uint32_t>(ok) << i;
            v[i] = *reinterpret_cast<const float4*>(p + (ok ? r * K + c : 0));
        }
    }
    __device__ void Store(float* s) const {
#pragma unroll
        for (int i = 0; i < kN; ++i) {
            const int idx = static_cast<int>(threadIdx.x) + kGemmThreads * i;
            *reinterpret_cast<float4*>(s + (idx >> 3) * kLd + 4 * (idx & 7)) =
                Mask4(v[i], ((keep >> i) & 1u) ? ~0u : 0u);
        }
    }
};

// A [128 outputs][32] tile of one block column of quantized W: thread tid
// decodes half tid & 1 (16 elements) of output row tid >> 1.  Rows past O
// read row 0 and are zeroed.
template <int QT>
struct QuantTile {
    uint32_t d;        // Q8_0 / Q4_0: the fp16 scale; Q4_1: d | m << 16
    uint32_t q[4];     // the 16 code bytes this thread needs
    uint32_t keep;     // ~0 when the row exists
    __device__ void Load(const uint8_t* w, int64_t O, int64_t row_bytes, int64_t n0, int64_t kb) {
        const int64_t n = n0 + (threadIdx.x >> 1);
        const int h = threadIdx.x & 1;
        keep = n < O ? ~0u : 0u;
        const uint8_t* blk = w + (n < O ? n : 0) * row_bytes + kb * Fmt<QT>::kBytes;
        if constexpr (QT == MLK_Q4_1) {
            const uint32_t* p = reinterpret_cast<const uint32_t*>(blk);
            d = p[0];
#pragma unroll
            for (int i = 0; i < 4; ++i) q[i] = p[1 + i];
        } else {
            // Q8_0: codes 16h .. 16h+15 at byte 2 + 16h; Q4_0: all 16 code
            // bytes at byte 2 (half h takes the low or high nibbles)
            const uint16_t* p = reinterpret_cast<const uint16_t*>(blk);
            d = p[0];
            const int o = QT == MLK_Q8_0 ? 1 + 8 * h : 1;
#pragma unroll
            for (int i = 0; i < 4; ++i) q[i] = p[o + 2 * i] | (static_cast<uint32_t>(p[o + 2 * i + 1]) << 16);
        }
    }
    __device__ void Store(float* s) const {
        const int h = threadIdx.x & 1;
        float* dst = s + (threadIdx.x >> 1) * kLd + 16 * h;
        float e[16];
        if constexpr (QT == MLK_Q8_0) {
            const float sc = HalfHw(d & 0xFFFFu);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int32_t code = static_cast<int32_t>(q[i / 4] << (24 - 8 * (i % 4))) >> 24;
                e[i] = sc * static_cast<float>(code);
            }
        } else if constexpr (QT == MLK_Q4_0) {
            const float sc = HalfHw(d & 0xFFFFu);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const uint32_t byte = (q[i / 4] >> (8 * (i % 4))) & 0xFFu;
                const int code = static_cast<int>(h ? byte >> 4 : byte & 15u);
                e[i] = sc * static_cast<float>(code - 8);
            }
        } else {
            const float sc = HalfHw(d & 0xFFFFu);
            const float mn = HalfHw(d >> 16);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const uint32_t byte = (q[i / 4] >> (8 * (i % 4))) & 0xFFu;
                const float code = static_cast<float>(h ? byte >> 4 : byte & 15u);
                e[i] = __fadd_rn(__fmul_rn(sc, code), mn);
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            *reinterpret_cast<float4*>(dst + 4 * i) =
                Mask4(make_float4(e[4 * i], e[4 * i + 1], e[4 * i + 2], e[4 * i + 3]), keep);
        }
    }
};

// The same tile from the planar layout: thread tid takes inputs 16h ..
// 16h + 15 (h = tid & 1) of block kb of row n0 + (tid >> 1), which lanes
// 32h + r and 32h + 16 + r of the row's tile hold; the decoded values are
// the block layout's (d * q, d * (code - 8)).
template <int QT>
struct PlanarTile {
    uint32_t d;
    uint32_t q[4];
    uint32_t keep;
    __device__ void Load(const uint8_t* w, int64_t O, int64_t K, int64_t n0, int64_t kb) {
        const int64_t n = n0 + (threadIdx.x >> 1);
        const int h = threadIdx.x & 1;
        keep = n < O ? ~0u : 0u;
        const int64_t row = n < O ? n : 0, rt = row / 16;
        const int r = static_cast<int>(row % 16);
        const int64_t tiles = (O + 15) / 16;
        const int64_t code_tile = QT == MLK_Q8_0 ? 16 * K : 8 * K;
        const uint8_t* scales = w + tiles * code_tile;
        d = *reinterpret_cast<const uint16_t*>(scales + ((rt * (K / 256) + kb / 8) * 16 + r) * 16 +
                                               (kb % 8) * 2);
        if constexpr (QT == MLK_Q8_0) {
            const uint8_t* c = w + rt * code_tile + ((kb / 2) * 64 + 32 * h + r) * 16 + (kb & 1) * 8;
            const uint2 a = *reinterpret_cast<const uint2*>(c);
            const uint2 b = *reinterpret_cast<const uint2*>(c + 16 * 16);
            q[0] = a.x;
            q[1] = a.y;
            q[2] = b.x;
            q[3] = b.y;
        } else {
            const uint8_t* c = w + rt * code_tile + ((kb / 4) * 64 + 32 * h + r) * 16 + (kb % 4) * 4;
            q[0] = *reinterpret_cast<const uint32_t*>(c);
            q[1] = *reinterpret_cast<const uint32_t*>(c + 16 * 16);
        }
    }
    __device__ void Store(float* s) const {
        const int h = threadIdx.x & 1;
        float* dst = s + (threadIdx.x >> 1) * kLd + 16 * h;
        const float sc = HalfHw(d);
        float e[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            int32_t code;
            if constexpr (QT == MLK_Q8_0) {
                code = static_cast<int32_t>(q[i / 4] << (24 - 8 * (i % 4))) >> 24;
            } else {  // input 8g + e: nibble e (low half of byte e, then high)
                const int e8 = i % 8;
                const int sh = e8 < 4 ? 8 * e8 : 8 * (e8 - 4) + 4;
                code = static_cast<int32_t>(q[i / 8] << (28 - sh)) >> 28;
            }
            e[i] = sc * static_cast<float>(code);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            *reinterpret_cast<float4*>(dst + 4 * i) =
                Mask4(make_float4(e[4 * i], e[4 * i + 1], e[4 * i + 2], e[4 * i + 3]), keep);
        }
    }
};

template <int WT>
struct WTile : QuantTile<WT> {
    __device__ void Load(const uint8_t* w, int64_t O, int64_t, int64_t row_bytes, int64_t n0,
                         int64_t k0) {
        QuantTile<WT>::Load(w, O, row_bytes, n0, k0 / kBK);
    }
};
template <>
struct WTile<kWPlanarQ8> : PlanarTile<MLK_Q8_0> {
    __device__ void Load(const uint8_t* w, int64_t O, int64_t K, int64_t, int64_t n0, int64_t k0) {
        PlanarTile<MLK_Q8_0>::Load(w, O, K, n0, k0 / kBK);
    }
};
template <>
struct WTile<kWPlanarQ4> : PlanarTile<MLK_Q4_0> {
    __device__ void Load(const uint8_t* w, int64_t O, int64_t K, int64_t, int64_t n0, int64_t k0) {
        PlanarTile<MLK_Q4_0>::Load(w, O, K, n0, k0 / kBK);
    }
};
template <>
struct WTile<kWF32> : F32Tile<kBN> {
    __device__ void Load(const uint8_t* w, int64_t O, int64_t K, int64_t, int64_t n0, int64_t k0) {
        F32Tile<kBN>::Load(reinterpret_cast<const float*>(w), O, K, n0, k0);
    }
};

// Instruction order of one K stage (the scheduler's groups, in order): the
// first half's operand reads; the next stage's global loads one per MFMA;
// the second half's operand reads one per MFMA; the rest of the first
// half's MFMAs; the next stage's LDS writes spread over the second half's
// MFMAs.  Left to itself the scheduler sinks the global loads to their use
// (the LDS writes after the MFMAs), which exposes the load latency every
// stage; with the loads first and the writes last it serializes the
// address and write work around the MFMA stream instead.
template <int MI>
__device__ inline void InterleaveStage() {
    constexpr int kMfma = 0x008, kVmemRead = 0x020, kDsRead = 0x100, kDsWrite = 0x200;
    constexpr int kOperands = MI + 4;   // b128 reads per half: MI x rows, 4 W rows
    constexpr int kHalf = 16 * MI;      // MFMAs per half stage
    __builtin_amdgcn_sched_group_barrier(kDsRead, kOperands, 0);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
        __builtin_amdgcn_sched_group_barrier(kVmemRead, 1, 0);
    }
#pragma unroll
    for (int i = 0; i < kOperands; ++i) {
        __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
        __builtin_amdgcn_sched_group_barrier(kDsRead, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(kMfma, kHalf - 8 - kOperands, 0);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        __builtin_amdgcn_sched_group_barrier(kMfma, kHalf / 8, 0);
        __builtin_amdgcn_sched_group_barrier(kDsWrite, 1, 0);
    }
}

// Workgroup (tile, split): split `sp` covers K stages [sp * per_split,
// min((sp + 1) * per_split, all)); with one split it writes y (+ bias),
// with more it writes its partial sums to partial[sp] ([T, O] each) for
// SplitKReduce.  A tile is BM token rows x 128 outputs; wave w owns rows
// (w / 2) * BM / 2 .. + BM / 2 and outputs (w % 2) * 64 .. + 64, i.e.
// MI = BM / 32 by 4 MFMA tiles.
template <int WT, int BM>
__global__ __launch_bounds__(kGemmThreads) void GemmMfma(const float* __restrict__ x,
                                                         const uint8_t* __restrict__ w,
                                                         const float* __restrict__ bias,
                                                         float* __restrict__ y, int64_t T,
                                                         int64_t K, int64_t O, int64_t row_bytes,
                                                         int tiles_m, int tiles,
                                                         int64_t per_split,
                                                         float* __restrict__ partial) {
    constexpr int MI = BM / 32;
    __shared__ GemmSmem<BM> sm;
    const int tile = static_cast<int>(blockIdx.x) % tiles;
    const int sp = static_cast<int>(blockIdx.x) / tiles;
    const int tm = tile % tiles_m;
    const int tn = tile / tiles_m;
    const int64_t m0 = static_cast<int64_t>(tm) * BM;
    const int64_t n0 = static_cast<int64_t>(tn) * kBN;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int wm = wave >> 1, wn = wave & 1;
    const int i16 = lane & 15, kq = lane >> 4;

    f32x4 acc[MI][4];
#pragma unroll
    for (int i = 0; i < MI; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    const int64_t all_stages = (K + kBK - 1) / kBK;
    const int64_t s0 = sp * per_split;
    const int64_t s1 = s0 + per_split < all_stages ? s0 + per_split : all_stages;
    F32Tile<BM> xt;
    WTile<WT> wt;
    xt.Load(x, T, K, m0, s0 * kBK);
    wt.Load(w, O, K, row_bytes, n0, s0 * kBK);
    xt.Store(sm.x[0]);
    wt.Store(sm.w[0]);
    __syncthreads();
    for (int64_t s = s0; s < s1; ++s) {
        const int buf = static_cast<int>((s - s0) & 1);
        // next stage's loads (the last stage reloads itself: no branch around
        // the loads, and the write below goes to a buffer no one reads again)
        const int64_t k_next = (s + 1 < s1 ? s + 1 : s) * kBK;
        xt.Load(x, T, K, m0, k_next);
        wt.Load(w, O, K, row_bytes, n0, k_next);
        const float* xs = sm.x[buf] + (wm * (BM / 2) + i16) * kLd + 4 * kq;
        const float* ws = sm.w[buf] + (wn * 64 + i16) * kLd + 4 * kq;
#pragma unroll
        for (int kk = 0; kk < kBK; kk += 16) {
            f32x4 a[MI], b[4];
#pragma unroll
            for (int i = 0; i < MI; ++i) a[i] = *reinterpret_cast<const f32x4*>(xs + 16 * i * kLd + kk);
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = *reinterpret_cast<const f32x4*>(ws + 16 * j * kLd + kk);
#pragma unroll
            for (int st = 0; st < 4; ++st) {
#pragma unroll
                for (int i = 0; i < MI; ++i) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][st], b[j][st],
                                                                         acc[i][j], 0, 0, 0);
                    }
                }
            }
        }
        xt.Store(sm.x[buf ^ 1]);
        wt.Store(sm.w[buf ^ 1]);
        InterleaveStage<MI>();
        __syncthreads();
    }

    float* out = partial != nullptr ? partial + sp * T * O : y;
    const float* add = partial != nullptr ? nullptr : bias;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t col = n0 + wn * 64 + 16 * j + i16;
        if (col >= O) continue;
        const float b = add != nullptr ? add[col] : 0.0f;
#pragma unroll
        for (int i = 0; i < MI; ++i) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t row = m0 + wm * (BM / 2) + 16 * i + 4 * kq + r;
                if (row < T) out[row * O + col] = acc[i][j][r] + b;
            }
        }
    }
}

// ------------------------------------------------ tiles on bf16 piece products
// The tiled GEMM for Q8_0 / Q4_0 weights (block or planar layout) with every
// product exact, as in GemmPlanar below: a code is a small integer, exact in
// bf16, and x is the exact sum of three bf16 pieces, so for each block
//   S = sum_i code_i x_i  (3 v_mfma_f32_16x16x32_bf16, fp32 sums only),
//   acc += d * S.
// Same tiling and split-K protocol as GemmMfma (128 token rows x 128
// outputs, one 32-input block per stage, wave w: rows (w / 2) * 64, outputs
// (w % 2) * 64, 4 x 4 MFMA tiles), 8x less matrix-core time per stage.  The
// thread that loads an x float4 splits it into pieces once per stage; x
// planes are [piece][128 rows][32 bf16] with the 16-byte group g of row r
// at g ^ ((r / 2) % 4), and W codes [128 rows][32 bf16 + 8] (80-byte rows),
// so the operand reads of 8 lanes meet 8 distinct bank quads.  Two stage
// buffers, 69 KB: two workgroups per compute unit.  NW = 8 waves take 256
// outputs per tile (90 KB, one workgroup per unit): each x split then
// serves twice the outputs, which halves the split work per product, the
// stage's largest VALU cost.
typedef __bf16 bf16x8g __attribute__((ext_vector_type(8)));
constexpr int kPcWRow = 20;  // W code row, dwords

template <int BNT>
struct __align__(16) PiecesSmem {
    uint32_t x[2][3 * 128 * 16];
    uint32_t w[2][BNT * kPcWRow];
    float d[2][BNT];
};

// The pieces of 4 floats, two per dword: o[0] high, o[1] middle, o[2] low.
// Finite values: mask and subtract; a wave with any inf or NaN takes
// SplitBf's form (the value whole in the high piece), so products with them
// are what fp32 products would be.  The low pieces of finite values are
// finite and below 2^-14 of them, so their sum is NaN exactly when some
// value is inf or NaN (inf - inf, NaN propagating): one test for four.
__device__ inline void PiecesOf4(float4 v, uint2 (&o)[3]) {
    const float x[4] = {v.x, v.y, v.z, v.w};
    uint32_t h[4], m[4], l[4];
    float lf[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t u = __float_as_uint(x[i]);
        const float r = x[i] - __uint_as_float(u & 0xFFFF0000u);
        h[i] = u;
        m[i] = __float_as_uint(r);
        lf[i] = r - __uint_as_float(m[i] & 0xFFFF0000u);
        l[i] = __float_as_uint(lf[i]);
    }
    const float chk = (lf[0] + lf[1]) + (lf[2] + lf[3]);
    if (__builtin_amdgcn_ballot_w64(chk != chk) != 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float p[3];
            SplitBf(x[i], p);
            h[i] = __float_as_uint(p[0]);
            m[i] = __float_as_uint(p[1]);
            l[i] = __float_as_uint(p[2]);
        }
    }
    o[0] = make_uint2(__builtin_amdgcn_perm(h[1], h[0], 0x07060302u),
                      __builtin_amdgcn_perm(h[3], h[2], 0x07060302u));
    o[1] = make_uint2(__builtin_amdgcn_perm(m[1], m[0], 0x07060302u),
                      __builtin_amdgcn_perm(m[3], m[2], 0x07060302u));
    o[2] = make_uint2(__builtin_amdgcn_perm(l[1], l[0], 0x07060302u),
                      __builtin_amdgcn_perm(l[3], l[2], 0x07060302u));
}

// The 16 signed codes a weight tile thread holds (inputs 16h .. 16h + 15 of
// its row's block), as the tiles' Store decodes them; block-layout Q4_0
// codes come as 16 x (nibble - 8) (CodeScale<WT>() undoes the 16 in the
// scale, exactly): each dword's nibbles of half h, XOR 8, moved to the high
// half of their bytes are those values as signed bytes, with no per-code
// select on h.
template <int WT>
__device__ constexpr float CodeScale() { return WT == MLK_Q4_0 ? 0.0625f : 1.0f; }

template <int WT>
__device__ inline void TileCodes(const WTile<WT>& t, int32_t (&c)[16]) {
    const int h = threadIdx.x & 1;
    uint32_t sb[4];
    if constexpr (WT == MLK_Q4_0) {
#pragma unroll
        for (int j = 0; j < 4; ++j) sb[j] = (((t.q[j] >> (4 * h)) & 0x0F0F0F0Fu) ^ 0x08080808u) << 4;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        if constexpr (WT == MLK_Q8_0 || WT == kWPlanarQ8) {
            c[i] = static_cast<int32_t>(t.q[i / 4] << (24 - 8 * (i % 4))) >> 24;
        } else if constexpr (WT == MLK_Q4_0) {
            c[i] = static_cast<int32_t>(sb[i / 4] << (24 - 8 * (i % 4))) >> 24;
        } else {  // planar Q4_0: input 8g + e is nibble e (low half of byte e, then high)
            const int e8 = i % 8;
            const int sh = e8 < 4 ? 8 * e8 : 8 * (e8 - 4) + 4;
            c[i] = static_cast<int32_t>(t.q[i / 8] << (28 - sh)) >> 28;
        }
    }
}

// Epilogues of GemmPieces (one K pass, no partial sums for the last two):
//   kPcStore   y = sum + bias, or the split's partial sums;
//   kPcAdd     y = y + (sum + bias), the residual add of the layer;
//   kPcSwiGlu  gate and up in one tile (NW = 8): W rows n0 .. n0 + 127 of
//              w (gate, waves with wn 0, 1) and of w2 (up, wn 2, 3); the gate
//              waves hand their sums + bias through LDS to the up waves that
//              hold the same outputs, which store SwiGlu(gate, up + bias2).
//   kPcPair    two matrices of O rows each in one launch (the layer's k and
//              v): the first half of the tiles along the outputs takes w,
//              bias and y, the second w2, bias2 and y2; stored as kPcStore.
// Each output's sum is the same as kPcStore's, so every epilogue gives the
// separate kernels' values (mlk_add_f32, mlk_swiglu_f32) bit for bit.
enum PiecesEpi { kPcStore = 0, kPcAdd = 1, kPcSwiGlu = 2, kPcPair = 3 };

typedef uint32_t u32x4p __attribute__((ext_vector_type(4)));

// kXP: x comes already split, as the planes StorePlanes writes ([K / 32
// blocks][3 pieces][T rows][16 dwords], the pieces PiecesOf4 makes, bit for
// bit, for every value): each stage copies 3 x 128 rows x 4 groups of 8
// inputs (16 B) into the swizzled LDS layout, with no split in the loop
// (the split was 7-8.5% of the linears' time at Llama-3-8B's T = 4096).
template <int WT, int NW, int EPI = kPcStore, bool kXP = false>
__global__ __launch_bounds__(64 * NW) void GemmPieces(const float* __restrict__ x,
                                                           const uint8_t* __restrict__ w,
                                                           const float* __restrict__ bias,
                                                           float* __restrict__ y, int64_t T,
                                                           int64_t K, int64_t O,
                                                           int64_t row_bytes, int tiles_m,
                                                           int tiles, int64_t per_split,
                                                           float* __restrict__ partial,
                                                           const uint8_t* __restrict__ w2,
                                                           const float* __restrict__ bias2,
                                                           float* __restrict__ y2,
                                                           const uint32_t* __restrict__ xp) {
    constexpr int BM = 128;
    constexpr int kThreads = 64 * NW;
    constexpr int BNT = 32 * NW;               // W rows per tile
    constexpr int kXN = BM * kBK / 4 / kThreads;  // x float4s per thread and stage
    constexpr int kXPN = 3 * BM * 4 / kThreads;   // kXP: 16-byte plane groups per thread and stage
    constexpr bool kDual = EPI == kPcSwiGlu;
    static_assert(!kDual || NW == 8, "gate / up tiles take 8 waves");
    __shared__ PiecesSmem<BNT> sm;
    const int tile = static_cast<int>(blockIdx.x) % tiles;
    const int sp = static_cast<int>(blockIdx.x) / tiles;
    const int tm = tile % tiles_m;
    const int tn = tile / tiles_m;
    const int64_t m0 = static_cast<int64_t>(tm) * BM;
    // kPcPair: the tile's matrix (the same for the whole workgroup)
    const int half_n = tiles / tiles_m / 2;
    const bool wg_second = EPI == kPcPair && tn >= half_n;
    const int64_t n0 = static_cast<int64_t>(wg_second ? tn - half_n : tn) * (kDual ? BNT / 2 : BNT);
    // the W rows this thread loads: gate rows n0 .. for the tile's first
    // half, up rows n0 .. (from w2) for the second when kDual
    const bool t_second = kDual && static_cast<int>(threadIdx.x >> 1) >= BNT / 2;
    const uint8_t* const wsrc = t_second || wg_second ? w2 : w;
    const int64_t n0w = t_second ? n0 - BNT / 2 : n0;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int wm = wave & 1, wn = wave >> 1;  // 64 token rows x 64 outputs per wave
    const int i16 = lane & 15, kq = lane >> 4;

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    const int64_t all_stages = (K + kBK - 1) / kBK;
    const int64_t s0 = sp * per_split;
    const int64_t s1 = s0 + per_split < all_stages ? s0 + per_split : all_stages;
    // x: thread tid holds float4 tid + kThreads i of the [128][32] stage, 8
    // per row.  Rows past T read row 0 and W rows past O their tile's row 0,
    // unmasked: the outputs they meet are never stored (K is a multiple of
    // 256, so no stage reads past K).
    // Stages are requested two ahead: registers A / B alternate, so the
    // stage stored at the end of stage s was requested at the start of
    // stage s - 1 and is in registers by then (requested one ahead, the
    // scheduler moved its split next to its request and every stage waited
    // out the load latency).
    using XRegs = typename std::conditional<kXP, u32x4p[kXPN], float4[kXN]>::type;
    auto load_x = [&](int64_t k0, XRegs& xv) {
        if constexpr (kXP) {
            // group idx: piece idx / 512, row (idx / 4) % 128, inputs 8 (idx % 4) ..
            const uint32_t* blk = xp + (k0 / kBK) * 3 * T * 16;
#pragma unroll
            for (int i = 0; i < kXPN; ++i) {
                const int idx = static_cast<int>(threadIdx.x) + kThreads * i;
                const int64_t r = m0 + ((idx >> 2) & (BM - 1));
                xv[i] = *reinterpret_cast<const u32x4p*>(
                    blk + ((idx >> 9) * T + (r < T ? r : 0)) * 16 + 4 * (idx & 3));
            }
        } else {
#pragma unroll
            for (int i = 0; i < kXN; ++i) {
                const int idx = static_cast<int>(threadIdx.x) + kThreads * i;
                const int64_t r = m0 + (idx >> 3);
                const int64_t c = k0 + 4 * (idx & 7);
                xv[i] = *reinterpret_cast<const float4*>(x + (r < T ? r * K + c : c));
            }
        }
    };
    // one stage into LDS buffer b: x pieces, W codes as bf16, scales
    auto store = [&](int b, const XRegs& xv, const WTile<WT>& wt) {
        if constexpr (kXP) {
#pragma unroll
            for (int i = 0; i < kXPN; ++i) {
                const int idx = static_cast<int>(threadIdx.x) + kThreads * i;
                const int r = (idx >> 2) & (BM - 1);
                const int at = (idx >> 9) * 128 * 16 + r * 16 + (((idx & 3) ^ ((r >> 1) & 3)) << 2);
                *reinterpret_cast<u32x4p*>(&sm.x[b][at]) = xv[i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < kXN; ++i) {
                const int idx = static_cast<int>(threadIdx.x) + kThreads * i;
                const int r = idx >> 3, c8 = idx & 7;
                uint2 pc[3];
                PiecesOf4(xv[i], pc);
                const int at = r * 16 + (((c8 >> 1) ^ ((r >> 1) & 3)) << 2) + 2 * (c8 & 1);
#pragma unroll
                for (int p = 0; p < 3; ++p) {
                    *reinterpret_cast<uint2*>(&sm.x[b][p * 128 * 16 + at]) = pc[p];
                }
            }
        }
        int32_t c[16];
        TileCodes<WT>(wt, c);
        uint32_t pk[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) pk[i] = PackBf(static_cast<float>(c[2 * i]), static_cast<float>(c[2 * i + 1]));
        const int row = threadIdx.x >> 1, h = threadIdx.x & 1;
        uint4* dst = reinterpret_cast<uint4*>(&sm.w[b][row * kPcWRow + 8 * h]);
        dst[0] = make_uint4(pk[0], pk[1], pk[2], pk[3]);
        dst[1] = make_uint4(pk[4], pk[5], pk[6], pk[7]);
        if (h == 0) sm.d[b][row] = HalfHw(wt.d & 0xFFFFu) * CodeScale<WT>();
    };
    // stage s in LDS buffer (s - s0) & 1, stage s + 1 in registers `held`;
    // stage s + 2 requested into `next` (past the last stage: the last again,
    // never stored where it is read)
    auto step = [&](int64_t s, const XRegs& held_x, const WTile<WT>& held_w, XRegs& next_x,
                    WTile<WT>& next_w) {
        const int buf = static_cast<int>((s - s0) & 1);
        const int64_t k2 = (s + 2 < s1 ? s + 2 : s1 - 1) * kBK;
        load_x(k2, next_x);
        next_w.Load(wsrc, O, K, row_bytes, n0w, k2);
        __builtin_amdgcn_sched_barrier(0);
        bf16x8g b[4];
        float dj[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int row = wn * 64 + 16 * j + i16;
            b[j] = *reinterpret_cast<const bf16x8g*>(&sm.w[buf][row * kPcWRow + 4 * kq]);
            dj[j] = sm.d[buf][row];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = wm * 64 + 16 * i + i16;
            const int at = r * 16 + ((kq ^ ((r >> 1) & 3)) << 2);
            bf16x8g a[3];
#pragma unroll
            for (int p = 0; p < 3; ++p) a[p] = *reinterpret_cast<const bf16x8g*>(&sm.x[buf][p * 128 * 16 + at]);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                f32x4 S = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[2], b[j], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                S = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[1], b[j], S, 0, 0, 0);
                S = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0], b[j], S, 0, 0, 0);
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4) acc[i][j][r4] += dj[j] * S[r4];
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        store(buf ^ 1, held_x, held_w);
        __syncthreads();
    };
    XRegs xa, xb;
    WTile<WT> wa, wb;
    load_x(s0 * kBK, xa);
    wa.Load(wsrc, O, K, row_bytes, n0w, s0 * kBK);
    {
        const int64_t k1 = (s0 + 1 < s1 ? s0 + 1 : s0) * kBK;
        load_x(k1, xb);
        wb.Load(wsrc, O, K, row_bytes, n0w, k1);
    }
    store(0, xa, wa);
    __syncthreads();
    for (int64_t s = s0; s < s1; s += 2) {
        step(s, xb, wb, xa, wa);
        if (s + 1 < s1) step(s + 1, xa, wa, xb, wb);
    }

    if constexpr (kDual) {
        // The stage buffers are free (the last stage's reads are behind the
        // loop's last barrier).  Gate wave (wm, wn) and up wave (wm, wn + 2)
        // hold the same outputs in the same registers, so lane l of one
        // hands lane l of the other its 64 sums, 16 float4s at a stride of
        // 64 lanes (1 KB per instruction, no bank conflicts).
        static_assert(sizeof(PiecesSmem<BNT>) >= 4 * 16 * 64 * sizeof(float4),
                      "the gate sums fit the stage buffers");
        float4* const xch = reinterpret_cast<float4*>(&sm) + (wm * 2 + (wn & 1)) * 16 * 64 + lane;
        if (wn < 2) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int64_t col = n0 + wn * 64 + 16 * j + i16;
                const float bg = bias != nullptr && col < O ? bias[col] : 0.0f;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    xch[(4 * i + j) * 64] = make_float4(acc[i][j][0] + bg, acc[i][j][1] + bg,
                                                        acc[i][j][2] + bg, acc[i][j][3] + bg);
                }
            }
        }
        __syncthreads();
        if (wn >= 2) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int64_t col = n0 + (wn - 2) * 64 + 16 * j + i16;
                if (col >= O) continue;
                const float bu = bias2 != nullptr ? bias2[col] : 0.0f;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float4 g4 = xch[(4 * i + j) * 64];
                    const float g[4] = {g4.x, g4.y, g4.z, g4.w};
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int64_t row = m0 + wm * 64 + 16 * i + 4 * kq + r;
                        if (row < T) y[row * O + col] = SwiGluF(g[r], acc[i][j][r] + bu);
                    }
                }
            }
        }
        return;
    }
    float* out = partial != nullptr ? partial + sp * T * O : (wg_second ? y2 : y);
    const float* add = partial != nullptr ? nullptr : (wg_second ? bias2 : bias);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t col = n0 + wn * 64 + 16 * j + i16;
        if (col >= O) continue;
        const float bb = add != nullptr ? add[col] : 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t row = m0 + wm * 64 + 16 * i + 4 * kq + r;
                if (row >= T) continue;
                if constexpr (EPI == kPcAdd) {
                    out[row * O + col] = out[row * O + col] + (acc[i][j][r] + bb);
                } else {
                    out[row * O + col] = acc[i][j][r] + bb;
                }
            }
        }
    }
}

// For each n: p[n][0] + p[n][stride] + ... + p[n][(splits - 1) * stride],
// added in that order (splits >= 1).  The loads of all N sums go out 8
// splits at a time, a group's indices past the last split reading the last
// one (not added): a rolled remainder loop would wait for each load.
template <int N>
__device__ inline void SumSplitsN(const float* const (&p)[N], int splits, int64_t stride,
                                  float (&v)[N]) {
#pragma unroll
    for (int n = 0; n < N; ++n) v[n] = 0.0f;
    for (int sp = 0; sp < splits; sp += 8) {
        float t[N][8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int64_t at = static_cast<int64_t>(sp + j < splits ? sp + j : splits - 1) * stride;
#pragma unroll
            for (int n = 0; n < N; ++n) t[n][j] = p[n][at];
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (sp + j < splits) {
#pragma unroll
                for (int n = 0; n < N; ++n) v[n] = sp + j == 0 ? t[n][j] : v[n] + t[n][j];
            }
        }
    }
}

__device__ inline float SumSplits(const float* p, int splits, int64_t stride) {
    const float* q[1] = {p};
    float v[1];
    SumSplitsN<1>(q, splits, stride, v);
    return v[0];
}

// y = sum of the splits' partial sums, in split order, + bias.
__global__ __launch_bounds__(kGemmThreads) void SplitKReduce(const float* __restrict__ partial,
                                                             int splits,
                                                             const float* __restrict__ bias,
                                                             float* __restrict__ y, int64_t T,
                                                             int64_t O) {
    const int64_t n = T * O;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const float v = SumSplits(partial + i, splits, n);
        y[i] = bias != nullptr ? v + bias[i % O] : v;
    }
}

// K splits for a T x O x K product: doubled while the grid holds fewer than
// two workgroups per CU and every split keeps at least 8 stages (K >= 256).
struct SplitPlan {
    int splits = 1;
    int64_t per_split = 0;
};

// Token rows per tile: the smallest of 32, 64, 128 that covers T, 128 beyond.
int TileRows(int64_t T) { return T <= 32 ? 32 : (T <= 64 ? 64 : 128); }

SplitPlan PlanSplits(int64_t T, int64_t K, int64_t O) {
    const int bm = TileRows(T);
    const int64_t tiles = ((T + bm - 1) / bm) * ((O + kBN - 1) / kBN);
    const int64_t stages = (K + kBK - 1) / kBK;
    const int64_t target = 2 * static_cast<int64_t>(ComputeUnits());
    int64_t sp = 1;
    while (tiles * sp < target && stages / (2 * sp) >= 8 && sp < 32) sp *= 2;
    SplitPlan p;
    p.per_split = (stages + sp - 1) / sp;
    p.splits = static_cast<int>((stages + p.per_split - 1) / p.per_split);
    return p;
}

// ------------------------------------------------------------- skinny
// Few token rows: the weights dominate, so each wave streams its 16
// output rows of W straight from HBM into MFMA B-operand registers (no LDS
// round trip for W), the whole chunk's loads in flight at once, and only x,
// small and shared by the workgroup, goes through LDS.  Which inputs a
// lane's k-slot takes per stage is set by WChunk (below); x is read from LDS
// in the same order.  Workgroup = 4 waves = 64 output rows x all T rows x
// one K chunk; the chunks' partial sums are added by SplitKReduce in chunk
// order.

constexpr int kSkThreads = 256;
constexpr int kSkRows = 64;  // output rows per workgroup (16 per wave)

// A lane's weights of one K chunk, and the chunk offset of the inputs its
// k-slot takes in stage u (8 consecutive inputs per stage; A and B use the
// same assignment, so each product x[t, k] * w[o, k] is formed once).
//   F32    4 stages of 32 inputs: the lane's k-slot q reads 8q .. 8q + 7 of
//          each 32 (two 16-byte non-temporal loads per stage).
//   Q8_0 / Q4_0 / Q4_1   8 stages: the lane owns a piece, the two blocks 2q
//          and 2q + 1 of the 8-block chunk (68 / 36 / 40 bytes, 4-byte
//          aligned, read as 16-byte loads), and stage u takes its inputs
//          8u .. 8u + 7; byte and nibble positions are compile-time constants.
typedef uint32_t u32x4a __attribute__((ext_vector_type(4), aligned(4)));

template <int WT>
struct WChunk;

template <>
struct WChunk<kWF32> {
    static constexpr int kStages = 4;
    static constexpr bool kPieces = false;
    f32x4 a[kStages], b[kStages];
    __device__ void Load(const uint8_t* w, int64_t row, int64_t row_bytes, int64_t k0, int q) {
#pragma unroll
        for (int u = 0; u < kStages; ++u) {
            const f32x4* p =
                reinterpret_cast<const f32x4*>(w + row * row_bytes) + (k0 + 32 * u + 8 * q) / 4;
            a[u] = __builtin_nontemporal_load(p);
            b[u] = __builtin_nontemporal_load(p + 1);
        }
    }
    __device__ float Get(int u, int j) const { return j < 4 ? a[u][j & 3] : b[u][j & 3]; }
    __device__ static int XOff(int u, int q) { return 32 * u + 8 * q; }
};

template <int QT>
struct PieceChunk {
    static constexpr int kStages = 8;
    static constexpr bool kPieces = true;
    static constexpr int kBlock = QT == MLK_Q8_0 ? 34 : (QT == MLK_Q4_0 ? 18 : 20);
    static constexpr int kWords = 2 * kBlock / 4;
    uint32_t wd[kWords];
    __device__ void Load(const uint8_t* w, int64_t row, int64_t row_bytes, int64_t k0, int q) {
        const uint32_t* p = reinterpret_cast<const uint32_t*>(w + row * row_bytes +
                                                              (k0 / 32 + 2 * q) * kBlock);
#pragma unroll
        for (int i = 0; i + 4 <= kWords; i += 4) {
            const u32x4a v = *reinterpret_cast<const u32x4a*>(p + i);
            wd[i] = v.x;
            wd[i + 1] = v.y;
            wd[i + 2] = v.z;
            wd[i + 3] = v.w;
        }
#pragma unroll
        for (int i = kWords / 4 * 4; i < kWords; ++i) wd[i] = p[i];
    }
    __device__ uint32_t Byte(int b) const { return (wd[b / 4] >> (8 * (b % 4))) & 0xFFu; }
    __device__ float Get(int u, int j) const {
        const int e = 8 * u + j;  // input within the piece
        const int blk = e / 32, i = e % 32;
        if constexpr (QT == MLK_Q8_0) {
            const uint32_t d = blk == 0 ? wd[0] & 0xFFFFu : wd[8] >> 16;
            const int b = 34 * blk + 2 + i;
            const int32_t code = static_cast<int32_t>(wd[b / 4] << (24 - 8 * (b % 4))) >> 24;
            return HalfHw(d) * static_cast<float>(code);
        } else if constexpr (QT == MLK_Q4_0) {
            const uint32_t d = blk == 0 ? wd[0] & 0xFFFFu : wd[4] >> 16;
            const uint32_t byte = Byte(18 * blk + 2 + i % 16);
            const int code = static_cast<int>(i < 16 ? byte & 15u : byte >> 4);
            return HalfHw(d) * static_cast<float>(code - 8);
        } else {
            const uint32_t dm = wd[5 * blk];
            const uint32_t byte = Byte(20 * blk + 4 + i % 16);
            const float code = static_cast<float>(i < 16 ? byte & 15u : byte >> 4);
            return __fadd_rn(__fmul_rn(HalfHw(dm & 0xFFFFu), code), HalfHw(dm >> 16));
        }
    }
    // inputs 64q + 8u .. of the chunk, in the padded LDS layout (4 floats
    // after every 64, so the 4 k-slots' reads start on different banks)
    __device__ static int XOff(int u, int q) { return 68 * q + 8 * u; }
};

template <>
struct WChunk<MLK_Q8_0> : PieceChunk<MLK_Q8_0> {};
template <>
struct WChunk<MLK_Q4_0> : PieceChunk<MLK_Q4_0> {};
template <>
struct WChunk<MLK_Q4_1> : PieceChunk<MLK_Q4_1> {};

// The x rows of one K chunk, [16 TT][chunk] in LDS (rows RS floats apart;
// with kPad, input k of a row at k + 4 (k / 64)), staged through registers.
template <int TT, int CHUNK, bool kPad>
struct XChunk {
    static constexpr int kRows = 16 * TT;
    static constexpr int RS = (kPad ? CHUNK + CHUNK / 16 : CHUNK) + 4;
    static constexpr int kN = kRows * CHUNK / 4 / kSkThreads;  // 4-float vectors per thread
    f32x4 v[kN];
    __device__ void Load(const float* x, int64_t T, int64_t K, int64_t k0) {
#pragma unroll
        for (int i = 0; i < kN; ++i) {
            const int idx = static_cast<int>(threadIdx.x) + kSkThreads * i;
            const int64_t t = idx / (CHUNK / 4);
            const int64_t r = t < T ? t : T - 1;
            v[i] = *reinterpret_cast<const f32x4*>(x + r * K + k0 + 4 * (idx % (CHUNK / 4)));
        }
    }
    __device__ void Store(float* s) const {
#pragma unroll
        for (int i = 0; i < kN; ++i) {
            const int idx = static_cast<int>(threadIdx.x) + kSkThreads * i;
            const int k = 4 * (idx % (CHUNK / 4));
            *reinterpret_cast<f32x4*>(s + (idx / (CHUNK / 4)) * RS + (kPad ? k + 4 * (k / 64) : k)) =
                v[i];
        }
    }
};

// Up to three weight matrices with the same K in one launch: their row
// groups are numbered one segment after another, and their partial sums
// fill adjacent columns of the partial rows (segment s from column col0[s]).
// One segment without a partial buffer writes y (+ bias) directly.
struct SkinnyArgs {
    const uint8_t* w[3];
    int64_t rows[3];
    int64_t col0[3];
    int g0[3];       // first row group of each segment
    int n_seg;
    int row_groups;  // all segments
    int64_t cols;    // columns of a partial row: the segments' rows together
    const float* bias;
    float* y;
};

// Workgroup (row group, chunk): 64 output rows over one K chunk of 32 D.
// Every weight load and the chunk's x rows are issued before anything is
// computed (one round of memory latency per workgroup); the chunk's sums go
// to partial[chunk] for the reduction, or straight to y (+ bias) when K is
// one chunk.
// NP > 1 (quantized weights): the workgroup takes NP
// consecutive chunks, all of their loads in flight at once, so the partial
// sums (written and read once each by the reduction) shrink NP times.
template <int WT, int TT, int NP>
__global__ __launch_bounds__(kSkThreads) void GemmSkinny(const float* __restrict__ x,
                                                         SkinnyArgs a, int64_t T, int64_t K,
                                                         int64_t row_bytes,
                                                         float* __restrict__ partial) {
    using WC = WChunk<WT>;
    constexpr int D = WC::kStages;
    constexpr int kSub = 32 * D;  // inputs of one chunk
    constexpr int kChunk = kSub * NP;
    static_assert(NP == 1 || WC::kPieces, "several chunks per workgroup: quantized weights");
    // padded LDS offset of chunk p's inputs (4 floats after every 64)
    constexpr int kSubX = WC::kPieces ? kSub + kSub / 16 : kSub;
    using XC = XChunk<TT, kChunk, WC::kPieces>;
    __shared__ __align__(16) float xs[16 * TT * XC::RS];
    const int rgall = static_cast<int>(blockIdx.x) % a.row_groups;
    const int sp = static_cast<int>(blockIdx.x) / a.row_groups;
    const int seg = (a.n_seg > 2 && rgall >= a.g0[2]) ? 2 : ((a.n_seg > 1 && rgall >= a.g0[1]) ? 1 : 0);
    const int rg = rgall - (seg == 2 ? a.g0[2] : (seg == 1 ? a.g0[1] : 0));
    const int64_t O = seg == 2 ? a.rows[2] : (seg == 1 ? a.rows[1] : a.rows[0]);
    const uint8_t* w = seg == 2 ? a.w[2] : (seg == 1 ? a.w[1] : a.w[0]);
    const int64_t col0 = seg == 2 ? a.col0[2] : (seg == 1 ? a.col0[1] : 0);
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int i16 = lane & 15, q = lane >> 4;
    const int64_t row = static_cast<int64_t>(rg) * kSkRows + wave * 16 + i16;
    const int64_t wrow = row < O ? row : O - 1;
    const int64_t k0 = static_cast<int64_t>(sp) * kChunk;

    WC wc[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) wc[p].Load(w, wrow, row_bytes, k0 + p * kSub, q);
    XC xc;
    xc.Load(x, T, K, k0);
    xc.Store(xs);
    __syncthreads();
    f32x4 acc[TT];
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) acc[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int pu = 0; pu < NP * D; ++pu) {
        const int p = pu / D, u = pu % D;
        float xa[TT][8];
#pragma unroll
        for (int tt = 0; tt < TT; ++tt) {
            const float* src = xs + (tt * 16 + i16) * XC::RS + p * kSubX + WC::XOff(u, q);
            const f32x4 lo = *reinterpret_cast<const f32x4*>(src);
            const f32x4 hi = *reinterpret_cast<const f32x4*>(src + 4);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                xa[tt][e] = lo[e];
                xa[tt][4 + e] = hi[e];
            }
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float wv = wc[p].Get(u, j);
#pragma unroll
            for (int tt = 0; tt < TT; ++tt) {
                acc[tt] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[tt][j], wv, acc[tt], 0, 0, 0);
            }
        }
    }
    if (row >= O) return;
    if (partial != nullptr) {
        float* out = partial + sp * T * a.cols + col0 + row;
#pragma unroll
        for (int tt = 0; tt < TT; ++tt) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t t = tt * 16 + 4 * q + r;
                if (t < T) out[t * a.cols] = acc[tt][r];
            }
        }
        return;
    }
    const float b = a.bias != nullptr ? a.bias[row] : 0.0f;
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t t = tt * 16 + 4 * q + r;
            if (t < T) a.y[t * O + row] = acc[tt][r] + b;
        }
    }
}

// ------------------------------------------------------- planar weights, bf16 products
// Q8_0 and Q4_0 weights on the bf16 matrix cores, with every product exact.
// A code (q, or a Q4_0 code minus 8) is a small integer, exact in bf16, and
// an fp32 x is the exact sum of three bf16 pieces: xh = x with its low 16
// bits cleared, xm = the same of x - xh, xl = x - xh - xm (at most 8
// significant bits left).  So each q * piece is exact in fp32, three
// v_mfma_f32_16x16x32_bf16 (one per piece) give one block's
// S = sum_i q_i x_i with fp32 summation only, and the block scale follows:
// acc += d * S.  That is the reference's sum_k x_k * (d q_k) (d q is exact
// in fp32) up to fp32 summation error, the bound every kernel here meets.
// A bf16 instruction does 8x the work of an fp32 one in half the cycles,
// so the matrix cores stop being the limit of the few-token projections.
//
// The weights come in the planar layout (mlk_quant_to_planar, below), in
// which a wave's 16-byte loads of one row tile are 1 KB contiguous and each
// lane's bytes are its MFMA operand: lane l = 16 g + r of row tile rt takes
// row 16 rt + r and inputs 8g .. 8g + 7 of every block (A and B share the
// assignment, so each product is formed once).  SplitXBf writes x once as
// three bf16 planes per block, [piece][token][32 inputs].
// GemmPlanar: workgroup = 4 waves = 128 output rows (wave: two 16-row
// tiles; one, 64 rows, when that leaves too few workgroups) x T tokens
// (16 per tile) x one K range of 2 * NP blocks; the
// ranges' partial sums are added by the split-K reductions, as
// GemmSkinny's.  Every weight load of the range is issued first, the
// range's x planes (token rows < T) are copied to LDS, and after one
// barrier the waves run on their own.  Operands: x is A (lane l: token
// l % 16), the weights are B, so the C registers of lane l are tokens
// 4(l / 16) + r of the lane's own row, whose scale it holds.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// PT: 16-row weight tiles per wave (2, or 1 for the shapes whose two-tile
// workgroups would be fewer than two per compute unit); a workgroup covers
// 4 * 16 * PT output rows.

// Bytes 2j, 2j + 1 of v as signed integers in bf16, in one dword.
__device__ inline uint32_t BytesBf(uint32_t v, int j) {
    return PackBf(static_cast<float>(static_cast<int8_t>(v >> (16 * j))),
                  static_cast<float>(static_cast<int8_t>(v >> (16 * j + 8))));
}

// Block b of a lane's planar codes (cw: the range's 16-byte code loads of one
// row tile, sw: its scale loads) as the MFMA's bf16 weight operand, and the
// block's scale.
template <int QT, int NP>
__device__ inline bf16x8 PlanarBlockOperand(const u32x4 (&cw)[QT == MLK_Q8_0 ? NP : NP / 2],
                                            const u32x4 (&sw)[NP / 4], int b, float* d) {
    const uint32_t sv = sw[b / 8][(b % 8) / 2];
    const uint32_t h16 = (b & 1) ? sv >> 16 : sv & 0xFFFFu;
    u32x4 q;
    if constexpr (QT == MLK_Q8_0) {
        const uint32_t lo = (b & 1) ? cw[b / 2][2] : cw[b / 2][0];
        const uint32_t hi = (b & 1) ? cw[b / 2][3] : cw[b / 2][1];
        q = u32x4{BytesBf(lo, 0), BytesBf(lo, 1), BytesBf(hi, 0), BytesBf(hi, 1)};
        *d = HalfHw(h16);
    } else {
        // nibbles (code - 8, two's complement) moved to the high half of each
        // byte: signed bytes of 16 (code - 8), scale d / 16
        const uint32_t v = cw[b / 4][b % 4];
        const uint32_t lo = (v << 4) & 0xF0F0F0F0u, hi = v & 0xF0F0F0F0u;
        q = u32x4{BytesBf(lo, 0), BytesBf(lo, 1), BytesBf(hi, 0), BytesBf(hi, 1)};
        *d = HalfHw(h16) * 0.0625f;
    }
    return __builtin_bit_cast(bf16x8, q);
}

// acc += d * (the block's three piece products): the exact products summed
// on the matrix cores, then one fp32 FMA with the block's scale.
template <int TT>
__device__ inline void PlanarBlockProducts(const bf16x8 (&xa)[TT][3], bf16x8 wb, float d,
                                           f32x4 (&acc)[TT]) {
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
        f32x4 s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[tt][0], wb, f32x4{0.f, 0.f, 0.f, 0.f},
                                                          0, 0, 0);
        s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[tt][1], wb, s, 0, 0, 0);
        s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[tt][2], wb, s, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[tt][r] = __builtin_fmaf(d, s[r], acc[tt][r]);
    }
}

// The x planes of tokens t < T: one thread per (block, token, input pair).
__global__ __launch_bounds__(kGemmThreads) void SplitXBf(const float* __restrict__ x, int64_t T,
                                                         int64_t K, uint32_t* __restrict__ planes) {
    const int64_t n = (K / 32) * T * 16;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int sp = static_cast<int>(i % 16);
        const int64_t t = (i / 16) % T;
        const int64_t b = i / (16 * T);
        const float* src = x + t * K + 32 * b + 2 * sp;
        StorePlanes(planes, T, t, 32 * b + 2 * sp, src[0], src[1]);
    }
}

// One K range's x planes in LDS: (block, piece, token slot) rows of 16
// dwords, kTok = 16 TT slots; slots t < T copied, the rest zero.  (Rows
// padded to 20 dwords measured no faster, with slightly more bank-conflict
// cycles.)
template <int TT, int NP>
struct PlanarX {
    static constexpr int kTok = 16 * TT;
    static constexpr int kRowWords = 16;
    static constexpr int kRows = 2 * NP * 3 * kTok;
    static constexpr int kWords = kRows * kRowWords;  // the LDS array
    static constexpr int kIter = kRows * 4 / kSkThreads;  // 16-byte copies per thread
    static_assert(kRows * 4 % kSkThreads == 0, "whole copy rounds");
    u32x4 v[kIter];
    __device__ void Load(const uint32_t* planes, int sp, int64_t T) {
        const u32x4* src = reinterpret_cast<const u32x4*>(planes) +
                           static_cast<int64_t>(sp) * 2 * NP * 3 * T * 4;
#pragma unroll
        for (int k = 0; k < kIter; ++k) {
            const int i = static_cast<int>(threadIdx.x) + kSkThreads * k;
            const int t = (i / 4) % kTok, bp = i / (4 * kTok);
            v[k] = u32x4{0u, 0u, 0u, 0u};
            if (t < T) v[k] = src[(bp * T + t) * 4 + i % 4];
        }
    }
    __device__ void Store(uint32_t* xs) const {
#pragma unroll
        for (int k = 0; k < kIter; ++k) {
            const int i = static_cast<int>(threadIdx.x) + kSkThreads * k;
            *reinterpret_cast<u32x4*>(xs + (i / 4) * kRowWords + 4 * (i % 4)) = v[k];
        }
    }
    // block b's three pieces as the A operands of the lane (token i16 of
    // each 16-token tile, inputs 8g .. 8g + 7)
    // (lo: the lane's offset in dwords, LaneOffset)
    __device__ static int LaneOffset(int i16, int g) { return i16 * kRowWords + 4 * g; }
    __device__ static void Read(const uint32_t* xs, int lo, int b, bf16x8 (&xa)[TT][3]) {
#pragma unroll
        for (int tt = 0; tt < TT; ++tt) {
#pragma unroll
            for (int p = 0; p < 3; ++p) {
                xa[tt][p] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(
                    xs + lo + ((b * 3 + p) * kTok + tt * 16) * kRowWords));
            }
        }
    }
};

template <int QT, int TT, int NP, int PT>
__global__ __launch_bounds__(kSkThreads) void GemmPlanar(const uint32_t* __restrict__ planes,
                                                         SkinnyArgs a, int64_t T, int64_t K,
                                                         float* __restrict__ partial) {
    constexpr int kCodeVecs = QT == MLK_Q8_0 ? NP : NP / 2;  // 16-byte code loads per tile
    __shared__ __align__(16) uint32_t xs[PlanarX<TT, NP>::kWords];
    const int rgall = static_cast<int>(blockIdx.x) % a.row_groups;
    const int sp = static_cast<int>(blockIdx.x) / a.row_groups;
    const int seg = (a.n_seg > 2 && rgall >= a.g0[2]) ? 2 : ((a.n_seg > 1 && rgall >= a.g0[1]) ? 1 : 0);
    const int rg = rgall - (seg == 2 ? a.g0[2] : (seg == 1 ? a.g0[1] : 0));
    const int64_t O = seg == 2 ? a.rows[2] : (seg == 1 ? a.rows[1] : a.rows[0]);
    const uint8_t* w = seg == 2 ? a.w[2] : (seg == 1 ? a.w[1] : a.w[0]);
    const int64_t col0 = seg == 2 ? a.col0[2] : (seg == 1 ? a.col0[1] : 0);
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int i16 = lane & 15, g = lane >> 4;
    const int64_t tiles = (O + 15) / 16;
    const int64_t tile0 = static_cast<int64_t>(rg) * (4 * PT) + wave * PT;
    const int64_t code_tile = QT == MLK_Q8_0 ? 16 * K : 8 * K;  // bytes per row tile
    const uint8_t* scales = w + tiles * code_tile;

    // every weight load of the range first (tiles past the last read it)
    u32x4 cw[PT][kCodeVecs];
    u32x4 sw[PT][NP / 4];
#pragma unroll
    for (int n = 0; n < PT; ++n) {
        const int64_t tile = tile0 + n < tiles ? tile0 + n : tiles - 1;
        const u32x4* c = reinterpret_cast<const u32x4*>(w + tile * code_tile) +
                         static_cast<int64_t>(sp) * kCodeVecs * 64 + lane;
#pragma unroll
        for (int v = 0; v < kCodeVecs; ++v) cw[n][v] = __builtin_nontemporal_load(c + 64 * v);
        const u32x4* sc = reinterpret_cast<const u32x4*>(scales + tile * (K / 32) * 32) +
                          static_cast<int64_t>(sp) * (NP / 4) * 16 + i16;
#pragma unroll
        for (int v = 0; v < NP / 4; ++v) sw[n][v] = sc[16 * v];
    }
    // the range's x planes into LDS (all loads before the stores)
    PlanarX<TT, NP> xv;
    xv.Load(planes, sp, T);
    xv.Store(xs);
    __syncthreads();

    f32x4 acc[PT][TT];
#pragma unroll
    for (int n = 0; n < PT; ++n) {
#pragma unroll
        for (int tt = 0; tt < TT; ++tt) acc[n][tt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int b = 0; b < 2 * NP; ++b) {
        bf16x8 xa[TT][3];
        PlanarX<TT, NP>::Read(xs, PlanarX<TT, NP>::LaneOffset(i16, g), b, xa);
#pragma unroll
        for (int n = 0; n < PT; ++n) {
            float d;
            const bf16x8 wb = PlanarBlockOperand<QT, NP>(cw[n], sw[n], b, &d);
            PlanarBlockProducts<TT>(xa, wb, d, acc[n]);
        }
    }
#pragma unroll
    for (int n = 0; n < PT; ++n) {
        const int64_t row = 16 * (tile0 + n) + i16;
        if (row >= O) continue;
        float* out = partial != nullptr ? partial + sp * T * a.cols + col0 + row : a.y + row;
        const int64_t stride = partial != nullptr ? a.cols : O;
        const float bias = partial == nullptr && a.bias != nullptr ? a.bias[row] : 0.0f;
#pragma unroll
        for (int tt = 0; tt < TT; ++tt) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t t = tt * 16 + 4 * g + r;
                if (t < T) out[t * stride] = acc[n][tt][r] + bias;
            }
        }
    }
}

// GemmPlanarStream: GemmPlanar's products, in its order, by workgroups that
// stay on one K range.  The range's x planes go to LDS once; then each wave
// streams steps (PT 16-row tiles of one segment) gw, gw + S, gw + 2S, ...
// (gw: the wave among the range's S = 4 wgs waves), computing one step
// while the codes and scales of the next D are in flight.  Weight loads
// are buffer loads against the segment's bytes; a tile past the segment's
// last, or a step past the launch's last, has an empty range and reads
// zeros without a memory access.  a.g0 / a.row_groups count steps here.
// Needs each segment's planar bytes below 2^31 and 16 TT x a partial row
// (or x O) below 2^30 bytes (the offsets are 32-bit); no bias (partial sums get theirs in
// the reduction; a direct output with a bias runs GemmPlanar).
// A segment's field (selects: the arguments are not indexed dynamically).
template <typename V>
__device__ inline V Seg3(int seg, V v0, V v1, V v2) {
    return seg == 2 ? v2 : (seg == 1 ? v1 : v0);
}

template <int QT, int NP, int PT>
struct PlanarStep {
    static constexpr int kCodeVecs = QT == MLK_Q8_0 ? NP : NP / 2;
    u32x4 cw[PT][kCodeVecs];
    u32x4 sw[PT][NP / 4];
};

template <int QT, int TT, int NP, int PT, int D>
__global__ __launch_bounds__(kSkThreads) void GemmPlanarStream(const uint32_t* __restrict__ planes,
                                                               SkinnyArgs a, int64_t T, int64_t K,
                                                               float* __restrict__ partial,
                                                               int wgs) {
    using Step = PlanarStep<QT, NP, PT>;
    constexpr int kCodeVecs = Step::kCodeVecs;
    __shared__ __align__(16) uint32_t xs[PlanarX<TT, NP>::kWords];
    const int sp = static_cast<int>(blockIdx.x) / wgs;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
    const int lane = threadIdx.x % kWave;
    const int i16 = lane & 15, g = lane >> 4;
    const int waves = 4 * wgs;
    const int first = (static_cast<int>(blockIdx.x) % wgs) * 4 + wave;
    const uint32_t code_tile = static_cast<uint32_t>(QT == MLK_Q8_0 ? 16 * K : 8 * K);
    const uint32_t code_lane = static_cast<uint32_t>(sp * kCodeVecs * 1024 + lane * 16);
    const uint32_t scale_lane = static_cast<uint32_t>(sp * (NP / 4) * 256 + i16 * 16);

    // the segment of step s, and its first tile
    auto locate = [&](int s, int* seg, int64_t* tile0) {
        *seg = (a.n_seg > 2 && s >= a.g0[2]) ? 2 : ((a.n_seg > 1 && s >= a.g0[1]) ? 1 : 0);
        *tile0 = static_cast<int64_t>(s - Seg3(*seg, 0, a.g0[1], a.g0[2])) * PT;
    };
    auto load = [&](int s, Step& st) {
        int seg;
        int64_t tile0;
        locate(s, &seg, &tile0);
        const int64_t tiles = (Seg3(seg, a.rows[0], a.rows[1], a.rows[2]) + 15) / 16;
        const uint32_t bytes = static_cast<uint32_t>(tiles * (code_tile + K));
#pragma unroll
        for (int n = 0; n < PT; ++n) {
            const bool live = s < a.row_groups && tile0 + n < tiles;
            const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<uint8_t*>(Seg3(seg, a.w[0], a.w[1], a.w[2])), 0, live ? bytes : 0u, 0x00020000);
            const uint32_t tile = static_cast<uint32_t>(live ? tile0 + n : 0);
            const uint32_t c = tile * code_tile + code_lane;
            const uint32_t sc = static_cast<uint32_t>(tiles) * code_tile +
                                tile * static_cast<uint32_t>(K) + scale_lane;
#pragma unroll
            for (int v = 0; v < kCodeVecs; ++v) {
                st.cw[n][v] = __builtin_bit_cast(
                    u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, c + 1024 * v, 0, 2));
            }
#pragma unroll
            for (int v = 0; v < NP / 4; ++v) {
                st.sw[n][v] = __builtin_bit_cast(
                    u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, sc + 256 * v, 0, 0));
            }
        }
    };

    // x loads first, then the first step's weights; the x planes stored to
    // LDS; then the other steps of the ring
    Step ring[D];
    {
        PlanarX<TT, NP> xv;
        xv.Load(planes, sp, T);
        load(first, ring[0]);
        xv.Store(xs);
    }
#pragma unroll
    for (int d = 1; d < D; ++d) load(first + d * waves, ring[d]);
    __syncthreads();

    // the output: this range's partial rows, or y; buffer stores, so rows
    // t >= T fall outside the range and are dropped (as are rows past a
    // segment's last, sent past it)
    const int64_t stride = partial != nullptr ? a.cols : a.rows[0];
    float* const out_base = partial != nullptr ? partial + sp * T * a.cols : a.y;
    const __amdgpu_buffer_rsrc_t out_r = __builtin_amdgcn_make_buffer_rsrc(
        out_base, 0, static_cast<uint32_t>(T * stride * 4), 0x00020000);

    // Every path through a step issues the slot's next loads, and the loop
    // exits only at its head: the memory counter then holds the same loads on
    // every path into the head, so each wait there is for one step's loads.
    for (int s0 = first; s0 < a.row_groups; s0 += D * waves) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const int s = s0 + d * waves;
            if (s < a.row_groups) {
                f32x4 acc[PT][TT];
#pragma unroll
                for (int n = 0; n < PT; ++n) {
#pragma unroll
                    for (int tt = 0; tt < TT; ++tt) acc[n][tt] = f32x4{0.f, 0.f, 0.f, 0.f};
                }
                // the x reads stay in the step (an opaque offset): hoisted
                // out of the loop, all blocks' pieces would take 192 registers
                int lo = PlanarX<TT, NP>::LaneOffset(i16, g);
                asm volatile("" : "+v"(lo));
#pragma unroll
                for (int b = 0; b < 2 * NP; ++b) {
                    bf16x8 xa[TT][3];
                    PlanarX<TT, NP>::Read(xs, lo, b, xa);
#pragma unroll
                    for (int n = 0; n < PT; ++n) {
                        float dd;
                        const bf16x8 wb =
                            PlanarBlockOperand<QT, NP>(ring[d].cw[n], ring[d].sw[n], b, &dd);
                        PlanarBlockProducts<TT>(xa, wb, dd, acc[n]);
                    }
                }
                int seg;
                int64_t tile0;
                locate(s, &seg, &tile0);
                const int64_t O = Seg3(seg, a.rows[0], a.rows[1], a.rows[2]);
                const int64_t col0 = Seg3(seg, a.col0[0], a.col0[1], a.col0[2]);
#pragma unroll
                for (int n = 0; n < PT; ++n) {
                    const int64_t row = 16 * (tile0 + n) + i16;
                    const uint32_t o0 = static_cast<uint32_t>((col0 + row) * 4);
#pragma unroll
                    for (int tt = 0; tt < TT; ++tt) {
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int64_t t = tt * 16 + 4 * g + r;
                            const uint32_t off =
                                row < O ? o0 + static_cast<uint32_t>(t * stride * 4) : 0x7FFFFFF0u;
                            // (__float_as_uint: this compiler's __builtin_bit_cast
                            // of a vector element reads element 0)
                            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc[n][tt][r]),
                                                                  out_r, off, 0, 0);
                        }
                    }
                }
            }
            // then the slot's next step (after the last use of the slot, so
            // the new values take the same registers: no copies at the loop's
            // back edge, which would wait for these loads)
            load(s + D * waves, ring[d]);
        }
    }
}

// Block layout -> planar layout (described at mlk_quant_to_planar): one
// thread per 16 code bytes of a lane (a block pair of Q8_0, a block quad of
// Q4_0), then one per row's 8 scales.  Rows past O get zero codes and scales.
template <int QT>
__global__ __launch_bounds__(kGemmThreads) void ToPlanar(const uint8_t* __restrict__ blocks,
                                                         int64_t O, int64_t K,
                                                         uint8_t* __restrict__ out) {
    constexpr int kBB = QT == MLK_Q8_0 ? 34 : 18;
    constexpr int kPer = QT == MLK_Q8_0 ? 2 : 4;  // blocks per 16-byte lane vector
    const int64_t tiles = (O + 15) / 16, nb = K / 32, row_bytes = nb * kBB;
    const int64_t code_vecs = tiles * (nb / kPer) * 64;
    const int64_t n = code_vecs + tiles * (nb / 8) * 16;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        if (i < code_vecs) {
            const int lane = static_cast<int>(i % 64), g = lane >> 4;
            const int64_t v = (i / 64) % (nb / kPer), tile = i / (64 * (nb / kPer));
            const int64_t row = 16 * tile + (lane & 15);
            uint8_t bytes[16];
#pragma unroll
            for (int j = 0; j < kPer; ++j) {
                const uint8_t* blk = blocks + row * row_bytes + (kPer * v + j) * kBB + 2;
#pragma unroll
                for (int e = 0; e < 16 / kPer; ++e) {
                    uint8_t b = 0;
                    if (row < O) {
                        if constexpr (QT == MLK_Q8_0) {
                            b = blk[8 * g + e];
                        } else {  // input 8g + e (low nibble) and 8g + e + 4 (high), as code ^ 8
                            const int c0 = 8 * g + e, c1 = c0 + 4;
                            const uint32_t n0 = c0 < 16 ? blk[c0] & 15u : blk[c0 - 16] >> 4;
                            const uint32_t n1 = c1 < 16 ? blk[c1] & 15u : blk[c1 - 16] >> 4;
                            b = static_cast<uint8_t>((n0 ^ 8u) | ((n1 ^ 8u) << 4));
                        }
                    }
                    bytes[(16 / kPer) * j + e] = b;
                }
            }
            u32x4 o;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                o[k] = bytes[4 * k] | (bytes[4 * k + 1] << 8) | (bytes[4 * k + 2] << 16) |
                       (static_cast<uint32_t>(bytes[4 * k + 3]) << 24);
            }
            reinterpret_cast<u32x4*>(out)[i] = o;
        } else {
            const int64_t j = i - code_vecs;
            const int r = static_cast<int>(j % 16);
            const int64_t grp = (j / 16) % (nb / 8), tile = j / (16 * (nb / 8));
            const int64_t row = 16 * tile + r;
            uint32_t h[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint8_t* blk = blocks + row * row_bytes + (8 * grp + e) * kBB;
                h[e] = row < O ? blk[0] | (static_cast<uint32_t>(blk[1]) << 8) : 0u;
            }
            u32x4 o;
#pragma unroll
            for (int k = 0; k < 4; ++k) o[k] = h[2 * k] | (h[2 * k + 1] << 16);
            const int64_t code_bytes = tiles * (QT == MLK_Q8_0 ? 16 : 8) * K;
            reinterpret_cast<u32x4*>(out + code_bytes)[j] = o;
        }
    }
}

// The reduction of a fused skinny launch: each output's partial sums added in
// chunk order (as SplitKReduce), then (+ bias) and the mode's epilogue:
// plain y_s = v; add y_s = res_s + v; SwiGLU y_1 = SwiGlu(gate, up) with
// gate and up the two segments' sums for the same row.
__global__ __launch_bounds__(kGemmThreads) void SplitKReduceFused(const float* __restrict__ partial,
                                                                  int splits, int64_t T,
                                                                  int64_t cols, StreamArgs a,
                                                                  int mode, int64_t out_cols) {
    const int64_t n = T * out_cols, stride = T * cols;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t t = i / out_cols, c = i % out_cols;
        const float* row = partial + t * cols;
        auto sum = [&](int64_t col) { return SumSplits(row + col, splits, stride); };
        auto sum2 = [&](int64_t c0, int64_t c1, float* a0, float* a1) {
            const float* q[2] = {row + c0, row + c1};
            float v[2];
            SumSplitsN<2>(q, splits, stride, v);
            *a0 = v[0];
            *a1 = v[1];
        };
        if (mode == kStreamSwiGlu) {
            const int64_t F = a.seg[0].rows;
            auto swiglu = [&](int64_t col) {
                float g, u;
                sum2(col, F + col, &g, &u);
                if (a.seg[0].bias != nullptr) g += a.seg[0].bias[col];
                if (a.seg[1].bias != nullptr) u += a.seg[1].bias[col];
                return SwiGluF(g, u);
            };
            const float yv = swiglu(c);
            a.seg[1].y[t * F + c] = yv;
            if (a.planes != nullptr) StorePlanes1(a.planes, T, t, c, yv);
            continue;
        }
        if (mode == kStreamQkvRope) {
            // unit c: a (2i, 2i+1) pair of the q then k columns, then one v column
            const RopeArgs& r = a.rope;
            const int32_t pos = r.positions != nullptr ? r.positions[t]
                                                       : r.pos0 + static_cast<int32_t>(t);
            const bool cache_ok = pos >= 0 && pos < r.max_seq;
            if (c == 0 && !cache_ok) RaiseFlag(r.err, 1);
            const int64_t QD = a.seg[0].rows, KD = a.seg[1].rows, pairs = (QD + KD) / 2;
            if (c >= pairs) {
                const int64_t local = c - pairs;
                float v = sum(QD + KD + local);
                if (a.seg[2].bias != nullptr) v += a.seg[2].bias[local];
                if (cache_ok) a.seg[2].y[pos * r.kv_stride + local] = v;
                continue;
            }
            const int64_t col = 2 * c;
            const bool is_k = col >= QD;
            const StreamSeg& sg = is_k ? a.seg[1] : a.seg[0];
            const int64_t local = is_k ? col - QD : col;
            float x0, x1;
            sum2(col, col + 1, &x0, &x1);
            if (sg.bias != nullptr) {
                x0 += sg.bias[local];
                x1 += sg.bias[local + 1];
            }
            float r0 = x0, r1 = x1;
            if (pos >= 0) {
                double cs, sn;
                RopeCosSin(pos, r.freq.inv[static_cast<int>(local % r.head_dim) / 2], &cs, &sn);
                RopeRotate(x0, x1, cs, sn, &r0, &r1);
            }
            if (is_k && !cache_ok) continue;
            float* y = is_k ? sg.y + pos * r.kv_stride : sg.y + t * QD;
            y[local] = r0;
            y[local + 1] = r1;
            continue;
        }
        const int s = (a.n_seg > 2 && c >= a.seg[0].rows + a.seg[1].rows) ? 2
                      : ((a.n_seg > 1 && c >= a.seg[0].rows) ? 1 : 0);
        const StreamSeg& sg = s == 2 ? a.seg[2] : (s == 1 ? a.seg[1] : a.seg[0]);
        const int64_t local = c - (s == 2 ? a.seg[0].rows + a.seg[1].rows : (s == 1 ? a.seg[0].rows : 0));
        float v = sum(c);
        if (sg.bias != nullptr) v += sg.bias[local];
        const int64_t at = t * sg.rows + local;
        sg.y[at] = mode == kStreamAdd ? sg.res[at] + v : v;
    }
}

int SkinnyChunk(int wt) { return wt == kWF32 ? 32 * WChunk<kWF32>::kStages : 32 * 8; }

// Chunks per workgroup: two for quantized weights when K is a multiple of
// two chunks, else one.
int SkinnyPieces(int wt, int64_t T, int64_t K) {
    return wt != kWF32 && T <= 32 && K % (2 * SkinnyChunk(wt)) == 0 ? 2 : 1;
}

// The skinny kernel takes SkinnyPieces chunks per workgroup: K / (that many
// chunks) splits.
SplitPlan PlanSkinny(int wt, int64_t T, int64_t K) {
    const int64_t chunk = SkinnyChunk(wt) * SkinnyPieces(wt, T, K);
    SplitPlan p;
    p.per_split = chunk;
    p.splits = static_cast<int>(K / chunk);
    return p;
}

// Where the skinny kernel measured faster than the tiled one on the 8B
// layer's projections: the quantized types up to 32 rows (F32 stays tiled).
bool SkinnyApplies(int wt, int64_t T, int64_t K) {
    const bool rows = wt >= MLK_Q8_0 && wt <= MLK_Q4_1 && T <= 32;
    return rows && K % SkinnyChunk(wt) == 0 && K / SkinnyChunk(wt) <= 4096;
}

template <int TT, int NP>
void LaunchSkinnyT(int wt, dim3 grid, hipStream_t s, const float* x, const SkinnyArgs& a,
                   int64_t T, int64_t K, int64_t row_bytes, float* partial) {
    switch (wt) {
        case MLK_Q8_0:
            hipLaunchKernelGGL((GemmSkinny<MLK_Q8_0, TT, NP>), grid, dim3(kSkThreads), 0, s, x, a,
                               T, K, row_bytes, partial);
            break;
        case MLK_Q4_0:
            hipLaunchKernelGGL((GemmSkinny<MLK_Q4_0, TT, NP>), grid, dim3(kSkThreads), 0, s, x, a,
                               T, K, row_bytes, partial);
            break;
        case MLK_Q4_1:
            hipLaunchKernelGGL((GemmSkinny<MLK_Q4_1, TT, NP>), grid, dim3(kSkThreads), 0, s, x, a,
                               T, K, row_bytes, partial);
            break;
        default:
            if constexpr (NP == 1) {
                hipLaunchKernelGGL((GemmSkinny<kWF32, TT, 1>), grid, dim3(kSkThreads), 0, s, x, a,
                                   T, K, row_bytes, partial);
            }
            break;
    }
}

mlk_status LaunchSkinny(int wt, const float* x, const SkinnyArgs& a, int64_t T, int64_t K,
                        int64_t row_bytes, int splits, float* partial, hipStream_t s) {
    if (static_cast<int64_t>(a.row_groups) * splits > 0x7FFFFFFF) {
        return Fail(MLK_ERR_INVALID, "linear: %lld output rows exceed one launch",
                    static_cast<long long>(a.cols));
    }
    const dim3 grid(static_cast<unsigned>(static_cast<int64_t>(a.row_groups) * splits));
    if (SkinnyPieces(wt, T, K) == 2) {
        if (T <= 16) {
            LaunchSkinnyT<1, 2>(wt, grid, s, x, a, T, K, row_bytes, partial);
        } else {
            LaunchSkinnyT<2, 2>(wt, grid, s, x, a, T, K, row_bytes, partial);
        }
    } else if (T <= 16) {
        LaunchSkinnyT<1, 1>(wt, grid, s, x, a, T, K, row_bytes, partial);
    } else {
        LaunchSkinnyT<2, 1>(wt, grid, s, x, a, T, K, row_bytes, partial);
    }
    return CheckLaunch("GemmSkinny");
}

// false: no kernel of this epilogue for wt (the fused epilogues are built
// for block-layout Q8_0 / Q4_0 only; x from planes (xp) for them too, with
// 8 waves)
template <int NW, int EPI = kPcStore>
bool LaunchPieces(int wt, dim3 grid, hipStream_t s, const float* x, const uint8_t* w,
                  const float* bias, float* y, int64_t T, int64_t K, int64_t O, int64_t row_bytes,
                  int tiles_m, int tiles, int64_t per_split, float* partial,
                  const uint8_t* w2 = nullptr, const float* bias2 = nullptr,
                  float* y2 = nullptr, const uint32_t* xp = nullptr) {
    const dim3 block(64 * NW);
    if (xp != nullptr) {
        // 8 waves only: at 4 the planes' registers leave one wave a SIMD
        if constexpr (NW == 8) {
            if (wt == MLK_Q8_0) {
                hipLaunchKernelGGL((GemmPieces<MLK_Q8_0, NW, EPI, true>), grid, block, 0, s, x, w,
                                   bias, y, T, K, O, row_bytes, tiles_m, tiles, per_split,
                                   partial, w2, bias2, y2, xp);
                return true;
            }
            if (wt == MLK_Q4_0) {
                hipLaunchKernelGGL((GemmPieces<MLK_Q4_0, NW, EPI, true>), grid, block, 0, s, x, w,
                                   bias, y, T, K, O, row_bytes, tiles_m, tiles, per_split,
                                   partial, w2, bias2, y2, xp);
                return true;
            }
        }
        return false;
    }
    switch (wt) {
        case MLK_Q8_0:
            hipLaunchKernelGGL((GemmPieces<MLK_Q8_0, NW, EPI>), grid, block, 0, s, x, w, bias, y,
                               T, K, O, row_bytes, tiles_m, tiles, per_split, partial, w2, bias2,
                               y2, nullptr);
            return true;
        case MLK_Q4_0:
            hipLaunchKernelGGL((GemmPieces<MLK_Q4_0, NW, EPI>), grid, block, 0, s, x, w, bias, y,
                               T, K, O, row_bytes, tiles_m, tiles, per_split, partial, w2, bias2,
                               y2, nullptr);
            return true;
        default:
            break;
    }
    if constexpr (EPI == kPcStore) {
        if (wt == kWPlanarQ8) {
            hipLaunchKernelGGL((GemmPieces<kWPlanarQ8, NW>), grid, block, 0, s, x, w, bias, y, T,
                               K, O, row_bytes, tiles_m, tiles, per_split, partial, w2, bias2,
                               y2, nullptr);
            return true;
        }
        if (wt == kWPlanarQ4) {
            hipLaunchKernelGGL((GemmPieces<kWPlanarQ4, NW>), grid, block, 0, s, x, w, bias, y, T,
                               K, O, row_bytes, tiles_m, tiles, per_split, partial, w2, bias2,
                               y2, nullptr);
            return true;
        }
    }
    return false;
}

template <int BM>
void LaunchTiles(int wt, dim3 grid, hipStream_t s, const float* x, const uint8_t* w,
                 const float* bias, float* y, int64_t T, int64_t K, int64_t O, int64_t row_bytes,
                 int tiles_m, int tiles, int64_t per_split, float* partial) {
    // 128-row tiles of Q8_0 / Q4_0 on bf16 piece products; K % 256 == 0 keeps
    // each product's fp32 roundings (block sum, scale, K / 32 block adds)
    // under the K of the fp32 kernel's bound
    if (BM == 128 && K % 256 == 0 &&
        (wt == MLK_Q8_0 || wt == MLK_Q4_0 || wt == kWPlanarQ8 || wt == kWPlanarQ4)) {
        // 256-output tiles when they still fill two workgroups per CU and K
        // is not split; else 128
        const int64_t tiles8 = static_cast<int64_t>(tiles_m) * ((O + 255) / 256);
        if (per_split >= (K + kBK - 1) / kBK && tiles8 >= 2 * static_cast<int64_t>(ComputeUnits())) {
            LaunchPieces<8>(wt, dim3(static_cast<unsigned>(tiles8)), s, x, w, bias, y, T, K, O,
                            row_bytes, tiles_m, static_cast<int>(tiles8), per_split, partial);
        } else {
            LaunchPieces<4>(wt, grid, s, x, w, bias, y, T, K, O, row_bytes, tiles_m, tiles,
                            per_split, partial);
        }
        return;
    }
    switch (wt) {
        case MLK_Q8_0:
            hipLaunchKernelGGL((GemmMfma<MLK_Q8_0, BM>), grid, dim3(kGemmThreads), 0, s, x, w,
                               bias, y, T, K, O, row_bytes, tiles_m, tiles, per_split, partial);
            break;
        case MLK_Q4_0:
            hipLaunchKernelGGL((GemmMfma<MLK_Q4_0, BM>), grid, dim3(kGemmThreads), 0, s, x, w,
                               bias, y, T, K, O, row_bytes, tiles_m, tiles, per_split, partial);
            break;
        case MLK_Q4_1:
            hipLaunchKernelGGL((GemmMfma<MLK_Q4_1, BM>), grid, dim3(kGemmThreads), 0, s, x, w,
                               bias, y, T, K, O, row_bytes, tiles_m, tiles, per_split, partial);
            break;
        case kWPlanarQ8:
            hipLaunchKernelGGL((GemmMfma<kWPlanarQ8, BM>), grid, dim3(kGemmThreads), 0, s, x, w,
                               bias, y, T, K, O, row_bytes, tiles_m, tiles, per_split, partial);
            break;
        case kWPlanarQ4:
            hipLaunchKernelGGL((GemmMfma<kWPlanarQ4, BM>), grid, dim3(kGemmThreads), 0, s, x, w,
                               bias, y, T, K, O, row_bytes, tiles_m, tiles, per_split, partial);
            break;
        default:
            hipLaunchKernelGGL((GemmMfma<kWF32, BM>), grid, dim3(kGemmThreads), 0, s, x, w, bias,
                               y, T, K, O, row_bytes, tiles_m, tiles, per_split, partial);
            break;
    }
}

}  // namespace

int64_t GemmWorkspaceBytes(int wt, int64_t T, int64_t K, int64_t O) {
    const SplitPlan p = SkinnyApplies(wt, T, K) ? PlanSkinny(wt, T, K) : PlanSplits(T, K, O);
    return p.splits > 1 ? static_cast<int64_t>(p.splits) * T * O * 4 : 0;
}

// Launches GemmMfma for a shape the caller has validated: K % 4 == 0 and
// x / fp32 W 16-byte aligned; for quantized W, K % 32 == 0 and W aligned to
// its loads (2 bytes, 4 for Q4_1).  K is split over workgroups when the
// workspace holds GemmWorkspaceBytes(wt, T, K, O) bytes, else not.  Shapes
// SkinnyApplies accepts take GemmSkinny (when K is more than one chunk, only
// with the workspace; without it the tiled kernel).
mlk_status LaunchGemm(int wt, const float* x, const void* w, const float* bias, float* y,
                      int64_t T, int64_t K, int64_t O, int64_t row_bytes, void* workspace,
                      size_t workspace_bytes, hipStream_t s) {
    const SplitPlan sk = PlanSkinny(wt, T, K);
    const bool sk_ws = sk.splits == 1 ||
                       (workspace != nullptr && Aligned(workspace, 16) &&
                        workspace_bytes >= static_cast<size_t>(sk.splits) * T * O * 4);
    if (SkinnyApplies(wt, T, K) && sk_ws) {
        const SplitPlan plan = sk;
        float* partial = plan.splits > 1 ? static_cast<float*>(workspace) : nullptr;
        const int64_t groups = (O + kSkRows - 1) / kSkRows;
        if (groups > 0x7FFFFFFF) {
            return Fail(MLK_ERR_INVALID, "linear: %lld output rows exceed one launch",
                        static_cast<long long>(O));
        }
        SkinnyArgs a{};
        a.w[0] = static_cast<const uint8_t*>(w);
        a.rows[0] = O;
        a.n_seg = 1;
        a.row_groups = static_cast<int>(groups);
        a.cols = O;
        a.bias = bias;
        a.y = y;
        mlk_status st = LaunchSkinny(wt, x, a, T, K, row_bytes, plan.splits, partial, s);
        if (st != MLK_OK || partial == nullptr) return st;
        hipLaunchKernelGGL(SplitKReduce, dim3(GridFor(T * O, kGemmThreads, 8)),
                           dim3(kGemmThreads), 0, s, partial, plan.splits, bias, y, T, O);
        return CheckLaunch("SplitKReduce");
    }
    const int bm = TileRows(T);
    const int64_t tiles_m = (T + bm - 1) / bm;
    const int64_t tiles_n = (O + kBN - 1) / kBN;
    const int64_t stages = (K + kBK - 1) / kBK;
    SplitPlan plan = PlanSplits(T, K, O);
    float* partial = nullptr;
    if (plan.splits > 1 && workspace != nullptr &&
        workspace_bytes >= static_cast<size_t>(plan.splits) * T * O * 4 && Aligned(workspace, 16)) {
        partial = static_cast<float*>(workspace);
    } else {
        plan.splits = 1;
        plan.per_split = stages;
    }
    if (tiles_m * tiles_n * plan.splits > 0x7FFFFFFF || tiles_m > 0x7FFFFFFF) {
        return Fail(MLK_ERR_INVALID, "linear: %lld x %lld tiles exceed one launch",
                    static_cast<long long>(tiles_m), static_cast<long long>(tiles_n));
    }
    const int tiles = static_cast<int>(tiles_m * tiles_n);
    const dim3 grid(static_cast<unsigned>(static_cast<int64_t>(tiles) * plan.splits));
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    const int tm = static_cast<int>(tiles_m);
    if (bm == 32) {
        LaunchTiles<32>(wt, grid, s, x, wb, bias, y, T, K, O, row_bytes, tm, tiles, plan.per_split,
                        partial);
    } else if (bm == 64) {
        LaunchTiles<64>(wt, grid, s, x, wb, bias, y, T, K, O, row_bytes, tm, tiles, plan.per_split,
                        partial);
    } else {
        LaunchTiles<128>(wt, grid, s, x, wb, bias, y, T, K, O, row_bytes, tm, tiles,
                         plan.per_split, partial);
    }
    mlk_status st = CheckLaunch("GemmMfma");
    if (st != MLK_OK || partial == nullptr) return st;
    hipLaunchKernelGGL(SplitKReduce, dim3(GridFor(T * O, kGemmThreads, 8)), dim3(kGemmThreads), 0,
                       s, partial, plan.splits, bias, y, T, O);
    return CheckLaunch("SplitKReduce");
}

bool TiledFusedApplies(int wt, int64_t T, int64_t K, int64_t O, int mode) {
    if ((wt != MLK_Q8_0 && wt != MLK_Q4_0) || K % 256 != 0 || TileRows(T) != 128 || O <= 0) {
        return false;
    }
    const int64_t tiles_m = (T + 127) / 128;
    if (mode == kStreamPlain) {  // a pair in one pass, where that fills the GPU on its own
        const int64_t tiles = tiles_m * 2 * ((O + 127) / 128);
        return tiles >= 2 * static_cast<int64_t>(ComputeUnits()) && tiles <= 0x7FFFFFFF;
    }
    if (PlanSplits(T, K, O).splits != 1) return false;
    if (mode == kStreamSwiGlu) {
        const int64_t tiles = tiles_m * ((O + 127) / 128);
        return tiles >= 2 * static_cast<int64_t>(ComputeUnits()) && tiles <= 0x7FFFFFFF;
    }
    return mode == kStreamAdd && tiles_m * ((O + 127) / 128) <= 0x7FFFFFFF;
}

bool TiledTakesPlanes(int64_t T, int64_t O) {
    return ((T + 127) / 128) * ((O + 255) / 256) >= 2 * static_cast<int64_t>(ComputeUnits());
}

mlk_status LinearTiledFused(int wt, const float* x, int64_t T, int64_t K, const StreamArgs& sa,
                            int mode, hipStream_t s) {
    const StreamSeg& g0 = sa.seg[0];
    const int64_t O = g0.rows;
    const bool single = mode == kStreamPlain && sa.n_seg == 1;
    if (!TiledFusedApplies(wt, T, K, O, single ? kStreamAdd : mode) || !Aligned(x, 16) ||
        (sa.x_planes != nullptr && !Aligned(sa.x_planes, 16))) {
        return Fail(MLK_ERR_INVALID, "linear (tiled, fused): unsupported shape");
    }
    if (single) {
        if (g0.w == nullptr || g0.y == nullptr || !Aligned(g0.w, 2)) {
            return Fail(MLK_ERR_INVALID, "linear (tiled, fused): bad segment");
        }
    } else if (mode == kStreamSwiGlu || mode == kStreamPlain) {
        const StreamSeg& g1 = sa.seg[1];
        if (sa.n_seg != 2 || g1.rows != O || g0.w == nullptr || g1.w == nullptr ||
            g1.y == nullptr || (mode == kStreamPlain && g0.y == nullptr) || !Aligned(g0.w, 2) ||
            !Aligned(g1.w, 2)) {
            return Fail(MLK_ERR_INVALID, "linear (tiled, fused): bad segment pair");
        }
    } else if (sa.n_seg != 1 || g0.w == nullptr || g0.y == nullptr || g0.res != g0.y ||
               !Aligned(g0.w, 2)) {
        // the residual add runs in place: y = y + sum
        return Fail(MLK_ERR_INVALID, "linear (tiled, fused): the residual must be y");
    }
    // the outputs are written while other workgroups still read x
    const auto overlaps_x = [&](const float* y) {
        return y != nullptr && y < x + T * K && x < y + T * O;
    };
    if (overlaps_x(g0.y) || (sa.n_seg == 2 && overlaps_x(sa.seg[1].y))) {
        return Fail(MLK_ERR_INVALID, "linear (tiled, fused): outputs must not overlap x");
    }
    const int64_t row_bytes = (K / 32) * BlockBytes(wt);
    const int64_t stages = K / kBK;
    const int tm = static_cast<int>((T + 127) / 128);
    bool ok = false;
    const uint32_t* xp = sa.x_planes;
    if (single) {
        // the tile width LaunchTiles takes for the plain product
        const int64_t tiles8 = static_cast<int64_t>(tm) * ((O + 255) / 256);
        if (tiles8 >= 2 * static_cast<int64_t>(ComputeUnits())) {
            const int tiles = static_cast<int>(tiles8);
            ok = LaunchPieces<8>(wt, dim3(static_cast<unsigned>(tiles)), s, x, g0.w, g0.bias, g0.y,
                                 T, K, O, row_bytes, tm, tiles, stages, nullptr, nullptr, nullptr,
                                 nullptr, xp);
        } else {
            // 4-wave tiles split x themselves (no planes variant)
            const int tiles = static_cast<int>(tm * ((O + 127) / 128));
            ok = LaunchPieces<4>(wt, dim3(static_cast<unsigned>(tiles)), s, x, g0.w, g0.bias, g0.y,
                                 T, K, O, row_bytes, tm, tiles, stages, nullptr);
        }
    } else if (mode == kStreamPlain) {
        // 256-output tiles (TiledFusedApplies leaves at least one a CU):
        // each x split serves twice the outputs of a 128-output tile;
        // measured at Llama-3-8B's k / v (256 tiles) as fast as 512 tiles
        // of 128 outputs, or slightly faster
        const int tiles = static_cast<int>(static_cast<int64_t>(tm) * 2 * ((O + 255) / 256));
        const StreamSeg& g1 = sa.seg[1];
        ok = LaunchPieces<8, kPcPair>(wt, dim3(static_cast<unsigned>(tiles)), s, x, g0.w, g0.bias,
                                      g0.y, T, K, O, row_bytes, tm, tiles, stages, nullptr, g1.w,
                                      g1.bias, g1.y, xp);
    } else if (mode == kStreamSwiGlu) {
        const int tiles = static_cast<int>(tm * ((O + 127) / 128));
        ok = LaunchPieces<8, kPcSwiGlu>(wt, dim3(static_cast<unsigned>(tiles)), s, x, g0.w,
                                        g0.bias, sa.seg[1].y, T, K, O, row_bytes, tm, tiles,
                                        stages, nullptr, sa.seg[1].w, sa.seg[1].bias, nullptr,
                                        xp);
    } else {
        // the tile width LaunchTiles takes for the plain product
        const int64_t tiles8 = static_cast<int64_t>(tm) * ((O + 255) / 256);
        if (tiles8 >= 2 * static_cast<int64_t>(ComputeUnits())) {
            const int tiles = static_cast<int>(tiles8);
            ok = LaunchPieces<8, kPcAdd>(wt, dim3(static_cast<unsigned>(tiles)), s, x, g0.w,
                                         g0.bias, g0.y, T, K, O, row_bytes, tm, tiles, stages,
                                         nullptr, nullptr, nullptr, nullptr, xp);
        } else {
            const int tiles = static_cast<int>(tm * ((O + 127) / 128));
            ok = LaunchPieces<4, kPcAdd>(wt, dim3(static_cast<unsigned>(tiles)), s, x, g0.w,
                                         g0.bias, g0.y, T, K, O, row_bytes, tm, tiles, stages,
                                         nullptr);
        }
    }
    if (!ok) return Fail(MLK_ERR_INVALID, "linear (tiled, fused): weight type %d", wt);
    return CheckLaunch("GemmPieces (fused)");
}

bool SkinnyFusedApplies(int wt, int64_t T, int64_t K) {
    return wt != kWF32 && T >= 1 && SkinnyApplies(wt, T, K);
}

int64_t SkinnyFusedWorkspaceBytes(int wt, int64_t T, int64_t K, int64_t cols) {
    return static_cast<int64_t>(PlanSkinny(wt, T, K).splits) * T * cols * 4;
}

// T token rows through up to three quantized weight matrices with the same K
// (StreamArgs segments) in one skinny launch, then one reduction with the
// mode's epilogue.  The partial sums always go through the workspace.
mlk_status LinearSkinnyFused(int wt, const float* x, int64_t T, int64_t K, const StreamArgs& sa,
                             int mode, void* workspace, size_t workspace_bytes, hipStream_t s) {
    if (!SkinnyFusedApplies(wt, T, K) || sa.n_seg < 1 || sa.n_seg > 3 || !Aligned(x, 16) ||
        (mode == kStreamSwiGlu && (sa.n_seg != 2 || sa.seg[0].rows != sa.seg[1].rows)) ||
        (mode == kStreamQkvRope && !QkvRopeArgsOk(sa))) {
        return Fail(MLK_ERR_INVALID, "linear (fused rows): unsupported shape");
    }
    SkinnyArgs a{};
    int64_t cols = 0, groups = 0;
    for (int i = 0; i < sa.n_seg; ++i) {
        const StreamSeg& g = sa.seg[i];
        if (g.w == nullptr || g.y == nullptr || g.rows <= 0 || !Aligned(g.w, 4) ||
            (mode == kStreamAdd && g.res == nullptr)) {
            return Fail(MLK_ERR_INVALID, "linear (fused rows): bad segment %d", i);
        }
        a.w[i] = g.w;
        a.rows[i] = g.rows;
        a.col0[i] = cols;
        a.g0[i] = static_cast<int>(groups);
        cols += g.rows;
        groups += (g.rows + kSkRows - 1) / kSkRows;
    }
    a.n_seg = sa.n_seg;
    a.row_groups = static_cast<int>(groups);
    a.cols = cols;
    const SplitPlan plan = PlanSkinny(wt, T, K);
    const int64_t need = static_cast<int64_t>(plan.splits) * T * cols * 4;
    if (workspace == nullptr || !Aligned(workspace, 16) ||
        static_cast<int64_t>(workspace_bytes) < need || groups > 0x3FFFFFFF) {
        return Fail(MLK_ERR_INVALID, "linear (fused rows): workspace of %lld bytes needed",
                    static_cast<long long>(need));
    }
    float* partial = static_cast<float*>(workspace);
    const int64_t row_bytes = (K / 32) * BlockBytes(wt);
    mlk_status st = LaunchSkinny(wt, x, a, T, K, row_bytes, plan.splits, partial, s);
    if (st != MLK_OK) return st;
    const int64_t out_cols = mode == kStreamSwiGlu    ? sa.seg[0].rows
                             : mode == kStreamQkvRope ? (sa.seg[0].rows + sa.seg[1].rows) / 2 +
                                                            sa.seg[2].rows
                                                      : cols;
    hipLaunchKernelGGL(SplitKReduceFused, dim3(GridFor(T * out_cols, kGemmThreads, 8)),
                       dim3(kGemmThreads), 0, s, partial, plan.splits, T, cols, sa, mode,
                       out_cols);
    return CheckLaunch("SplitKReduceFused");
}

// ------------------------------------------------------- planar launches
int64_t PlanarBytes(int qt, int64_t O, int64_t K) {
    if ((qt != MLK_Q8_0 && qt != MLK_Q4_0) || O <= 0 || K <= 0 || K % 256 != 0) return 0;
    const int64_t tiles = (O + 15) / 16;
    return tiles * (qt == MLK_Q8_0 ? 16 : 8) * K + tiles * (K / 32) * 32;
}

mlk_status LaunchToPlanar(int qt, const void* blocks, int64_t O, int64_t K, void* planar,
                          hipStream_t s) {
    const int64_t tiles = (O + 15) / 16, nb = K / 32;
    const int64_t n = tiles * (nb / (qt == MLK_Q8_0 ? 2 : 4)) * 64 + tiles * (nb / 8) * 16;
    const dim3 grid(GridFor(n, kGemmThreads, 8));
    const uint8_t* b = static_cast<const uint8_t*>(blocks);
    uint8_t* o = static_cast<uint8_t*>(planar);
    if (qt == MLK_Q8_0) {
        hipLaunchKernelGGL(ToPlanar<MLK_Q8_0>, grid, dim3(kGemmThreads), 0, s, b, O, K, o);
    } else {
        hipLaunchKernelGGL(ToPlanar<MLK_Q4_0>, grid, dim3(kGemmThreads), 0, s, b, O, K, o);
    }
    return CheckLaunch("ToPlanar");
}

namespace {

// GemmPlanar's plan: token tiles, block pairs per K range, ranges (splits),
// and the workspace: partial sums (splits > 1, or always with `partials`: a
// fused launch's reduction applies its epilogue), then the x planes.
struct PlanarPlan {
    int tt = 1, np = 4, splits = 1, pt = 2;
    int wgs = 0;  // > 0: GemmPlanarStream, with this many workgroups per K range
    int64_t partial_bytes = 0, plane_bytes = 0;
    int64_t Bytes() const { return partial_bytes + plane_bytes; }
};

PlanarPlan PlanPlanar(int64_t T, int64_t K, int64_t cols, bool partials) {
    PlanarPlan p;
    p.tt = T <= 16 ? 1 : 2;
    p.np = p.tt == 1 && K % 512 == 0 ? 8 : 4;
    p.splits = static_cast<int>(K / (64 * p.np));
    p.partial_bytes = p.splits > 1 || partials
                          ? (static_cast<int64_t>(p.splits) * T * cols * 4 + 255) / 256 * 256
                          : 0;
    p.plane_bytes = (K / 32) * 3 * T * 64;
    return p;
}

template <int QT, int PT>
void LaunchPlanarPt(const PlanarPlan& p, dim3 grid, hipStream_t s, const uint32_t* planes,
                    const SkinnyArgs& a, int64_t T, int64_t K, float* partial) {
    if (p.tt == 1 && p.np == 8) {
        hipLaunchKernelGGL((GemmPlanar<QT, 1, 8, PT>), grid, dim3(kSkThreads), 0, s, planes, a,
                           T, K, partial);
    } else if (p.tt == 1) {
        hipLaunchKernelGGL((GemmPlanar<QT, 1, 4, PT>), grid, dim3(kSkThreads), 0, s, planes, a,
                           T, K, partial);
    } else {
        hipLaunchKernelGGL((GemmPlanar<QT, 2, 4, PT>), grid, dim3(kSkThreads), 0, s, planes, a,
                           T, K, partial);
    }
}

// GemmPlanarStream's shape: steps of kStreamPt tiles, a ring of kStreamD
// steps per wave, about kStreamWgsPerCu workgroups per compute unit.
constexpr int kStreamPt = 1;
constexpr int kStreamD = 3;
constexpr int kStreamWgsPerCu = 2;
constexpr int kStreamMinWgsPerCu = 4;

template <int QT>
void LaunchPlanarStream(const PlanarPlan& p, dim3 grid, hipStream_t s, const uint32_t* planes,
                        const SkinnyArgs& a, int64_t T, int64_t K, float* partial) {
    constexpr int P = kStreamPt, D = kStreamD;
    if (p.tt == 1 && p.np == 8) {
        hipLaunchKernelGGL((GemmPlanarStream<QT, 1, 8, P, D>), grid, dim3(kSkThreads), 0, s,
                           planes, a, T, K, partial, p.wgs);
    } else if (p.tt == 1) {
        hipLaunchKernelGGL((GemmPlanarStream<QT, 1, 4, P, D>), grid, dim3(kSkThreads), 0, s,
                           planes, a, T, K, partial, p.wgs);
    } else {
        hipLaunchKernelGGL((GemmPlanarStream<QT, 2, 4, P, D>), grid, dim3(kSkThreads), 0, s,
                           planes, a, T, K, partial, p.wgs);
    }
}

template <int QT>
void LaunchPlanarT(const PlanarPlan& p, dim3 grid, hipStream_t s, const uint32_t* planes,
                   const SkinnyArgs& a, int64_t T, int64_t K, float* partial) {
    if (p.wgs > 0) {
        LaunchPlanarStream<QT>(p, grid, s, planes, a, T, K, partial);
    } else if (p.pt == 1) {
        LaunchPlanarPt<QT, 1>(p, grid, s, planes, a, T, K, partial);
    } else {
        LaunchPlanarPt<QT, 2>(p, grid, s, planes, a, T, K, partial);
    }
}

// x split into planes (after the partial sums in the workspace; or the
// caller's planes of x when planes_in is set), then GemmPlanar over the
// segments' row groups x the plan's ranges.  a.w, a.rows, a.n_seg set; the
// rest filled in here.  The caller reduces.
mlk_status RunPlanar(int qt, const float* x, const uint32_t* planes_in, SkinnyArgs& a, int64_t T,
                     int64_t K, bool partials, void* workspace, size_t workspace_bytes,
                     int* splits, float** partial, hipStream_t s) {
    // a direct output is one [T, rows] matrix: several segments go through
    // partial sums (the fused launches' reductions place each segment)
    if (a.n_seg > 1 && !partials) {
        return Fail(MLK_ERR_INVALID, "linear (planar): several segments need partial sums");
    }
    int64_t cols = 0;
    for (int i = 0; i < a.n_seg; ++i) {
        if (!Aligned(a.w[i], 16)) return Fail(MLK_ERR_INVALID, "linear (planar): weights not 16-byte aligned");
        a.col0[i] = cols;
        cols += a.rows[i];
    }
    PlanarPlan p = PlanPlanar(T, K, cols, partials);
    // row groups of 4 waves x pt tiles: one tile per wave when two would
    // leave fewer than two workgroups per compute unit
    auto count_groups = [&](int pt) {
        int64_t g = 0;
        for (int i = 0; i < a.n_seg; ++i) g += (a.rows[i] + 64 * pt - 1) / (64 * pt);
        return g;
    };
    // The streaming kernel where GemmPlanar's grid would take more than
    // kStreamMinWgsPerCu workgroups per compute unit (the 8B gate/up with
    // 16 tokens, 7: measured 34.3 -> 27.6 us; at 1-4 per unit GemmPlanar's
    // one round of loads per workgroup measured as fast or faster: the 8B
    // q/k/v 11.6 vs 12.7 us, wo 9 vs 11, down 20 vs 20.4), and where its
    // offsets fit 31 bits, unless y takes a bias.
    const int64_t out_row = p.partial_bytes > 0 ? cols : a.rows[0];
    // (every token slot of the tiles, t < 16 tt, not only t < T: the stores
    // of slots past T must land past the output's range, unwrapped)
    bool stream = count_groups(2) * p.splits > kStreamMinWgsPerCu * ComputeUnits() &&
                  !(p.partial_bytes == 0 && a.bias != nullptr) &&
                  16 * p.tt * out_row * 4 < (int64_t{1} << 30);
    for (int i = 0; i < a.n_seg; ++i) {
        const int64_t tiles = (a.rows[i] + 15) / 16;
        stream = stream && tiles * ((qt == MLK_Q8_0 ? 16 : 8) * K + K) < (int64_t{1} << 31);
    }
    int64_t groups = 0;
    if (stream) {
        // steps of kStreamPt tiles per segment; per K range as many
        // workgroups as give each wave the same count of steps, within
        // kStreamWgsPerCu per compute unit over all ranges
        for (int i = 0; i < a.n_seg; ++i) {
            a.g0[i] = static_cast<int>(groups);
            groups += ((a.rows[i] + 15) / 16 + kStreamPt - 1) / kStreamPt;
        }
        const int64_t cap = std::max<int64_t>(1, kStreamWgsPerCu * ComputeUnits() / p.splits);
        const int64_t per_wave = std::max<int64_t>(1, (groups + 4 * cap - 1) / (4 * cap));
        p.wgs = static_cast<int>((groups + 4 * per_wave - 1) / (4 * per_wave));
    } else {
        if (count_groups(2) * p.splits < 2 * ComputeUnits()) p.pt = 1;
        for (int i = 0; i < a.n_seg; ++i) {
            a.g0[i] = static_cast<int>(groups);
            groups += (a.rows[i] + 64 * p.pt - 1) / (64 * p.pt);
        }
    }
    if (workspace == nullptr || !Aligned(workspace, 16) ||
        static_cast<int64_t>(workspace_bytes) < p.Bytes()) {
        return Fail(MLK_ERR_INVALID, "linear (planar): workspace of %lld bytes needed",
                    static_cast<long long>(p.Bytes()));
    }
    if ((p.wgs > 0 ? p.wgs : groups) * p.splits > 0x7FFFFFFF) {
        return Fail(MLK_ERR_INVALID, "linear (planar): %lld output rows exceed one launch",
                    static_cast<long long>(cols));
    }
    if (planes_in != nullptr && !Aligned(planes_in, 16)) {
        return Fail(MLK_ERR_INVALID, "linear (planar): x planes not 16-byte aligned");
    }
    a.row_groups = static_cast<int>(groups);
    a.cols = cols;
    *splits = p.splits;
    *partial = p.partial_bytes > 0 ? static_cast<float*>(workspace) : nullptr;
    const uint32_t* planes = planes_in;
    if (planes == nullptr) {
        uint32_t* own = reinterpret_cast<uint32_t*>(static_cast<char*>(workspace) + p.partial_bytes);
        hipLaunchKernelGGL(SplitXBf, dim3(GridFor((K / 32) * T * 16, kGemmThreads, 4)),
                           dim3(kGemmThreads), 0, s, x, T, K, own);
        mlk_status st = CheckLaunch("SplitXBf");
        if (st != MLK_OK) return st;
        planes = own;
    }
    const dim3 grid(static_cast<unsigned>((p.wgs > 0 ? p.wgs : groups) * p.splits));
    if (qt == MLK_Q8_0) {
        LaunchPlanarT<MLK_Q8_0>(p, grid, s, planes, a, T, K, *partial);
    } else {
        LaunchPlanarT<MLK_Q4_0>(p, grid, s, planes, a, T, K, *partial);
    }
    return CheckLaunch("GemmPlanar");
}

}  // namespace

bool PlanarApplies(int qt, int64_t T, int64_t K) {
    return (qt == MLK_Q8_0 || qt == MLK_Q4_0) && T >= 1 && T <= 32 && K % 256 == 0;
}

int64_t PlanarWorkspaceBytes(int64_t T, int64_t K, int64_t cols, bool partials) {
    return PlanPlanar(T, K, cols, partials).Bytes();
}

mlk_status LinearPlanar(int qt, const float* x, const void* w, const float* bias, float* y,
                        int64_t T, int64_t K, int64_t O, void* workspace, size_t workspace_bytes,
                        hipStream_t s, const uint32_t* planes) {
    if (!PlanarApplies(qt, T, K)) {  // many rows: the tiled GEMM on the planar tiles
        return LaunchGemm(qt == MLK_Q8_0 ? kWPlanarQ8 : kWPlanarQ4, x, w, bias, y, T, K, O, 0,
                          workspace, workspace_bytes, s);
    }
    SkinnyArgs a{};
    a.w[0] = static_cast<const uint8_t*>(w);
    a.rows[0] = O;
    a.n_seg = 1;
    a.bias = bias;
    a.y = y;
    int splits = 1;
    float* partial = nullptr;
    mlk_status st = RunPlanar(qt, x, planes, a, T, K, false, workspace, workspace_bytes,
                              &splits, &partial, s);
    if (st != MLK_OK || partial == nullptr) return st;
    hipLaunchKernelGGL(SplitKReduce, dim3(GridFor(T * O, kGemmThreads, 8)), dim3(kGemmThreads), 0,
                       s, partial, splits, bias, y, T, O);
    return CheckLaunch("SplitKReduce");
}

mlk_status LinearPlanarPartials(int qt, const float* x, const void* w, int64_t T, int64_t K,
                                int64_t O, void* workspace, size_t workspace_bytes,
                                hipStream_t s, const uint32_t* planes, float** partial,
                                int* splits) {
    if (!PlanarApplies(qt, T, K) || !Aligned(x, 16)) {
        return Fail(MLK_ERR_INVALID, "linear (planar): unsupported shape");
    }
    SkinnyArgs a{};
    a.w[0] = static_cast<const uint8_t*>(w);
    a.rows[0] = O;
    a.n_seg = 1;
    return RunPlanar(qt, x, planes, a, T, K, true, workspace, workspace_bytes, splits, partial, s);
}

mlk_status LinearPlanarFused(int qt, const float* x, int64_t T, int64_t K, const StreamArgs& sa,
                             int mode, void* workspace, size_t workspace_bytes, hipStream_t s,
                             const uint32_t* planes) {
    if (sa.planes != nullptr &&
        (mode != kStreamSwiGlu || sa.seg[0].rows % 32 != 0 || !Aligned(sa.planes, 16))) {
        return Fail(MLK_ERR_INVALID, "linear (planar, fused rows): planes out only after SwiGLU");
    }
    if (!PlanarApplies(qt, T, K) || sa.n_seg < 1 || sa.n_seg > 3 || !Aligned(x, 16) ||
        (mode == kStreamSwiGlu && (sa.n_seg != 2 || sa.seg[0].rows != sa.seg[1].rows)) ||
        (mode == kStreamQkvRope && !QkvRopeArgsOk(sa))) {
        return Fail(MLK_ERR_INVALID, "linear (planar, fused rows): unsupported shape");
    }
    SkinnyArgs a{};
    for (int i = 0; i < sa.n_seg; ++i) {
        const StreamSeg& g = sa.seg[i];
        if (g.w == nullptr || g.y == nullptr || g.rows <= 0 ||
            (mode == kStreamAdd && g.res == nullptr)) {
            return Fail(MLK_ERR_INVALID, "linear (planar, fused rows): bad segment %d", i);
        }
        a.w[i] = g.w;
        a.rows[i] = g.rows;
    }
    a.n_seg = sa.n_seg;
    int splits = 1;
    float* partial = nullptr;
    mlk_status st = RunPlanar(qt, x, planes, a, T, K, true, workspace, workspace_bytes, &splits,
                              &partial, s);
    if (st != MLK_OK) return st;
    const int64_t cols = a.cols;
    const int64_t out_cols = mode == kStreamSwiGlu    ? sa.seg[0].rows
                             : mode == kStreamQkvRope ? (sa.seg[0].rows + sa.seg[1].rows) / 2 +
                                                            sa.seg[2].rows
                                                      : cols;
    hipLaunchKernelGGL(SplitKReduceFused, dim3(GridFor(T * out_cols, kGemmThreads, 8)),
                       dim3(kGemmThreads), 0, s, partial, splits, T, cols, sa, mode, out_cols);
    return CheckLaunch("SplitKReduceFused");
}

}  // namespace mlk
