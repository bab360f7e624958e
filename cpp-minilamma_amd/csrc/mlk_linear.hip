// mlk_linear.hip -- linear layers y = x W^T (+ bias) with F32 or block-
// quantized weights, and the F32 Matmul.
//
// Semantics (the reference, paths under its tree):
//   quantized  y[t, j] = sum_k x[t, k] * dequant(W)[j, k]   LinearQ80/Q40/Q41
//              (src/quant.cc:393-463), device kernels Q80/Q40/Q41LinearKernel
//              (src/cuda_quant.cu:29-97): one thread per output, a serial
//              loop over every block of the weight row.
//   F32        the same with W [out, in] fp32: LinearNative
//              (matumal/matuml_ops.cc:146-163), cublasSgemm on the device
//              (src/cuda_matmul.cc:142-186).
//   bias       added to the finished fp32 sum (the reference adds it on the
//              host after download, src/cuda_quant.cu:99-110).
// Sums are fp32 in a different order than the reference's serial loop; both
// are within the recursive-summation bound gamma_K * sum_k |x_k w_k| of the
// exact value, which is what the parity tests hold them to.
//
// Decode-shaped calls (a few token rows, the forward pass's one-token
// steps) are weight-streaming GEMVs bound by HBM: every weight byte is read
// once, x stays in L1.  Layout of the work:
//   - a wave owns kRows consecutive weight rows; each lane owns "pairs" of
//     two consecutive blocks (64 inputs) of those rows, p = lane, lane + 64,
//     ..., so a wave's loads cover contiguous spans of every row;
//   - a pair is 68 / 36 / 40 bytes (Q8_0 / Q4_0 / Q4_1), a whole number of
//     dwords at a dword-aligned offset when in_features % 64 == 0, so it is
//     read with dwordx4 loads and the codes realigned with v_alignbyte;
//   - per block, s = sum code * x over the 32 inputs, then the block's
//     scale is applied once (Q4_0: d * (s - 8 sum x), Q4_1: d * s + m sum x,
//     with sum x per block shared by the wave's rows);
//   - the 64 lane partials are summed with a butterfly at the end.
// Shapes outside that (in_features % 64 != 0, unaligned pointers) take a
// one-wave-per-row kernel with byte loads.
#include "mlk_quant.h"

namespace mlk {
namespace {

constexpr int kThreads = 256;
constexpr int kWavesPerBlock = kThreads / kWave;
constexpr int kRows = 4;      // weight rows per wave in the GEMV kernels
constexpr int kMaxTok = 4;    // token rows per GEMV launch

typedef uint32_t U32x4A4 __attribute__((ext_vector_type(4), aligned(4)));

__device__ inline float WaveSumF(float v) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) {
        v += __shfl_xor(v, off, kWave);
    }
    return v;
}

template <int QT>
struct Pair {
    static constexpr int kBytes = 2 * Fmt<QT>::kBytes;  // 68, 36, 40
    static constexpr int kWords = kBytes / 4;           // 17, 9, 10
};

// The dwords of one block pair (dword-aligned), as dwordx4 loads plus a tail.
template <int QT>
__device__ inline void LoadPair(const uint8_t* p, uint32_t (&u)[Pair<QT>::kWords]) {
    const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
    constexpr int n4 = Pair<QT>::kWords / 4;
#pragma unroll
    for (int i = 0; i < n4; ++i) {
        const U32x4A4 v = *reinterpret_cast<const U32x4A4*>(q + 4 * i);
        u[4 * i + 0] = v.x;
        u[4 * i + 1] = v.y;
        u[4 * i + 2] = v.z;
        u[4 * i + 3] = v.w;
    }
#pragma unroll
    for (int i = 4 * n4; i < Pair<QT>::kWords; ++i) {
        u[i] = q[i];
    }
}

// Block B (0 or 1) of a pair: scale, min (Q4_1) and the code dwords, four
// elements per dword for Q8_0 (8 dwords), low/high nibble pairs for Q4
// (4 dwords: byte j of dword i holds elements 4i + j and 16 + 4i + j).
template <int QT, int B>
struct BlockOf;

template <int B>
struct BlockOf<MLK_Q8_0, B> {
    float d;
    uint32_t c[8];
    __device__ inline explicit BlockOf(const uint32_t (&u)[17]) {
        if (B == 0) {
            d = HalfHw(u[0] & 0xFFFFu);
#pragma unroll
            for (int i = 0; i < 8; ++i) c[i] = __builtin_amdgcn_alignbyte(u[i + 1], u[i], 2);
        } else {
            d = HalfHw(u[8] >> 16);
#pragma unroll
            for (int i = 0; i < 8; ++i) c[i] = u[9 + i];
        }
    }
};

template <int B>
struct BlockOf<MLK_Q4_0, B> {
    float d;
    uint32_t c[4];
    __device__ inline explicit BlockOf(const uint32_t (&u)[9]) {
        if (B == 0) {
            d = HalfHw(u[0] & 0xFFFFu);
#pragma unroll
            for (int i = 0; i < 4; ++i) c[i] = __builtin_amdgcn_alignbyte(u[i + 1], u[i], 2);
        } else {
            d = HalfHw(u[4] >> 16);
#pragma unroll
            for (int i = 0; i < 4; ++i) c[i] = u[5 + i];
        }
    }
};

template <int B>
struct BlockOf<MLK_Q4_1, B> {
    float d, m;
    uint32_t c[4];
    __device__ inline explicit BlockOf(const uint32_t (&u)[10]) {
        const uint32_t dm = u[5 * B];
        d = HalfHw(dm & 0xFFFFu);
        m = HalfHw(dm >> 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) c[i] = u[5 * B + 1 + i];
    }
};

__device__ inline float SByte(uint32_t w, int j) {
    return static_cast<float>(static_cast<int32_t>(w << (24 - 8 * j)) >> 24);
}
__device__ inline float UByte(uint32_t w, int j) {
    return static_cast<float>((w >> (8 * j)) & 0xFFu);
}

// Adds block B of pair u, times the x block xb (32 inputs for each token),
// into acc[t].  xsum[t] = sum of the token's 32 inputs (Q4 formats).
template <int QT, int B, int R>
__device__ inline void BlockDot(const uint32_t (&u)[Pair<QT>::kWords], const float4 (&xb)[R][8],
                                const float (&xsum)[R], float (&acc)[R]) {
    const BlockOf<QT, B> blk(u);
    float s[R];
#pragma unroll
    for (int t = 0; t < R; ++t) s[t] = 0.0f;
    if constexpr (QT == MLK_Q8_0) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t c = blk.c[i];
            const float q0 = SByte(c, 0), q1 = SByte(c, 1), q2 = SByte(c, 2), q3 = SByte(c, 3);
#pragma unroll
            for (int t = 0; t < R; ++t) {
                s[t] = fmaf(q0, xb[t][i].x, s[t]);
                s[t] = fmaf(q1, xb[t][i].y, s[t]);
                s[t] = fmaf(q2, xb[t][i].z, s[t]);
                s[t] = fmaf(q3, xb[t][i].w, s[t]);
            }
        }
#pragma unroll
        for (int t = 0; t < R; ++t) acc[t] = fmaf(blk.d, s[t], acc[t]);
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo = blk.c[i] & 0x0F0F0F0Fu;
            const uint32_t hi = (blk.c[i] >> 4) & 0x0F0F0F0Fu;
            const float l0 = UByte(lo, 0), l1 = UByte(lo, 1), l2 = UByte(lo, 2), l3 = UByte(lo, 3);
            const float h0 = UByte(hi, 0), h1 = UByte(hi, 1), h2 = UByte(hi, 2), h3 = UByte(hi, 3);
#pragma unroll
            for (int t = 0; t < R; ++t) {
                s[t] = fmaf(l0, xb[t][i].x, s[t]);
                s[t] = fmaf(l1, xb[t][i].y, s[t]);
                s[t] = fmaf(l2, xb[t][i].z, s[t]);
                s[t] = fmaf(l3, xb[t][i].w, s[t]);
                s[t] = fmaf(h0, xb[t][i + 4].x, s[t]);
                s[t] = fmaf(h1, xb[t][i + 4].y, s[t]);
                s[t] = fmaf(h2, xb[t][i + 4].z, s[t]);
                s[t] = fmaf(h3, xb[t][i + 4].w, s[t]);
            }
        }
        if constexpr (QT == MLK_Q4_0) {
#pragma unroll
            for (int t = 0; t < R; ++t) acc[t] = fmaf(blk.d, fmaf(-8.0f, xsum[t], s[t]), acc[t]);
        } else {
#pragma unroll
            for (int t = 0; t < R; ++t) acc[t] = fmaf(blk.m, xsum[t], fmaf(blk.d, s[t], acc[t]));
        }
    }
}

// Loads the 32 inputs k0..k0+31 of each of R tokens (16-byte aligned rows);
// tokens past n_tok repeat the last valid one (their sums are discarded).
template <int R>
__device__ inline void LoadXBlock(const float* x, int64_t K, int n_tok, int64_t k0,
                                  float4 (&xb)[R][8], float (&xsum)[R], bool want_sum) {
#pragma unroll
    for (int t = 0; t < R; ++t) {
        const int tt = t < n_tok ? t : n_tok - 1;
        const float4* p = reinterpret_cast<const float4*>(x + tt * K + k0);
#pragma unroll
        for (int i = 0; i < 8; ++i) xb[t][i] = p[i];
        float sx = 0.0f;
        if (want_sum) {
#pragma unroll
            for (int i = 0; i < 8; ++i) sx += (xb[t][i].x + xb[t][i].y) + (xb[t][i].z + xb[t][i].w);
        }
        xsum[t] = sx;
    }
}

// Sums acc over the wave and writes y[t, row0 + r] (+ bias) for valid rows
// and tokens, one output per lane.
template <int R>
__device__ inline void StoreRows(float (&acc)[kRows][R], const float* bias, float* y, int64_t O,
                                 int64_t row0, int n_tok, int lane) {
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
#pragma unroll
        for (int t = 0; t < R; ++t) {
            const float v = WaveSumF(acc[r][t]);
            if (lane == r * R + t && t < n_tok && row0 + r < O) {
                y[t * O + row0 + r] = bias != nullptr ? v + bias[row0 + r] : v;
            }
        }
    }
}

template <int QT, int R>
__global__ __launch_bounds__(kThreads) void GemvQuantKernel(
    const float* __restrict__ x, const uint8_t* __restrict__ w, const float* __restrict__ bias,
    float* __restrict__ y, int64_t K, int64_t O, int64_t row_bytes, int n_tok) {
    const int lane = threadIdx.x % kWave;
    const int64_t row0 =
        (static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + threadIdx.x / kWave) * kRows;
    if (row0 >= O) return;  // wave-uniform
    const int64_t P = K / 64;
    const uint8_t* wr[kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
        wr[r] = w + (row0 + r < O ? row0 + r : O - 1) * row_bytes;
    }
    float acc[kRows][R];
#pragma unroll
    for (int r = 0; r < kRows; ++r)
#pragma unroll
        for (int t = 0; t < R; ++t) acc[r][t] = 0.0f;

    for (int64_t p = lane; p < P; p += kWave) {
        uint32_t u[kRows][Pair<QT>::kWords];
#pragma unroll
        for (int r = 0; r < kRows; ++r) LoadPair<QT>(wr[r] + p * Pair<QT>::kBytes, u[r]);
        float4 xb[R][8];
        float xsum[R];
        LoadXBlock<R>(x, K, n_tok, p * 64, xb, xsum, QT != MLK_Q8_0);
#pragma unroll
        for (int r = 0; r < kRows; ++r) BlockDot<QT, 0, R>(u[r], xb, xsum, acc[r]);
        LoadXBlock<R>(x, K, n_tok, p * 64 + 32, xb, xsum, QT != MLK_Q8_0);
#pragma unroll
        for (int r = 0; r < kRows; ++r) BlockDot<QT, 1, R>(u[r], xb, xsum, acc[r]);
    }
    StoreRows<R>(acc, bias, y, O, row0, n_tok, lane);
}

template <int R>
__global__ __launch_bounds__(kThreads) void GemvF32Kernel(
    const float* __restrict__ x, const float* __restrict__ w, const float* __restrict__ bias,
    float* __restrict__ y, int64_t K, int64_t O, int n_tok) {
    const int lane = threadIdx.x % kWave;
    const int64_t row0 =
        (static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + threadIdx.x / kWave) * kRows;
    if (row0 >= O) return;
    const int64_t C = K / 4;
    const float4* wr[kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
        wr[r] = reinterpret_cast<const float4*>(w + (row0 + r < O ? row0 + r : O - 1) * K);
    }
    const float4* xr[R];
#pragma unroll
    for (int t = 0; t < R; ++t) xr[t] = reinterpret_cast<const float4*>(x + (t < n_tok ? t : n_tok - 1) * K);
    float acc[kRows][R];
#pragma unroll
    for (int r = 0; r < kRows; ++r)
#pragma unroll
        for (int t = 0; t < R; ++t) acc[r][t] = 0.0f;
    for (int64_t c = lane; c < C; c += kWave) {
        float4 wv[kRows];
#pragma unroll
        for (int r = 0; r < kRows; ++r) wv[r] = LoadNT(wr[r] + c);
#pragma unroll
        for (int t = 0; t < R; ++t) {
            const float4 xv = xr[t][c];
#pragma unroll
            for (int r = 0; r < kRows; ++r) {
                float a = acc[r][t];
                a = fmaf(xv.x, wv[r].x, a);
                a = fmaf(xv.y, wv[r].y, a);
                a = fmaf(xv.z, wv[r].z, a);
                a = fmaf(xv.w, wv[r].w, a);
                acc[r][t] = a;
            }
        }
    }
    StoreRows<R>(acc, bias, y, O, row0, n_tok, lane);
}

// Any shape and alignment: one wave per weight row, every token, byte loads.
template <int QT>
__device__ inline float DecodeAny(const uint8_t* row, int64_t k) {
    const uint8_t* blk = row + (k / 32) * Fmt<QT>::kBytes;
    const int i = static_cast<int>(k % 32);
    const float d = HalfBits(static_cast<uint32_t>(blk[0]) | (static_cast<uint32_t>(blk[1]) << 8));
    if (QT == MLK_Q8_0) {
        return d * static_cast<float>(static_cast<int8_t>(blk[2 + i]));
    } else if (QT == MLK_Q4_0) {
        const uint32_t b = blk[2 + (i & 15)];
        return d * static_cast<float>(static_cast<int>(i < 16 ? (b & 15u) : (b >> 4)) - 8);
    } else {
        const float m = HalfBits(static_cast<uint32_t>(blk[2]) | (static_cast<uint32_t>(blk[3]) << 8));
        const uint32_t b = blk[4 + (i & 15)];
        return fmaf(d, static_cast<float>(i < 16 ? (b & 15u) : (b >> 4)), m);
    }
}

template <int QT>  // QT < 0: F32 weights
__global__ __launch_bounds__(kThreads) void GemvAnyKernel(
    const float* __restrict__ x, const void* __restrict__ w, const float* __restrict__ bias,
    float* __restrict__ y, int64_t K, int64_t O, int64_t row_bytes, int64_t T) {
    const int lane = threadIdx.x % kWave;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + threadIdx.x / kWave;
    if (row >= O) return;
    const uint8_t* wr = static_cast<const uint8_t*>(w) + row * row_bytes;
    for (int64_t t = 0; t < T; ++t) {
        float s = 0.0f;
        for (int64_t k = lane; k < K; k += kWave) {
            float wk;
            if constexpr (QT < 0) {
                wk = reinterpret_cast<const float*>(wr)[k];
            } else {
                wk = DecodeAny<QT>(wr, k);
            }
            s = fmaf(x[t * K + k], wk, s);
        }
        s = WaveSumF(s);
        if (lane == 0) y[t * O + row] = bias != nullptr ? s + bias[row] : s;
    }
}

// c = a @ b for a [m, k], b [k, n]: 16 x 16 output tiles, k staged through
// LDS in steps of 16 (the reference's Matmul is a test-surface op).
constexpr int kMmTile = 16;

__global__ __launch_bounds__(kMmTile* kMmTile) void MatmulKernel(const float* __restrict__ a,
                                                                 const float* __restrict__ b,
                                                                 float* __restrict__ c, int64_t M,
                                                                 int64_t Kd, int64_t N) {
    __shared__ float ta[kMmTile][kMmTile + 1];
    __shared__ float tb[kMmTile][kMmTile + 1];
    const int tx = threadIdx.x % kMmTile, ty = threadIdx.x / kMmTile;
    const int64_t row = static_cast<int64_t>(blockIdx.y) * kMmTile + ty;
    const int64_t col = static_cast<int64_t>(blockIdx.x) * kMmTile + tx;
    float s = 0.0f;
    for (int64_t k0 = 0; k0 < Kd; k0 += kMmTile) {
        ta[ty][tx] = (row < M && k0 + tx < Kd) ? a[row * Kd + k0 + tx] : 0.0f;
        tb[ty][tx] = (k0 + ty < Kd && col < N) ? b[(k0 + ty) * N + col] : 0.0f;
        __syncthreads();
#pragma unroll
        for (int i = 0; i < kMmTile; ++i) s = fmaf(ta[ty][i], tb[i][tx], s);
        __syncthreads();
    }
    if (row < M && col < N) c[row * N + col] = s;
}

mlk_status CheckLinear(const char* fn, const float* x, const void* w, float* y, int64_t T,
                       int64_t K, int64_t O) {
    if (x == nullptr || w == nullptr || y == nullptr) {
        return Fail(MLK_ERR_INVALID, "%s: x, weight and y must not be null", fn);
    }
    if (T <= 0 || K <= 0 || O <= 0) {
        return Fail(MLK_ERR_INVALID, "%s: dimensions must be positive (rows %lld, in %lld, out %lld)",
                    fn, static_cast<long long>(T), static_cast<long long>(K),
                    static_cast<long long>(O));
    }
    if (static_cast<const void*>(y) == static_cast<const void*>(x) ||
        static_cast<const void*>(y) == w) {
        return Fail(MLK_ERR_INVALID, "%s: y must not alias x or the weight", fn);
    }
    if (!Aligned(x, 4) || !Aligned(y, 4)) {
        return Fail(MLK_ERR_INVALID, "%s: x and y must be 4-byte aligned", fn);
    }
    return MLK_OK;
}

unsigned GemvGrid(int64_t O, int rows_per_wave) {
    return FullGrid(O, static_cast<int64_t>(kWavesPerBlock) * rows_per_wave);
}

template <int QT, int R>
void LaunchGemvQuant(const float* x, const uint8_t* w, const float* bias, float* y, int64_t K,
                     int64_t O, int64_t row_bytes, int n, hipStream_t s) {
    hipLaunchKernelGGL((GemvQuantKernel<QT, R>), dim3(GemvGrid(O, kRows)), dim3(kThreads), 0, s,
                       x, w, bias, y, K, O, row_bytes, n);
}

template <int QT>
void GemvQuantChunk(const float* x, const uint8_t* w, const float* bias, float* y, int64_t K,
                    int64_t O, int64_t row_bytes, int n, hipStream_t s) {
    if (n == 1) {
        LaunchGemvQuant<QT, 1>(x, w, bias, y, K, O, row_bytes, n, s);
    } else if (n == 2) {
        LaunchGemvQuant<QT, 2>(x, w, bias, y, K, O, row_bytes, n, s);
    } else {
        LaunchGemvQuant<QT, 4>(x, w, bias, y, K, O, row_bytes, n, s);
    }
}

}  // namespace
}  // namespace mlk

using namespace mlk;

extern "C" {

mlk_status mlk_linear_quant(int32_t quant_type, const float* x, const void* w_blocks,
                            const float* bias, float* y, int64_t rows, int64_t in_features,
                            int64_t out_features, void* stream) {
    if (quant_type < MLK_Q8_0 || quant_type > MLK_Q4_1) {
        return Fail(MLK_ERR_INVALID, "mlk_linear_quant: unknown quantization type %d", quant_type);
    }
    mlk_status st = CheckLinear("mlk_linear_quant", x, w_blocks, y, rows, in_features,
                                out_features);
    if (st != MLK_OK) return st;
    if (!Aligned(w_blocks, 2)) {
        return Fail(MLK_ERR_INVALID, "mlk_linear_quant: weight blocks must be 2-byte aligned");
    }
    const int64_t K = in_features, O = out_features;
    const int64_t row_bytes = ((K + 31) / 32) * BlockBytes(quant_type);
    const uint8_t* w = static_cast<const uint8_t*>(w_blocks);
    const hipStream_t s = AsStream(stream);
    const bool fast = K % 64 == 0 && Aligned(w_blocks, 4) && Aligned(x, 16);
    if (!fast) {
        const unsigned grid = FullGrid(O, kWavesPerBlock);
        switch (quant_type) {
            case MLK_Q8_0:
                hipLaunchKernelGGL(GemvAnyKernel<MLK_Q8_0>, dim3(grid), dim3(kThreads), 0, s, x, w,
                                   bias, y, K, O, row_bytes, rows);
                break;
            case MLK_Q4_0:
                hipLaunchKernelGGL(GemvAnyKernel<MLK_Q4_0>, dim3(grid), dim3(kThreads), 0, s, x, w,
                                   bias, y, K, O, row_bytes, rows);
                break;
            default:
                hipLaunchKernelGGL(GemvAnyKernel<MLK_Q4_1>, dim3(grid), dim3(kThreads), 0, s, x, w,
                                   bias, y, K, O, row_bytes, rows);
                break;
        }
        return CheckLaunch("GemvAnyKernel");
    }
    for (int64_t t0 = 0; t0 < rows; t0 += kMaxTok) {
        const int n = static_cast<int>(rows - t0 < kMaxTok ? rows - t0 : kMaxTok);
        const float* xt = x + t0 * K;
        float* yt = y + t0 * O;
        switch (quant_type) {
            case MLK_Q8_0: GemvQuantChunk<MLK_Q8_0>(xt, w, bias, yt, K, O, row_bytes, n, s); break;
            case MLK_Q4_0: GemvQuantChunk<MLK_Q4_0>(xt, w, bias, yt, K, O, row_bytes, n, s); break;
            default: GemvQuantChunk<MLK_Q4_1>(xt, w, bias, yt, K, O, row_bytes, n, s); break;
        }
        st = CheckLaunch("GemvQuantKernel");
        if (st != MLK_OK) return st;
    }
    return MLK_OK;
}

mlk_status mlk_linear_f32(const float* x, const float* w, const float* bias, float* y,
                          int64_t rows, int64_t in_features, int64_t out_features, void* stream) {
    mlk_status st = CheckLinear("mlk_linear_f32", x, w, y, rows, in_features, out_features);
    if (st != MLK_OK) return st;
    if (!Aligned(w, 4)) {
        return Fail(MLK_ERR_INVALID, "mlk_linear_f32: weight must be 4-byte aligned");
    }
    const int64_t K = in_features, O = out_features;
    const hipStream_t s = AsStream(stream);
    if (K % 4 != 0 || !Aligned(x, 16) || !Aligned(w, 16)) {
        hipLaunchKernelGGL(GemvAnyKernel<-1>, dim3(FullGrid(O, kWavesPerBlock)), dim3(kThreads), 0,
                           s, x, static_cast<const void*>(w), bias, y, K, O, K * 4, rows);
        return CheckLaunch("GemvAnyKernel");
    }
    for (int64_t t0 = 0; t0 < rows; t0 += kMaxTok) {
        const int n = static_cast<int>(rows - t0 < kMaxTok ? rows - t0 : kMaxTok);
        const float* xt = x + t0 * K;
        float* yt = y + t0 * O;
        const dim3 grid(GemvGrid(O, kRows));
        if (n == 1) {
            hipLaunchKernelGGL(GemvF32Kernel<1>, grid, dim3(kThreads), 0, s, xt, w, bias, yt, K, O, n);
        } else if (n == 2) {
            hipLaunchKernelGGL(GemvF32Kernel<2>, grid, dim3(kThreads), 0, s, xt, w, bias, yt, K, O, n);
        } else {
            hipLaunchKernelGGL(GemvF32Kernel<4>, grid, dim3(kThreads), 0, s, xt, w, bias, yt, K, O, n);
        }
        st = CheckLaunch("GemvF32Kernel");
        if (st != MLK_OK) return st;
    }
    return MLK_OK;
}

mlk_status mlk_matmul_f32(const float* a, const float* b, float* c, int64_t m, int64_t k,
                          int64_t n, void* stream) {
    if (a == nullptr || b == nullptr || c == nullptr) {
        return Fail(MLK_ERR_INVALID, "mlk_matmul_f32: pointers must not be null");
    }
    if (m <= 0 || k <= 0 || n <= 0) {
        return Fail(MLK_ERR_INVALID, "mlk_matmul_f32: dimensions must be positive");
    }
    if (c == a || c == b) {
        return Fail(MLK_ERR_INVALID, "mlk_matmul_f32: c must not alias a or b");
    }
    if ((n + kMmTile - 1) / kMmTile > 0x7FFFFFFF || (m + kMmTile - 1) / kMmTile > 65535) {
        return Fail(MLK_ERR_INVALID, "mlk_matmul_f32: matrix too large");
    }
    const dim3 grid(static_cast<unsigned>((n + kMmTile - 1) / kMmTile),
                    static_cast<unsigned>((m + kMmTile - 1) / kMmTile));
    hipLaunchKernelGGL(MatmulKernel, grid, dim3(kMmTile * kMmTile), 0, AsStream(stream), a, b, c,
                       m, k, n);
    return CheckLaunch("MatmulKernel");
}

}  // extern "C"
