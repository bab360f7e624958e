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
// once.  One token row of quantized weights with in_features % 64 == 0
// takes GemvStream (two-block pieces per lane, x in LDS, described at the
// kernel); other calls below 8 rows take GemvSplitK.  Layout of the work
// (GemvSplitK):
//   - a workgroup of four waves owns RW consecutive weight rows; the four
//     waves split K: wave w takes spans w, w + 4, w + 8, ... (two spans per
//     loop trip, so each lane has 2 * RW span loads in flight);
//   - a span is the part of K one wave covers in one step, with every lane
//     owning a contiguous slice, so that consecutive lanes read consecutive
//     bytes of the weight row and consecutive float4 of x:
//       Q8_0  8 blocks (256 inputs); lane: block lane/8, inputs 4*(lane%8)+0..3
//             (fp16 scale and the four code bytes as three aligned u16 loads)
//       Q4_0  16 blocks (512 inputs); lane: block lane/4, code bytes
//             4*(lane%4)+0..3, i.e. inputs 4j..4j+3 (low nibbles) and
//             16+4j..16+4j+3 (high nibbles), j = lane%4
//       Q4_1  as Q4_0, with d|m and the code bytes as aligned u32 loads
//       F32   256 inputs; lane: one float4 (non-temporal load)
//   - per slice, s = sum code * x, then the block scale is applied once
//     (Q8_0: d * s; Q4_0: d * (s - 8 * sum x); Q4_1: d * s + m * sum x, the
//     sum of x taken in the same order as s, so that a Q4_0 slice of all-8
//     codes folds to exactly zero);
//   - each lane ends with RW * R partial sums; a transpose-reduce over the
//     wave leaves one output per lane group, and the four waves' totals are
//     added in wave order through LDS (deterministic order).
// The first span of each wave is w, so the four waves of a workgroup read
// adjacent spans of the same rows at the same time.  Spans past the last
// block (in_features % 256 or % 512 != 0) are masked per lane.  Token rows
// come in launches of up to four; RW is 4 for outputs >= 4096 (x reused over
// more rows) and 2 below (more workgroups for the small K/V projections).
// Shapes outside that (in_features % 32 != 0, unaligned pointers) take a
// one-wave-per-row kernel with byte loads.
#include "mlk_quant.h"

namespace mlk {
namespace {

constexpr int kThreads = 256;
constexpr int kWavesPerBlock = kThreads / kWave;
constexpr int kMaxTok = 4;    // token rows per GEMV launch
constexpr int kGemmMinRows = 8;  // from here on, the matrix-core GEMM (mlk_gemm.hip)
constexpr int kF32 = -1;      // QT value of F32 weights

__device__ inline float WaveSumF(float v) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

__device__ inline float SByte(uint32_t w, int j) {
    return static_cast<float>(static_cast<int32_t>(w << (24 - 8 * j)) >> 24);
}
__device__ inline float UByte(uint32_t w, int j) {
    return static_cast<float>((w >> (8 * j)) & 0xFFu);
}

// w & 0x0F0F0F0F as one instruction the optimizer cannot see through.  In
// plain C++ the mask folds into every byte's extraction (a bit-field extract
// per nibble, then a convert); kept whole, each nibble converts straight
// from its byte (v_cvt_f32_ubyte0..3): 11 instead of 16 VALU ops per 8 codes.
__device__ inline uint32_t LowNibbles(uint32_t w) {
    uint32_t r;
    asm("v_and_b32 %0, 0x0f0f0f0f, %1" : "=v"(r) : "v"(w));
    return r;
}


// Zero (m == 0) or keep (m == ~0) the bits of four floats.  Masking with
// integer ANDs after unconditional loads keeps the compiler from turning a
// select of loaded values into a branch around each load (which serializes
// the loads of a span behind one another).
__device__ inline float4 MaskBits(float4 v, uint32_t m) {
    return make_float4(__uint_as_float(__float_as_uint(v.x) & m),
                       __uint_as_float(__float_as_uint(v.y) & m),
                       __uint_as_float(__float_as_uint(v.z) & m),
                       __uint_as_float(__float_as_uint(v.w) & m));
}

// One lane's slice of one span: Load reads it from a weight row (a masked
// lane, past the row's nb blocks / K inputs, reads block 0 and zeroes the
// bits with m), XOff locates the matching x.
template <int QT>
struct Span;

template <>
struct Span<MLK_Q8_0> {
    static constexpr int kElems = 256;
    static constexpr int kXs = 1;  // float4 of x per token per lane
    struct Raw {
        uint32_t d, c;
    };
    __device__ static bool Valid(int64_t s, int lane, int64_t nb) { return s * 8 + lane / 8 < nb; }
    __device__ static Raw Load(const uint8_t* row, int64_t s, int lane, bool ok, uint32_t m) {
        const uint16_t* b = reinterpret_cast<const uint16_t*>(row + (ok ? (s * 8 + lane / 8) * 34 : 0));
        const int j = lane % 8;
        Raw r;
        r.d = b[0] & m;
        r.c = (static_cast<uint32_t>(b[1 + 2 * j]) | (static_cast<uint32_t>(b[2 + 2 * j]) << 16)) & m;
        return r;
    }
    __device__ static int64_t XOff(int64_t s, int lane, int i) {
        (void)i;
        return s * 256 + 4 * lane;
    }
};

template <>
struct Span<MLK_Q4_0> {
    static constexpr int kElems = 512;
    static constexpr int kXs = 2;
    struct Raw {
        uint32_t d, c;
    };
    __device__ static bool Valid(int64_t s, int lane, int64_t nb) { return s * 16 + lane / 4 < nb; }
    __device__ static Raw Load(const uint8_t* row, int64_t s, int lane, bool ok, uint32_t m) {
        const uint16_t* b = reinterpret_cast<const uint16_t*>(row + (ok ? (s * 16 + lane / 4) * 18 : 0));
        const int j = lane % 4;
        Raw r;
        r.d = b[0] & m;
        r.c = (static_cast<uint32_t>(b[1 + 2 * j]) | (static_cast<uint32_t>(b[2 + 2 * j]) << 16)) & m;
        return r;
    }
    __device__ static int64_t XOff(int64_t s, int lane, int i) {
        return s * 512 + (lane / 4) * 32 + 4 * (lane % 4) + 16 * i;
    }
};

template <>
struct Span<MLK_Q4_1> {
    static constexpr int kElems = 512;
    static constexpr int kXs = 2;
    struct Raw {
        uint32_t d, c;  // d: fp16 d | fp16 m << 16
    };
    __device__ static bool Valid(int64_t s, int lane, int64_t nb) { return s * 16 + lane / 4 < nb; }
    __device__ static Raw Load(const uint8_t* row, int64_t s, int lane, bool ok, uint32_t m) {
        const uint32_t* b = reinterpret_cast<const uint32_t*>(row + (ok ? (s * 16 + lane / 4) * 20 : 0));
        Raw r;
        r.d = b[0] & m;
        r.c = b[1 + lane % 4] & m;
        return r;
    }
    __device__ static int64_t XOff(int64_t s, int lane, int i) {
        return s * 512 + (lane / 4) * 32 + 4 * (lane % 4) + 16 * i;
    }
};

template <>
struct Span<kF32> {
    static constexpr int kElems = 256;
    static constexpr int kXs = 1;
    struct Raw {
        float4 w;
    };
    // nb here is K / 4 (float4 per row)
    __device__ static bool Valid(int64_t s, int lane, int64_t nb) { return s * 64 + lane < nb; }
    __device__ static Raw Load(const uint8_t* row, int64_t s, int lane, bool ok, uint32_t m) {
        Raw r;
        r.w = MaskBits(LoadNT(reinterpret_cast<const float4*>(row) + (ok ? s * 64 + lane : 0)), m);
        return r;
    }
    __device__ static int64_t XOff(int64_t s, int lane, int i) {
        (void)i;
        return s * 256 + 4 * lane;
    }
};

// acc[t] += the lane's slice of one weight row times token t's x slice.
template <int QT, int R>
__device__ inline void SliceDot(const typename Span<QT>::Raw& raw,
                                const float4 (&xv)[R][Span<QT>::kXs], const float (&xs)[R],
                                float (&acc)[R]) {
    if constexpr (QT == kF32) {
#pragma unroll
        for (int t = 0; t < R; ++t) {
            float a = acc[t];
            a = fmaf(raw.w.x, xv[t][0].x, a);
            a = fmaf(raw.w.y, xv[t][0].y, a);
            a = fmaf(raw.w.z, xv[t][0].z, a);
            a = fmaf(raw.w.w, xv[t][0].w, a);
            acc[t] = a;
        }
    } else if constexpr (QT == MLK_Q8_0) {
        const float d = HalfHw(raw.d);
        const float q0 = SByte(raw.c, 0), q1 = SByte(raw.c, 1), q2 = SByte(raw.c, 2),
                    q3 = SByte(raw.c, 3);
#pragma unroll
        for (int t = 0; t < R; ++t) {
            float s = q0 * xv[t][0].x;
            s = fmaf(q1, xv[t][0].y, s);
            s = fmaf(q2, xv[t][0].z, s);
            s = fmaf(q3, xv[t][0].w, s);
            acc[t] = fmaf(d, s, acc[t]);
        }
    } else {
        const uint32_t lo = LowNibbles(raw.c);
        const uint32_t hi = LowNibbles(raw.c >> 4);
        const float l0 = UByte(lo, 0), l1 = UByte(lo, 1), l2 = UByte(lo, 2), l3 = UByte(lo, 3);
        const float h0 = UByte(hi, 0), h1 = UByte(hi, 1), h2 = UByte(hi, 2), h3 = UByte(hi, 3);
        const float d = HalfHw(raw.d & 0xFFFFu);
#pragma unroll
        for (int t = 0; t < R; ++t) {
            float s = l0 * xv[t][0].x;
            s = fmaf(l1, xv[t][0].y, s);
            s = fmaf(l2, xv[t][0].z, s);
            s = fmaf(l3, xv[t][0].w, s);
            s = fmaf(h0, xv[t][1].x, s);
            s = fmaf(h1, xv[t][1].y, s);
            s = fmaf(h2, xv[t][1].z, s);
            s = fmaf(h3, xv[t][1].w, s);
            if constexpr (QT == MLK_Q4_0) {
                acc[t] = fmaf(d, fmaf(-8.0f, xs[t], s), acc[t]);
            } else {
                const float m = HalfHw(raw.d >> 16);
                acc[t] = fmaf(m, xs[t], fmaf(d, s, acc[t]));
            }
        }
    }
}

// The lane's x slices of span s for R token rows (rows past n_tok repeat the
// last valid one; their sums are discarded), zero when the slice is masked.
// xs = sum of the slice in the order SliceDot sums the codes (Q4 formats).
template <int QT, int R>
__device__ inline void LoadX(const float* x, int64_t K, int n_tok, int64_t s, int lane, bool ok,
                             uint32_t m, float4 (&xv)[R][Span<QT>::kXs], float (&xs)[R]) {
#pragma unroll
    for (int t = 0; t < R; ++t) {
        const int tt = t < n_tok ? t : n_tok - 1;
#pragma unroll
        for (int i = 0; i < Span<QT>::kXs; ++i) {
            xv[t][i] = MaskBits(
                *reinterpret_cast<const float4*>(x + tt * K + (ok ? Span<QT>::XOff(s, lane, i) : 0)),
                m);
        }
        if constexpr (QT == MLK_Q4_0 || QT == MLK_Q4_1) {
            float a = xv[t][0].x;
            a += xv[t][0].y;
            a += xv[t][0].z;
            a += xv[t][0].w;
            a += xv[t][1].x;
            a += xv[t][1].y;
            a += xv[t][1].z;
            a += xv[t][1].w;
            xs[t] = a;
        } else {
            xs[t] = 0.0f;
        }
    }
}

// Sums N = 2^n values per lane over the wave.  Each step halves the values
// a lane holds: lanes whose bit o is clear keep the lower half and add the
// partner's lower half, the others the upper half; after log2(N) steps a
// lane holds one value, index ReduceIdx(lane), and a plain butterfly over
// the remaining lane bits completes it.  N - 1 + (6 - log2 N) shuffles
// instead of 6 * N.
template <int N>
__device__ inline float TransposeReduce(float (&v)[N], int lane) {
#pragma unroll
    for (int h = N / 2, o = kWave / 2; h >= 1; h /= 2, o /= 2) {
        const bool upper = (lane & o) != 0;
#pragma unroll
        for (int i = 0; i < h; ++i) {
            const float send = upper ? v[i] : v[i + h];
            const float keep = upper ? v[i + h] : v[i];
            v[i] = keep + __shfl_xor(send, o, kWave);
        }
    }
    float r = v[0];
    constexpr int steps = __builtin_ctz(N);
#pragma unroll
    for (int o = (kWave / 2) >> steps; o >= 1; o /= 2) r += __shfl_xor(r, o, kWave);
    return r;
}

template <int N>
__device__ inline int ReduceIdx(int lane) {
    int idx = 0;
    int o = kWave / 2;
#pragma unroll
    for (int h = N / 2; h >= 1; h /= 2, o /= 2) idx += (lane & o) ? h : 0;
    return idx;
}

// nb: blocks per weight row (quantized) or K / 4 (F32).  kTail: K is not a
// whole number of spans, so the last span is masked per lane (otherwise no
// lane is ever masked and the masks fold away).
template <int QT, int R, int RW, bool kTail>
__global__ __launch_bounds__(kThreads) void GemvSplitK(const float* __restrict__ x,
                                                       const uint8_t* __restrict__ w,
                                                       const float* __restrict__ bias,
                                                       float* __restrict__ y, int64_t K,
                                                       int64_t O, int64_t row_bytes, int64_t nb,
                                                       int n_tok) {
    using S = Span<QT>;
    constexpr int N = RW * R;
    static_assert(N <= kWave && (N & (N - 1)) == 0, "RW * R must be a power of two <= 64");
    __shared__ float red[kWavesPerBlock][N];
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int64_t row0 = static_cast<int64_t>(blockIdx.x) * RW;
    const uint8_t* wr[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) wr[r] = w + (row0 + r < O ? row0 + r : O - 1) * row_bytes;
    float acc[RW][R];
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
        for (int t = 0; t < R; ++t) acc[r][t] = 0.0f;
    const int64_t NS = (K + S::kElems - 1) / S::kElems;
    int64_t s = wave;
    for (; s + kWavesPerBlock < NS; s += 2 * kWavesPerBlock) {
        const int64_t s1 = s + kWavesPerBlock;
        const bool ok0 = !kTail || S::Valid(s, lane, nb), ok1 = !kTail || S::Valid(s1, lane, nb);
        const uint32_t m0 = ok0 ? ~0u : 0u, m1 = ok1 ? ~0u : 0u;
        typename S::Raw raw0[RW], raw1[RW];
#pragma unroll
        for (int r = 0; r < RW; ++r) raw0[r] = S::Load(wr[r], s, lane, ok0, m0);
#pragma unroll
        for (int r = 0; r < RW; ++r) raw1[r] = S::Load(wr[r], s1, lane, ok1, m1);
        float4 xv[R][S::kXs];
        float xs[R];
        LoadX<QT, R>(x, K, n_tok, s, lane, ok0, m0, xv, xs);
#pragma unroll
        for (int r = 0; r < RW; ++r) SliceDot<QT, R>(raw0[r], xv, xs, acc[r]);
        LoadX<QT, R>(x, K, n_tok, s1, lane, ok1, m1, xv, xs);
#pragma unroll
        for (int r = 0; r < RW; ++r) SliceDot<QT, R>(raw1[r], xv, xs, acc[r]);
    }
    if (s < NS) {
        const bool ok0 = !kTail || S::Valid(s, lane, nb);
        const uint32_t m0 = ok0 ? ~0u : 0u;
        typename S::Raw raw0[RW];
#pragma unroll
        for (int r = 0; r < RW; ++r) raw0[r] = S::Load(wr[r], s, lane, ok0, m0);
        float4 xv[R][S::kXs];
        float xs[R];
        LoadX<QT, R>(x, K, n_tok, s, lane, ok0, m0, xv, xs);
#pragma unroll
        for (int r = 0; r < RW; ++r) SliceDot<QT, R>(raw0[r], xv, xs, acc[r]);
    }
    float v[N];
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
        for (int t = 0; t < R; ++t) v[r * R + t] = acc[r][t];
    const float tot = TransposeReduce<N>(v, lane);
    if ((lane & (kWave / N - 1)) == 0) red[wave][ReduceIdx<N>(lane)] = tot;
    __syncthreads();
    if (threadIdx.x < N) {
        const int i = threadIdx.x;
        const float sum = ((red[0][i] + red[1][i]) + red[2][i]) + red[3][i];
        const int r = i / R, t = i % R;
        const int64_t row = row0 + r;
        if (t < n_tok && row < O) y[t * O + row] = bias != nullptr ? sum + bias[row] : sum;
    }
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

template <int QT>  // QT == kF32: F32 weights
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
            if constexpr (QT == kF32) {
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

// ------------------------------------------------------------ piece GEMV
// Quantized weights with in_features % 64 == 0 and 4-byte aligned blocks:
// a lane owns a piece -- two consecutive blocks of one weight row, 68 / 36 /
// 40 bytes (Q8_0 / Q4_0 / Q4_1), read with 4-byte aligned 16-byte loads --
// and the 64 lanes of a wave cover 4096 inputs of the row per pass, so a
// wave reads a 4096-wide row as one contiguous run.  The loads are plain,
// not non-temporal: a lane's 16-byte loads are 68 bytes apart, so each
// cache line is read by several of a piece's loads, and a non-temporal
// load, which does not keep the line in L1, fetches it again from L2 for
// each (measured about 1.5x slower).  A wave owns R rows; the R pieces at
// one position are decoded against the same x values.  Per block, the codes
// are summed against x and the scale applied once, as in GemvSplitK; the
// byte and nibble positions inside a piece are compile-time constants (one
// v_cvt_f32_i32 with a byte select and one FMA per Q8_0 weight).  The
// partial sums of the 64 lanes are added by one transpose-reduce.
typedef uint32_t u32x4a __attribute__((ext_vector_type(4), aligned(4)));

template <int QT>
struct Piece;
template <>
struct Piece<MLK_Q8_0> {
    static constexpr int kWords = 17;
};
template <>
struct Piece<MLK_Q4_0> {
    static constexpr int kWords = 9;
};
template <>
struct Piece<MLK_Q4_1> {
    static constexpr int kWords = 10;
};

template <int N>
__device__ inline void LoadWords(const uint8_t* p, uint32_t (&w)[N]) {
    const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
#pragma unroll
    for (int i = 0; i + 4 <= N; i += 4) {
        const u32x4a v = *reinterpret_cast<const u32x4a*>(q + i);
        w[i] = v.x;
        w[i + 1] = v.y;
        w[i + 2] = v.z;
        w[i + 3] = v.w;
    }
#pragma unroll
    for (int i = N / 4 * 4; i < N; ++i) w[i] = q[i];
}

// Byte `b` of a piece (static), as the word index and bit shift.
__device__ constexpr int WordOf(int b) { return b / 4; }
__device__ constexpr int ShiftOf(int b) { return 8 * (b % 4); }

// x[t][32 blk .. + 31] of the lane's 64 inputs (xp[t]) into registers.
template <int T>
__device__ inline void LoadBlockX(const float* const (&xp)[T], int blk, float (&xv)[T][32]) {
#pragma unroll
    for (int t = 0; t < T; ++t) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 v = *reinterpret_cast<const float4*>(xp[t] + 32 * blk + 4 * i);
            xv[t][4 * i] = v.x;
            xv[t][4 * i + 1] = v.y;
            xv[t][4 * i + 2] = v.z;
            xv[t][4 * i + 3] = v.w;
        }
    }
}

// acc[r][t] += block `blk` of the R pieces times xv[t] (that block's x).
template <int QT, int R, int T, int blk>
__device__ inline void PieceBlock(const uint32_t (&wd)[R][Piece<QT>::kWords],
                                  const float (&xv)[T][32], float (&acc)[R][T]) {
    if constexpr (QT == MLK_Q8_0) {
        constexpr int base = 34 * blk;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float d = HalfHw(blk == 0 ? wd[r][0] & 0xFFFFu : wd[r][8] >> 16);
            float sv[T];
#pragma unroll
            for (int i = 0; i < 32; ++i) {
                const int b = base + 2 + i;
                const float c = SByte(wd[r][WordOf(b)], ShiftOf(b) / 8);
#pragma unroll
                for (int t = 0; t < T; ++t) sv[t] = i == 0 ? c * xv[t][0] : fmaf(c, xv[t][i], sv[t]);
            }
#pragma unroll
            for (int t = 0; t < T; ++t) acc[r][t] = fmaf(d, sv[t], acc[r][t]);
        }
    } else {
        // byte j of the block's codes holds element j (low nibble) and j + 16
        constexpr int base = QT == MLK_Q4_0 ? 18 * blk + 2 : 20 * blk + 4;
        float xs[T];
#pragma unroll
        for (int t = 0; t < T; ++t) {
            float a = xv[t][0];
            a += xv[t][16];
#pragma unroll
            for (int j = 1; j < 16; ++j) {
                a += xv[t][j];
                a += xv[t][16 + j];
            }
            xs[t] = a;
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float sv[T];
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int b = base + j;
                const uint32_t word = wd[r][WordOf(b)];
                const float lo = UByte(LowNibbles(word), ShiftOf(b) / 8);
                const float hi = UByte(LowNibbles(word >> 4), ShiftOf(b) / 8);
#pragma unroll
                for (int t = 0; t < T; ++t) {
                    sv[t] = j == 0 ? lo * xv[t][0] : fmaf(lo, xv[t][j], sv[t]);
                    sv[t] = fmaf(hi, xv[t][16 + j], sv[t]);
                }
            }
            if constexpr (QT == MLK_Q4_0) {
                const float d = HalfHw(blk == 0 ? wd[r][0] & 0xFFFFu : wd[r][4] >> 16);
#pragma unroll
                for (int t = 0; t < T; ++t) acc[r][t] = fmaf(d, fmaf(-8.0f, xs[t], sv[t]), acc[r][t]);
            } else {
                const uint32_t dm = wd[r][5 * blk];
                const float d = HalfHw(dm & 0xFFFFu), m = HalfHw(dm >> 16);
#pragma unroll
                for (int t = 0; t < T; ++t) acc[r][t] = fmaf(m, xs[t], fmaf(d, sv[t], acc[r][t]));
            }
        }
    }
}

// The streaming kernel: a workgroup of 8 waves requests its first weight
// step, then copies x into LDS (input k at k + 4 (k / 64): each lane's 64
// inputs start 68 floats after the previous lane's, so the 16-byte reads of
// 16 lanes fall on 64 distinct banks).  Each wave then walks `per_wave`
// consecutive groups of R rows, one step per (group, 4096-input pass), and
// issues the next step's weight loads before computing the current step, so
// the loads of one step overlap the decode and FMAs of the previous one.
// Without that every wave loads, waits, then computes (measured: 8B layer,
// Q8_0, 88 -> 68 us).  Loading two steps ahead measured slower than one.
// Lanes past the row's last piece (K % 4096 != 0, kTail) read piece 0 with
// their weight words masked to zero.
constexpr int kStreamThreads = 512;
constexpr int kStreamDepth = 1;  // steps loaded ahead of the one computed
// (the kernel asks for 4 waves per SIMD, at most 128 VGPRs: two 8-wave
// workgroups per CU)
constexpr int kStreamWaves = kStreamThreads / kWave;

__host__ __device__ inline int64_t XPad(int64_t k) { return k + 4 * (k / 64); }

__device__ inline const StreamSeg& SegAt(const StreamArgs& a, int s) {
    return s == 0 ? a.seg[0] : (s == 1 ? a.seg[1] : a.seg[2]);
}

struct StreamStep {
    int seg;
    int64_t row0;
    int pass;
    // The passes of a group in order, then: (plain, add) the next R rows,
    // moving to the next segment at the end of one; (SwiGLU) the same rows of
    // the up segment, then the next R rows of the gate segment.
    template <int MODE>
    __device__ void Advance(const StreamArgs& a, int passes, int rows) {
        if (++pass < passes) return;
        pass = 0;
        if constexpr (MODE == kStreamSwiGlu) {
            if (seg == 0) {
                seg = 1;
                return;
            }
            seg = 0;
            row0 += rows;
            return;
        }
        row0 += rows;
        if (row0 >= SegAt(a, seg).rows && seg + 1 < a.n_seg) {
            ++seg;
            row0 = 0;
        }
    }
};

// `live` false: a prefetch past the wave's last step, which every lane
// points at the first piece of the first matrix (one cache line, never used).
template <int QT, int R, bool kTail>
__device__ inline void StreamLoad(const StreamArgs& a, const StreamStep& st, int64_t row_bytes,
                                  int lane, int64_t pieces, bool live,
                                  uint32_t (&wd)[R][Piece<QT>::kWords]) {
    constexpr int PB = 4 * Piece<QT>::kWords;
    const StreamSeg& sg = SegAt(a, st.seg);
    const int64_t piece = static_cast<int64_t>(st.pass) * kWave + lane;
    const bool ok = !kTail || piece < pieces;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int64_t row = st.row0 + r < sg.rows ? st.row0 + r : sg.rows - 1;
        LoadWords(live ? sg.w + row * row_bytes + (ok ? piece : 0) * PB : a.seg[0].w, wd[r]);
    }
    if constexpr (kTail) {
        const uint32_t m = ok ? ~0u : 0u;
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int i = 0; i < Piece<QT>::kWords; ++i) wd[r][i] &= m;
    }
}

template <int QT, int R, bool kTail>
__device__ inline void StreamCompute(const uint32_t (&wd)[R][Piece<QT>::kWords],
                                     const float* xs, int pass, int lane, int64_t pieces,
                                     float (&acc)[R][1]) {
    const int64_t piece = static_cast<int64_t>(pass) * kWave + lane;
    const bool ok = !kTail || piece < pieces;
    const float* const xp[1] = {xs + (ok ? XPad(64 * piece) : 0)};
    float xv[1][32];
    LoadBlockX(xp, 0, xv);
    PieceBlock<QT, R, 1, 0>(wd, xv, acc);
    LoadBlockX(xp, 1, xv);
    PieceBlock<QT, R, 1, 1>(wd, xv, acc);
}

// The R rows' sums over the wave, then the epilogue.  SwiGLU: the gate
// segment's sums stay in `gate` (the lanes that will write each row hold
// it) until the up segment's step for the same rows.  q/k/v RoPE: with one
// row per step an even q or k row waits in `gate` for its odd partner (a
// wave's run starts at an even group, so the pair is its next step); with
// two, the pair is the step's two rows, exchanged between the wave halves.
template <int R, int MODE>
__device__ inline void StreamFinish(float (&acc)[R][1], const StreamArgs& a, const StreamStep& st,
                                    int lane, float& gate, int32_t pos, const double2* rope_cs) {
    float v[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        v[r] = acc[r][0];
        acc[r][0] = 0.0f;
    }
    const float tot = TransposeReduce<R>(v, lane);
    const StreamSeg& sg = SegAt(a, st.seg);
    const int64_t row = st.row0 + ReduceIdx<R>(lane);
    const float val = row < sg.rows && sg.bias != nullptr ? tot + sg.bias[row] : tot;
    if constexpr (MODE == kStreamSwiGlu) {
        if (st.seg == 0) {
            gate = val;
            return;
        }
    }
    if constexpr (MODE == kStreamQkvRope) {
        static_assert(R == 1 || R == 2, "pairs are one step of two rows or two steps of one");
        const bool writer = (lane & (kWave / R - 1)) == 0;
        const bool cache_ok = pos >= 0 && pos < a.rope.max_seq;
        if (st.seg == 2) {
            if (writer && cache_ok) sg.y[pos * a.rope.kv_stride + row] = val;
            return;
        }
        float x0, x1;
        if constexpr (R == 1) {
            if ((row & 1) == 0) {
                gate = val;
                return;
            }
            x0 = gate;
            x1 = val;
        } else {
            const float other = __shfl_xor(val, kWave / 2, kWave);
            x0 = (row & 1) ? other : val;
            x1 = (row & 1) ? val : other;
        }
        float r0 = x0, r1 = x1;
        if (pos >= 0) {
            const double2 cs = rope_cs[static_cast<int>(row % a.rope.head_dim) / 2];
            RopeRotate(x0, x1, cs.x, cs.y, &r0, &r1);
        }
        if (!writer || (st.seg == 1 && !cache_ok)) return;
        float* y = st.seg == 1 ? sg.y + pos * a.rope.kv_stride : sg.y;
        if constexpr (R == 1) {
            y[row - 1] = r0;
            y[row] = r1;
        } else {
            y[row] = (row & 1) ? r1 : r0;
        }
        return;
    }
    if ((lane & (kWave / R - 1)) != 0 || row >= sg.rows) return;
    if constexpr (MODE == kStreamSwiGlu) {
        sg.y[row] = SwiGluF(gate, val);
    } else if constexpr (MODE == kStreamAdd) {
        sg.y[row] = sg.res[row] + val;
    } else {
        sg.y[row] = val;
    }
}

// The RMSNorm of residual row x (+ delta) into xs (StreamNorm): the
// separate norm kernel's threads are emulated here, virtual thread vt =
// tid + 512 j of its 64 * waves (waves 8 or 16), each summing the squares
// of its float4s vt, vt + 64 * waves (vpt of them, at most 2) in order, in
// float64; each virtual wave's sum by the same butterfly, then the wave
// sums in order; each float4 then scaled as that kernel scales it.  Load()
// issues every load (x, delta, the norm weight); Finish() waits for them,
// reduces (one barrier) and writes xs, so a caller can issue loads of its
// own in between.  VPT: float4s per norm thread held (n.vpt <= VPT).
constexpr int kNormVpt = 2;  // float4s per norm thread the staging handles

template <int VPT = kNormVpt>
struct NormStager {
    static constexpr int NJ = 1024 / kStreamThreads;  // virtual threads per thread, at most
    float4 r[NJ][VPT], w[NJ][VPT], d[NJ][VPT];
    bool ok[NJ][VPT];

    __device__ int64_t Index(const StreamNorm& n, int j, int v) const {
        return threadIdx.x + j * kStreamThreads + static_cast<int64_t>(v) * (kWave * n.waves);
    }

    // Every load is issued (lanes past the row read its first float4, and
    // without a delta x stands in for it), so no branch joins after a load
    // and the caller's own loads issued next are not waited for early.
    __device__ void Load(const StreamNorm& n, const float* x, int64_t K) {
        const int nv = kWave * n.waves;
        const float4* xs4 = reinterpret_cast<const float4*>(x);
        const float4* ws4 = reinterpret_cast<const float4*>(n.weight);
        const float4* ds4 = reinterpret_cast<const float4*>(n.delta != nullptr ? n.delta : x);
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
#pragma unroll
            for (int v = 0; v < VPT; ++v) {
                const int64_t i = Index(n, j, v);
                ok[j][v] = j * kStreamThreads < nv && v < n.vpt && i < K / 4;
                const int64_t ic = ok[j][v] ? i : 0;
                r[j][v] = xs4[ic];
                w[j][v] = ws4[ic];
                d[j][v] = ds4[ic];
            }
        }
    }

    __device__ void Finish(const StreamNorm& n, int64_t K, float* xs, double* wsum) {
#pragma clang fp contract(off)
        const int nv = kWave * n.waves;
        const int lane = threadIdx.x % kWave, rw = threadIdx.x / kWave;
        const bool writer = blockIdx.x == 0 && n.res_out != nullptr;
        if (n.delta != nullptr) {
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
#pragma unroll
                for (int v = 0; v < VPT; ++v) {
                    r[j][v].x += d[j][v].x;
                    r[j][v].y += d[j][v].y;
                    r[j][v].z += d[j][v].z;
                    r[j][v].w += d[j][v].w;
                }
            }
        }
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            if (j * kStreamThreads >= nv) break;
            double ss = 0.0;
#pragma unroll
            for (int v = 0; v < VPT; ++v) {
                if (ok[j][v]) {
                    if (writer) reinterpret_cast<float4*>(n.res_out)[Index(n, j, v)] = r[j][v];
                    const double a = r[j][v].x, b = r[j][v].y, c = r[j][v].z, e = r[j][v].w;
                    ss += a * a;
                    ss += b * b;
                    ss += c * c;
                    ss += e * e;
                }
            }
            ss = WaveSum(ss);
            if (lane == 0) wsum[rw + j * kStreamWaves] = ss;
        }
        __syncthreads();
        double total = 0.0;
        for (int k = 0; k < n.waves; ++k) total += wsum[k];
        const double scale =
            1.0 / sqrt(total / static_cast<double>(K) + static_cast<double>(n.eps));
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
#pragma unroll
            for (int v = 0; v < VPT; ++v) {
                if (ok[j][v]) {
                    const float4 a = r[j][v], b = w[j][v];
                    float4 o;
                    o.x = static_cast<float>(static_cast<double>(a.x) * static_cast<double>(b.x) * scale);
                    o.y = static_cast<float>(static_cast<double>(a.y) * static_cast<double>(b.y) * scale);
                    o.z = static_cast<float>(static_cast<double>(a.z) * static_cast<double>(b.z) * scale);
                    o.w = static_cast<float>(static_cast<double>(a.w) * static_cast<double>(b.w) * scale);
                    *reinterpret_cast<float4*>(xs + XPad(4 * Index(n, j, v))) = o;
                }
            }
        }
    }
};

template <int VPT = kNormVpt>
__device__ void StageNorm(const StreamNorm& n, const float* x, int64_t K, float* xs,
                          double* wsum) {
    NormStager<VPT> st;
    st.Load(n, x, K);
    st.Finish(n, K, xs, wsum);
}

// x and the weights are not __restrict__: loads through restrict-qualified
// read-only pointers are marked invariant, and the compiler then sinks the
// first steps' weight loads past the barrier to their first use.
template <int QT, int R, bool kTail, int MODE>
__global__ __launch_bounds__(kStreamThreads, 4) void GemvStream(const float* x, StreamArgs a,
                                                             int64_t K, int64_t row_bytes,
                                                             int64_t groups, int per_wave) {
    extern __shared__ __align__(16) float xs[];
    const int lane = threadIdx.x % kWave;
    // wave-uniform (scalar) loop bounds, so the step loop needs no exec masks
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / kWave));
    const int64_t g_first = (static_cast<int64_t>(blockIdx.x) * kStreamWaves + wave) * per_wave;
    // a wave past the last group loads group 0 and leaves after the barrier
    const int64_t g0 = g_first < groups ? g_first : 0;
    const int64_t pieces = K / 64;
    const int passes = static_cast<int>((pieces + kWave - 1) / kWave);
    const int per_group = MODE == kStreamSwiGlu ? 2 * passes : passes;
    const int64_t n_steps = ((g0 + per_wave < groups ? g0 + per_wave : groups) - g0) * per_group;
    // the first group's segment and row
    StreamStep first{0, 0, 0};
    if constexpr (MODE == kStreamSwiGlu) {
        first.row0 = g0 * R;
    } else {
        int64_t g = g0;
        while (first.seg + 1 < a.n_seg && g >= SegAt(a, first.seg).groups) {
            g -= SegAt(a, first.seg).groups;
            ++first.seg;
        }
        first.row0 = g * R;
    }
    float acc[R][1];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r][0] = 0.0f;
    float gate = 0.0f;
    // the token's position (q/k/v RoPE): a uniform load, requested first
    int32_t pos = 0;
    if constexpr (MODE == kStreamQkvRope) {
        pos = a.rope.positions != nullptr ? a.rope.positions[0] : a.rope.pos0;
    }
    // Steps in order (StreamStep::Advance).  D + 1 register buffers: step
    // st + D is loaded while step st is computed.  `ld` is the next step to
    // load, `cur` the one computed.  The prefetches are unconditional (past
    // the last step they read one shared line): a load issued on one path
    // only makes the compiler wait for every outstanding load before the next
    // step's arithmetic.
    constexpr int D = kStreamDepth;
    uint32_t wbuf[D + 1][R][Piece<QT>::kWords];
    StreamStep ld = first, cur = first;
    // the first D steps are requested before x is copied to LDS, so the copy
    // and the barrier overlap their latency
    int64_t next = 0;  // the next step to load
#pragma unroll
    for (int b = 0; b < D; ++b) {
        StreamLoad<QT, R, kTail>(a, ld, row_bytes, lane, pieces, next < n_steps, wbuf[b]);
        ld.Advance<MODE>(a, passes, R);
        ++next;
    }
    __builtin_amdgcn_sched_barrier(0);
    if (a.norm.weight != nullptr) {  // x's RMSNorm (the same thread stages and scales each float4)
        __shared__ double wsum[16];
        StageNorm(a.norm, x, K, xs, wsum);
    } else {
        for (int64_t i = threadIdx.x; i < K / 4; i += kStreamThreads) {
            *reinterpret_cast<float4*>(xs + XPad(4 * i)) = reinterpret_cast<const float4*>(x)[i];
        }
    }
    // q/k/v RoPE: the (cos, sin) of every pair index of a head, after x in
    // LDS, computed once per workgroup while the first steps load (the
    // epilogue then only rotates, so the float64 sin and cos take no
    // registers in the step loop)
    double2* rope_cs = reinterpret_cast<double2*>(xs + XPad(K));
    if constexpr (MODE == kStreamQkvRope) {
        if (pos >= 0) {
            for (int i = threadIdx.x; i < a.rope.head_dim / 2; i += kStreamThreads) {
                double cs, sn;
                RopeCosSin(pos, a.rope.freq.inv[i], &cs, &sn);
                rope_cs[i] = make_double2(cs, sn);
            }
        }
        if (blockIdx.x == 0 && threadIdx.x == 0 && (pos < 0 || pos >= a.rope.max_seq)) {
            RaiseFlag(a.rope.err, 1);
        }
    }
    __syncthreads();
    if (g_first >= groups) return;
    for (int64_t st = 0; st < n_steps; st += D + 1) {
#pragma unroll
        for (int b = 0; b <= D; ++b) {
            StreamLoad<QT, R, kTail>(a, ld, row_bytes, lane, pieces, next < n_steps,
                                     wbuf[(b + D) % (D + 1)]);
            ld.Advance<MODE>(a, passes, R);
            ++next;
            __builtin_amdgcn_sched_barrier(0);
            if (st + b < n_steps) {
                StreamCompute<QT, R, kTail>(wbuf[b], xs, cur.pass, lane, pieces, acc);
                if (cur.pass == passes - 1) StreamFinish<R, MODE>(acc, a, cur, lane, gate, pos, rope_cs);
                cur.Advance<MODE>(a, passes, R);
            }
        }
    }
}

// ------------------------------------------------ one token, planar weights
// One token row over Q8_0 / Q4_0 weights in the planar layout
// (mlk_quant_to_planar), with GemvStream's modes and epilogues (StreamArgs):
//   - a workgroup owns one or two 16-row tiles (SwiGLU: the gate and the up
//     tile of the same rows, waves [0, nwm) on gate and [nwm, 2 nwm) on up);
//     its waves split each tile's K into 256-input chunks, ncw consecutive
//     chunks per wave;
//   - a chunk is 4 KB (Q8_0) or 2 KB (Q4_0) of codes, each load 1 KB
//     contiguous per wave, plus 16 bytes of scales per lane (its row's 8
//     blocks); lane l = 16 g + r takes row r and inputs 8g .. 8g + 7 of every
//     block: per block s = sum code * x in input order, then acc += d * s,
//     blocks in order;
//   - a chunk's acc is summed over the lane groups, (g0 + g1) + (g2 + g3),
//     into LDS, and a row's total adds the chunks in a fixed order: four
//     running sums over chunks c = q (mod 4), c ascending, then (s0 + s1) +
//     (s2 + s3).  The sums depend on K alone, not on how many waves a launch
//     uses, so the fused launches (norm staged, q/k/v with RoPE, gate/up with
//     SwiGLU) give the plain launch's sums bit for bit;
//   - each thread requests its float4s of x (or of its RMSNorm's operands)
//     first, then its wave's first two chunks, then stages x: loads complete
//     in order, so the staging waits for x alone while the chunks are in
//     flight; from there each wave loads the next chunk while it computes
//     one.
// Every load is 16-byte aligned and contiguous across the wave, unlike the
// block layout's 34- / 18-byte blocks; q/k/v RoPE's (cos, sin) are computed
// by the finishing wave's lanes for their own rows while the loads are in
// flight.
constexpr int kRowPlanarMaxWaves = 16;

template <int QT>
constexpr int PlanarLoads() { return QT == MLK_Q8_0 ? 4 : 2; }

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int QT>
struct PlanarChunk {
    u32x4 c[PlanarLoads<QT>()];
    u32x4 s;
};

__device__ inline float HalfOf(uint32_t w, int hi) {
    return static_cast<float>(
        __builtin_bit_cast(_Float16, static_cast<uint16_t>(hi ? w >> 16 : w & 0xFFFFu)));
}

__device__ inline float I8Of(uint32_t w, int byte) {
    return static_cast<float>(static_cast<int8_t>(w >> (8 * byte)));
}

__device__ inline float4 XsAt(const float* p) { return *reinterpret_cast<const float4*>(p); }

// codes: the tile's first chunk + 16 * lane; scales: the tile's scales of
// row r (16 bytes a chunk)
template <int QT>
__device__ inline void LoadPlanarChunk(const uint8_t* codes, const uint8_t* scales, int c,
                                       PlanarChunk<QT>& b) {
    constexpr int L = PlanarLoads<QT>();
    const u32x4* cp = reinterpret_cast<const u32x4*>(codes + static_cast<int64_t>(c) * L * 1024);
#pragma unroll
    for (int i = 0; i < L; ++i) b.c[i] = __builtin_nontemporal_load(cp + 64 * i);
    b.s = __builtin_nontemporal_load(
        reinterpret_cast<const u32x4*>(scales + static_cast<int64_t>(c) * 256));
}

// The lane's part of one chunk, from xc = xs + XPad(256 * chunk) + 8 g
// (= xs + 272 * chunk + 8 g): a 256-input chunk starts 64-aligned, so input
// 32 b + 8 g + e of it sits at xc + 32 b + 4 (b / 2) + e, an immediate
// offset per block.  Q4_0: each code word spreads into two words of
// sign-extended bytes holding 16 * the code's value (low nibbles shifted
// up, high nibbles in place), converted one instruction a byte as Q8_0's
// are; the chunk's sums then carry a factor 16, exact in binary floating
// point, taken out once at the end, so the result is that of the values
// themselves bit for bit.
template <int QT>
__device__ inline float PlanarChunkDot(const PlanarChunk<QT>& b, const float* xc) {
    float acc = 0.0f;
    if constexpr (QT == MLK_Q8_0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {  // block pair i: blocks 2i, 2i + 1 of the chunk
            const float* q = xc + 68 * i;
            const float4 a0 = XsAt(q), a1 = XsAt(q + 4);
            const float4 b0 = XsAt(q + 32), b1 = XsAt(q + 36);
            const u32x4 c = b.c[i];
            float s0 = I8Of(c.x, 0) * a0.x;
            s0 = fmaf(I8Of(c.x, 1), a0.y, s0);
            s0 = fmaf(I8Of(c.x, 2), a0.z, s0);
            s0 = fmaf(I8Of(c.x, 3), a0.w, s0);
            s0 = fmaf(I8Of(c.y, 0), a1.x, s0);
            s0 = fmaf(I8Of(c.y, 1), a1.y, s0);
            s0 = fmaf(I8Of(c.y, 2), a1.z, s0);
            s0 = fmaf(I8Of(c.y, 3), a1.w, s0);
            float s1 = I8Of(c.z, 0) * b0.x;
            s1 = fmaf(I8Of(c.z, 1), b0.y, s1);
            s1 = fmaf(I8Of(c.z, 2), b0.z, s1);
            s1 = fmaf(I8Of(c.z, 3), b0.w, s1);
            s1 = fmaf(I8Of(c.w, 0), b1.x, s1);
            s1 = fmaf(I8Of(c.w, 1), b1.y, s1);
            s1 = fmaf(I8Of(c.w, 2), b1.z, s1);
            s1 = fmaf(I8Of(c.w, 3), b1.w, s1);
            const uint32_t d = b.s[i];
            acc = fmaf(HalfOf(d, 0), s0, acc);
            acc = fmaf(HalfOf(d, 1), s1, acc);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 2; ++i) {  // blocks 4i .. 4i + 3 of the chunk
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int blk = 4 * i + j;
                const float* q = xc + 32 * blk + 4 * (blk / 2);
                const float4 a0 = XsAt(q), a1 = XsAt(q + 4);
                const uint32_t w = b.c[i][j];  // byte e: input e (low nibble), e + 4 (high)
                const uint32_t lo = (w << 4) & 0xF0F0F0F0u, hi = w & 0xF0F0F0F0u;
                float s = I8Of(lo, 0) * a0.x;
                s = fmaf(I8Of(lo, 1), a0.y, s);
                s = fmaf(I8Of(lo, 2), a0.z, s);
                s = fmaf(I8Of(lo, 3), a0.w, s);
                s = fmaf(I8Of(hi, 0), a1.x, s);
                s = fmaf(I8Of(hi, 1), a1.y, s);
                s = fmaf(I8Of(hi, 2), a1.z, s);
                s = fmaf(I8Of(hi, 3), a1.w, s);
                acc = fmaf(HalfOf(b.s[2 * i + j / 2], j & 1), s, acc);
            }
        }
        acc *= 0.0625f;
    }
    return acc;
}

// Dynamic LDS: x (XPad(K) floats, 16-byte aligned), then the chunk sums
// [tiles of the workgroup][matrices][K / 256][16].  A wave's work is the
// flat sequence of steps s = (tile s / ncw of the workgroup, chunk c_lo +
// s % ncw), two chunks in registers: while one is computed the other is
// loading.  A prefetch past the last step (one step, or an odd count) reads
// one line per load (the matrix's first bytes, the same for every lane), so
// every weight load is issued unconditionally and each step waits only for
// its own chunk.
template <int QT, int MODE, int NVPT, int NB>
__global__ __launch_bounds__(kRowPlanarMaxWaves* kWave) void GemvRowPlanar(
    const float* x, StreamArgs a, int64_t K, int nwm, int ncw, int tpw) {
    extern __shared__ __align__(16) float xs[];
    constexpr int L = PlanarLoads<QT>();
    constexpr int kMats = MODE == kStreamSwiGlu ? 2 : 1;
    constexpr int64_t kChunkBytes = L * 1024;
    const int nch = static_cast<int>(K / 256);
    float* part = xs + (XPad(K) + 3) / 4 * 4;
    const int lane = threadIdx.x % kWave, g = lane / 16, r = lane % 16;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / kWave));
    // the workgroup's segment and first tile, the matrix this wave reads
    int seg = 0, mat = 0, w_in = wave;
    int64_t tile0 = static_cast<int64_t>(blockIdx.x) * tpw;
    if constexpr (MODE == kStreamSwiGlu) {
        mat = wave >= nwm ? 1 : 0;
        w_in = wave - mat * nwm;
    } else {
        while (seg + 1 < a.n_seg && tile0 >= SegAt(a, seg).groups) {
            tile0 -= SegAt(a, seg).groups;
            ++seg;
        }
    }
    const StreamSeg& ls = SegAt(a, MODE == kStreamSwiGlu ? mat : seg);
    const int ntile = static_cast<int>(ls.groups - tile0 < tpw ? ls.groups - tile0 : tpw);
    const int c_lo = w_in * ncw;
    const int n_w = nch - c_lo < ncw ? nch - c_lo : ncw;  // <= 0: an idle wave
    const int steps = ntile * ncw;
    const int lg = 31 - __builtin_clz(ncw);  // ncw is a power of two
    const uint8_t* scale0 = ls.w + ls.groups * nch * kChunkBytes + 16 * r;
    auto load = [&](int st, PlanarChunk<QT>& b) {
        const uint8_t* cp = ls.w;
        const uint8_t* sp = ls.w;
        if (st < steps) {
            const int j = st & (ncw - 1);
            const int64_t q = (tile0 + (st >> lg)) * nch + (c_lo + j < nch ? c_lo + j : nch - 1);
            cp += q * kChunkBytes + 16 * lane;
            sp = scale0 + q * 256;
        }
        LoadPlanarChunk<QT>(cp, sp, 0, b);
    };
    // the norm's operands first (x itself, without a norm, after the
    // chunks: its loop would wait for every load before it either way)
    // q/k/v RoPE (one tile a workgroup): the token's position and, in the
    // finishing wave, each lane's inverse frequency, requested before the
    // weights (loads complete in order, so a wait for them later would
    // also wait for every chunk requested before)
    int32_t pos = 0;
    double inv = 0.0;
    const bool rope_rows = MODE == kStreamQkvRope && wave == 0 && seg < 2;
    if constexpr (MODE == kStreamQkvRope) {
        // every lane loads (no branch joins after a load), through a global
        // pointer (a generic one would make a flat load, which every later
        // wait must cover); without positions the weights stand in
        typedef const int32_t __attribute__((address_space(1)))* GlobalI32;
        const int32_t* pp = a.rope.positions != nullptr
                                ? a.rope.positions : reinterpret_cast<const int32_t*>(ls.w);
        const int32_t p0 = *(GlobalI32)pp;
        pos = a.rope.positions != nullptr ? p0 : a.rope.pos0;
        inv = a.rope.freq.inv[static_cast<int>((tile0 * 16 + r) % a.rope.head_dim) / 2];
    }
    NormStager<(NVPT > 0 ? NVPT : 1)> ns;
    // no norm: x's float4s tid + i * threads, i < 4 (named, not an array,
    // which the compiler would keep in scratch memory)
    float4 xq0, xq1, xq2, xq3;
    const int64_t k4 = K / 4;
    auto x_at = [&](int i) {  // unconditional (past x: its last float4)
        const int64_t e = threadIdx.x + static_cast<int64_t>(i) * blockDim.x;
        return reinterpret_cast<const float4*>(x)[e < k4 ? e : k4 - 1];
    };
    if constexpr (NVPT > 0) {
        ns.Load(a.norm, x, K);
    } else {
        xq0 = x_at(0);
        xq1 = x_at(1);
        xq2 = x_at(2);
        xq3 = x_at(3);
    }
    PlanarChunk<QT> b[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) load(i, b[i]);
    __builtin_amdgcn_sched_barrier(0);
    // the (cos, sin) of each finishing lane's row, while the chunks load
    double rc = 1.0, rs = 0.0;
    if constexpr (MODE == kStreamQkvRope) {
        if (rope_rows && pos >= 0) RopeCosSin(pos, inv, &rc, &rs);
        if (blockIdx.x == 0 && threadIdx.x == 0 && (pos < 0 || pos >= a.rope.max_seq)) {
            RaiseFlag(a.rope.err, 1);
        }
    }
    if constexpr (NVPT > 0) {  // the launcher sets kStreamThreads threads, a.norm.vpt <= NVPT
        __shared__ double wsum[16];
        ns.Finish(a.norm, K, xs, wsum);
    } else {
        auto put = [&](int i, const float4& v) {
            const int64_t e = threadIdx.x + static_cast<int64_t>(i) * blockDim.x;
            if (e < k4) *reinterpret_cast<float4*>(xs + XPad(4 * e)) = v;
        };
        put(0, xq0);
        put(1, xq1);
        put(2, xq2);
        put(3, xq3);
        // x past four float4s a thread (K beyond 16 * threads)
        for (int64_t e = threadIdx.x + 4 * static_cast<int64_t>(blockDim.x); e < k4;
             e += blockDim.x) {
            *reinterpret_cast<float4*>(xs + XPad(4 * e)) = reinterpret_cast<const float4*>(x)[e];
        }
    }
    __syncthreads();
    auto compute = [&](const PlanarChunk<QT>& b, int st) {
        const int j = st & (ncw - 1);
        if (j >= n_w) return;
        const int c = c_lo + j;
        float v = PlanarChunkDot<QT>(b, xs + 272 * c + 8 * g);
        v += __shfl_xor(v, 16);
        v += __shfl_xor(v, 32);
        if (g == 0) part[(((st >> lg) * kMats + mat) * nch + c) * 16 + r] = v;
    };
    // b[i] holds step st + i; each computed buffer takes the step NB ahead,
    // and the last NB steps take no further loads (a load still in flight
    // would hold up the barrier below)
    int st = 0;
    for (; st + NB < steps; st += NB) {
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            compute(b[i], st + i);
            load(st + i + NB, b[i]);
        }
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        if (st + i < steps) compute(b[i], st + i);
    }
    __syncthreads();
    if (wave >= ntile) return;  // wave t finishes tile t
    const int64_t tile = tile0 + wave;
    auto total = [&](int m) {
        const float* p = part + (wave * kMats + m) * nch * 16 + r;
        float v[16];  // chunks g, g + 4, ... (at most 64 chunks fit the LDS)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int c = g + 4 * i;
            v[i] = c < nch ? p[c * 16] : 0.0f;
        }
        float t = v[0];
#pragma unroll
        for (int i = 1; i < 16; ++i) t += v[i];
        t += __shfl_xor(t, 16);
        t += __shfl_xor(t, 32);
        return t;
    };
    const int64_t row = tile * 16 + r;
    if constexpr (MODE == kStreamSwiGlu) {
        const float tg = total(0), tu = total(1);
        const StreamSeg& gs = a.seg[0];
        const StreamSeg& us = a.seg[1];
        if (g != 0 || row >= us.rows) return;
        const float gv = gs.bias != nullptr ? tg + gs.bias[row] : tg;
        const float uv = us.bias != nullptr ? tu + us.bias[row] : tu;
        us.y[row] = SwiGluF(gv, uv);
        return;
    }
    const float tot = total(0);
    const StreamSeg& sg = SegAt(a, seg);
    const bool valid = row < sg.rows;
    const float val = valid && sg.bias != nullptr ? tot + sg.bias[row] : tot;
    if constexpr (MODE == kStreamQkvRope) {
        const bool cache_ok = pos >= 0 && pos < a.rope.max_seq;
        if (seg == 2) {
            if (g == 0 && valid && cache_ok) sg.y[pos * a.rope.kv_stride + row] = val;
            return;
        }
        const float other = __shfl_xor(val, 1);
        const float x0 = (r & 1) ? other : val, x1 = (r & 1) ? val : other;
        float r0 = x0, r1 = x1;
        if (pos >= 0) RopeRotate(x0, x1, rc, rs, &r0, &r1);
        if (g != 0 || !valid || (seg == 1 && !cache_ok)) return;
        float* y = seg == 1 ? sg.y + pos * a.rope.kv_stride : sg.y;
        y[row] = (r & 1) ? r1 : r0;
        return;
    }
    if (g != 0 || !valid) return;
    if constexpr (MODE == kStreamAdd) {
        sg.y[row] = sg.res[row] + val;
    } else {
        sg.y[row] = val;
    }
}

// The shape of a one-token planar launch: waves per matrix (nwm), chunks
// per wave (ncw) and tiles per workgroup (tpw).  With a staged norm the
// workgroup is kStreamThreads threads (StageNorm's shape), else the fewest
// chunks per wave (2, 4 or 8; 1 only for K = 256: a wave with one chunk
// has nothing to overlap its load with) that keep the waves within 8 a
// workgroup,
// or within kRowPlanarMaxWaves when there are fewer than two tiles per
// compute unit (the kernel holds 76 registers, so a compute unit runs 24
// waves: three 8-wave workgroups, or one of 16; few tiles need the larger
// workgroups to fill it).  Workgroups take two tiles (one segment, or
// SwiGLU's pairs) when that still leaves a workgroup per compute unit,
// halving the copies of x (and of its norm) staged.  False: K has more
// chunks than the waves cover.
struct RowPlanarPlan {
    int nwm = 0, ncw = 0, tpw = 1;
};

bool RowPlanarShape(int64_t K, int mode, bool norm, int64_t tiles, RowPlanarPlan* p) {
    const int64_t nch = K / 256;
    const int mats = mode == kStreamSwiGlu ? 2 : 1;
    const int wg = norm ? kStreamWaves
                        : (tiles < 2 * ComputeUnits() ? kRowPlanarMaxWaves : kStreamWaves);
    const int most = wg / mats;
    for (const int c : {1, 2, 4, 8}) {
        const int64_t w = (nch + c - 1) / c;
        if (w <= most && (c > 1 || nch == 1 || norm)) {
            p->nwm = norm ? most : static_cast<int>(w);
            p->ncw = c;
            return true;
        }
    }
    return false;
}

size_t RowPlanarLds(int64_t K, int mode, int tpw) {
    const int mats = mode == kStreamSwiGlu ? 2 : 1;
    return static_cast<size_t>((XPad(K) + 3) / 4 * 4 + tpw * mats * (K / 256) * 16) * 4;
}

constexpr size_t kRowPlanarLdsMax = 64 * 1024 - 16 * sizeof(double);  // StageNorm's sums

template <int QT, int MODE, int NB>
void LaunchRowPlanarNb(unsigned grid, int threads, size_t lds, hipStream_t s, const float* x,
                       const StreamArgs& a, int64_t K, const RowPlanarPlan& p) {
    if (a.norm.weight == nullptr) {
        hipLaunchKernelGGL((GemvRowPlanar<QT, MODE, 0, NB>), dim3(grid), dim3(threads), lds, s, x,
                           a, K, p.nwm, p.ncw, p.tpw);
    } else if (a.norm.vpt == 1) {
        hipLaunchKernelGGL((GemvRowPlanar<QT, MODE, 1, NB>), dim3(grid), dim3(threads), lds, s, x,
                           a, K, p.nwm, p.ncw, p.tpw);
    } else {
        hipLaunchKernelGGL((GemvRowPlanar<QT, MODE, 2, NB>), dim3(grid), dim3(threads), lds, s, x,
                           a, K, p.nwm, p.ncw, p.tpw);
    }
}

// Two chunks in flight per wave.  Four (16 KB of Q8_0 weights requested per
// wave) measured slower on the 8B decode layer (Q8_0 77.4 -> 80.6 us): the
// extra registers cost a wave per SIMD, and the weights streamed no faster.
template <int QT, int MODE>
void LaunchRowPlanar(unsigned grid, int threads, size_t lds, hipStream_t s, const float* x,
                     const StreamArgs& a, int64_t K, const RowPlanarPlan& p) {
    LaunchRowPlanarNb<QT, MODE, 2>(grid, threads, lds, s, x, a, K, p);
}

template <int QT>
void LaunchRowPlanarMode(int mode, unsigned grid, int threads, size_t lds, hipStream_t s,
                         const float* x, const StreamArgs& a, int64_t K, const RowPlanarPlan& p) {
    switch (mode) {
        case kStreamAdd: LaunchRowPlanar<QT, kStreamAdd>(grid, threads, lds, s, x, a, K, p); break;
        case kStreamSwiGlu: LaunchRowPlanar<QT, kStreamSwiGlu>(grid, threads, lds, s, x, a, K, p); break;
        case kStreamQkvRope: LaunchRowPlanar<QT, kStreamQkvRope>(grid, threads, lds, s, x, a, K, p); break;
        default: LaunchRowPlanar<QT, kStreamPlain>(grid, threads, lds, s, x, a, K, p); break;
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
    if (O > (int64_t{1} << 30)) {
        return Fail(MLK_ERR_INVALID, "%s: out_features %lld exceeds 2^30", fn,
                    static_cast<long long>(O));
    }
    return MLK_OK;
}

// Token rows in launches of up to kMaxTok; RW weight rows per workgroup.
template <int QT, int RW, bool kTail>
mlk_status GemvRows(const float* x, const uint8_t* w, const float* bias, float* y, int64_t K,
                    int64_t O, int64_t row_bytes, int64_t nb, int64_t rows, hipStream_t s) {
    const dim3 grid(static_cast<unsigned>((O + RW - 1) / RW));
    for (int64_t t0 = 0; t0 < rows; t0 += kMaxTok) {
        const int n = static_cast<int>(rows - t0 < kMaxTok ? rows - t0 : kMaxTok);
        const float* xt = x + t0 * K;
        float* yt = y + t0 * O;
        if (n == 1) {
            hipLaunchKernelGGL((GemvSplitK<QT, 1, RW, kTail>), grid, dim3(kThreads), 0, s, xt, w,
                               bias, yt, K, O, row_bytes, nb, n);
        } else if (n == 2) {
            hipLaunchKernelGGL((GemvSplitK<QT, 2, RW, kTail>), grid, dim3(kThreads), 0, s, xt, w,
                               bias, yt, K, O, row_bytes, nb, n);
        } else {
            hipLaunchKernelGGL((GemvSplitK<QT, 4, RW, kTail>), grid, dim3(kThreads), 0, s, xt, w,
                               bias, yt, K, O, row_bytes, nb, n);
        }
        const mlk_status st = CheckLaunch("GemvSplitK");
        if (st != MLK_OK) return st;
    }
    return MLK_OK;
}

// One token row (the decode step) with in_features % 64 == 0, 4-byte
// aligned blocks and x small enough for LDS; two or more rows take
// GemvSplitK, whose registers hold several rows' x.  Each wave gets enough
// row groups for about four waves per SIMD over the whole GPU.
// Rows per wave: two for the Q4 formats (x read from LDS once per two rows);
// one for Q8_0, whose double-buffered pieces would otherwise take 68
// registers and leave one 8-wave workgroup per CU.
template <int QT>
constexpr int StreamRows() { return QT == MLK_Q8_0 ? 1 : 2; }

template <int QT, int R, int MODE>
void LaunchStreamT(dim3 grid, size_t lds, hipStream_t s, const float* x, const StreamArgs& a,
                   int64_t K, int64_t row_bytes, int64_t groups, int per_wave) {
    if (K % 4096 != 0) {
        hipLaunchKernelGGL((GemvStream<QT, R, true, MODE>), grid, dim3(kStreamThreads), lds, s, x,
                           a, K, row_bytes, groups, per_wave);
    } else {
        hipLaunchKernelGGL((GemvStream<QT, R, false, MODE>), grid, dim3(kStreamThreads), lds, s, x,
                           a, K, row_bytes, groups, per_wave);
    }
}

template <int QT>
mlk_status StreamLaunch(const float* x, StreamArgs a, int mode, int64_t K, int64_t row_bytes,
                        hipStream_t s) {
    constexpr int R = StreamRows<QT>();
    int64_t groups = 0;
    for (int i = 0; i < a.n_seg; ++i) {
        a.seg[i].groups = (a.seg[i].rows + R - 1) / R;
        groups += a.seg[i].groups;
    }
    if (mode == kStreamSwiGlu) groups = a.seg[0].groups;
    const int64_t want = static_cast<int64_t>(ComputeUnits()) * 16;
    int64_t per_wave = groups > want ? (groups + want - 1) / want : 1;
    // q/k/v RoPE with one row per group: runs of whole pairs (the segments'
    // group counts are even, so every run starts on an even row)
    if (mode == kStreamQkvRope && R == 1) per_wave += per_wave % 2;
    const int64_t waves = (groups + per_wave - 1) / per_wave;
    const dim3 grid(static_cast<unsigned>((waves + kStreamWaves - 1) / kStreamWaves));
    // x, then (q/k/v RoPE) a (cos, sin) pair per pair index of a head, 8-byte aligned
    size_t lds = static_cast<size_t>(XPad(K)) * 4;
    if (mode == kStreamQkvRope) lds = (lds + 15) / 16 * 16 + static_cast<size_t>(a.rope.head_dim / 2) * 16;
    const int pw = static_cast<int>(per_wave);
    switch (mode) {
        case kStreamAdd: LaunchStreamT<QT, R, kStreamAdd>(grid, lds, s, x, a, K, row_bytes, groups, pw); break;
        case kStreamSwiGlu: LaunchStreamT<QT, R, kStreamSwiGlu>(grid, lds, s, x, a, K, row_bytes, groups, pw); break;
        case kStreamQkvRope: LaunchStreamT<QT, R, kStreamQkvRope>(grid, lds, s, x, a, K, row_bytes, groups, pw); break;
        default: LaunchStreamT<QT, R, kStreamPlain>(grid, lds, s, x, a, K, row_bytes, groups, pw); break;
    }
    return CheckLaunch("GemvStream");
}

// RW = 4 reuses each x slice over more rows; below 4096 outputs, RW = 2
// gives the small projections (K/V: 1024 outputs) enough workgroups.
template <int QT>
mlk_status Gemv(const float* x, const uint8_t* w, const float* bias, float* y, int64_t K,
                int64_t O, int64_t row_bytes, int64_t nb, int64_t rows, hipStream_t s) {
    if (K % Span<QT>::kElems != 0) {
        return O >= 4096 ? GemvRows<QT, 4, true>(x, w, bias, y, K, O, row_bytes, nb, rows, s)
                         : GemvRows<QT, 2, true>(x, w, bias, y, K, O, row_bytes, nb, rows, s);
    }
    return O >= 4096 ? GemvRows<QT, 4, false>(x, w, bias, y, K, O, row_bytes, nb, rows, s)
                     : GemvRows<QT, 2, false>(x, w, bias, y, K, O, row_bytes, nb, rows, s);
}

}  // namespace

bool QkvRopeArgsOk(const StreamArgs& a) {
    const int64_t hd = a.rope.head_dim;
    return a.n_seg == 3 && hd > 0 && hd % 2 == 0 && hd <= 2 * kRopePairs &&
           a.seg[0].rows % hd == 0 &&
           a.seg[1].rows % hd == 0 && a.seg[2].rows % 2 == 0 &&
           a.rope.kv_stride >= a.seg[1].rows && a.rope.kv_stride >= a.seg[2].rows &&
           a.rope.max_seq > 0;
}

bool StreamFits(int64_t K) { return K % 64 == 0 && K > 0 && XPad(K) * 4 <= 64 * 1024; }

bool StreamRopeFits(int64_t K, int64_t head_dim) {
    return StreamFits(K) && head_dim > 0 && XPad(K) * 4 + head_dim / 2 * 16 <= 64 * 1024;
}

// no norm, or one StageNorm can stage (the norm kernel's 8 or 16 waves, at
// most kNormVpt float4s per thread covering K)
bool NormArgsOk(const StreamNorm& n, int64_t K) {
    return n.weight == nullptr ||
           ((n.waves == 8 || n.waves == 16) && n.vpt >= 1 && n.vpt <= kNormVpt &&
            K / 4 <= static_cast<int64_t>(n.vpt) * kWave * n.waves && Aligned(n.weight, 16) &&
            Aligned(n.delta, 16) && Aligned(n.res_out, 16) && n.eps > 0.0f);
}

mlk_status LinearRowStream(int qt, const float* x, int64_t K, const StreamArgs& a, int mode,
                           hipStream_t s) {
    if (qt < MLK_Q8_0 || qt > MLK_Q4_1 || !StreamFits(K) || !Aligned(x, 16) || a.n_seg < 1 ||
        a.n_seg > 3 || (mode == kStreamSwiGlu && (a.n_seg != 2 || a.seg[0].rows != a.seg[1].rows))) {
        return Fail(MLK_ERR_INVALID, "linear (one row): unsupported shape for the streaming kernel");
    }
    for (int i = 0; i < a.n_seg; ++i) {
        if (a.seg[i].w == nullptr || !Aligned(a.seg[i].w, 4) || a.seg[i].y == nullptr ||
            a.seg[i].rows <= 0 || (mode == kStreamAdd && a.seg[i].res == nullptr)) {
            return Fail(MLK_ERR_INVALID, "linear (one row): bad segment %d", i);
        }
    }
    if (mode == kStreamQkvRope && (!QkvRopeArgsOk(a) || !StreamRopeFits(K, a.rope.head_dim))) {
        return Fail(MLK_ERR_INVALID, "linear (one row): bad q/k/v RoPE segments");
    }
    if (!NormArgsOk(a.norm, K)) {
        return Fail(MLK_ERR_INVALID, "linear (one row): bad input RMSNorm");
    }
    const int64_t row_bytes = (K / 32) * BlockBytes(qt);
    switch (qt) {
        case MLK_Q8_0: return StreamLaunch<MLK_Q8_0>(x, a, mode, K, row_bytes, s);
        case MLK_Q4_0: return StreamLaunch<MLK_Q4_0>(x, a, mode, K, row_bytes, s);
        default: return StreamLaunch<MLK_Q4_1>(x, a, mode, K, row_bytes, s);
    }
}

bool RowPlanarApplies(int qt, int64_t K, int mode, bool norm) {
    RowPlanarPlan p;  // the 8-wave shape covers fewer chunks than the 16-wave one
    return (qt == MLK_Q8_0 || qt == MLK_Q4_0) && K > 0 && K % 256 == 0 &&
           RowPlanarLds(K, mode, 1) <= kRowPlanarLdsMax &&
           RowPlanarShape(K, mode, norm, int64_t{1} << 40, &p);
}

mlk_status LinearRowPlanar(int qt, const float* x, int64_t K, const StreamArgs& a, int mode,
                           hipStream_t s) {
    const bool norm = a.norm.weight != nullptr;
    if (!RowPlanarApplies(qt, K, mode, norm) || !Aligned(x, 16) || a.n_seg < 1 || a.n_seg > 3 ||
        a.planes != nullptr ||
        (mode == kStreamSwiGlu && (a.n_seg != 2 || a.seg[0].rows != a.seg[1].rows))) {
        return Fail(MLK_ERR_INVALID, "linear (one row, planar): unsupported shape");
    }
    StreamArgs b = a;
    int64_t tiles = 0;
    for (int i = 0; i < b.n_seg; ++i) {
        StreamSeg& g = b.seg[i];
        if (g.w == nullptr || !Aligned(g.w, 16) || g.y == nullptr || g.rows <= 0 ||
            (mode == kStreamAdd && g.res == nullptr)) {
            return Fail(MLK_ERR_INVALID, "linear (one row, planar): bad segment %d", i);
        }
        g.groups = (g.rows + 15) / 16;
        tiles += g.groups;
    }
    if (mode == kStreamSwiGlu) tiles = b.seg[0].groups;
    if (mode == kStreamQkvRope && !QkvRopeArgsOk(b)) {
        return Fail(MLK_ERR_INVALID, "linear (one row, planar): bad q/k/v RoPE segments");
    }
    if (!NormArgsOk(b.norm, K)) {
        return Fail(MLK_ERR_INVALID, "linear (one row, planar): bad input RMSNorm");
    }
    RowPlanarPlan p;
    RowPlanarShape(K, mode, norm, tiles, &p);
    const int waves = p.nwm * (mode == kStreamSwiGlu ? 2 : 1);
    if ((b.n_seg == 1 || mode == kStreamSwiGlu) && tiles >= 2 * ComputeUnits() &&
        waves >= 2 && RowPlanarLds(K, mode, 2) <= kRowPlanarLdsMax) {
        p.tpw = 2;
    }
    const int64_t grid = (tiles + p.tpw - 1) / p.tpw;
    if (grid > 0x7FFFFFFF) return Fail(MLK_ERR_INVALID, "linear (one row, planar): too many rows");
    const size_t lds = RowPlanarLds(K, mode, p.tpw);
    if (qt == MLK_Q8_0) {
        LaunchRowPlanarMode<MLK_Q8_0>(mode, static_cast<unsigned>(grid), waves * kWave, lds, s, x,
                                      b, K, p);
    } else {
        LaunchRowPlanarMode<MLK_Q4_0>(mode, static_cast<unsigned>(grid), waves * kWave, lds, s, x,
                                      b, K, p);
    }
    return CheckLaunch("GemvRowPlanar");
}

}  // namespace mlk

using namespace mlk;

extern "C" {

int64_t mlk_linear_workspace_bytes(int64_t rows, int64_t in_features, int64_t out_features) {
    if (rows < kGemmMinRows || rows <= 0 || in_features <= 0 || out_features <= 0) return 0;
    // the plans differ by weight type (the skinny kernel's K chunk): the
    // larger serves every type
    int64_t most = 0;
    for (const int wt : {kF32, static_cast<int>(MLK_Q8_0), static_cast<int>(MLK_Q4_0),
                         static_cast<int>(MLK_Q4_1)}) {
        const int64_t b = GemmWorkspaceBytes(wt, rows, in_features, out_features);
        if (b > most) most = b;
    }
    return most;
}

mlk_status mlk_linear_quant(int32_t quant_type, const float* x, const void* w_blocks,
                            const float* bias, float* y, int64_t rows, int64_t in_features,
                            int64_t out_features, void* workspace, size_t workspace_bytes,
                            void* stream) {
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
    const bool fast = K % 32 == 0 && Aligned(x, 16) &&
                      (quant_type != MLK_Q4_1 || Aligned(w_blocks, 4));
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
    if (rows >= kGemmMinRows) {
        return LaunchGemm(quant_type, x, w_blocks, bias, y, rows, K, O, row_bytes, workspace,
                          workspace_bytes, s);
    }
    if (rows == 1 && StreamFits(K) && Aligned(w_blocks, 4)) {
        StreamArgs a{};
        a.seg[0] = StreamSeg{w, bias, y, nullptr, O, 0};
        a.n_seg = 1;
        return LinearRowStream(quant_type, x, K, a, kStreamPlain, s);
    }
    const int64_t nb = K / 32;
    switch (quant_type) {
        case MLK_Q8_0: return Gemv<MLK_Q8_0>(x, w, bias, y, K, O, row_bytes, nb, rows, s);
        case MLK_Q4_0: return Gemv<MLK_Q4_0>(x, w, bias, y, K, O, row_bytes, nb, rows, s);
        default: return Gemv<MLK_Q4_1>(x, w, bias, y, K, O, row_bytes, nb, rows, s);
    }
}

mlk_status mlk_linear_f32(const float* x, const float* w, const float* bias, float* y,
                          int64_t rows, int64_t in_features, int64_t out_features,
                          void* workspace, size_t workspace_bytes, void* stream) {
    mlk_status st = CheckLinear("mlk_linear_f32", x, w, y, rows, in_features, out_features);
    if (st != MLK_OK) return st;
    if (!Aligned(w, 4)) {
        return Fail(MLK_ERR_INVALID, "mlk_linear_f32: weight must be 4-byte aligned");
    }
    const int64_t K = in_features, O = out_features;
    const hipStream_t s = AsStream(stream);
    if (K % 4 != 0 || !Aligned(x, 16) || !Aligned(w, 16)) {
        hipLaunchKernelGGL(GemvAnyKernel<kF32>, dim3(FullGrid(O, kWavesPerBlock)), dim3(kThreads), 0,
                           s, x, static_cast<const void*>(w), bias, y, K, O, K * 4, rows);
        return CheckLaunch("GemvAnyKernel");
    }
    if (rows >= kGemmMinRows) {
        return LaunchGemm(kF32, x, w, bias, y, rows, K, O, K * 4, workspace, workspace_bytes, s);
    }
    return Gemv<kF32>(x, reinterpret_cast<const uint8_t*>(w), bias, y, K, O, K * 4, K / 4, rows,
                      s);
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

int64_t mlk_quant_planar_bytes(int32_t quant_type, int64_t rows, int64_t cols) {
    return PlanarBytes(quant_type, rows, cols);
}

mlk_status mlk_quant_to_planar(int32_t quant_type, const void* blocks, int64_t rows,
                               int64_t cols, void* planar, void* stream) {
    if (PlanarBytes(quant_type, rows, cols) == 0) {
        return Fail(MLK_ERR_INVALID,
                    "mlk_quant_to_planar: no planar layout for type %d, %lld x %lld (Q8_0 or "
                    "Q4_0, cols a positive multiple of 256)",
                    quant_type, static_cast<long long>(rows), static_cast<long long>(cols));
    }
    if (blocks == nullptr || planar == nullptr) {
        return Fail(MLK_ERR_INVALID, "mlk_quant_to_planar: null pointer");
    }
    if (!Aligned(planar, 16)) {
        return Fail(MLK_ERR_INVALID, "mlk_quant_to_planar: the planar buffer must be 16-byte aligned");
    }
    return LaunchToPlanar(quant_type, blocks, rows, cols, planar, AsStream(stream));
}

int64_t mlk_linear_planar_workspace_bytes(int64_t rows, int64_t in_features,
                                          int64_t out_features) {
    if (rows <= 0 || in_features <= 0 || out_features <= 0 || in_features % 256 != 0) return 0;
    if (rows == 1 && RowPlanarApplies(MLK_Q8_0, in_features, kStreamPlain, false)) return 0;
    if (!PlanarApplies(MLK_Q8_0, rows, in_features)) {
        return GemmWorkspaceBytes(kWPlanarQ8, rows, in_features, out_features);
    }
    return PlanarWorkspaceBytes(rows, in_features, out_features, false);
}

mlk_status mlk_linear_planar(int32_t quant_type, const float* x, const void* w_planar,
                             const float* bias, float* y, int64_t rows, int64_t in_features,
                             int64_t out_features, void* workspace, size_t workspace_bytes,
                             void* stream) {
    if (quant_type != MLK_Q8_0 && quant_type != MLK_Q4_0) {
        return Fail(MLK_ERR_INVALID, "mlk_linear_planar: type %d has no planar layout",
                    quant_type);
    }
    mlk_status st = CheckLinear("mlk_linear_planar", x, w_planar, y, rows, in_features,
                                out_features);
    if (st != MLK_OK) return st;
    if (in_features % 256 != 0 || !Aligned(w_planar, 16) || !Aligned(x, 16)) {
        return Fail(MLK_ERR_INVALID,
                    "mlk_linear_planar: in_features must be a multiple of 256, the weights and x "
                    "16-byte aligned");
    }
    if (rows == 1 && RowPlanarApplies(quant_type, in_features, kStreamPlain, false)) {
        StreamArgs a{};
        a.seg[0] = StreamSeg{static_cast<const uint8_t*>(w_planar), bias, y, nullptr,
                             out_features, 0};
        a.n_seg = 1;
        return LinearRowPlanar(quant_type, x, in_features, a, kStreamPlain, AsStream(stream));
    }
    return LinearPlanar(quant_type, x, w_planar, bias, y, rows, in_features, out_features,
                        workspace, workspace_bytes, AsStream(stream));
}

}  // extern "C"
