// mlk_common.h -- shared host/device helpers for the gfx950 kernels.
//
// Every .hip file of libminilamma_hip.so includes this header.  It holds the
// thread-local error message behind mlk_last_error(), the launch-check
// helper, per-device properties used to size grids, and the wave64 / block
// reductions the row kernels share.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>

#include "minilamma_hip.h"

namespace mlk {

constexpr int kWave = 64;  // CDNA wavefront width

// ---------------------------------------------------------------- errors

// Records a printf-style message for mlk_last_error() and returns `status`.
mlk_status Fail(mlk_status status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Turns a HIP error into MLK_ERR_HIP with "<what>: <hip message>".
mlk_status FromHip(hipError_t err, const char* what);

// Checks the launch that was just issued.
inline mlk_status CheckLaunch(const char* kernel) {
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? MLK_OK : FromHip(err, kernel);
}

inline hipStream_t AsStream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool Aligned(const void* p, uintptr_t n) {
    return (reinterpret_cast<uintptr_t>(p) & (n - 1)) == 0;
}

// Compute units of the current device (cached per device id).
int ComputeUnits();

// Grid size for a grid-stride kernel: enough workgroups to cover `work`
// units of `per_block` each, capped at `waves_per_cu` resident workgroups
// per compute unit.
inline unsigned GridFor(int64_t work, int64_t per_block, int blocks_per_cu) {
    const int64_t need = (work + per_block - 1) / per_block;
    const int64_t cap = static_cast<int64_t>(ComputeUnits()) * blocks_per_cu;
    const int64_t g = need < cap ? need : cap;
    return static_cast<unsigned>(g < 1 ? 1 : g);
}

// Grid for a kernel that gives every workgroup its own chunk (no grid-stride
// reuse of workgroups); the kernels still loop, so a capped grid is correct.
inline unsigned FullGrid(int64_t work, int64_t per_block) {
    const int64_t need = (work + per_block - 1) / per_block;
    const int64_t cap = int64_t{1} << 30;
    return static_cast<unsigned>(need < 1 ? 1 : (need < cap ? need : cap));
}

// ------------------------------------------------------- streaming memory
// Non-temporal 16-byte loads and stores (global_load/store_dwordx4 ... nt):
// data that is touched once per kernel should not displace what the next
// op wants from L2 and the MALL.  On MI355X the hint is worth ~15% of
// streaming bandwidth for the read-read-write pattern of these ops.

typedef float F32x4 __attribute__((ext_vector_type(4)));
typedef float F32x2 __attribute__((ext_vector_type(2)));

__device__ inline float4 LoadNT(const float4* p) {
    const F32x4 v = __builtin_nontemporal_load(reinterpret_cast<const F32x4*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}

__device__ inline void StoreNT(float4* p, float4 v) {
    F32x4 t = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(t, reinterpret_cast<F32x4*>(p));
}

__device__ inline float2 LoadNT(const float2* p) {
    const F32x2 v = __builtin_nontemporal_load(reinterpret_cast<const F32x2*>(p));
    return make_float2(v.x, v.y);
}

__device__ inline void StoreNT(float2* p, float2 v) {
    F32x2 t = {v.x, v.y};
    __builtin_nontemporal_store(t, reinterpret_cast<F32x2*>(p));
}

__device__ inline float LoadNT(const float* p) { return __builtin_nontemporal_load(p); }
__device__ inline void StoreNT(float* p, float v) { __builtin_nontemporal_store(v, p); }

// ------------------------------------------------------------ reductions

// Sum over the 64 lanes of a wave; every lane receives the total.  The
// xor-butterfly gives each lane the same association order, so the result
// is identical on all lanes and from run to run.
__device__ inline double WaveSum(double v) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) {
        v += __shfl_xor(v, off, kWave);
    }
    return v;
}

__device__ inline float WaveMax(float v) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) {
        v = fmaxf(v, __shfl_xor(v, off, kWave));
    }
    return v;
}

// Block-wide sum for blocks of NW waves.  `scratch` holds NW doubles and must
// not be reused by the caller before the next __syncthreads().  Every thread
// returns the same value, summed in wave order.
template <int NW>
__device__ inline double BlockSum(double v, double* scratch) {
    v = WaveSum(v);
    const int wave = threadIdx.x / kWave;
    if ((threadIdx.x % kWave) == 0) {
        scratch[wave] = v;
    }
    __syncthreads();
    double total = 0.0;
#pragma unroll
    for (int i = 0; i < NW; ++i) {
        total += scratch[i];
    }
    return total;
}

template <int NW>
__device__ inline float BlockMax(float v, float* scratch) {
    v = WaveMax(v);
    const int wave = threadIdx.x / kWave;
    if ((threadIdx.x % kWave) == 0) {
        scratch[wave] = v;
    }
    __syncthreads();
    float m = scratch[0];
#pragma unroll
    for (int i = 1; i < NW; ++i) {
        m = fmaxf(m, scratch[i]);
    }
    return m;
}

// SwiGLU of one element: s = g * (1 / (1 + exp(-g))) rounded to float, then
// s * u (src/ops.cc:135-151), without contraction; shared by the element-wise
// kernel and the fused gate/up GEMV so both round alike.
__device__ inline float SwiGluF(float g, float u) {
#pragma clang fp contract(off)
    const float sig = 1.0f / (1.0f + expf(-g));
    const float s = g * sig;
    return s * u;
}

// sin and cos of a float64 angle a.  The angle is first reduced by whole
// turns: a / pi is formed as a double-double, with the product by 1/pi's
// leading double split exactly by an fma (Dekker's two-product) and the
// product by its trailing double added, then the nearest even integer n is
// subtracted exactly (|a / pi| < 2^52), which is Cody and Waite's additive
// reduction.  sincospi of the remainder, in [-1, 1], then equals sin / cos
// of a within a few float64 ulps for |a| < 2^31, the angles RoPE forms.
// Unlike a general sincos this keeps no large-argument (Payne-Hanek)
// reduction, whose registers would be allocated across the whole kernel.
__device__ inline void SinCosAngle(double a, double* s, double* c) {
    constexpr double kInvPiHi = 0x1.45f306dc9c883p-2;    // 1/pi rounded to float64
    constexpr double kInvPiLo = -0x1.6b01ec5417056p-56;  // 1/pi - kInvPiHi, rounded
    const double p = a * kInvPiHi;
    const double e = fma(a, kInvPiHi, -p) + a * kInvPiLo;
    const double n = 2.0 * rint(0.5 * p);
    sincospi((p - n) + e, s, c);
}

// RoPE's inverse frequencies theta^(-2i / head_dim), one per pair index i,
// evaluated on the host with the C library's pow exactly as the CPU Rope
// does (src/ops.cc:200-206), so every angle pos * inv[i] equals the
// reference's bit for bit; kernels take the table by value (kernel
// arguments), so no device memory or copy is involved.  head_dim up to
// 2 * kRopePairs.
constexpr int kRopePairs = 128;
struct RopeFreqs {
    double inv[kRopePairs];
};
// Fills the table for head_dim / 2 pairs (head_dim even, <= 2 * kRopePairs).
RopeFreqs MakeRopeFreqs(float theta, int head_dim);

// RoPE of one pair (x0, x1) of a head at position pos with inverse
// frequency inv_freq (src/ops.cc:177-224): angle = (double) pos * inv_freq,
// cos and sin in float64, each output rounded once to float.  The fused
// q/k/v epilogues use these; the RoPE kernels write the same expressions.
__device__ inline void RopeCosSin(int32_t pos, double inv_freq, double* c, double* s) {
    SinCosAngle(static_cast<double>(pos) * inv_freq, s, c);
}

__device__ inline void RopeRotate(float x0, float x1, double c, double s, float* r0, float* r1) {
#pragma clang fp contract(off)
    const double a0 = x0, a1 = x1;
    *r0 = static_cast<float>(a0 * c - a1 * s);
    *r1 = static_cast<float>(a0 * s + a1 * c);
}

// x for the planar bf16 linear layers (mlk_gemm.hip) as three bf16 planes:
// v = p[0] + p[1] + p[2] exactly, each p[i] exact in bf16 (p[0] = v with its
// low 16 bits cleared, p[1] the same of v - p[0], p[2] the rest, at most 8
// significant bits).  Inf and NaN go whole into p[0] (NaN as the quiet NaN,
// whose payload bit survives in bf16), so products with them are what fp32
// products would be.
__device__ inline void SplitBf(float v, float (&p)[3]) {
    if (!__builtin_isfinite(v)) {
        p[0] = v != v ? __builtin_nanf("") : v;
        p[1] = p[2] = 0.0f;
        return;
    }
    p[0] = __uint_as_float(__float_as_uint(v) & 0xFFFF0000u);
    const float r = v - p[0];  // exact: the low 16 bits of v's significand
    p[1] = __uint_as_float(__float_as_uint(r) & 0xFFFF0000u);
    p[2] = r - p[1];
}

// Two floats whose values are exact in bf16, as one dword of bf16 (a low).
__device__ inline uint32_t PackBf(float a, float b) {
    return __builtin_amdgcn_perm(__float_as_uint(b), __float_as_uint(a), 0x07060302u);
}

// Inputs k, k + 1 (k even) of token row t of a [T, K] x into its planes
// ([K / 32 blocks][3 pieces][T tokens][16 dwords], dword j of a block
// holding inputs 2j, 2j + 1).
__device__ inline void StorePlanes(uint32_t* planes, int64_t T, int64_t t, int64_t k, float v0,
                                   float v1) {
    float p0[3], p1[3];
    SplitBf(v0, p0);
    SplitBf(v1, p1);
    uint32_t* d = planes + ((k / 32) * 3 * T + t) * 16 + (k % 32) / 2;
#pragma unroll
    for (int p = 0; p < 3; ++p) d[p * T * 16] = PackBf(p0[p], p1[p]);
}

// Inputs k .. k + 3 (k a multiple of 4): two dwords of each plane, one
// 8-byte store per piece.
__device__ inline void StorePlanes4(uint32_t* planes, int64_t T, int64_t t, int64_t k, float v0,
                                    float v1, float v2, float v3) {
    float p0[3], p1[3], p2[3], p3[3];
    SplitBf(v0, p0);
    SplitBf(v1, p1);
    SplitBf(v2, p2);
    SplitBf(v3, p3);
    uint32_t* d = planes + ((k / 32) * 3 * T + t) * 16 + (k % 32) / 2;
#pragma unroll
    for (int p = 0; p < 3; ++p) {
        *reinterpret_cast<uint2*>(d + p * T * 16) = make_uint2(PackBf(p0[p], p1[p]),
                                                               PackBf(p2[p], p3[p]));
    }
}

// Input k alone: its three bf16 halves of the planes' dwords.
__device__ inline void StorePlanes1(uint32_t* planes, int64_t T, int64_t t, int64_t k, float v) {
    float p[3];
    SplitBf(v, p);
    uint16_t* d = reinterpret_cast<uint16_t*>(planes + ((k / 32) * 3 * T + t) * 16) + k % 32;
#pragma unroll
    for (int i = 0; i < 3; ++i) d[i * T * 32] = static_cast<uint16_t>(__float_as_uint(p[i]) >> 16);
}

// Raises a device-side error flag (the flag is only ever set, never read
// back here, so any nonzero store is enough).
__device__ inline void RaiseFlag(int32_t* err, int32_t code) {
    if (err != nullptr) {
        atomicOr(err, code);
    }
}

}  // namespace mlk
