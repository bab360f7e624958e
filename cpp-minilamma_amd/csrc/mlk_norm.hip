// mlk_norm.hip -- residual add fused with RMSNorm, and plain RMSNorm, over
// [n_rows, dim] fp32 rows.
//
// Semantics follow the CPU ops the reference checks its GPU path against:
// ForwardAdd (src/forward.cc:213-222) then RmsNorm (src/ops.cc:82-112):
//   r   = x + delta                          (fp32, written back in place)
//   ss  = sum((double) r_i^2)
//   y_i = (float)((double) r_i * (double) w_i * (1 / sqrt(ss / dim + eps)))
// The reference's device path (src/cuda_ops.cu:151-164, :335-355) used three
// launches, one float atomicAdd per element into a single address and a
// stream synchronize; here one workgroup owns one row, keeps it in
// registers between the reduction and the scaling, and reduces with wave64
// shuffles (plus one LDS exchange when a row spans several waves).  The float64
// arithmetic is free at this arithmetic intensity (the kernel is HBM bound)
// and makes y equal the CPU result except for the order of the sum.
//
// HBM bytes per row (fused): read x, delta (8*dim), write x', y (8*dim),
// all with non-temporal hints; w (4*dim) is shared by all rows and stays in
// L2 (normal loads).  One workgroup per row, one row per workgroup.
#include "mlk_common.h"
#include "mlk_quant.h"

#include <cmath>

namespace mlk {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;

// Vector path: dim % 4 == 0.  One workgroup owns one row and holds it in
// registers, VPT float4 per lane, with as many waves as the row needs up to
// 16 (1024 lanes: one float4 per lane at dim 4096).  Measured on MI355X at
// [4096, 4096]: 16 waves x 1 float4 beats 1 wave x 16 float4 by 25%, and
// non-temporal hints are worth another ~12%.
// kPlanes: y also goes to `planes`, split into the three bf16 planes the
// planar linear layers read (StorePlanes; dim % 32 == 0).  splits > 1 or
// dbias: delta is a linear layer's split-K partial sums ([splits][rows][dim],
// split_stride floats apart), added in split order, then dbias: the
// reduction SplitKReduce would do, fused here.
template <int kWaves, int VPT, bool kDelta, bool kWriteBack, bool kPlanes = false,
          bool kPartials = false>
__global__ __launch_bounds__(kWave * kWaves) void AddRmsNormVec(
    float* residual, const float* __restrict__ delta, const float* __restrict__ weight, float* y,
    int64_t n_rows, int64_t dim, float eps, uint32_t* planes, int splits, int64_t split_stride,
    const float* __restrict__ dbias) {
#pragma clang fp contract(off)
    constexpr int lanes = kWave * kWaves;
    __shared__ double partial[2][kWaves];
    const int tid = threadIdx.x;
    const int64_t dim4 = dim >> 2;
    const double ddim = static_cast<double>(dim);
    int parity = 0;
    // the norm weight is the same for every row: loaded once, before the
    // first row's reduction, so no row waits on it after its sum
    const float4* wr = reinterpret_cast<const float4*>(weight);
    float4 wv[VPT];
#pragma unroll
    for (int v = 0; v < VPT; ++v) {
        const int64_t i = tid + static_cast<int64_t>(v) * lanes;
        wv[v] = i < dim4 ? wr[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    for (int64_t row = blockIdx.x; row < n_rows; row += gridDim.x, parity ^= 1) {
        float4* xr = reinterpret_cast<float4*>(residual + row * dim);
        const float4* dr = reinterpret_cast<const float4*>(delta + (kDelta ? row * dim : 0));
        float4 r[VPT];
#pragma unroll
        for (int v = 0; v < VPT; ++v) {
            const int64_t i = tid + static_cast<int64_t>(v) * lanes;
            r[v] = i < dim4 ? LoadNT(xr + i) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        if (kDelta) {
#pragma unroll
            for (int v = 0; v < VPT; ++v) {
                const int64_t i = tid + static_cast<int64_t>(v) * lanes;
                if (i < dim4) {
                    float4 d = LoadNT(dr + i);
                    if (kPartials && splits > 1) {
                        // splits 1.. added in order; loads 8 at a time, indices
                        // past the last split reading the last one (not added)
                        for (int sp = 1; sp < splits; sp += 8) {
                            float4 t[8];
#pragma unroll
                            for (int j = 0; j < 8; ++j) {
                                const int64_t at = sp + j < splits ? sp + j : splits - 1;
                                t[j] = LoadNT(dr + at * (split_stride / 4) + i);
                            }
#pragma unroll
                            for (int j = 0; j < 8; ++j) {
                                if (sp + j < splits) {
                                    d.x += t[j].x;
                                    d.y += t[j].y;
                                    d.z += t[j].z;
                                    d.w += t[j].w;
                                }
                            }
                        }
                    }
                    if (kPartials && dbias != nullptr) {
                        const float4 b = reinterpret_cast<const float4*>(dbias)[i];
                        d.x += b.x;
                        d.y += b.y;
                        d.z += b.z;
                        d.w += b.w;
                    }
                    r[v].x += d.x;
                    r[v].y += d.y;
                    r[v].z += d.z;
                    r[v].w += d.w;
                }
            }
        }
        double ss = 0.0;
#pragma unroll
        for (int v = 0; v < VPT; ++v) {
            const int64_t i = tid + static_cast<int64_t>(v) * lanes;
            if (i < dim4) {
                if (kWriteBack) StoreNT(xr + i, r[v]);
                const double a = r[v].x, b = r[v].y, c = r[v].z, d = r[v].w;
                ss += a * a;
                ss += b * b;
                ss += c * c;
                ss += d * d;
            }
        }
        ss = kWaves > 1 ? BlockSum<kWaves>(ss, partial[parity]) : WaveSum(ss);
        const double scale = 1.0 / sqrt(ss / ddim + static_cast<double>(eps));
        float4* yr = reinterpret_cast<float4*>(y + row * dim);
#pragma unroll
        for (int v = 0; v < VPT; ++v) {
            const int64_t i = tid + static_cast<int64_t>(v) * lanes;
            if (i < dim4) {
                const float4 w = wv[v];
                float4 o;
                o.x = static_cast<float>(static_cast<double>(r[v].x) * static_cast<double>(w.x) * scale);
                o.y = static_cast<float>(static_cast<double>(r[v].y) * static_cast<double>(w.y) * scale);
                o.z = static_cast<float>(static_cast<double>(r[v].z) * static_cast<double>(w.z) * scale);
                o.w = static_cast<float>(static_cast<double>(r[v].w) * static_cast<double>(w.w) * scale);
                StoreNT(yr + i, o);
                if (kPlanes) StorePlanes4(planes, n_rows, row, 4 * i, o.x, o.y, o.z, o.w);
            }
        }
    }
}

// Any width: two passes over the row, the second re-reading the elements
// the same thread wrote in the first.
template <bool kDelta, bool kWriteBack>
__global__ __launch_bounds__(kThreads) void AddRmsNormAny(float* residual,
                                                          const float* __restrict__ delta,
                                                          const float* __restrict__ weight,
                                                          float* y, int64_t n_rows, int64_t dim,
                                                          float eps) {
#pragma clang fp contract(off)
    __shared__ double partial[2][kWaves];
    const double ddim = static_cast<double>(dim);
    int parity = 0;
    for (int64_t row = blockIdx.x; row < n_rows; row += gridDim.x, parity ^= 1) {
        float* xr = residual + row * dim;
        double ss = 0.0;
        for (int64_t i = threadIdx.x; i < dim; i += kThreads) {
            float r = xr[i];
            if (kDelta) r += delta[row * dim + i];
            if (kWriteBack) xr[i] = r;
            const double a = r;
            ss += a * a;
        }
        ss = BlockSum<kWaves>(ss, partial[parity]);
        const double scale = 1.0 / sqrt(ss / ddim + static_cast<double>(eps));
        for (int64_t i = threadIdx.x; i < dim; i += kThreads) {
            float r = xr[i];
            if (kDelta && !kWriteBack) r += delta[row * dim + i];
            y[row * dim + i] =
                static_cast<float>(static_cast<double>(r) * static_cast<double>(weight[i]) * scale);
        }
    }
}

// AddRmsNormVec's block for rows of dim floats: waves doubled up to 16
// while the row has more float4s than threads, then float4s per thread.
void NormShapeOf(int64_t dim, int* waves, int* vpt) {
    const int64_t dim4 = dim / 4;
    int w = 1;
    while (w < 16 && static_cast<int64_t>(w) * kWave < dim4) w *= 2;
    *waves = w;
    *vpt = static_cast<int>((dim4 + w * kWave - 1) / (w * kWave));
}

bool VecApplies(const float* residual, const float* delta, const float* weight, const float* y,
                int64_t dim) {
    return (dim % 4) == 0 && dim / 4 <= 1024 * 8 && Aligned(residual, 16) &&
           Aligned(weight, 16) && Aligned(y, 16) && (delta == nullptr || Aligned(delta, 16));
}

template <bool kDelta, bool kWriteBack, bool kPlanes = false, bool kPartials = false>
mlk_status Launch(float* residual, const float* delta, const float* weight, float* y,
                  int64_t n_rows, int64_t dim, float eps, hipStream_t stream,
                  uint32_t* planes = nullptr, int splits = 1, const float* dbias = nullptr) {
    const unsigned grid = FullGrid(n_rows, 1);
    const bool vec = VecApplies(residual, kDelta ? delta : nullptr, weight, y, dim);
    if (vec) {  // beyond 8 float4 per lane the row would spill
        int waves = 0, vpt = 0;
        NormShapeOf(dim, &waves, &vpt);
#define MLK_NORM_CASE(W, V)                                                                    \
    if (waves == (W) && vpt <= (V)) {                                                         \
        hipLaunchKernelGGL((AddRmsNormVec<W, V, kDelta, kWriteBack, kPlanes, kPartials>),      \
                           dim3(grid),                                                         \
                           dim3(kWave * (W)), 0, stream, residual, delta, weight, y, n_rows,   \
                           dim, eps, planes, splits, n_rows * dim, dbias);                     \
        return CheckLaunch("AddRmsNormVec");                                                   \
    }
        MLK_NORM_CASE(1, 1)
        MLK_NORM_CASE(2, 1)
        MLK_NORM_CASE(4, 1)
        MLK_NORM_CASE(8, 1)
        MLK_NORM_CASE(16, 1)
        MLK_NORM_CASE(16, 2)
        MLK_NORM_CASE(16, 4)
        MLK_NORM_CASE(16, 8)
#undef MLK_NORM_CASE
    }
    if (kPlanes || splits > 1 || dbias != nullptr) {
        return Fail(MLK_ERR_INVALID, "rmsnorm (planes / partial sums): unsupported row layout");
    }
    hipLaunchKernelGGL((AddRmsNormAny<kDelta, kWriteBack>), dim3(grid), dim3(kThreads), 0,
                       stream, residual, delta, weight, y, n_rows, dim, eps);
    return CheckLaunch("AddRmsNormAny");
}

mlk_status CheckNormArgs(const char* caller, const void* x, const void* weight, const void* y,
                         int64_t n_rows, int64_t dim, float eps) {
    if (x == nullptr || weight == nullptr || y == nullptr) {
        return Fail(MLK_ERR_INVALID, "%s: input, weight and output pointers must not be null",
                    caller);
    }
    if (n_rows <= 0 || dim <= 0) {
        return Fail(MLK_ERR_INVALID, "%s: rows and dim must be positive (got %lld x %lld)", caller,
                    static_cast<long long>(n_rows), static_cast<long long>(dim));
    }
    if (!std::isfinite(eps) || eps <= 0.0f) {
        return Fail(MLK_ERR_INVALID, "%s: eps must be finite and positive", caller);
    }
    return MLK_OK;
}

}  // namespace

bool NormShape(const float* residual, const float* delta, const float* weight, const float* y,
               int64_t dim, int* waves, int* vpt) {
    if (!VecApplies(residual, delta, weight, y, dim)) return false;
    NormShapeOf(dim, waves, vpt);
    return *vpt <= 8;
}

bool NormPlanesApplies(const float* residual, const float* delta, const float* weight,
                       const float* y, int64_t dim) {
    return dim % 32 == 0 && VecApplies(residual, delta, weight, y, dim);
}

mlk_status AddRmsNormPlanes(float* residual, const float* delta, const float* weight, float* y,
                            uint32_t* planes, int64_t n_rows, int64_t dim, float eps,
                            hipStream_t s, int splits, const float* dbias) {
    if (!NormPlanesApplies(residual, delta, weight, y, dim) || !Aligned(planes, 16) ||
        (dbias != nullptr && !Aligned(dbias, 16)) || splits < 1) {
        return Fail(MLK_ERR_INVALID, "rmsnorm (planes): unsupported row layout");
    }
    if (delta == nullptr) {
        return Launch<false, false, true>(residual, nullptr, weight, y, n_rows, dim, eps, s, planes);
    }
    if (splits > 1 || dbias != nullptr) {
        return Launch<true, true, true, true>(residual, delta, weight, y, n_rows, dim, eps, s,
                                              planes, splits, dbias);
    }
    return Launch<true, true, true>(residual, delta, weight, y, n_rows, dim, eps, s, planes);
}

}  // namespace mlk

using namespace mlk;

extern "C" {

mlk_status mlk_add_rmsnorm_f32(float* residual, const float* delta, const float* weight,
                               float* y, int64_t n_rows, int64_t dim, float eps, void* stream) {
    const mlk_status st =
        CheckNormArgs("mlk_add_rmsnorm_f32", residual, weight, y, n_rows, dim, eps);
    if (st != MLK_OK) return st;
    if (delta == nullptr) {
        return Launch<false, false>(residual, nullptr, weight, y, n_rows, dim, eps,
                                    AsStream(stream));
    }
    if (y == residual || y == delta) {
        return Fail(MLK_ERR_INVALID, "mlk_add_rmsnorm_f32: output must not alias the residual");
    }
    return Launch<true, true>(residual, delta, weight, y, n_rows, dim, eps, AsStream(stream));
}

mlk_status mlk_rmsnorm_f32(const float* x, const float* weight, float* y, int64_t n_rows,
                           int64_t dim, float eps, void* stream) {
    const mlk_status st = CheckNormArgs("mlk_rmsnorm_f32", x, weight, y, n_rows, dim, eps);
    if (st != MLK_OK) return st;
    // x is only read (kWriteBack = false), so casting away const is safe.
    return Launch<false, false>(const_cast<float*>(x), nullptr, weight, y, n_rows, dim, eps,
                                AsStream(stream));
}

}  // extern "C"
