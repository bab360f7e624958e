// mlk_rope.hip -- rotary position embedding, in place, on Q and K of a batch
// of tokens with per-token positions.
//
// Semantics of Rope (src/ops.cc:177-224): for pair i < head_dim / 2,
//   angle = (double) pos * pow((double) theta, -2.0 * i / head_dim)
//   (x0, x1) <- ((float)(x0 c - x1 s), (float)(x0 s + x1 c)),  c, s in double
// Normal pairs (2i, 2i+1); NeoX pairs (i, i + head_dim/2).  The reference's
// device kernel (src/cuda_ops.cu:254-299) used fp32 powf/cosf/sinf, whose
// angle drifts from the double one by ~4e-4 rad at pos 8191 (theta 5e5);
// here the angle, cos and sin are float64, so the result equals the CPU's.
// The pow factors are evaluated once per call on the host with the C
// library's pow (the CPU's own), so the angles are the reference's bit for
// bit, and handed to the kernel in its arguments.
//
// Work layout: workgroups walk the tokens (about four per workgroup at
// T = 4096).  The threads form `rows` rows of `lanes` lanes; a lane owns PV
// consecutive pairs of a head, computes its inverse frequencies once per
// kernel and, per token, issues the loads of its first kBatch heads before
// evaluating the float64 sin and cos, so the transcendental latency hides under
// the memory latency; the same angles then serve every head the row visits.
// Q and K are one launch (the reference made two per token).  The update is
// in place with non-temporal loads and stores: on MI355X a cold
// read-modify-write stream reaches ~6.0 TB/s with them against ~5.3 TB/s
// with plain ones (plain ones only look faster when the data is still in the
// 256 MB MALL).
//
// HBM bytes per token: 8 * (n_heads + n_kv_heads) * head_dim (read + write).
#include "mlk_common.h"

#include <climits>
#include <cmath>

namespace mlk {
namespace {

constexpr int kThreads = 256;
constexpr int kBatch = 5;  // heads loaded per lane before the first rotation

template <int PV, bool kNeoX>
struct Pairs;

// Normal layout, two pairs per lane: one float4 at element 4g.
template <>
struct Pairs<2, false> {
    float4 v;
    __device__ void Load(const float* head, int g, int) {
        v = LoadNT(reinterpret_cast<const float4*>(head) + g);
    }
    __device__ void Rotate(const double* c, const double* s) {
        const double a0 = v.x, a1 = v.y, b0 = v.z, b1 = v.w;
        v.x = static_cast<float>(a0 * c[0] - a1 * s[0]);
        v.y = static_cast<float>(a0 * s[0] + a1 * c[0]);
        v.z = static_cast<float>(b0 * c[1] - b1 * s[1]);
        v.w = static_cast<float>(b0 * s[1] + b1 * c[1]);
    }
    __device__ void Store(float* head, int g, int) const {
        StoreNT(reinterpret_cast<float4*>(head) + g, v);
    }
    // byte offset of the lane's elements from a row base (32-bit, so the
    // address is a scalar base plus a 32-bit lane offset)
    static __device__ uint32_t LaneBytes(int g, int) { return 16u * g; }
    __device__ void LoadAt(const char* base, uint32_t o, uint32_t) {
        v = LoadNT(reinterpret_cast<const float4*>(base + o));
    }
    __device__ void StoreAt(char* base, uint32_t o, uint32_t) const {
        StoreNT(reinterpret_cast<float4*>(base + o), v);
    }
};

// Normal layout, one pair per lane.
template <>
struct Pairs<1, false> {
    float x0, x1;
    __device__ void Load(const float* head, int g, int) {
        x0 = LoadNT(head + 2 * g);
        x1 = LoadNT(head + 2 * g + 1);
    }
    __device__ void Rotate(const double* c, const double* s) {
        const double a0 = x0, a1 = x1;
        x0 = static_cast<float>(a0 * c[0] - a1 * s[0]);
        x1 = static_cast<float>(a0 * s[0] + a1 * c[0]);
    }
    __device__ void Store(float* head, int g, int) const {
        StoreNT(head + 2 * g, x0);
        StoreNT(head + 2 * g + 1, x1);
    }
    static __device__ uint32_t LaneBytes(int g, int) { return 8u * g; }
    __device__ void LoadAt(const char* base, uint32_t o, uint32_t) {
        x0 = LoadNT(reinterpret_cast<const float*>(base + o));
        x1 = LoadNT(reinterpret_cast<const float*>(base + (o + 4u)));
    }
    __device__ void StoreAt(char* base, uint32_t o, uint32_t) const {
        StoreNT(reinterpret_cast<float*>(base + o), x0);
        StoreNT(reinterpret_cast<float*>(base + (o + 4u)), x1);
    }
};

// NeoX layout, two pairs per lane: float2 at 2g and at half + 2g.
template <>
struct Pairs<2, true> {
    float2 lo, hi;
    __device__ void Load(const float* head, int g, int half) {
        lo = LoadNT(reinterpret_cast<const float2*>(head) + g);
        hi = LoadNT(reinterpret_cast<const float2*>(head + half) + g);
    }
    __device__ void Rotate(const double* c, const double* s) {
        const double a0 = lo.x, a1 = hi.x, b0 = lo.y, b1 = hi.y;
        lo.x = static_cast<float>(a0 * c[0] - a1 * s[0]);
        hi.x = static_cast<float>(a0 * s[0] + a1 * c[0]);
        lo.y = static_cast<float>(b0 * c[1] - b1 * s[1]);
        hi.y = static_cast<float>(b0 * s[1] + b1 * c[1]);
    }
    __device__ void Store(float* head, int g, int half) const {
        StoreNT(reinterpret_cast<float2*>(head) + g, lo);
        StoreNT(reinterpret_cast<float2*>(head + half) + g, hi);
    }
    static __device__ uint32_t LaneBytes(int g, int) { return 8u * g; }
    __device__ void LoadAt(const char* base, uint32_t o, uint32_t half_bytes) {
        lo = LoadNT(reinterpret_cast<const float2*>(base + o));
        hi = LoadNT(reinterpret_cast<const float2*>(base + (o + half_bytes)));
    }
    __device__ void StoreAt(char* base, uint32_t o, uint32_t half_bytes) const {
        StoreNT(reinterpret_cast<float2*>(base + o), lo);
        StoreNT(reinterpret_cast<float2*>(base + (o + half_bytes)), hi);
    }
};

// NeoX layout, one pair per lane.
template <>
struct Pairs<1, true> {
    float x0, x1;
    __device__ void Load(const float* head, int g, int half) {
        x0 = LoadNT(head + g);
        x1 = LoadNT(head + g + half);
    }
    __device__ void Rotate(const double* c, const double* s) {
        const double a0 = x0, a1 = x1;
        x0 = static_cast<float>(a0 * c[0] - a1 * s[0]);
        x1 = static_cast<float>(a0 * s[0] + a1 * c[0]);
    }
    __device__ void Store(float* head, int g, int half) const {
        StoreNT(head + g, x0);
        StoreNT(head + g + half, x1);
    }
    static __device__ uint32_t LaneBytes(int g, int) { return 4u * g; }
    __device__ void LoadAt(const char* base, uint32_t o, uint32_t half_bytes) {
        x0 = LoadNT(reinterpret_cast<const float*>(base + o));
        x1 = LoadNT(reinterpret_cast<const float*>(base + (o + half_bytes)));
    }
    __device__ void StoreAt(char* base, uint32_t o, uint32_t half_bytes) const {
        StoreNT(reinterpret_cast<float*>(base + o), x0);
        StoreNT(reinterpret_cast<float*>(base + (o + half_bytes)), x1);
    }
};

// General form (any head count and even head_dim): inverse frequencies from
// the host table when head_dim <= 2 * kRopePairs, else from the device pow
// (same expression; it may differ from the C library's in the last bit).
template <int PV, bool kNeoX>
__global__ __launch_bounds__(kThreads) void RopeKernel(float* q, float* k, int64_t n_tokens,
                                                       int n_heads, int n_kv_heads, int head_dim,
                                                       int64_t q_stride, int64_t k_stride,
                                                       const int32_t* positions, int32_t pos0,
                                                       float theta, const RopeFreqs f,
                                                       int32_t* err) {
#pragma clang fp contract(off)
    const int tid = threadIdx.x;
    const int half = head_dim / 2;
    const int groups = half / PV;
    const int lanes = groups < kThreads ? groups : kThreads;
    const int rows = kThreads / lanes;
    const int lane = tid % lanes;
    const int row = tid / lanes;
    if (row >= rows) {
        return;  // spare threads when kThreads is not a multiple of lanes
    }
    const int heads = n_heads + n_kv_heads;
    for (int g = lane; g < groups; g += lanes) {
        double inv_freq[PV];
#pragma unroll
        for (int p = 0; p < PV; ++p) {
            const int i = g * PV + p;
            inv_freq[p] = half <= kRopePairs ? f.inv[i]
                                             : pow(static_cast<double>(theta), -2.0 * i / head_dim);
        }
        for (int64_t t = blockIdx.x; t < n_tokens; t += gridDim.x) {
            const int32_t pos = positions != nullptr ? positions[t] : pos0 + static_cast<int32_t>(t);
            if (pos < 0) {
                if (tid == 0 && g == 0) RaiseFlag(err, 1);
                continue;
            }
            float* qt = q + t * q_stride;
            float* kt = k + t * k_stride;
            double c[PV], s[PV];
            bool have_angles = false;
            for (int h0 = row; h0 < heads; h0 += rows * kBatch) {
                Pairs<PV, kNeoX> v[kBatch];
                float* base[kBatch];
#pragma unroll
                for (int b = 0; b < kBatch; ++b) {
                    const int h = h0 + b * rows;
                    base[b] = nullptr;
                    if (h < heads) {
                        base[b] = h < n_heads ? qt + static_cast<int64_t>(h) * head_dim
                                              : kt + static_cast<int64_t>(h - n_heads) * head_dim;
                        v[b].Load(base[b], g, half);
                    }
                }
                if (!have_angles) {
                    // evaluated while the first batch of loads is in flight
#pragma unroll
                    for (int p = 0; p < PV; ++p) {
                        SinCosAngle(static_cast<double>(pos) * inv_freq[p], &s[p], &c[p]);
                    }
                    have_angles = true;
                }
#pragma unroll
                for (int b = 0; b < kBatch; ++b) {
                    if (base[b] != nullptr) {
                        v[b].Rotate(c, s);
                        v[b].Store(base[b], g, half);
                    }
                }
            }
        }
    }
}

// Common case: every lane rotates at most kBatch heads of one pair group per
// token, so one batch of loads covers the token.  The threads form `rows`
// rows; batch slot b < q_slots holds Q head b * rows + row, the later slots
// K heads (b - q_slots) * rows + row, so which of Q and K a slot reads is
// uniform and the token's Q and K row addresses stay scalar, each lane
// keeping one 32-bit offset per slot (256 threads for 8B heads: rows 8,
// slots 4 + 1; 512 for 70B: rows 16, slots 4 + 1).
// The workgroup's tokens are t = blockIdx.x + j * gridDim.x; the next
// token's heads load while the current one's float64 sin, cos and rotation
// run (two register sets, loop unrolled by two with the last one or two
// tokens peeled, so no load sits under a branch and no token is loaded
// twice: a reload would come from HBM, the loads being non-temporal).
// Same arithmetic as RopeKernel.  The Llama path (normal layout, two pairs
// a lane) fits 128 registers and takes workgroups of up to 1024 threads;
// the NeoX and one-pair forms need a few more registers than that (their
// two register sets of 2 x 5 heads, and the extra address of NeoX's second
// half), so they are built for at most 512 threads (up to 256 registers,
// no scratch) -- every Llama / Qwen head shape fits 512.
template <int PV, bool kNeoX>
constexpr int PipeMaxThreads() { return PV == 2 && !kNeoX ? 1024 : 512; }

template <int PV, bool kNeoX>
__global__ __launch_bounds__((PipeMaxThreads<PV, kNeoX>())) void RopePipe(float* q, float* k, int64_t n_tokens,
                                                 int n_heads, int n_kv_heads, int head_dim,
                                                 int64_t q_stride, int64_t k_stride,
                                                 const int32_t* positions, int32_t pos0,
                                                 const RopeFreqs f, int rows, int q_slots,
                                                 int32_t* err) {
#pragma clang fp contract(off)
    const int tid = threadIdx.x;
    const int half = head_dim / 2;
    const int lanes = half / PV;
    const int lane = tid % lanes;
    const int row = tid / lanes;
    if (row >= rows) return;
    const int64_t nt = (n_tokens - blockIdx.x + gridDim.x - 1) / gridDim.x;
    auto token = [&](int64_t j) { return static_cast<int64_t>(blockIdx.x) + j * gridDim.x; };
    double inv_freq[PV];
#pragma unroll
    for (int p = 0; p < PV; ++p) inv_freq[p] = f.inv[lane * PV + p];
    using V = Pairs<PV, kNeoX>;
    uint32_t off[kBatch];  // byte offset of the lane's elements of the slot's head
    bool ok[kBatch];       // the slot holds a head
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
        const int h = (b < q_slots ? b : b - q_slots) * rows + row;
        ok[b] = h < (b < q_slots ? n_heads : n_kv_heads);
        off[b] = 4u * static_cast<uint32_t>(h) * static_cast<uint32_t>(head_dim) +
                 V::LaneBytes(lane, half);
    }
    const uint32_t half_bytes = 4u * static_cast<uint32_t>(half);
    // the token's Q or K row: uniform across the workgroup
    auto row_base = [&](int64_t t, int b) {
        return reinterpret_cast<char*>(b < q_slots ? q + t * q_stride : k + t * k_stride);
    };
    auto load = [&](int64_t t, V (&v)[kBatch]) {
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            if (ok[b]) v[b].LoadAt(row_base(t, b), off[b], half_bytes);
        }
    };
    auto rotate = [&](int64_t t, V (&v)[kBatch]) {
        const int32_t pos = positions != nullptr ? positions[t] : pos0 + static_cast<int32_t>(t);
        if (pos < 0) {  // leave the token unrotated, raise the flag
            if (tid == 0) RaiseFlag(err, 1);
            return;
        }
        double c[PV], sn[PV];
#pragma unroll
        for (int p = 0; p < PV; ++p) SinCosAngle(static_cast<double>(pos) * inv_freq[p], &sn[p], &c[p]);
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            if (ok[b]) {
                v[b].Rotate(c, sn);
                v[b].StoreAt(row_base(t, b), off[b], half_bytes);
            }
        }
    };
    V va[kBatch], vb[kBatch];
    load(token(0), va);
    int64_t j = 0;
    for (; j + 2 < nt; j += 2) {  // tokens j, j+1 and j+2 exist
        load(token(j + 1), vb);
        rotate(token(j), va);
        load(token(j + 2), va);
        rotate(token(j + 1), vb);
    }
    // one or two tokens left, j's already loaded; both branches complete,
    // so no load is pending across a join
    if (j + 1 < nt) {
        load(token(j + 1), vb);
        rotate(token(j), va);
        rotate(token(j + 1), vb);
    } else {
        rotate(token(j), va);
    }
}

// Smallest row count whose Q and K slots fit kBatch, or 0 when the rows
// would need more than max_threads threads.
inline int PipeRows(int n_heads, int n_kv_heads, int lanes, int max_threads) {
    for (int rows = (n_heads + n_kv_heads + kBatch - 1) / kBatch; rows * lanes <= max_threads;
         ++rows) {
        if ((n_heads + rows - 1) / rows + (n_kv_heads + rows - 1) / rows <= kBatch) return rows;
    }
    return 0;
}

template <int PV, bool kNeoX>
mlk_status LaunchRope(float* q, float* k, int64_t n_tokens, int n_heads, int n_kv_heads,
                      int head_dim, int64_t qs, int64_t ks, const int32_t* positions,
                      int32_t pos0, float theta, int32_t* err, hipStream_t stream) {
    const int lanes = head_dim / 2 / PV;
    const bool table = head_dim / 2 <= kRopePairs;
    const RopeFreqs f = MakeRopeFreqs(theta, table ? head_dim : 2);
    const int rows = table ? PipeRows(n_heads, n_kv_heads, lanes, PipeMaxThreads<PV, kNeoX>()) : 0;
    // byte offsets within a token's Q or K row are 32-bit
    const bool offsets_fit =
        4 * static_cast<int64_t>(n_heads > n_kv_heads ? n_heads : n_kv_heads) * head_dim <= UINT32_MAX;
    if (rows > 0 && offsets_fit) {
        const int64_t threads = (static_cast<int64_t>(lanes) * rows + kWave - 1) / kWave * kWave;
        // about 1024 resident threads' worth of workgroups per CU
        const int per_cu = static_cast<int>(1024 / threads);
        const unsigned grid = GridFor(n_tokens, 1, per_cu);
        const int q_slots = (n_heads + rows - 1) / rows;
        hipLaunchKernelGGL((RopePipe<PV, kNeoX>), dim3(grid), dim3(threads), 0, stream, q, k,
                           n_tokens, n_heads, n_kv_heads, head_dim, qs, ks, positions, pos0,
                           f, rows, q_slots, err);
        return CheckLaunch("RopePipe");
    }
    const unsigned grid = GridFor(n_tokens, 1, 4);
    hipLaunchKernelGGL((RopeKernel<PV, kNeoX>), dim3(grid), dim3(kThreads), 0, stream, q, k,
                       n_tokens, n_heads, n_kv_heads, head_dim, qs, ks, positions, pos0, theta,
                       f, err);
    return CheckLaunch("RopeKernel");
}

}  // namespace
}  // namespace mlk

using namespace mlk;

extern "C" {

mlk_status mlk_rope_f32(float* q, float* k, int64_t n_tokens, int32_t n_heads,
                        int32_t n_kv_heads, int32_t head_dim, int64_t q_row_stride,
                        int64_t k_row_stride, const int32_t* positions, int32_t pos0,
                        float theta, int32_t rope_type, int32_t* err, void* stream) {
    const char* caller = "mlk_rope_f32";
    if (q == nullptr || k == nullptr) {
        return Fail(MLK_ERR_INVALID, "%s: q and k pointers must not be null", caller);
    }
    if (n_tokens < 0) {
        return Fail(MLK_ERR_INVALID, "%s: n_tokens must not be negative", caller);
    }
    if (n_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0 || head_dim % 2 != 0) {
        return Fail(MLK_ERR_INVALID,
                    "%s: head counts must be positive and head_dim must be positive and even",
                    caller);
    }
    if (!std::isfinite(theta) || theta <= 0.0f) {
        return Fail(MLK_ERR_INVALID, "%s: theta must be finite and positive", caller);
    }
    if (rope_type != MLK_ROPE_NORMAL && rope_type != MLK_ROPE_NEOX) {
        return Fail(MLK_ERR_INVALID, "%s: unknown rope type %d", caller, rope_type);
    }
    const int64_t q_width = static_cast<int64_t>(n_heads) * head_dim;
    const int64_t k_width = static_cast<int64_t>(n_kv_heads) * head_dim;
    if (q_row_stride < q_width || k_row_stride < k_width) {
        return Fail(MLK_ERR_INVALID, "%s: row strides must cover n_heads * head_dim", caller);
    }
    if (positions == nullptr) {
        if (pos0 < 0) return Fail(MLK_ERR_RANGE, "%s: pos must be non-negative", caller);
        if (n_tokens > 0 && static_cast<int64_t>(pos0) + n_tokens - 1 > INT32_MAX) {
            return Fail(MLK_ERR_RANGE, "%s: positions exceed the int32 range", caller);
        }
    }
    if (n_tokens == 0) return MLK_OK;
    const hipStream_t s = AsStream(stream);
    const bool neox = rope_type == MLK_ROPE_NEOX;
    const bool two = head_dim % 4 == 0;
    if (!neox) {
        const bool v4 = two && Aligned(q, 16) && Aligned(k, 16) && q_row_stride % 4 == 0 &&
                        k_row_stride % 4 == 0;
        return v4 ? LaunchRope<2, false>(q, k, n_tokens, n_heads, n_kv_heads, head_dim,
                                         q_row_stride, k_row_stride, positions, pos0, theta, err, s)
                  : LaunchRope<1, false>(q, k, n_tokens, n_heads, n_kv_heads, head_dim,
                                         q_row_stride, k_row_stride, positions, pos0, theta, err, s);
    }
    const bool v2 = two && Aligned(q, 8) && Aligned(k, 8) && q_row_stride % 2 == 0 &&
                    k_row_stride % 2 == 0;
    return v2 ? LaunchRope<2, true>(q, k, n_tokens, n_heads, n_kv_heads, head_dim, q_row_stride,
                                    k_row_stride, positions, pos0, theta, err, s)
              : LaunchRope<1, true>(q, k, n_tokens, n_heads, n_kv_heads, head_dim, q_row_stride,
                                    k_row_stride, positions, pos0, theta, err, s);
}

}  // extern "C"
