// mlk_quant.h -- block formats and the fp16 decode shared by the quantized
// gather and the quantized linear kernels.
//
// Packed blocks of 32 elements (include/quantized_tensor.h:10-35 of the
// reference, little-endian):
//   Q8_0  34 B: u16 d | i8 qs[32]            w = d * q
//   Q4_0  18 B: u16 d | u8 qs[16]            w = d * (code - 8)
//   Q4_1  20 B: u16 d | u16 m | u8 qs[16]    w = d * code + m
// For Q4 formats, element i < 16 is the low nibble of qs[i] and element
// i >= 16 the high nibble of qs[i - 16].
#pragma once

#include "mlk_common.h"

namespace mlk {

template <int QT>
struct Fmt;
template <>
struct Fmt<MLK_Q8_0> {
    static constexpr int kBytes = 34;
};
template <>
struct Fmt<MLK_Q4_0> {
    static constexpr int kBytes = 18;
};
template <>
struct Fmt<MLK_Q4_1> {
    static constexpr int kBytes = 20;
};

__host__ __device__ inline int BlockBytes(int qt) {
    return qt == MLK_Q8_0 ? 34 : (qt == MLK_Q4_0 ? 18 : 20);
}

// IEEE binary16 -> binary32 with integer operations only, so no denormal
// mode can flush a subnormal scale; inf and NaN payloads are kept.
__device__ inline float HalfBits(uint32_t h) {
    const uint32_t sign = (h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 31u;
    const uint32_t f = h & 1023u;
    uint32_t bits;
    if (e == 31u) {
        bits = sign | 0x7F800000u | (f << 13);
    } else if (e != 0u) {
        bits = sign | ((e + 112u) << 23) | (f << 13);
    } else if (f == 0u) {
        bits = sign;
    } else {
        const uint32_t sh = static_cast<uint32_t>(__clz(f)) - 21u;  // moves the top bit to bit 10
        bits = sign | ((113u - sh) << 23) | (((f << sh) & 1023u) << 13);
    }
    return __uint_as_float(bits);
}

// The same conversion with the hardware instruction (v_cvt_f32_f16), for
// the inner loops of the linear kernels where the integer sequence costs ~10
// VALU ops per block.  gfx950 runs with f16/f64 denormals preserved (the HIP
// default mode), so subnormal scales convert exactly; the parity tests hold
// subnormal-scale blocks to keep that assumption checked.
__device__ inline float HalfHw(uint32_t h16) {
    const _Float16 v = __builtin_bit_cast(_Float16, static_cast<uint16_t>(h16));
    return static_cast<float>(v);
}

// One token row through the streaming GEMV (mlk_linear.hip), for up to three
// weight matrices with the same in_features in one launch.  Segment i: its
// blocks w (4-byte aligned), rows outputs y[0 .. rows) (+ bias), and for
// kStreamAdd the residual res (y[row] = res[row] + sum; res may be y).
// kStreamSwiGlu: segments 0 and 1 are gate and up with equal rows, y of
// segment 1 receives SwiGlu(gate, up) (segment 0's y is not written).
// kStreamQkvRope: segments q, k and v of attention heads of `rope.head_dim`
// (both even row counts, multiples of head_dim); each token's q and k rows
// are rotated in normal-layout pairs (2i, 2i+1) at the token's position as
// mlk_rope_f32 does (RopeRotatePair), q lands in segment 0's y and k and v in
// their cache rows: y + pos * rope.kv_stride for segments 1 and 2.  A
// position outside [0, max_seq) raises rope.err and writes no cache row (q is
// still rotated when pos >= 0, left as is below 0), as mlk_rope_f32 followed
// by mlk_kv_write_f32 would.
enum StreamMode { kStreamPlain = 0, kStreamAdd = 1, kStreamSwiGlu = 2, kStreamQkvRope = 3 };

struct StreamSeg {
    const uint8_t* w;
    const float* bias;
    float* y;
    const float* res;
    int64_t rows;
    int64_t groups;  // set by the launcher
};

struct RopeArgs {
    const int32_t* positions;  // per token, or null: pos0 + t
    int32_t pos0;
    int32_t head_dim;           // <= 2 * kRopePairs
    int64_t kv_stride;  // floats between cache rows of consecutive positions
    int64_t max_seq;
    int32_t* err;
    RopeFreqs freq;             // inverse frequencies of the head's pairs
};

// The one-token streaming GEMV can take its input as the RMSNorm of a
// residual row (plus delta), staged straight into its LDS: the same float64
// sums in the same order as AddRmsNormVec's block of `waves` waves with
// `vpt` float4s per thread (NormShape), so the staged row equals that
// kernel's output bit for bit.  res_out (when set) receives x + delta from
// workgroup 0 (the residual stream's next value, which x itself cannot take
// while other workgroups still read it).
struct StreamNorm {
    const float* weight = nullptr;  // null: no norm, the GEMV reads x as is
    const float* delta = nullptr;
    float* res_out = nullptr;
    float eps = 0.0f;
    int waves = 0, vpt = 0;
};

struct StreamArgs {
    StreamSeg seg[3];
    int n_seg;
    StreamNorm norm;  // the input row's RMSNorm (LinearRowStream, LinearRowPlanar)
    RopeArgs rope;  // kStreamQkvRope only
    // kStreamSwiGlu of the planar launches only: when set, the SwiGLU
    // outputs also go here as bf16 planes (StorePlanes, mlk_common.h) for
    // the next planar layer; F % 32 == 0
    uint32_t* planes = nullptr;
    // LinearTiledFused only: x already split into planes (StorePlanes
    // layout, 16-byte aligned), read instead of x by 8-wave tiles
    const uint32_t* x_planes = nullptr;
};

// in_features % 64 == 0 and x (16-byte aligned) fits the kernel's LDS
bool StreamFits(int64_t K);
// the shape rules of kStreamQkvRope above, and x plus its (cos, sin) table
// within the streaming kernel's LDS
bool QkvRopeArgsOk(const StreamArgs& a);
bool StreamRopeFits(int64_t K, int64_t head_dim);
mlk_status LinearRowStream(int qt, const float* x, int64_t K, const StreamArgs& a, int mode,
                           hipStream_t s);
// The same for one token over planar Q8_0 / Q4_0 weights (segments' w in
// the layout at mlk_quant_to_planar, 16-byte aligned; no `planes` out):
// contiguous 1 KB loads per wave, sums that depend on K only, so every mode
// and a staged norm give the plain launch's sums bit for bit.  Applies when
// K % 256 == 0 and x plus the chunk sums fit the kernel's LDS (K up to
// about 14.5 K inputs).
bool RowPlanarApplies(int qt, int64_t K, int mode, bool norm);
mlk_status LinearRowPlanar(int qt, const float* x, int64_t K, const StreamArgs& a, int mode,
                           hipStream_t s);

// T token rows (up to 32) through up to three quantized weight matrices with
// the same K (a multiple of 256) in one skinny launch (mlk_gemm.hip), then
// one split-K reduction with the mode's epilogue (segments and modes as for
// LinearRowStream).  The workspace holds SkinnyFusedWorkspaceBytes(wt, T, K,
// sum of the segments' rows) bytes.
bool SkinnyFusedApplies(int wt, int64_t T, int64_t K);
int64_t SkinnyFusedWorkspaceBytes(int wt, int64_t T, int64_t K, int64_t cols);
mlk_status LinearSkinnyFused(int wt, const float* x, int64_t T, int64_t K, const StreamArgs& a,
                             int mode, void* workspace, size_t workspace_bytes, hipStream_t s);

// Prefill-shaped linear on the matrix cores (mlk_gemm.hip): y [T, O] =
// x [T, K] W^T (+ bias), W fp32 (wt = -1) or MLK_Q8_0/Q4_0/Q4_1 blocks of
// row_bytes per output row.  Needs K % 4 == 0 and 16-byte aligned x (and
// fp32 W); quantized W needs K % 32 == 0 and its load alignment (2 bytes,
// 4 for Q4_1).
// K is split over workgroups when `workspace` holds GemmWorkspaceBytes(wt, T,
// K, O) bytes (16-byte aligned), else not.
mlk_status LaunchGemm(int wt, const float* x, const void* w, const float* bias, float* y,
                      int64_t T, int64_t K, int64_t O, int64_t row_bytes, void* workspace,
                      size_t workspace_bytes, hipStream_t s);
int64_t GemmWorkspaceBytes(int wt, int64_t T, int64_t K, int64_t O);
// The same tiled product with the layer's epilogue in one launch (no
// workspace) for many token rows: block-layout Q8_0 / Q4_0, K % 256 == 0,
// T > 64, O rows per matrix, and only where LaunchGemm would not split K
// either, so each output's sum is LaunchGemm's.  kStreamAdd: one segment
// with res == y (y = y + (sum + bias), mlk_add_f32's value).  kStreamSwiGlu:
// gate and up segments of O rows each, seg[1].y = SwiGlu(gate, up) as
// mlk_swiglu_f32 computes it, when the gate / up tiles fill two workgroups
// per CU.  kStreamPlain: two matrices of O rows each (segments 0 and 1,
// each to its own y) in one launch without a K split, when their tiles
// together fill two workgroups per CU (where LaunchGemm would split each:
// the sums are then the unsplit product's, LaunchGemm's without a
// workspace); with one segment, that matrix alone, under kStreamAdd's shape
// rule (LaunchGemm's sums).  a.x_planes, when set, holds x as StorePlanes
// writes it and the 8-wave tiles read it instead of splitting x (the same
// sums; 4-wave tiles still read x).  x 16-byte aligned, W 2-byte aligned.
bool TiledFusedApplies(int wt, int64_t T, int64_t K, int64_t O, int mode);
// A one-matrix or residual-add launch of O rows takes the 8-wave tiles,
// which read x_planes (the pair and SwiGLU launches always do).
bool TiledTakesPlanes(int64_t T, int64_t O);
mlk_status LinearTiledFused(int wt, const float* x, int64_t T, int64_t K, const StreamArgs& a,
                            int mode, hipStream_t s);

// Planar Q8_0 / Q4_0 weights (layout at mlk_quant_to_planar, minilamma_hip.h;
// mlk_gemm.hip).  wt values of LaunchGemm for them:
constexpr int kWPlanarQ8 = 16, kWPlanarQ4 = 17;
// bytes of the layout (0: unsupported shape) and the repack
int64_t PlanarBytes(int qt, int64_t O, int64_t K);
mlk_status LaunchToPlanar(int qt, const void* blocks, int64_t O, int64_t K, void* planar,
                          hipStream_t s);
// Up to 32 token rows on the bf16 matrix cores: one matrix, or up to three
// with the same K fused as LinearSkinnyFused (modes and epilogues alike).
// The workspace (16-byte aligned) holds PlanarWorkspaceBytes(T, K, rows of
// all segments, fused) bytes: partial sums, then x split into bf16 planes.
// planes: x's planes already made (StorePlanes layout, 16-byte aligned),
// or null.
bool PlanarApplies(int qt, int64_t T, int64_t K);
int64_t PlanarWorkspaceBytes(int64_t T, int64_t K, int64_t cols, bool fused);
mlk_status LinearPlanar(int qt, const float* x, const void* w, const float* bias, float* y,
                        int64_t T, int64_t K, int64_t O, void* workspace, size_t workspace_bytes,
                        hipStream_t s, const uint32_t* planes = nullptr);
mlk_status LinearPlanarFused(int qt, const float* x, int64_t T, int64_t K, const StreamArgs& a,
                             int mode, void* workspace, size_t workspace_bytes, hipStream_t s,
                             const uint32_t* planes = nullptr);

// Residual add + RMSNorm (mlk_norm.hip; delta may be null: plain RMSNorm of
// residual, which is then only read) that also writes y's bf16 planes for
// the planar layers (StorePlanes, mlk_common.h), when NormPlanesApplies.
// splits > 1 or dbias: delta holds a linear layer's split-K partial sums
// ([splits][n_rows][dim]), reduced here in split order, then + dbias, as
// SplitKReduce would.
bool NormPlanesApplies(const float* residual, const float* delta, const float* weight,
                       const float* y, int64_t dim);
// AddRmsNormVec's block for rows of dim floats (false: another kernel takes
// such rows, or a pointer is not 16-byte aligned)
bool NormShape(const float* residual, const float* delta, const float* weight, const float* y,
               int64_t dim, int* waves, int* vpt);
mlk_status AddRmsNormPlanes(float* residual, const float* delta, const float* weight, float* y,
                            uint32_t* planes, int64_t n_rows, int64_t dim, float eps,
                            hipStream_t s, int splits = 1, const float* dbias = nullptr);
// The planar GEMM alone, partial sums always in the workspace: *partial,
// *splits for the caller's reduction (e.g. AddRmsNormPlanes).
mlk_status LinearPlanarPartials(int qt, const float* x, const void* w, int64_t T, int64_t K,
                                int64_t O, void* workspace, size_t workspace_bytes,
                                hipStream_t s, const uint32_t* planes, float** partial,
                                int* splits);

}  // namespace mlk
