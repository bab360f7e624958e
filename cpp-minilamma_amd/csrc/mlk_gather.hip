// mlk_gather.hip -- token-embedding gather from F32 and block-quantized
// tables, and the device block quantizer.
//
// F32 gather: out[t] = table[ids[t]], a bit-exact row copy (Embedding,
// src/forward.cc:198-205; device EmbeddingKernel src/cuda_ops.cu:187-192,
// which copied one token per launch with 32-bit element offsets).  Offsets
// here are 64-bit: the 70B-class tables exceed 2^31 bytes.
//
// Quantized gather: out[t] = dequant(table row ids[t]) with the semantics of
// Q80ToTensor / Q40ToTensor / Q41ToTensor (src/quant.cc:175-368):
//   Q8_0  d * q                         q int8
//   Q4_0  d * (code - 8)                code = low nibble of byte i for
//   Q4_1  d * code + m                  element i < 16, high nibble of byte
//                                       i - 16 otherwise
// with d, m IEEE binary16 (subnormals, inf and NaN payloads kept, decoded by
// integer ops so no denormal mode can flush them).  fp16 * (<= 8-bit int)
// is exact in fp32, so only the Q4_1 "+ m" rounds and the result equals the
// CPU one bit for bit.
//
// Table rows are read with normal loads (Zipf-distributed ids repeat hot
// rows, which then come from L2 / the MALL); output rows are written with
// non-temporal stores.  A 1024-lane workgroup takes one token row at a time;
// each lane decodes four consecutive outputs of one block with aligned u16 /
// u32 loads of the scale(s) and code bytes and writes them as one float4.
// (An LDS-staged variant -- 16-byte loads of the packed row, barrier, decode
// from LDS -- measured 15-25% slower on MI355X: the gather is write-bound
// and the staging round trip only added latency.)
#include "mlk_quant.h"

#include <type_traits>

namespace mlk {
namespace {

constexpr int kThreads = 256;
constexpr int kQThreads = 1024;  // one float4 per lane of a 4096-wide row

__device__ inline uint32_t LoadU16(const uint8_t* p) {
    return static_cast<uint32_t>(p[0]) | (static_cast<uint32_t>(p[1]) << 8);
}

// Decodes element w (0..31) of a block with byte loads (any alignment).
template <int QT>
__device__ inline float Decode1(const uint8_t* blk, int w) {
#pragma clang fp contract(off)
    const float d = HalfBits(LoadU16(blk));
    if (QT == MLK_Q8_0) {
        return d * static_cast<float>(static_cast<int8_t>(blk[2 + w]));
    } else if (QT == MLK_Q4_0) {
        const uint32_t byte = blk[2 + (w & 15)];
        const int code = static_cast<int>(w < 16 ? (byte & 15u) : (byte >> 4)) - 8;
        return d * static_cast<float>(code);
    } else {
        const float m = HalfBits(LoadU16(blk + 2));
        const uint32_t byte = blk[4 + (w & 15)];
        const int code = static_cast<int>(w < 16 ? (byte & 15u) : (byte >> 4));
        return d * static_cast<float>(code) + m;
    }
}

// Decodes elements w..w+3 (w % 4 == 0) of block `blk` straight from global
// memory with aligned loads.  The scales go through the hardware conversion
// (v_cvt_f32_f16, one instruction instead of the integer sequence of
// HalfBits, which made the Q4_1 gather VALU-bound); gfx950 keeps fp16
// denormals, so subnormal scales convert exactly (the parity tests hold
// blocks with scale 0x0001), and a NaN scale still gives NaN outputs (its
// quiet bit is set one step earlier than on the CPU, where the product
// sets it).  Every block starts at an even byte offset
// (34, 18 and 20 are even and rows start 16-byte aligned), so d and m are
// u16 loads; Q4_1 blocks start 4-byte aligned (20b) so d|m and the four code
// bytes (20b + 4 + 4k) are one u32 each, Q8_0 / Q4_0 code bytes two u16.
// The block's bytes are shared by 8 neighbouring lanes, so these small
// loads hit in L1 after the first.
template <int QT>
__device__ inline float4 Decode4(const uint8_t* blk, int w) {
#pragma clang fp contract(off)
    float d, m = 0.0f;
    uint32_t codes;  // four code bytes, little-endian
    if (QT == MLK_Q4_1) {
        const uint32_t dm = *reinterpret_cast<const uint32_t*>(blk);
        d = HalfHw(dm & 0xFFFFu);
        m = HalfHw(dm >> 16);
        codes = *reinterpret_cast<const uint32_t*>(blk + 4 + (w & 15));
    } else {
        d = HalfHw(*reinterpret_cast<const uint16_t*>(blk));
        const uint16_t* p =
            reinterpret_cast<const uint16_t*>(blk + 2 + (QT == MLK_Q8_0 ? w : (w & 15)));
        codes = static_cast<uint32_t>(p[0]) | (static_cast<uint32_t>(p[1]) << 16);
    }
    float4 o;
    if (QT == MLK_Q8_0) {
        o.x = d * static_cast<float>(static_cast<int8_t>(codes & 0xFFu));
        o.y = d * static_cast<float>(static_cast<int8_t>((codes >> 8) & 0xFFu));
        o.z = d * static_cast<float>(static_cast<int8_t>((codes >> 16) & 0xFFu));
        o.w = d * static_cast<float>(static_cast<int8_t>(codes >> 24));
    } else {
        // element w + j is the low nibble of byte j (w < 16) or its high nibble
        const uint32_t nib = w < 16 ? codes : (codes >> 4);
        const int bias = QT == MLK_Q4_0 ? 8 : 0;
        const float c0 = static_cast<float>(static_cast<int>(nib & 15u) - bias);
        const float c1 = static_cast<float>(static_cast<int>((nib >> 8) & 15u) - bias);
        const float c2 = static_cast<float>(static_cast<int>((nib >> 16) & 15u) - bias);
        const float c3 = static_cast<float>(static_cast<int>((nib >> 24) & 15u) - bias);
        if (QT == MLK_Q4_0) {
            o.x = d * c0;
            o.y = d * c1;
            o.z = d * c2;
            o.w = d * c3;
        } else {
            o.x = d * c0 + m;
            o.y = d * c1 + m;
            o.z = d * c2 + m;
            o.w = d * c3 + m;
        }
    }
    return o;
}

// A workgroup takes one token row per iteration (grid-stride over tokens;
// the launch gives every token its own workgroup up to 16 per CU).
// U > 0: dim == 4 * U * kQThreads and aligned buffers (the 8B and 70B
// widths): each lane decodes U float4 at compile-time offsets, all their
// loads issued before the first store.  U == 0: any width; vec (dim % 4 ==
// 0, aligned buffers) -> one float4 per lane per step with Decode4,
// otherwise one element per lane with Decode1 (byte loads).
template <int QT, int U>
__global__ __launch_bounds__(kQThreads) void GatherQuantKernel(const uint8_t* __restrict__ blocks,
                                                               int64_t vocab, int64_t dim,
                                                               const int32_t* __restrict__ ids,
                                                               int32_t token, int64_t n_tokens,
                                                               float* __restrict__ out,
                                                               int32_t* err, int vec) {
    constexpr int kBB = Fmt<QT>::kBytes;
    const int tid = threadIdx.x;
    const int64_t row_bytes = ((dim + 31) / 32) * kBB;
    for (int64_t t = blockIdx.x; t < n_tokens; t += gridDim.x) {
        const int32_t id = ids != nullptr ? ids[t] : token;
        float* dst = out + t * dim;
        if (id < 0 || id >= vocab) {
            if (tid == 0) RaiseFlag(err, 1);
            for (int64_t i = tid; i < dim; i += kQThreads) dst[i] = 0.0f;
            continue;
        }
        const uint8_t* row = blocks + static_cast<int64_t>(id) * row_bytes;
        if constexpr (U > 0) {
            float4 v[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int e = 4 * (tid + u * kQThreads);
                v[u] = Decode4<QT>(row + (e >> 5) * kBB, e & 31);
            }
            float4* d4 = reinterpret_cast<float4*>(dst);
#pragma unroll
            for (int u = 0; u < U; ++u) StoreNT(d4 + tid + u * kQThreads, v[u]);
        } else if (vec) {
            float4* d4 = reinterpret_cast<float4*>(dst);
            for (int64_t j = tid; j < dim / 4; j += kQThreads) {
                const int64_t e = 4 * j;
                StoreNT(d4 + j, Decode4<QT>(row + (e >> 5) * kBB, static_cast<int>(e & 31)));
            }
        } else {
            for (int64_t e = tid; e < dim; e += kQThreads) {
                dst[e] = Decode1<QT>(row + (e >> 5) * kBB, static_cast<int>(e & 31));
            }
        }
    }
}

template <int VPT>
__global__ __launch_bounds__(kThreads) void GatherF32Vec(const float4* __restrict__ table,
                                                         int64_t vocab, int64_t dim4,
                                                         const int32_t* __restrict__ ids,
                                                         int32_t token, int64_t n_tokens,
                                                         float4* __restrict__ out, int32_t* err) {
    const int tid = threadIdx.x;
    for (int64_t t = blockIdx.x; t < n_tokens; t += gridDim.x) {
        const int32_t id = ids != nullptr ? ids[t] : token;
        float4* dst = out + t * dim4;
        const bool ok = id >= 0 && id < vocab;
        if (!ok && tid == 0) RaiseFlag(err, 1);
        const float4* src = table + (ok ? static_cast<int64_t>(id) : 0) * dim4;
        for (int64_t base = tid; base < dim4; base += static_cast<int64_t>(kThreads) * VPT) {
            float4 v[VPT];
#pragma unroll
            for (int u = 0; u < VPT; ++u) {
                const int64_t i = base + static_cast<int64_t>(u) * kThreads;
                v[u] = (ok && i < dim4) ? src[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int u = 0; u < VPT; ++u) {
                const int64_t i = base + static_cast<int64_t>(u) * kThreads;
                if (i < dim4) StoreNT(dst + i, v[u]);
            }
        }
    }
}

__global__ __launch_bounds__(kThreads) void GatherF32Any(const float* __restrict__ table,
                                                         int64_t vocab, int64_t dim,
                                                         const int32_t* __restrict__ ids,
                                                         int32_t token, int64_t n_tokens,
                                                         float* __restrict__ out, int32_t* err) {
    for (int64_t t = blockIdx.x; t < n_tokens; t += gridDim.x) {
        const int32_t id = ids != nullptr ? ids[t] : token;
        const bool ok = id >= 0 && id < vocab;
        if (!ok && threadIdx.x == 0) RaiseFlag(err, 1);
        const float* src = table + (ok ? static_cast<int64_t>(id) : 0) * dim;
        for (int64_t i = threadIdx.x; i < dim; i += kThreads) {
            out[t * dim + i] = ok ? src[i] : 0.0f;
        }
    }
}

// ------------------------------------------------------------- quantizer

// The exact float operations of TensorToQ80/Q40/Q41 (src/quant.cc:136-331).
__device__ inline uint32_t FloatToHalfBits(float value) {
    const uint32_t bits = __float_as_uint(value);
    const uint32_t sign = (bits >> 16) & 0x8000u;
    const uint32_t exp8 = (bits >> 23) & 255u;
    const uint32_t man = bits & 0x7FFFFFu;
    if (exp8 == 255u) {
        return man == 0u ? (sign | 0x7C00u) : (sign | 0x7E00u | (man >> 13));
    }
    const int e = static_cast<int>(exp8) - 112;
    if (e >= 31) return sign | 0x7C00u;
    if (e <= 0) {
        if (e < -10) return sign;
        const uint32_t sig = man | 0x800000u;
        const int shift = 14 - e;
        uint32_t q = sig >> shift;
        const uint32_t rem = sig & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1);
        q += (rem > half || (rem == half && (q & 1u))) ? 1u : 0u;
        return sign | q;
    }
    uint32_t q = (static_cast<uint32_t>(e) << 10) | (man >> 13);
    const uint32_t rem = man & 0x1FFFu;
    q += (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ? 1u : 0u;
    return sign | q;
}

__device__ inline float StdMax(float a, float b) { return a < b ? b : a; }
__device__ inline float StdMin(float a, float b) { return b < a ? b : a; }

template <int QT>
__global__ __launch_bounds__(kThreads) void QuantizeKernel(const float* __restrict__ x, int64_t rows,
                                                           int64_t cols, uint8_t* __restrict__ out) {
#pragma clang fp contract(off)
    constexpr int kBB = Fmt<QT>::kBytes;
    const int64_t nb = (cols + 31) / 32;
    const int64_t total = rows * nb;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
    for (int64_t idx = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; idx < total;
         idx += stride) {
        const int64_t r = idx / nb;
        const int64_t b = idx - r * nb;
        const float* src = x + r * cols + b * 32;
        const int64_t left = cols - b * 32;
        const int len = left < 32 ? static_cast<int>(left) : 32;
        float v[32];
#pragma unroll
        for (int i = 0; i < 32; ++i) v[i] = i < len ? src[i] : 0.0f;
        uint8_t bytes[kBB];
        if (QT == MLK_Q8_0) {
            float amax = fabsf(v[0]);
#pragma unroll
            for (int i = 1; i < 32; ++i) amax = StdMax(amax, fabsf(v[i]));
            const float d = amax / 127.0f;
            const uint32_t h = FloatToHalfBits(d);
            bytes[0] = static_cast<uint8_t>(h & 0xFFu);
            bytes[1] = static_cast<uint8_t>(h >> 8);
#pragma unroll
            for (int i = 0; i < 32; ++i) {
                const float q = d != 0.0f ? roundf(v[i] / d) : 0.0f;
                bytes[2 + i] = static_cast<uint8_t>(static_cast<int8_t>(q));
            }
        } else if (QT == MLK_Q4_0) {
            float amax = fabsf(v[0]);
            float vmax = v[0];
#pragma unroll
            for (int i = 1; i < 32; ++i) {
                if (fabsf(v[i]) > amax) {
                    amax = fabsf(v[i]);
                    vmax = v[i];
                }
            }
            const float d = vmax / -8.0f;
            const float inv_d = d != 0.0f ? 1.0f / d : 0.0f;
            const uint32_t h = FloatToHalfBits(d);
            bytes[0] = static_cast<uint8_t>(h & 0xFFu);
            bytes[1] = static_cast<uint8_t>(h >> 8);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float lo = v[i] * inv_d;
                const float hi = v[i + 16] * inv_d;
                const int u0 = min(15, static_cast<int>(lo + 8.5f));
                const int u1 = min(15, static_cast<int>(hi + 8.5f));
                bytes[2 + i] = static_cast<uint8_t>(u0 | (u1 << 4));
            }
        } else {
            float lo = v[0];
            float hi = v[0];
#pragma unroll
            for (int i = 1; i < 32; ++i) {
                lo = StdMin(lo, v[i]);
                hi = StdMax(hi, v[i]);
            }
            const float m = lo;
            const float d = (hi - lo) / 15.0f;
            const float inv_d = d != 0.0f ? 1.0f / d : 0.0f;
            const uint32_t hd = FloatToHalfBits(d);
            const uint32_t hm = FloatToHalfBits(m);
            bytes[0] = static_cast<uint8_t>(hd & 0xFFu);
            bytes[1] = static_cast<uint8_t>(hd >> 8);
            bytes[2] = static_cast<uint8_t>(hm & 0xFFu);
            bytes[3] = static_cast<uint8_t>(hm >> 8);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float a = (v[i] - m) * inv_d + 0.5f;
                const float c = (v[i + 16] - m) * inv_d + 0.5f;
                const int u0 = min(15, static_cast<int>(a));
                const int u1 = min(15, static_cast<int>(c));
                bytes[4 + i] = static_cast<uint8_t>(u0 | (u1 << 4));
            }
        }
        // every block starts at an even byte offset: store 16-bit words
        uint16_t* dst = reinterpret_cast<uint16_t*>(out + idx * kBB);
#pragma unroll
        for (int i = 0; i < kBB / 2; ++i) {
            dst[i] = static_cast<uint16_t>(bytes[2 * i] | (bytes[2 * i + 1] << 8));
        }
    }
}

mlk_status CheckGather(const char* caller, const void* table, int64_t vocab, int64_t dim,
                       const int32_t* ids, int32_t token, int64_t n_tokens, const float* out) {
    if (table == nullptr) {
        return Fail(MLK_ERR_INVALID, "%s: embedding weight pointer must not be null", caller);
    }
    if (vocab <= 0 || dim <= 0 || vocab > INT32_MAX) {
        return Fail(MLK_ERR_INVALID, "%s: weight dimensions must be positive", caller);
    }
    if (n_tokens < 0) {
        return Fail(MLK_ERR_INVALID, "%s: n_tokens must not be negative", caller);
    }
    if (out == nullptr && n_tokens > 0) {
        return Fail(MLK_ERR_INVALID, "%s: output pointer must not be null", caller);
    }
    if (ids == nullptr) {
        if (n_tokens != 1) {
            return Fail(MLK_ERR_INVALID, "%s: a host token id gathers exactly one row", caller);
        }
        if (token < 0 || token >= vocab) {
            return Fail(MLK_ERR_RANGE, "%s: token_id must be in [0, vocab_size)", caller);
        }
    }
    return MLK_OK;
}

}  // namespace
}  // namespace mlk

using namespace mlk;

extern "C" {

mlk_status mlk_gather_f32(const float* table, int64_t vocab, int64_t dim, const int32_t* ids,
                          int32_t token, int64_t n_tokens, float* out, int32_t* err,
                          void* stream) {
    const mlk_status st = CheckGather("mlk_gather_f32", table, vocab, dim, ids, token, n_tokens, out);
    if (st != MLK_OK || n_tokens == 0) return st;
    const hipStream_t s = AsStream(stream);
    const unsigned grid = FullGrid(n_tokens, 1);
    if (dim % 4 == 0 && Aligned(table, 16) && Aligned(out, 16)) {
        hipLaunchKernelGGL(GatherF32Vec<4>, dim3(grid), dim3(kThreads), 0, s,
                           reinterpret_cast<const float4*>(table), vocab, dim / 4, ids, token,
                           n_tokens, reinterpret_cast<float4*>(out), err);
        return CheckLaunch("GatherF32Vec");
    }
    hipLaunchKernelGGL(GatherF32Any, dim3(grid), dim3(kThreads), 0, s, table, vocab, dim, ids,
                       token, n_tokens, out, err);
    return CheckLaunch("GatherF32Any");
}

int64_t mlk_quant_bytes(int32_t quant_type, int64_t rows, int64_t cols) {
    if (quant_type < MLK_Q8_0 || quant_type > MLK_Q4_1 || rows <= 0 || cols <= 0) return 0;
    return rows * ((cols + 31) / 32) * BlockBytes(quant_type);
}

mlk_status mlk_gather_quant(int32_t quant_type, const void* blocks, int64_t vocab, int64_t dim,
                            const int32_t* ids, int32_t token, int64_t n_tokens, float* out,
                            int32_t* err, void* stream) {
    if (quant_type < MLK_Q8_0 || quant_type > MLK_Q4_1) {
        return Fail(MLK_ERR_INVALID, "mlk_gather_quant: unknown quantization type %d", quant_type);
    }
    const mlk_status st =
        CheckGather("mlk_gather_quant", blocks, vocab, dim, ids, token, n_tokens, out);
    if (st != MLK_OK || n_tokens == 0) return st;
    // the vector path reads d|m and codes as aligned u16/u32 words
    const int vec = (dim % 4 == 0 && Aligned(out, 16) &&
                     Aligned(blocks, quant_type == MLK_Q4_1 ? 4 : 2)) ? 1 : 0;
    // one token per workgroup up to 16 workgroups per CU: measured 81-84% of
    // HBM peak by distinct rows at configs[3], against 66-78% with 8 per CU
    const unsigned grid = GridFor(n_tokens, 1, 16);
    const hipStream_t s = AsStream(stream);
    const uint8_t* b = static_cast<const uint8_t*>(blocks);
    const int u = !vec ? 0 : (dim == 4 * kQThreads ? 1 : (dim == 8 * kQThreads ? 2 : 0));
    auto launch = [&](auto qt) {
        constexpr int Q = decltype(qt)::value;
        if (u == 1) {
            hipLaunchKernelGGL((GatherQuantKernel<Q, 1>), dim3(grid), dim3(kQThreads), 0, s, b,
                               vocab, dim, ids, token, n_tokens, out, err, vec);
        } else if (u == 2) {
            hipLaunchKernelGGL((GatherQuantKernel<Q, 2>), dim3(grid), dim3(kQThreads), 0, s, b,
                               vocab, dim, ids, token, n_tokens, out, err, vec);
        } else {
            hipLaunchKernelGGL((GatherQuantKernel<Q, 0>), dim3(grid), dim3(kQThreads), 0, s, b,
                               vocab, dim, ids, token, n_tokens, out, err, vec);
        }
    };
    switch (quant_type) {
        case MLK_Q8_0: launch(std::integral_constant<int, MLK_Q8_0>{}); break;
        case MLK_Q4_0: launch(std::integral_constant<int, MLK_Q4_0>{}); break;
        default: launch(std::integral_constant<int, MLK_Q4_1>{}); break;
    }
    return CheckLaunch("GatherQuantKernel");
}

mlk_status mlk_quantize(int32_t quant_type, const float* x, int64_t rows, int64_t cols,
                        void* blocks, void* stream) {
    if (quant_type < MLK_Q8_0 || quant_type > MLK_Q4_1) {
        return Fail(MLK_ERR_INVALID, "mlk_quantize: unknown quantization type %d", quant_type);
    }
    if (x == nullptr || blocks == nullptr) {
        return Fail(MLK_ERR_INVALID, "mlk_quantize: pointers must not be null");
    }
    if (rows <= 0 || cols <= 0) {
        return Fail(MLK_ERR_INVALID, "mlk_quantize: dimensions must be positive");
    }
    if (!Aligned(blocks, 2)) {
        return Fail(MLK_ERR_INVALID, "mlk_quantize: block buffer must be 2-byte aligned");
    }
    const int64_t total = rows * ((cols + 31) / 32);
    const unsigned grid = GridFor(total, kThreads, 8);
    const hipStream_t s = AsStream(stream);
    uint8_t* out = static_cast<uint8_t*>(blocks);
    switch (quant_type) {
        case MLK_Q8_0:
            hipLaunchKernelGGL(QuantizeKernel<MLK_Q8_0>, dim3(grid), dim3(kThreads), 0, s, x, rows,
                               cols, out);
            break;
        case MLK_Q4_0:
            hipLaunchKernelGGL(QuantizeKernel<MLK_Q4_0>, dim3(grid), dim3(kThreads), 0, s, x, rows,
                               cols, out);
            break;
        default:
            hipLaunchKernelGGL(QuantizeKernel<MLK_Q4_1>, dim3(grid), dim3(kThreads), 0, s, x, rows,
                               cols, out);
            break;
    }
    return CheckLaunch("QuantizeKernel");
}

}  // extern "C"
