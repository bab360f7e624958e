/*
 * oracle.c -- CPU restatement of cpp-minilamma's per-layer ops.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h): the checker for the HIP kernels
 * and the "port" CPU baseline.  The product never links or loads it.
 *
 * Built with -ffp-contract=off so that a*b+c is never fused: the reference's
 * own build (CMakeLists.txt, no -march/-mfma) does not fuse either, which is
 * what makes the quantizer and dequantizer outputs bit-identical to it.
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stddef.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* ------------------------------------------------------------------ fp16 */

float orc_fp16_to_fp32(uint16_t h)
{
    /* IEEE-754 binary16 -> binary32, exact for every code; NaN payloads are
     * carried over (src/quant.cc:81-112). */
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const uint32_t exp5 = (h >> 10) & 31u;
    uint32_t frac = h & 1023u;
    uint32_t bits;
    if (exp5 == 31u) {
        bits = sign | 0x7F800000u | (frac << 13);
    } else if (exp5 != 0u) {
        bits = sign | ((exp5 + 112u) << 23) | (frac << 13);
    } else if (frac == 0u) {
        bits = sign;
    } else {
        /* subnormal: frac * 2^-24; normalise so bit 10 is the hidden one */
        uint32_t shift = 0;
        while ((frac & 0x400u) == 0u) {
            frac <<= 1;
            ++shift;
        }
        bits = sign | ((113u - shift) << 23) | ((frac & 1023u) << 13);
    }
    float f;
    memcpy(&f, &bits, sizeof f);
    return f;
}

uint16_t orc_fp32_to_fp16(float value)
{
    /* Round to nearest, ties to even (src/quant.cc:31-79). */
    uint32_t bits;
    memcpy(&bits, &value, sizeof bits);
    const uint32_t sign = (bits >> 16) & 0x8000u;
    const uint32_t exp8 = (bits >> 23) & 255u;
    const uint32_t man = bits & 0x7FFFFFu;
    if (exp8 == 255u) {
        /* inf stays inf; NaN keeps its top payload bits and is made quiet */
        return (uint16_t)(man == 0u ? (sign | 0x7C00u) : (sign | 0x7E00u | (man >> 13)));
    }
    const int e = (int)exp8 - 112; /* biased binary16 exponent */
    if (e >= 31) {
        return (uint16_t)(sign | 0x7C00u);
    }
    if (e <= 0) {
        if (e < -10) {
            return (uint16_t)sign; /* below half the smallest subnormal */
        }
        const uint32_t sig = man | 0x800000u;
        const int shift = 14 - e; /* 14..24 */
        uint32_t q = sig >> shift;
        const uint32_t rem = sig & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1);
        q += (rem > half || (rem == half && (q & 1u))) ? 1u : 0u;
        return (uint16_t)(sign | q);
    }
    uint32_t q = ((uint32_t)e << 10) | (man >> 13);
    const uint32_t rem = man & 0x1FFFu;
    /* a carry out of the fraction bumps the exponent (to inf at the top) */
    q += (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ? 1u : 0u;
    return (uint16_t)(sign | q);
}

void orc_fp16_to_fp32_array(const uint16_t* in, float* out, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) {
        out[i] = orc_fp16_to_fp32(in[i]);
    }
}

void orc_fp32_to_fp16_array(const float* in, uint16_t* out, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) {
        out[i] = orc_fp32_to_fp16(in[i]);
    }
}

/* ------------------------------------------------------------- blocks */

static void put_u16(uint8_t* p, uint16_t v)
{
    p[0] = (uint8_t)(v & 0xFFu);
    p[1] = (uint8_t)(v >> 8);
}

static uint16_t get_u16(const uint8_t* p)
{
    return (uint16_t)(p[0] | ((uint16_t)p[1] << 8));
}

static int64_t row_blocks(int64_t cols)
{
    return (cols + ORC_QK - 1) / ORC_QK;
}

/* Copy block b of a row into 32 floats, zero padded past the row end. */
static int load_padded(const float* row, int64_t cols, int64_t b, float out[ORC_QK])
{
    const int64_t off = b * ORC_QK;
    const int64_t left = cols - off;
    const int len = left < ORC_QK ? (int)left : ORC_QK;
    for (int i = 0; i < ORC_QK; ++i) {
        out[i] = i < len ? row[off + i] : 0.0f;
    }
    return len;
}

/* std::max / std::min over floats as the reference calls them. */
static float std_max(float a, float b) { return a < b ? b : a; }
static float std_min(float a, float b) { return b < a ? b : a; }

int orc_quantize_q8_0(const float* x, int64_t rows, int64_t cols, uint8_t* blocks)
{
    if (rows <= 0 || cols <= 0) {
        return ORC_EINVAL;
    }
    const int64_t nb = row_blocks(cols);
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t b = 0; b < nb; ++b) {
            float v[ORC_QK];
            load_padded(x + r * cols, cols, b, v);
            uint8_t* blk = blocks + (r * nb + b) * ORC_Q8_0_BYTES;
            float amax = fabsf(v[0]);
            for (int i = 1; i < ORC_QK; ++i) {
                amax = std_max(amax, fabsf(v[i]));
            }
            const float d = amax / 127.0f;
            put_u16(blk, orc_fp32_to_fp16(d));
            for (int i = 0; i < ORC_QK; ++i) {
                /* divide by the float scale, not the fp16-rounded one;
                 * roundf rounds halves away from zero like std::round */
                const float q = d != 0.0f ? roundf(v[i] / d) : 0.0f;
                blk[2 + i] = (uint8_t)(int8_t)q;
            }
        }
    }
    return ORC_OK;
}

int orc_quantize_q4_0(const float* x, int64_t rows, int64_t cols, uint8_t* blocks)
{
    if (rows <= 0 || cols <= 0) {
        return ORC_EINVAL;
    }
    const int64_t nb = row_blocks(cols);
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t b = 0; b < nb; ++b) {
            float v[ORC_QK];
            load_padded(x + r * cols, cols, b, v);
            uint8_t* blk = blocks + (r * nb + b) * ORC_Q4_0_BYTES;
            /* signed value of the first element with the largest magnitude */
            float amax = fabsf(v[0]);
            float vmax = v[0];
            for (int i = 1; i < ORC_QK; ++i) {
                if (fabsf(v[i]) > amax) {
                    amax = fabsf(v[i]);
                    vmax = v[i];
                }
            }
            const float d = vmax / -8.0f;
            const float inv_d = d != 0.0f ? 1.0f / d : 0.0f;
            put_u16(blk, orc_fp32_to_fp16(d));
            for (int i = 0; i < 16; ++i) {
                const float lo = v[i] * inv_d;
                const float hi = v[i + 16] * inv_d;
                int u0 = (int)(lo + 8.5f);
                int u1 = (int)(hi + 8.5f);
                u0 = u0 < 15 ? u0 : 15;
                u1 = u1 < 15 ? u1 : 15;
                blk[2 + i] = (uint8_t)(u0 | (u1 << 4));
            }
        }
    }
    return ORC_OK;
}

int orc_quantize_q4_1(const float* x, int64_t rows, int64_t cols, uint8_t* blocks)
{
    if (rows <= 0 || cols <= 0) {
        return ORC_EINVAL;
    }
    const int64_t nb = row_blocks(cols);
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t b = 0; b < nb; ++b) {
            float v[ORC_QK];
            load_padded(x + r * cols, cols, b, v);
            uint8_t* blk = blocks + (r * nb + b) * ORC_Q4_1_BYTES;
            /* the zero padding takes part in min/max */
            float lo = v[0];
            float hi = v[0];
            for (int i = 1; i < ORC_QK; ++i) {
                lo = std_min(lo, v[i]);
                hi = std_max(hi, v[i]);
            }
            const float m = lo;
            const float d = (hi - lo) / 15.0f;
            const float inv_d = d != 0.0f ? 1.0f / d : 0.0f;
            put_u16(blk, orc_fp32_to_fp16(d));
            put_u16(blk + 2, orc_fp32_to_fp16(m));
            for (int i = 0; i < 16; ++i) {
                int u0 = (int)((v[i] - m) * inv_d + 0.5f);
                int u1 = (int)((v[i + 16] - m) * inv_d + 0.5f);
                u0 = u0 < 15 ? u0 : 15;
                u1 = u1 < 15 ? u1 : 15;
                blk[4 + i] = (uint8_t)(u0 | (u1 << 4));
            }
        }
    }
    return ORC_OK;
}

/* One dequantized block: only the first len elements are written. */
static void dequant_block(int type, const uint8_t* blk, int len, float* out)
{
    const float d = orc_fp16_to_fp32(get_u16(blk));
    if (type == 0) {
        for (int i = 0; i < len; ++i) {
            out[i] = d * (float)(int8_t)blk[2 + i];
        }
    } else if (type == 1) {
        for (int i = 0; i < len; ++i) {
            const uint8_t byte = blk[2 + (i & 15)];
            const int code = (i < 16 ? (byte & 15) : (byte >> 4)) - 8;
            out[i] = d * (float)code;
        }
    } else {
        const float m = orc_fp16_to_fp32(get_u16(blk + 2));
        for (int i = 0; i < len; ++i) {
            const uint8_t byte = blk[4 + (i & 15)];
            const int code = i < 16 ? (byte & 15) : (byte >> 4);
            out[i] = d * (float)code + m;
        }
    }
}

static const int64_t kBlockBytes[3] = {ORC_Q8_0_BYTES, ORC_Q4_0_BYTES, ORC_Q4_1_BYTES};

static void dequant_row(int type, const uint8_t* row, int64_t cols, float* out)
{
    const int64_t nb = row_blocks(cols);
    for (int64_t b = 0; b < nb; ++b) {
        const int64_t left = cols - b * ORC_QK;
        const int len = left < ORC_QK ? (int)left : ORC_QK;
        dequant_block(type, row + b * kBlockBytes[type], len, out + b * ORC_QK);
    }
}

static int dequantize(int type, const uint8_t* blocks, int64_t rows, int64_t cols, float* out)
{
    if (rows <= 0 || cols <= 0) {
        return ORC_EINVAL;
    }
    const int64_t row_bytes = row_blocks(cols) * kBlockBytes[type];
    for (int64_t r = 0; r < rows; ++r) {
        dequant_row(type, blocks + r * row_bytes, cols, out + r * cols);
    }
    return ORC_OK;
}

int orc_dequantize_q8_0(const uint8_t* b, int64_t rows, int64_t cols, float* out)
{
    return dequantize(0, b, rows, cols, out);
}

int orc_dequantize_q4_0(const uint8_t* b, int64_t rows, int64_t cols, float* out)
{
    return dequantize(1, b, rows, cols, out);
}

int orc_dequantize_q4_1(const uint8_t* b, int64_t rows, int64_t cols, float* out)
{
    return dequantize(2, b, rows, cols, out);
}

/* -------------------------------------------------------------- gather */

static int ids_valid(const int32_t* ids, int64_t n, int64_t vocab)
{
    for (int64_t t = 0; t < n; ++t) {
        if (ids[t] < 0 || ids[t] >= vocab) {
            return 0;
        }
    }
    return 1;
}

int orc_gather_f32(const float* table, int64_t vocab, int64_t dim,
                   const int32_t* ids, int64_t n_tokens, float* out)
{
    if (vocab <= 0 || dim <= 0 || n_tokens < 0 || !ids_valid(ids, n_tokens, vocab)) {
        return ORC_EINVAL;
    }
    for (int64_t t = 0; t < n_tokens; ++t) {
        const float* row = table + (int64_t)ids[t] * dim;
        for (int64_t i = 0; i < dim; ++i) {
            out[t * dim + i] = row[i];
        }
    }
    return ORC_OK;
}

int orc_gather_quant(int quant_type, const uint8_t* blocks, int64_t vocab, int64_t dim,
                     const int32_t* ids, int64_t n_tokens, float* out)
{
    if (quant_type < 0 || quant_type > 2 || vocab <= 0 || dim <= 0 || n_tokens < 0 ||
        !ids_valid(ids, n_tokens, vocab)) {
        return ORC_EINVAL;
    }
    const int64_t row_bytes = row_blocks(dim) * kBlockBytes[quant_type];
    for (int64_t t = 0; t < n_tokens; ++t) {
        dequant_row(quant_type, blocks + (int64_t)ids[t] * row_bytes, dim, out + t * dim);
    }
    return ORC_OK;
}

/* ---------------------------------------------------------- elementwise */

void orc_add(const float* a, const float* b, float* y, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) {
        y[i] = a[i] + b[i];
    }
}

void orc_mul(const float* a, const float* b, float* y, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) {
        y[i] = a[i] * b[i];
    }
}

static float silu1(float v)
{
    const float sig = 1.0f / (1.0f + expf(-v));
    return v * sig;
}

void orc_silu(const float* x, float* y, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) {
        y[i] = silu1(x[i]);
    }
}

void orc_swiglu(const float* gate, const float* up, float* y, int64_t n)
{
    /* Silu first into a float, then the product: the same two roundings as
     * ElementwiseMul(Silu(gate), up). */
    for (int64_t i = 0; i < n; ++i) {
        const float s = silu1(gate[i]);
        y[i] = s * up[i];
    }
}

int orc_softmax(const float* x, float* y, int64_t n)
{
    if (n <= 0) {
        return ORC_EINVAL;
    }
    float mx = x[0];
    for (int64_t i = 1; i < n; ++i) {
        if (x[i] > mx) {
            mx = x[i];
        }
    }
    float sum = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
        y[i] = expf(x[i] - mx);
        sum += y[i];
    }
    for (int64_t i = 0; i < n; ++i) {
        y[i] /= sum;
    }
    return ORC_OK;
}

/* -------------------------------------------------------------- rmsnorm */

int orc_rmsnorm_row(const float* x, const float* w, float* y, int64_t dim, float eps)
{
    if (dim <= 0 || !isfinite(eps) || eps < 0.0f) {
        return ORC_EINVAL;
    }
    double ss = 0.0;
    for (int64_t i = 0; i < dim; ++i) {
        const double v = (double)x[i];
        ss += v * v;
    }
    const double den = sqrt(ss / (double)dim + (double)eps);
    if (!isfinite(den) || den <= 0.0) {
        return ORC_EINVAL;
    }
    const double scale = 1.0 / den;
    for (int64_t i = 0; i < dim; ++i) {
        y[i] = (float)((double)x[i] * (double)w[i] * scale);
    }
    return ORC_OK;
}

int orc_add_rmsnorm(float* residual, const float* delta, const float* w, float* y,
                    int64_t n_rows, int64_t dim, float eps)
{
    if (n_rows < 0 || dim <= 0 || !isfinite(eps) || eps < 0.0f) {
        return ORC_EINVAL;
    }
    for (int64_t r = 0; r < n_rows; ++r) {
        float* row = residual + r * dim;
        if (delta != NULL) {
            orc_add(row, delta + r * dim, row, dim);
        }
        const int rc = orc_rmsnorm_row(row, w, y + r * dim, dim, eps);
        if (rc != ORC_OK) {
            return rc;
        }
    }
    return ORC_OK;
}

/* ----------------------------------------------------------------- rope */

int orc_rope_token(float* q, float* k, int32_t n_heads, int32_t n_kv_heads,
                   int32_t head_dim, int32_t pos, float theta, int32_t rope_type)
{
    if (pos < 0 || !isfinite(theta) || theta <= 0.0f || n_heads <= 0 || n_kv_heads <= 0 ||
        head_dim <= 0 || (head_dim % 2) != 0 ||
        (rope_type != ORC_ROPE_NORMAL && rope_type != ORC_ROPE_NEOX)) {
        return ORC_EINVAL;
    }
    const int half = head_dim / 2;
    for (int i = 0; i < half; ++i) {
        /* angle, cos and sin in double, as the reference computes them */
        const double angle = (double)pos * pow((double)theta, -2.0 * i / head_dim);
        const double c = cos(angle);
        const double s = sin(angle);
        const size_t a = rope_type == ORC_ROPE_NORMAL ? (size_t)i * 2 : (size_t)i;
        const size_t b = rope_type == ORC_ROPE_NORMAL ? a + 1 : a + (size_t)half;
        for (int which = 0; which < 2; ++which) {
            float* base = which == 0 ? q : k;
            const int heads = which == 0 ? n_heads : n_kv_heads;
            for (int h = 0; h < heads; ++h) {
                float* v = base + (size_t)h * (size_t)head_dim;
                const double x0 = v[a];
                const double x1 = v[b];
                v[a] = (float)(x0 * c - x1 * s);
                v[b] = (float)(x0 * s + x1 * c);
            }
        }
    }
    return ORC_OK;
}

int orc_rope(float* q, float* k, int64_t n_tokens, int32_t n_heads, int32_t n_kv_heads,
             int32_t head_dim, const int32_t* positions, int32_t pos0,
             float theta, int32_t rope_type)
{
    if (n_tokens < 0 || n_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0) {
        return ORC_EINVAL;
    }
    const int64_t qs = (int64_t)n_heads * head_dim;
    const int64_t ks = (int64_t)n_kv_heads * head_dim;
    for (int64_t t = 0; t < n_tokens; ++t) {
        const int32_t pos = positions != NULL ? positions[t] : (int32_t)(pos0 + t);
        const int rc = orc_rope_token(q + t * qs, k + t * ks, n_heads, n_kv_heads,
                                      head_dim, pos, theta, rope_type);
        if (rc != ORC_OK) {
            return rc;
        }
    }
    return ORC_OK;
}

/* ------------------------------------------------------------- linear */

/* thread_pool/thread_pool.cc:31-90 ParallelFor: n tasks in static
 * contiguous chunks, the first n % threads chunks one longer; serial when
 * there are fewer than 16 tasks per thread. */
typedef void (*par_fn)(void* ctx, int64_t begin, int64_t end);

typedef struct {
    par_fn fn;
    void* ctx;
    int64_t begin, end;
} par_job;

static void* par_run(void* arg)
{
    par_job* j = (par_job*)arg;
    j->fn(j->ctx, j->begin, j->end);
    return NULL;
}

static int par_for(int64_t n, int n_threads, par_fn fn, void* ctx)
{
    const int nt = orc_parallel_threads(n_threads);
    if (n <= 0) {
        return ORC_OK;
    }
    if (nt <= 1 || n / 16 < nt) {
        fn(ctx, 0, n);
        return ORC_OK;
    }
    par_job* jobs = (par_job*)calloc((size_t)nt, sizeof(par_job));
    pthread_t* th = (pthread_t*)calloc((size_t)nt, sizeof(pthread_t));
    if (jobs == NULL || th == NULL) {
        free(jobs);
        free(th);
        return ORC_EINVAL;
    }
    const int64_t chunk = n / nt;
    const int64_t remain = n % nt;
    int64_t start = 0;
    int started = 0;
    for (int i = 0; i < nt; ++i) {
        jobs[i].fn = fn;
        jobs[i].ctx = ctx;
        jobs[i].begin = start;
        jobs[i].end = start + chunk + (i < remain ? 1 : 0);
        start = jobs[i].end;
        if (pthread_create(&th[i], NULL, par_run, &jobs[i]) != 0) {
            break;
        }
        ++started;
    }
    for (int i = 0; i < started; ++i) {
        pthread_join(th[i], NULL);
    }
    /* a thread that could not start leaves its chunk to the caller */
    for (int i = started; i < nt; ++i) {
        fn(ctx, jobs[i].begin, jobs[i].end);
    }
    free(jobs);
    free(th);
    return ORC_OK;
}

typedef struct {
    int type;  /* -1: F32 weights */
    const float* x;
    const void* w;
    const float* bias;
    float* y;
    int64_t in, out;
} linear_job;

static void linear_outputs(void* arg, int64_t begin, int64_t end)
{
    const linear_job* j = (const linear_job*)arg;
    const int64_t nb = row_blocks(j->in);
    for (int64_t index = begin; index < end; ++index) {
        const int64_t row = index / j->out;
        const int64_t col = index % j->out;
        const float* xr = j->x + row * j->in;
        float sum = 0.0f;
        if (j->type < 0) {
            const float* wr = (const float*)j->w + col * j->in;
            for (int64_t k = 0; k < j->in; ++k) {
                sum += xr[k] * wr[k];
            }
        } else {
            const int64_t bb = kBlockBytes[j->type];
            const uint8_t* wr = (const uint8_t*)j->w + col * nb * bb;
            for (int64_t b = 0; b < nb; ++b) {
                const int64_t left = j->in - b * ORC_QK;
                const int len = left < ORC_QK ? (int)left : ORC_QK;
                float w[ORC_QK];
                dequant_block(j->type, wr + b * bb, len, w);
                for (int i = 0; i < len; ++i) {
                    sum += xr[b * ORC_QK + i] * w[i];
                }
            }
        }
        if (j->bias != NULL) {
            sum += j->bias[col];
        }
        j->y[index] = sum;
    }
}

static int linear_common(int type, const float* x, const void* w, const float* bias, float* y,
                         int64_t rows, int64_t in, int64_t out, int n_threads)
{
    if (rows <= 0 || in <= 0 || out <= 0 || rows > 0x7FFFFFFF / out) {
        return ORC_EINVAL;
    }
    linear_job job = {type, x, w, bias, y, in, out};
    return par_for(rows * out, n_threads, linear_outputs, &job);
}

int orc_linear_quant(int quant_type, const float* x, const uint8_t* blocks, const float* bias,
                     float* y, int64_t rows, int64_t in_features, int64_t out_features,
                     int n_threads)
{
    if (quant_type < 0 || quant_type > 2) {
        return ORC_EINVAL;
    }
    return linear_common(quant_type, x, blocks, bias, y, rows, in_features, out_features,
                         n_threads);
}

int orc_linear_f32(const float* x, const float* w, const float* bias, float* y, int64_t rows,
                   int64_t in_features, int64_t out_features, int n_threads)
{
    return linear_common(-1, x, w, bias, y, rows, in_features, out_features, n_threads);
}

typedef struct {
    const float* a;
    const float* b;
    float* c;
    int64_t k, n;
} matmul_job;

static void matmul_outputs(void* arg, int64_t begin, int64_t end)
{
    const matmul_job* j = (const matmul_job*)arg;
    for (int64_t index = begin; index < end; ++index) {
        const int64_t row = index / j->n;
        const int64_t col = index % j->n;
        float sum = 0.0f;
        for (int64_t k = 0; k < j->k; ++k) {
            sum += j->a[row * j->k + k] * j->b[k * j->n + col];
        }
        j->c[index] = sum;
    }
}

int orc_matmul_f32(const float* a, const float* b, float* c, int64_t m, int64_t k, int64_t n,
                   int n_threads)
{
    if (m <= 0 || k <= 0 || n <= 0 || m > 0x7FFFFFFF / n) {
        return ORC_EINVAL;
    }
    matmul_job job = {a, b, c, k, n};
    return par_for(m * n, n_threads, matmul_outputs, &job);
}

/* ------------------------------------------------ attention, KV cache */

static int kv_args_ok(int64_t n_layers, int64_t max_seq, int32_t n_kv_heads, int32_t head_dim,
                      int64_t layer)
{
    return n_layers > 0 && max_seq > 0 && n_kv_heads > 0 && head_dim > 0 && layer >= 0 &&
           layer < n_layers;
}

int orc_kv_write(float* k_cache, float* v_cache, int64_t n_layers, int64_t max_seq,
                 int32_t n_kv_heads, int32_t head_dim, int64_t layer, const int32_t* positions,
                 int64_t n_tokens, const float* k, const float* v)
{
    if (!kv_args_ok(n_layers, max_seq, n_kv_heads, head_dim, layer) || n_tokens < 0) {
        return ORC_EINVAL;
    }
    const int64_t row = (int64_t)n_kv_heads * head_dim;
    for (int64_t t = 0; t < n_tokens; ++t) {
        if (positions[t] < 0 || positions[t] >= max_seq) {
            return ORC_EINVAL; /* KvCache::Write throws "Pos Out Of Range" */
        }
    }
    for (int64_t t = 0; t < n_tokens; ++t) {
        const int64_t slot = (layer * max_seq + positions[t]) * row;
        memcpy(k_cache + slot, k + t * row, (size_t)row * sizeof(float));
        memcpy(v_cache + slot, v + t * row, (size_t)row * sizeof(float));
    }
    return ORC_OK;
}

int orc_attention(const float* q, const float* k_cache, const float* v_cache, int64_t n_layers,
                  int64_t max_seq, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                  int64_t layer, const int32_t* positions, int64_t n_tokens, float* out)
{
    if (!kv_args_ok(n_layers, max_seq, n_kv_heads, head_dim, layer) || n_tokens < 0 ||
        n_heads <= 0 || n_heads % n_kv_heads != 0) {
        return ORC_EINVAL;
    }
    for (int64_t t = 0; t < n_tokens; ++t) {
        if (positions[t] < 0 || positions[t] >= max_seq) {
            return ORC_EINVAL;
        }
    }
    const int64_t hd = head_dim;
    const int64_t row = (int64_t)n_kv_heads * hd;
    const int32_t group = n_heads / n_kv_heads;
    const float scale = 1.0f / sqrtf((float)head_dim);
    float* scores = (float*)malloc((size_t)max_seq * sizeof(float));
    float* probs = (float*)malloc((size_t)max_seq * sizeof(float));
    if (scores == NULL || probs == NULL) {
        free(scores);
        free(probs);
        return ORC_EINVAL;
    }
    for (int64_t t = 0; t < n_tokens; ++t) {
        const int64_t pos = positions[t];
        for (int32_t i = 0; i < n_heads; ++i) {
            const int64_t kvh = i / group;
            const float* qh = q + (t * n_heads + i) * hd;
            for (int64_t j = 0; j <= pos; ++j) {
                const float* kr = k_cache + (layer * max_seq + j) * row + kvh * hd;
                float dot = 0.0f;
                for (int64_t d = 0; d < hd; ++d) {
                    dot += qh[d] * kr[d];
                }
                scores[j] = dot * scale;
            }
            orc_softmax(scores, probs, pos + 1);
            float* oh = out + (t * n_heads + i) * hd;
            for (int64_t d = 0; d < hd; ++d) {
                float val = 0.0f;
                for (int64_t j = 0; j <= pos; ++j) {
                    val += probs[j] * v_cache[(layer * max_seq + j) * row + kvh * hd + d];
                }
                oh[d] = val;
            }
        }
    }
    free(scores);
    free(probs);
    return ORC_OK;
}

/* --------------------------------------------------- CPU baseline port */

int orc_parallel_threads(int n_threads)
{
    if (n_threads > 0) {
        return n_threads;
    }
    const long n = sysconf(_SC_NPROCESSORS_ONLN);
    return n > 0 ? (int)n : 4; /* thread_pool/thread_pool.cc:13-22 */
}

typedef struct {
    const float* table;
    int64_t vocab, dim;
    const int32_t* ids;
    float* x;
    const float* delta;
    const float* norm_w;
    float* y;
    float eps;
    float* q;
    float* k;
    int32_t n_heads, n_kv_heads, head_dim;
    const int32_t* positions;
    float theta;
    const float* gate;
    const float* up;
    float* ffn_out;
    int64_t ffn_dim;
    int64_t begin, end;
    int rc;
} chain_job;

static void* chain_rows(void* arg)
{
    chain_job* j = (chain_job*)arg;
    const int64_t qs = (int64_t)j->n_heads * j->head_dim;
    const int64_t ks = (int64_t)j->n_kv_heads * j->head_dim;
    for (int64_t t = j->begin; t < j->end && j->rc == ORC_OK; ++t) {
        const int32_t id = j->ids[t];
        if (id < 0 || id >= j->vocab) {
            j->rc = ORC_EINVAL;
            break;
        }
        float* x = j->x + t * j->dim;
        memcpy(x, j->table + (int64_t)id * j->dim, (size_t)j->dim * sizeof(float));
        orc_add(x, j->delta + t * j->dim, x, j->dim);
        j->rc = orc_rmsnorm_row(x, j->norm_w, j->y + t * j->dim, j->dim, j->eps);
        if (j->rc != ORC_OK) {
            break;
        }
        j->rc = orc_rope_token(j->q + t * qs, j->k + t * ks, j->n_heads, j->n_kv_heads,
                               j->head_dim, j->positions[t], j->theta, ORC_ROPE_NORMAL);
        if (j->rc != ORC_OK) {
            break;
        }
        orc_swiglu(j->gate + t * j->ffn_dim, j->up + t * j->ffn_dim,
                   j->ffn_out + t * j->ffn_dim, j->ffn_dim);
    }
    return NULL;
}

int orc_chain(const float* table, int64_t vocab, int64_t dim, const int32_t* ids,
              float* x, const float* delta, const float* norm_w, float* y, float eps,
              float* q, float* k, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
              const int32_t* positions, float theta,
              const float* gate, const float* up, float* ffn_out, int64_t ffn_dim,
              int64_t n_tokens, int n_threads)
{
    if (n_tokens < 0 || n_tokens > 0x7FFFFFFF) {
        return ORC_EINVAL;
    }
    chain_job base = {table, vocab, dim, ids, x, delta, norm_w, y, eps, q, k,
                      n_heads, n_kv_heads, head_dim, positions, theta,
                      gate, up, ffn_out, ffn_dim, 0, n_tokens, ORC_OK};
    const int nt = orc_parallel_threads(n_threads);
    const int n = (int)n_tokens;
    /* ParallelFor: serial when there is less than 16 rows per thread */
    if (nt <= 1 || n / 16 < nt) {
        chain_rows(&base);
        return base.rc;
    }
    chain_job* jobs = (chain_job*)calloc((size_t)nt, sizeof(chain_job));
    pthread_t* th = (pthread_t*)calloc((size_t)nt, sizeof(pthread_t));
    if (jobs == NULL || th == NULL) {
        free(jobs);
        free(th);
        return ORC_EINVAL;
    }
    const int chunk = n / nt;
    const int remain = n % nt;
    int start = 0;
    int started = 0;
    for (int i = 0; i < nt; ++i) {
        jobs[i] = base;
        jobs[i].begin = start;
        jobs[i].end = start + chunk + (i < remain ? 1 : 0);
        start = (int)jobs[i].end;
        if (pthread_create(&th[i], NULL, chain_rows, &jobs[i]) != 0) {
            break;
        }
        ++started;
    }
    int rc = started == nt ? ORC_OK : ORC_EINVAL;
    for (int i = 0; i < started; ++i) {
        pthread_join(th[i], NULL);
        if (rc == ORC_OK && jobs[i].rc != ORC_OK) {
            rc = jobs[i].rc;
        }
    }
    free(jobs);
    free(th);
    return rc;
}
