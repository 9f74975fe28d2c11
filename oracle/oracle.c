/*
 * CPU oracle for the Q8_0 block-quantized linear path (TEST INFRASTRUCTURE ONLY; see oracle.h).
 *
 * A plain-C restatement of the reference's CPU kernels, written from their semantics: each function names the
 * reference lines it follows. Built with -O2 -ffp-contract=off, so every fused multiply-add below is an explicit
 * fmaf that mirrors either an _mm256_fmadd_ps in the reference or a contraction that GCC performs when it builds
 * the reference with -mfma (its default -ffp-contract=fast for C++).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define Q8_BLOCK 32
#define Q8_BYTES 34

/* ------------------------------------------------------------------------------------------------ fp16 */

float orc_half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t mant = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (mant << 13);
    } else if (exp != 0) {
        bits = sign | ((exp + 112u) << 23) | (mant << 13);
    } else if (mant == 0) {
        bits = sign;
    } else {
        /* subnormal half: mant * 2^-24, normalised */
        int e = -1;
        do {
            ++e;
            mant <<= 1;
        } while ((mant & 0x400u) == 0);
        bits = sign | ((uint32_t)(112 - e) << 23) | ((mant & 0x3ffu) << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t orc_float_to_half(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));  /* quiet NaN */
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);                         /* rounds to infinity */
    const uint32_t e = ax >> 23;
    if (e < 113) {
        /* below 2^-14: a half subnormal, h = round(value / 2^-24) with ties to even */
        if (ax < 0x33000000u) return sign;
        const uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
        const uint32_t s = 126u - e;
        uint32_t h = mant >> s;
        const uint32_t rem = mant & ((1u << s) - 1u), half = 1u << (s - 1u);
        if (rem > half || (rem == half && (h & 1u))) ++h;
        return (uint16_t)(sign | h);
    }
    uint32_t h = ((e - 112u) << 10) | ((ax >> 13) & 0x3ffu);
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
}

void orc_half_to_float_n(const uint16_t* h, int64_t count, float* out) {
    for (int64_t i = 0; i < count; ++i) out[i] = orc_half_to_float(h[i]);
}

void orc_float_to_half_n(const float* f, int64_t count, uint16_t* out) {
    for (int64_t i = 0; i < count; ++i) out[i] = orc_float_to_half(f[i]);
}

static inline float block_scale(const uint8_t* blk) { return orc_half_to_float((uint16_t)(blk[0] | (blk[1] << 8))); }

/* ------------------------------------------------------------------------------------------------ Q8_0 format */

/* ggml quantize_row_q8_0_ref as restated by gguf-py's Q8_0.quantize_blocks (called from
 * tools/export_full_gguf.py:332-335 and tests/python/test_fused_packed.py:40): d = amax / 127 in fp32,
 * id = d ? 1 / d : 0, q = round-half-away(x * id), d stored as fp16. */
void orc_q8_0_quantize(const float* w, int64_t n, int64_t k, uint8_t* blocks) {
    const int64_t nb = k / Q8_BLOCK;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < n; ++r)
        for (int64_t b = 0; b < nb; ++b) {
            const float* x = w + r * k + b * Q8_BLOCK;
            uint8_t* out = blocks + (r * nb + b) * Q8_BYTES;
            float amax = 0.0f;
            for (int t = 0; t < Q8_BLOCK; ++t) amax = fmaxf(amax, fabsf(x[t]));
            const float d = amax / 127.0f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            const uint16_t dh = orc_float_to_half(d);
            out[0] = (uint8_t)(dh & 0xff);
            out[1] = (uint8_t)(dh >> 8);
            for (int t = 0; t < Q8_BLOCK; ++t) out[2 + t] = (uint8_t)(int8_t)roundf(x[t] * id);
        }
}

/* tools/idol_packed.py:28-31,71 (codes * scale in fp32) and tools/idol_triton.py:24-33. */
void orc_q8_0_dequant(const uint8_t* blocks, int64_t n, int64_t k, float* w) {
    const int64_t nb = k / Q8_BLOCK;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < n; ++r)
        for (int64_t b = 0; b < nb; ++b) {
            const uint8_t* blk = blocks + (r * nb + b) * Q8_BYTES;
            const float d = block_scale(blk);
            for (int t = 0; t < Q8_BLOCK; ++t) w[r * k + b * Q8_BLOCK + t] = (float)(int8_t)blk[2 + t] * d;
        }
}

int64_t orc_panel_bytes(int64_t n, int64_t k) {
    /* src/kernels.cpp:512-514 for bits 8, group 32: (k / 32) * (64 + 2 * 32 * 8) bytes per 16-column panel */
    return ((n + 15) / 16) * (k / 32) * (64 + 2 * 32 * 8);
}

/* tools/gguf_to_decoder.py:16-40 (native_blob) into the panel layout of src/kernels.hpp:33-51 as written by
 * tools/idolq.py:137-166 for bits 8: per panel of 16 columns and group of 32 k, 16 fp16 scales, 16 fp16
 * minimums, then byte k * 16 + c holds the code of column c at depth k. */
int orc_q8_0_to_panel(const uint8_t* blocks, int64_t n, int64_t k, uint8_t* blob) {
    const int64_t nb = k / Q8_BLOCK, panels = (n + 15) / 16;
    const int64_t group_bytes = 64 + 2 * 32 * 8;
    memset(blob, 0, (size_t)orc_panel_bytes(n, k));
    for (int64_t p = 0; p < panels; ++p)
        for (int64_t g = 0; g < nb; ++g) {
            uint8_t* grp = blob + (p * nb + g) * group_bytes;
            for (int c = 0; c < 16; ++c) {
                const int64_t row = p * 16 + c;
                uint16_t sh = 0, mh = 0;
                if (row < n) {
                    const uint8_t* blk = blocks + (row * nb + g) * Q8_BYTES;
                    sh = (uint16_t)(blk[0] | (blk[1] << 8));
                    const float d = orc_half_to_float(sh);
                    const float minimum = -128.0f * d;
                    mh = orc_float_to_half(minimum);
                    if (!isfinite(d) || orc_half_to_float(mh) != minimum) return -1;
                    for (int t = 0; t < Q8_BLOCK; ++t) grp[64 + t * 16 + c] = (uint8_t)((int)(int8_t)blk[2 + t] + 128);
                }
                grp[2 * c] = (uint8_t)(sh & 0xff);
                grp[2 * c + 1] = (uint8_t)(sh >> 8);
                grp[32 + 2 * c] = (uint8_t)(mh & 0xff);
                grp[32 + 2 * c + 1] = (uint8_t)(mh >> 8);
            }
        }
    return 0;
}

/* ------------------------------------------------------------------------------------------------ exp and GELU */

/* src/kernels.cpp:806-824 (exp256), one lane. */
static float exp256_lane(float x) {
    x = x > -88.3762626647949f ? x : -88.3762626647949f;
    x = x < 88.3762626647949f ? x : 88.3762626647949f;
    const float fx = rintf(x * 1.44269504088896341f);
    /* GCC's intrinsics are plain vector operators, so x - fx * c is contracted into one FMA under -mfma */
    x = fmaf(-fx, 0.693359375f, x);
    x = fmaf(-fx, -2.12194440e-4f, x);
    const float z = x * x;
    float y = 1.9875691500e-4f;
    y = fmaf(y, x, 1.3981999507e-3f);
    y = fmaf(y, x, 8.3334519073e-3f);
    y = fmaf(y, x, 4.1665795894e-2f);
    y = fmaf(y, x, 1.6666665459e-1f);
    y = fmaf(y, x, 5.0000001201e-1f);
    y = fmaf(y, z, x);
    y = y + 1.0f;
    const uint32_t nbits = (uint32_t)((int32_t)fx + 127) << 23;
    float pow2n;
    memcpy(&pow2n, &nbits, 4);
    return y * pow2n;
}

/* src/kernels.cpp:826-841 (gelu256), one lane: erf from Abramowitz and Stegun 7.1.26. */
static float gelu256_lane(float x) {
    const float z = x * 0.70710678118654752f;
    const float az = fabsf(z);
    const float t = 1.0f / fmaf(0.3275911f, az, 1.0f);
    float p = 1.061405429f;
    p = fmaf(t, p, -1.453152027f);
    p = fmaf(t, p, 1.421413741f);
    p = fmaf(t, p, -0.284496736f);
    p = fmaf(t, p, 0.254829592f);
    p = t * p;
    const float decay = exp256_lane(0.0f - az * az);
    const float erf_abs = fmaf(-p, decay, 1.0f);
    const float erf = signbit(z) ? -erf_abs : erf_abs;
    return (0.5f * x) * (1.0f + erf);
}

/* src/kernels.cpp:843-850 (gelu_scalar), with the multiply-adds GCC fuses under -mfma. */
static float gelu_scalar_one(float x) {
    const float z = x * 0.70710678118654752f;
    const float az = fabsf(z);
    const float t = 1.0f / fmaf(0.3275911f, az, 1.0f);
    const float poly = fmaf(fmaf(fmaf(fmaf(1.061405429f, t, -1.453152027f), t, 1.421413741f), t, -0.284496736f), t,
                            0.254829592f);
    const float p = t * poly;
    const float erf_abs = fmaf(-p, expf(-az * az), 1.0f);
    return 0.5f * x * (1.0f + (z < 0.0f ? -erf_abs : erf_abs));
}

void orc_exp256(const float* x, int64_t count, float* y) {
    for (int64_t i = 0; i < count; ++i) y[i] = exp256_lane(x[i]);
}
void orc_gelu_erf(const float* x, int64_t count, float* y) {
    for (int64_t i = 0; i < count; ++i) y[i] = gelu256_lane(x[i]);
}
void orc_gelu_scalar(const float* x, int64_t count, float* y) {
    for (int64_t i = 0; i < count; ++i) y[i] = gelu_scalar_one(x[i]);
}

/* src/decoders.cpp:55-71 (gelu_tanh): tanh through exp256 on 8-wide blocks, libm tanhf on the tail. */
void orc_gelu_tanh(float* x, int64_t count) {
    const int64_t body = count / 8 * 8;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < body; ++i) {
        const float v = x[i];
        const float u = 0.7978845608028654f * fmaf(0.044715f * (v * v), v, v);
        const float e = exp256_lane(2.0f * u);
        const float t = 1.0f - 2.0f / (e + 1.0f);
        x[i] = (0.5f * v) * (1.0f + t);
    }
    for (int64_t i = body; i < count; ++i) {
        const float v = x[i];
        const float u = 0.7978845608028654f * fmaf(0.044715f * v * v, v, v);
        x[i] = 0.5f * v * (1.0f + tanhf(u));
    }
}

/* ------------------------------------------------------------------------------------------------ GEMM */

/* src/kernels.cpp:212-241 (finish_tile): bias, then the residual, then GELU; full 16-column tiles use gelu256 and
 * the ragged right edge gelu_scalar. */
static inline float finish(float acc, float bias, const float* residual, int gelu, int full_tile) {
    float v = acc + bias;
    if (residual) v = v + *residual;
    if (gelu) v = full_tile ? gelu256_lane(v) : gelu_scalar_one(v);
    return v;
}

/* src/kernels.cpp:552-565 -> 246-296 (gemm_quant) with microkernel_6x16 (:78-121) and dequant_chunk (:190-209):
 * each 32-deep chunk is a sequential FMA chain from zero, w = fma(code, scale, min) == q * d exactly, and the chunk
 * partials are added left to right. */
void orc_gemm_q8_float(const float* a, int64_t m, const uint8_t* w, int64_t n_total, int64_t k, const float* bias,
                       int64_t n_offset, int64_t n, const float* residual, int gelu, float* c) {
    (void)n_total;
    const int64_t nb = k / Q8_BLOCK;
    float* out = c;
    int64_t total = m * n;
    float* tmp = NULL;
    if (residual == c) {
        /* residual aliases c: compute into a scratch buffer first (each element reads only its own residual) */
        tmp = (float*)malloc(sizeof(float) * (size_t)(total > 0 ? total : 1));
        out = tmp;
    }
#pragma omp parallel for schedule(static)
    for (int64_t idx = 0; idx < total; ++idx) {
        const int64_t i = idx / n, j = idx % n;
        const float* arow = a + i * k;
        const uint8_t* wrow = w + (n_offset + j) * nb * Q8_BYTES;
        float tile = 0.0f;
        for (int64_t b = 0; b < nb; ++b) {
            const uint8_t* blk = wrow + b * Q8_BYTES;
            const float d = block_scale(blk);
            float part = 0.0f;
            for (int t = 0; t < Q8_BLOCK; ++t) part = fmaf(arow[b * Q8_BLOCK + t], (float)(int8_t)blk[2 + t] * d, part);
            tile = b == 0 ? part : tile + part;
        }
        const int full = (j / 16) * 16 + 16 <= n;
        out[idx] = finish(tile, bias ? bias[n_offset + j] : 0.0f, residual ? residual + idx : NULL, gelu, full);
    }
    if (tmp) {
        memcpy(c, tmp, sizeof(float) * (size_t)total);
        free(tmp);
    }
}

/* src/kernels.cpp:566-596 (gemm_packed, unquantized PackedLinear): dense fp32 weights [n_total x k], the same
 * 32-deep chunked FMA summation as the quantized float kernel, then finish_tile. */
void orc_gemm_dense(const float* a, int64_t m, const float* w, int64_t n_total, int64_t k, const float* bias,
                    int64_t n_offset, int64_t n, int gelu, float* c) {
    (void)n_total;
    const int64_t total = m * n;
#pragma omp parallel for schedule(static)
    for (int64_t idx = 0; idx < total; ++idx) {
        const int64_t i = idx / n, j = idx % n;
        const float* arow = a + i * k;
        const float* wrow = w + (n_offset + j) * k;
        float tile = 0.0f;
        for (int64_t k0 = 0; k0 < k; k0 += 32) {
            const int64_t kc = k - k0 < 32 ? k - k0 : 32;
            float part = 0.0f;
            for (int64_t t = 0; t < kc; ++t) part = fmaf(arow[k0 + t], wrow[k0 + t], part);
            tile = k0 == 0 ? part : tile + part;
        }
        const int full = (j / 16) * 16 + 16 <= n;
        c[idx] = finish(tile, bias ? bias[n_offset + j] : 0.0f, NULL, gelu, full);
    }
}

/* src/kernels.cpp:368-404 (quantize_activations) for group 32: amax, s = amax / 127, inv = 127 / amax (0 when
 * amax == 0), q = round-to-nearest-even(x * inv) as int8, qsum = sum of q. */
void orc_quantize_act(const float* a, int64_t m, int64_t k, int8_t* qa, float* scale, int32_t* qsum) {
    const int64_t ng = k / Q8_BLOCK;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < m; ++r)
        for (int64_t g = 0; g < ng; ++g) {
            const float* x = a + r * k + g * Q8_BLOCK;
            int8_t* q = qa + r * k + g * Q8_BLOCK;
            float amax = 0.0f;
            for (int t = 0; t < Q8_BLOCK; ++t) {
                const float ab = fabsf(x[t]);
                amax = amax > ab ? amax : ab;
            }
            const float s = amax / 127.0f, inv = amax > 0.0f ? 127.0f / amax : 0.0f;
            int32_t sum = 0;
            for (int t = 0; t < Q8_BLOCK; ++t) {
                const int32_t qi = (int32_t)rintf(x[t] * inv);
                q[t] = (int8_t)qi;
                sum += qi;
            }
            scale[r * ng + g] = s;
            qsum[r * ng + g] = sum;
        }
}

/* src/kernels.cpp:407-479 (vnni_task, gemm_quant_int8) on the Q8_0 -> panel mapping (code = q + 128,
 * min = -128 d): per group I_u = sum qa * code in int32, then t = fma(I_u, sw * sa, fma(mw, sa * qsum, t)). */
void orc_gemm_q8_int8(const float* a, int64_t m, const uint8_t* w, int64_t n_total, int64_t k, const float* bias,
                      int64_t n_offset, int64_t n, const float* residual, int gelu, float* c) {
    (void)n_total;
    const int64_t nb = k / Q8_BLOCK;
    int8_t* qa = (int8_t*)malloc((size_t)(m * k > 0 ? m * k : 1));
    float* sa = (float*)malloc(sizeof(float) * (size_t)(m * nb > 0 ? m * nb : 1));
    int32_t* qs = (int32_t*)malloc(sizeof(int32_t) * (size_t)(m * nb > 0 ? m * nb : 1));
    orc_quantize_act(a, m, k, qa, sa, qs);
    float* out = c;
    const int64_t total = m * n;
    float* tmp = NULL;
    if (residual == c) {
        tmp = (float*)malloc(sizeof(float) * (size_t)(total > 0 ? total : 1));
        out = tmp;
    }
#pragma omp parallel for schedule(static)
    for (int64_t idx = 0; idx < total; ++idx) {
        const int64_t i = idx / n, j = idx % n;
        const int8_t* qrow = qa + i * k;
        const uint8_t* wrow = w + (n_offset + j) * nb * Q8_BYTES;
        float t = 0.0f;
        for (int64_t g = 0; g < nb; ++g) {
            const uint8_t* blk = wrow + g * Q8_BYTES;
            int32_t acc = 0;
            for (int e = 0; e < Q8_BLOCK; ++e) acc += (int32_t)qrow[g * Q8_BLOCK + e] * ((int32_t)(int8_t)blk[2 + e] + 128);
            const float sw = block_scale(blk);
            const float mw = orc_half_to_float(orc_float_to_half(-128.0f * sw));
            const float s = sa[i * nb + g];
            const float sq = s * (float)qs[i * nb + g];
            t = fmaf((float)acc, sw * s, fmaf(mw, sq, t));
        }
        const int full = (j / 16) * 16 + 16 <= n;
        out[idx] = finish(t, bias ? bias[n_offset + j] : 0.0f, residual ? residual + idx : NULL, gelu, full);
    }
    if (tmp) {
        memcpy(c, tmp, sizeof(float) * (size_t)total);
        free(tmp);
    }
    free(qa);
    free(sa);
    free(qs);
}

/* The per-32-block int8 x int8 dot products that the integer kernel sums: I_q = I_u - 128 * qsum. */
void orc_block_dots(const int8_t* qa, int64_t m, const uint8_t* w, int64_t n_offset, int64_t n, int64_t k,
                    int32_t* dots) {
    const int64_t nb = k / Q8_BLOCK;
#pragma omp parallel for schedule(static)
    for (int64_t idx = 0; idx < m * n; ++idx) {
        const int64_t i = idx / n, j = idx % n;
        const uint8_t* wrow = w + (n_offset + j) * nb * Q8_BYTES;
        for (int64_t b = 0; b < nb; ++b) {
            int32_t acc = 0;
            for (int e = 0; e < Q8_BLOCK; ++e)
                acc += (int32_t)qa[i * k + b * Q8_BLOCK + e] * (int32_t)(int8_t)wrow[b * Q8_BYTES + 2 + e];
            dots[idx * nb + b] = acc;
        }
    }
}

/* ------------------------------------------------------------------------------------------------ norms */

/* src/kernels.cpp:599-618 (layer_norm), eps 1e-5, fp32 sums. */
void orc_layer_norm(const float* x, int64_t rows, int64_t dim, const float* gamma, const float* beta, float* y) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const float* in = x + r * dim;
        float* out = y + r * dim;
        float mean = 0.0f;
        for (int64_t d = 0; d < dim; ++d) mean += in[d];
        mean /= (float)dim;
        float var = 0.0f;
        for (int64_t d = 0; d < dim; ++d) {
            const float c = in[d] - mean;
            var = fmaf(c, c, var);
        }
        var /= (float)dim;
        const float inv = 1.0f / sqrtf(var + 1e-5f);
        for (int64_t d = 0; d < dim; ++d) out[d] = fmaf((in[d] - mean) * inv, gamma[d], beta[d]);
    }
}

/* src/decoders.cpp:23-42 (norm_rows): fp64 sums, eps as given, optional gamma/beta, optional adaLN
 * v * (1 + scale) + shift. */
void orc_norm_rows(const float* x, float* y, int64_t rows, int64_t dim, float eps, const float* gamma,
                   const float* beta, const float* shift, const float* scale, int64_t rows_per_batch) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const float* xr = x + r * dim;
        float* yr = y + r * dim;
        const int64_t bidx = rows_per_batch > 0 ? r / rows_per_batch : 0;
        const float* sh = shift ? shift + bidx * dim : NULL;
        const float* sc = scale ? scale + bidx * dim : NULL;
        double sum = 0.0;
        for (int64_t c = 0; c < dim; ++c) sum += xr[c];
        const float mean = (float)(sum / (double)dim);
        double sq = 0.0;
        for (int64_t c = 0; c < dim; ++c) {
            const double t = (double)(xr[c] - mean);
            sq = fma(t, t, sq);
        }
        const float inv = 1.0f / sqrtf((float)(sq / (double)dim) + eps);
        for (int64_t c = 0; c < dim; ++c) {
            float v = (xr[c] - mean) * inv;
            if (gamma) v = fmaf(v, gamma[c], beta[c]);
            if (sc) v = fmaf(v, 1.0f + sc[c], sh[c]);
            yr[c] = v;
        }
    }
}

/* ------------------------------------------------------------------------------------------------ attention */

/* src/kernels.cpp:58-64 (hsum) over eight lanes. */
static inline float hsum8(const float* l) {
    const float a0 = l[0] + l[4], a1 = l[1] + l[5], a2 = l[2] + l[6], a3 = l[3] + l[7];
    return (a0 + a1) + (a2 + a3);
}

/* The softmax of src/kernels.cpp:665-684 (and :782-796): max, exp256 over 8-wide blocks into eight lane sums,
 * libm expf on the tail, normalise by 1 / total. */
static void softmax_row(float* row, int64_t lk, float scale) {
    float mx = -INFINITY;
    for (int64_t j = 0; j < lk; ++j) mx = mx < row[j] ? row[j] : mx;
    float lanes[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int64_t j = 0;
    for (; j + 8 <= lk; j += 8)
        for (int l = 0; l < 8; ++l) {
            const float e = exp256_lane((row[j + l] - mx) * scale);
            row[j + l] = e;
            lanes[l] = lanes[l] + e;
        }
    float total = hsum8(lanes);
    for (; j < lk; ++j) {
        row[j] = expf((row[j] - mx) * scale);
        total += row[j];
    }
    const float inv = 1.0f / total;
    for (j = 0; j < lk; ++j) row[j] *= inv;
}

/* src/kernels.cpp:735-746 (attention) dispatching to attention_blocked (:629-731, head_dim % 16 == 0) or
 * attention_dot (:750-802). Both compute, per head, scores as FMA chains over head_dim, the softmax above, and
 * P*V as FMA chains over the keys; they differ only in how a score is summed. */
void orc_attention(const float* q, int64_t lq, int64_t ldq, const float* k, const float* v, int64_t lk, int64_t ldkv,
                   int64_t heads, int64_t head_dim, float* out, int64_t dim) {
    const float scale = 1.0f / sqrtf((float)head_dim);
    const char* env = getenv("IDOL_ATTENTION");
    const int blocked = head_dim % 16 == 0 && !(env && strcmp(env, "dot") == 0);
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
    for (int64_t h = 0; h < heads; ++h)
        for (int64_t i = 0; i < lq; ++i) {
            float* s = (float*)malloc(sizeof(float) * (size_t)(lk > 0 ? lk : 1));
            const float* qr = q + i * ldq + h * head_dim;
            for (int64_t j = 0; j < lk; ++j) {
                const float* kr = k + j * ldkv + h * head_dim;
                if (blocked) {
                    float acc = 0.0f;
                    for (int64_t d = 0; d < head_dim; ++d) acc = fmaf(qr[d], kr[d], acc);
                    s[j] = acc;
                } else {
                    /* dot(): eight lane accumulators, hsum, then a contracted scalar tail (src/kernels.cpp:66-72) */
                    float lanes[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                    int64_t d = 0;
                    for (; d + 8 <= head_dim; d += 8)
                        for (int l = 0; l < 8; ++l) lanes[l] = fmaf(qr[d + l], kr[d + l], lanes[l]);
                    float sum = hsum8(lanes);
                    for (; d < head_dim; ++d) sum = fmaf(qr[d], kr[d], sum);
                    s[j] = sum;
                }
            }
            softmax_row(s, lk, scale);
            float* o = out + i * dim + h * head_dim;
            for (int64_t d = 0; d < head_dim; ++d) {
                float acc = 0.0f;
                for (int64_t j = 0; j < lk; ++j) acc = fmaf(s[j], v[j * ldkv + h * head_dim + d], acc);
                o[d] = acc;
            }
            free(s);
        }
}

/* ------------------------------------------------------------------------------------------------ embedding */

/* src/decoders.cpp:215-230 (pos_embed) without the zero padding: per coordinate c, sin then cos of
 * (coord * freq) * pi for each frequency, written at out[row * ldo + c * 2 * nfreq + {j, nfreq + j}]. */
void orc_pos_embed(const float* freqs, int64_t nfreq, const float* coords, int64_t rows, float* out, int64_t ldo) {
    const float kPi = 3.14159265358979323846f;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        float* o = out + r * ldo;
        for (int c = 0; c < 3; ++c) {
            const float v = coords[r * 3 + c];
            for (int64_t j = 0; j < nfreq; ++j) {
                const float ang = (v * freqs[j]) * kPi;
                o[c * 2 * nfreq + j] = sinf(ang);
                o[c * 2 * nfreq + nfreq + j] = cosf(ang);
            }
        }
    }
}
