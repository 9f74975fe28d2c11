// Row-wise layer norm with optional affine and adaLN modulation: one wave per row with 16-byte accesses for aligned
// rows whose width is a multiple of 64 chunks (layernorm_rows_kernel), else one 256-thread workgroup per row.
// Mean and variance are accumulated in fp64 as the reference's norm_rows does; the per-element arithmetic is the
// reference's fp32 sequence ((x - mean) * inv, then fma with gamma/beta, then fma with 1 + scale and shift).
// HBM-bound: one read and one write of each row (the re-reads of a row hit L1/L2).
#include "common.h"

#include <type_traits>

namespace idolq {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ double block_sum(double v, double* red) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    double t = 0.0;
    for (int w = 0; w < kThreads / 64; ++w) t += red[w];
    __syncthreads();
    return t;
}

// PER values per thread kept in registers (dim <= PER * 256); PER == 0 re-reads the row for each pass.
template <int PER>
__global__ __launch_bounds__(kThreads) void layernorm_kernel(const void* x, int x_dt, int64_t dim,
                                                             int64_t ldx, float eps, const float* __restrict__ gamma,
                                                             const float* __restrict__ beta,
                                                             const float* __restrict__ shift,
                                                             const float* __restrict__ scale, int64_t rows_per_batch,
                                                             void* y, int y_dt, int64_t ldy) {
    __shared__ double red[kThreads / 64];
    const int64_t r = blockIdx.x;
    const int64_t xo = r * ldx;
    float vals[PER > 0 ? PER : 1];
    double sum = 0.0;
    if (PER > 0) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int64_t c = threadIdx.x + (int64_t)i * kThreads;
            vals[i] = c < dim ? load_as_float(x, x_dt, xo + c) : 0.0f;
            sum += (double)vals[i];
        }
    } else {
        for (int64_t c = threadIdx.x; c < dim; c += kThreads) sum += (double)load_as_float(x, x_dt, xo + c);
    }
    const float mean = (float)(block_sum(sum, red) / (double)dim);
    double sq = 0.0;
    if (PER > 0) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int64_t c = threadIdx.x + (int64_t)i * kThreads;
            if (c < dim) {
                const double t = (double)(vals[i] - mean);
                sq = fma(t, t, sq);
            }
        }
    } else {
        for (int64_t c = threadIdx.x; c < dim; c += kThreads) {
            const double t = (double)(load_as_float(x, x_dt, xo + c) - mean);
            sq = fma(t, t, sq);
        }
    }
    const float inv = 1.0f / sqrtf((float)(block_sum(sq, red) / (double)dim) + eps);
    const int64_t b = rows_per_batch > 0 ? r / rows_per_batch : 0;
    const float* sh = shift ? shift + b * dim : nullptr;
    const float* sc = scale ? scale + b * dim : nullptr;
    const int64_t yo = r * ldy;
    auto finish = [&](int64_t c, float xv) {
        float v = (xv - mean) * inv;
        if (gamma) v = fmaf(v, gamma[c], beta ? beta[c] : 0.0f);
        if (sc) v = fmaf(v, 1.0f + sc[c], sh ? sh[c] : 0.0f);
        store_from_float(y, y_dt, yo + c, v);
    };
    if (PER > 0) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int64_t c = threadIdx.x + (int64_t)i * kThreads;
            if (c < dim) finish(c, vals[i]);
        }
    } else {
        for (int64_t c = threadIdx.x; c < dim; c += kThreads) finish(c, load_as_float(x, x_dt, xo + c));
    }
}

// Vectorized rows: one wave per row, dim = 64 * NV * E (E = 16 / sizeof(T) elements per 16-byte chunk); lane l
// holds chunks j * 64 + l, j < NV, in registers. Same arithmetic as layernorm_kernel (fp32 values, fp64 sums reduced
// across the wave, fp32 normalization and modulation); x, y, the row strides and the parameter arrays are 16-byte
// aligned.
template <typename T, int NV>
__global__ __launch_bounds__(256) void layernorm_rows_kernel(const T* x, int64_t rows, int64_t ldx,
                                                              float eps, const float* __restrict__ gamma,
                                                              const float* __restrict__ beta,
                                                              const float* __restrict__ shift,
                                                              const float* __restrict__ scale, int64_t rows_per_batch,
                                                              T* y, int64_t ldy) {
    // x may be y (in place): a wave reads its whole row before it writes
    constexpr int E = 16 / sizeof(T);
    constexpr int dim = 64 * NV * E;
    const int lane = threadIdx.x & 63;
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    float v[NV][E];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const uint4 raw = *reinterpret_cast<const uint4*>(x + r * ldx + (j * 64 + lane) * E);
        const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int e = 0; e < E; ++e) {
            if (sizeof(T) == 4) v[j][e] = __uint_as_float(w[e]);
            else {
                const uint16_t b = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
                v[j][e] = std::is_same<T, __bf16>::value ? bf16_bits_to_float(b) : half_bits_to_float(b);
            }
        }
    }
    double sum = 0.0;
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int e = 0; e < E; ++e) sum += (double)v[j][e];
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
    const float mean = (float)(sum / (double)dim);
    double sq = 0.0;
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const double t = (double)(v[j][e] - mean);
            sq = fma(t, t, sq);
        }
    for (int off = 32; off > 0; off >>= 1) sq += __shfl_xor(sq, off);
    const float inv = 1.0f / sqrtf((float)(sq / (double)dim) + eps);
    const int64_t b = rows_per_batch > 0 ? r / rows_per_batch : 0;
    const float* sh = shift ? shift + b * dim : nullptr;
    const float* sc = scale ? scale + b * dim : nullptr;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int c0 = (j * 64 + lane) * E;
        float o[E];
#pragma unroll
        for (int e = 0; e < E; e += 4) {
            const float4 g = gamma ? *reinterpret_cast<const float4*>(gamma + c0 + e) : make_float4(1, 1, 1, 1);
            const float4 be = beta ? *reinterpret_cast<const float4*>(beta + c0 + e) : make_float4(0, 0, 0, 0);
            const float gg[4] = {g.x, g.y, g.z, g.w}, bb[4] = {be.x, be.y, be.z, be.w};
            float4 s4 = make_float4(0, 0, 0, 0), h4 = make_float4(0, 0, 0, 0);
            if (sc) {
                s4 = *reinterpret_cast<const float4*>(sc + c0 + e);
                h4 = *reinterpret_cast<const float4*>(sh + c0 + e);
            }
            const float ss[4] = {s4.x, s4.y, s4.z, s4.w}, hh[4] = {h4.x, h4.y, h4.z, h4.w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float t = (v[j][e + q] - mean) * inv;
                if (gamma) t = fmaf(t, gg[q], beta ? bb[q] : 0.0f);
                if (sc) t = fmaf(t, 1.0f + ss[q], hh[q]);
                o[e + q] = t;
            }
        }
        uint32_t w[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if (sizeof(T) == 4) w[q] = __float_as_uint(o[q]);
            else if (std::is_same<T, __bf16>::value)
                w[q] = (uint32_t)float_to_bf16_bits(o[2 * q]) | ((uint32_t)float_to_bf16_bits(o[2 * q + 1]) << 16);
            else
                w[q] = (uint32_t)float_to_half_bits(o[2 * q]) | ((uint32_t)float_to_half_bits(o[2 * q + 1]) << 16);
        }
        *reinterpret_cast<uint4*>(y + r * ldy + c0) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

template <typename T>
int launch_rows(const void* x, int64_t rows, int64_t dim, int64_t ldx, float eps, const float* gamma, const float* beta,
                const float* shift, const float* scale, int64_t rows_per_batch, void* y, int64_t ldy, hipStream_t s) {
    constexpr int E = 16 / sizeof(T);
    const dim3 grid((unsigned)((rows + 3) / 4)), block(256);
    const T* xt = static_cast<const T*>(x);
    T* yt = static_cast<T*>(y);
#define IDOLQ_ROWS(NV)                                                                                              \
    case NV:                                                                                                        \
        hipLaunchKernelGGL((layernorm_rows_kernel<T, NV>), grid, block, 0, s, xt, rows, ldx, eps, gamma, beta, shift, \
                           scale, rows_per_batch, yt, ldy);                                                         \
        break
    switch (dim / (64 * E)) {
        IDOLQ_ROWS(1);
        IDOLQ_ROWS(2);
        IDOLQ_ROWS(3);
        IDOLQ_ROWS(4);
        IDOLQ_ROWS(5);
        IDOLQ_ROWS(6);
        IDOLQ_ROWS(8);
        default: return -1;
    }
#undef IDOLQ_ROWS
    return check_launch("layernorm_rows_kernel");
}

bool rows_eligible(int x_dt, int y_dt, int64_t dim, const void* x, int64_t ldx, const void* y, int64_t ldy,
                   const float* gamma, const float* beta, const float* shift, const float* scale) {
    if (x_dt != y_dt) return false;
    const int esz = x_dt == IDOLQ_F32 ? 4 : 2, E = 16 / esz;
    const int64_t nv = dim / (64 * E);
    if (dim % (64 * E) != 0 || nv < 1 || nv > 8 || nv == 7) return false;
    auto al = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    return al(x) && al(y) && (ldx * esz) % 16 == 0 && (ldy * esz) % 16 == 0 && (!gamma || al(gamma)) &&
           (!beta || al(beta)) && (!shift || al(shift)) && (!scale || al(scale));
}

}  // namespace
}  // namespace idolq

using namespace idolq;

extern "C" int idolq_layernorm(const void* x, int x_dtype, int64_t rows, int64_t dim, int64_t ldx, float eps,
                               const float* gamma, const float* beta, const float* shift, const float* scale,
                               int64_t rows_per_batch, void* y, int y_dtype, int64_t ldy, void* stream) {
    if (!dtype_ok(x_dtype) || !dtype_ok(y_dtype)) return fail(IDOLQ_EINVAL, "unknown dtype code");
    if (rows < 0 || dim <= 0 || ldx < dim || ldy < dim) return fail(IDOLQ_EINVAL, "bad layer norm shape");
    if (rows == 0) return IDOLQ_OK;
    if (!x || !y) return fail(IDOLQ_EINVAL, "x and y must be non-null");
    if (x == y && (x_dtype != y_dtype || ldx != ldy)) return fail(IDOLQ_EINVAL, "in place needs equal dtypes and strides");
    if ((shift == nullptr) != (scale == nullptr)) return fail(IDOLQ_EINVAL, "adaLN needs both shift and scale");
    if (rows == 0) return IDOLQ_OK;
    if (rows > 0x7fffffff) return fail(IDOLQ_EINVAL, "too many rows");
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (rows_eligible(x_dtype, y_dtype, dim, x, ldx, y, ldy, gamma, beta, shift, scale)) {
        int rc;
        if (x_dtype == IDOLQ_BF16)
            rc = launch_rows<__bf16>(x, rows, dim, ldx, eps, gamma, beta, shift, scale, rows_per_batch, y, ldy, s);
        else if (x_dtype == IDOLQ_F16)
            rc = launch_rows<_Float16>(x, rows, dim, ldx, eps, gamma, beta, shift, scale, rows_per_batch, y, ldy, s);
        else
            rc = launch_rows<float>(x, rows, dim, ldx, eps, gamma, beta, shift, scale, rows_per_batch, y, ldy, s);
        if (rc != -1) return rc;
    }
    const dim3 grid((unsigned)rows), block(kThreads);
    if (dim <= 8 * kThreads)
        hipLaunchKernelGGL(layernorm_kernel<8>, grid, block, 0, s, x, x_dtype, dim, ldx, eps, gamma, beta, shift, scale,
                           rows_per_batch, y, y_dtype, ldy);
    else
        hipLaunchKernelGGL(layernorm_kernel<0>, grid, block, 0, s, x, x_dtype, dim, ldx, eps, gamma, beta, shift, scale,
                           rows_per_batch, y, y_dtype, ldy);
    return check_launch("layernorm_kernel");
}
