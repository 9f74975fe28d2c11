// Row-wise layer norm with optional affine and adaLN modulation, one 256-thread workgroup per row.
// Mean and variance are accumulated in fp64 as the reference's norm_rows does; the per-element arithmetic is the
// reference's fp32 sequence ((x - mean) * inv, then fma with gamma/beta, then fma with 1 + scale and shift).
// HBM-bound: one read and one write of each row (the re-reads of a row hit L1/L2).
#include "common.h"

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
    const dim3 grid((unsigned)rows), block(kThreads);
    if (dim <= 8 * kThreads)
        hipLaunchKernelGGL(layernorm_kernel<8>, grid, block, 0, s, x, x_dtype, dim, ldx, eps, gamma, beta, shift, scale,
                           rows_per_batch, y, y_dtype, ldy);
    else
        hipLaunchKernelGGL(layernorm_kernel<0>, grid, block, 0, s, x, x_dtype, dim, ldx, eps, gamma, beta, shift, scale,
                           rows_per_batch, y, y_dtype, ldy);
    return check_launch("layernorm_kernel");
}
