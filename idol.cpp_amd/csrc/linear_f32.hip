// Dense fp32 linear layer: y = act(x * W^T + bias), W fp32 [n x k] held in LDS, one output row per thread.
//
// The depth is summed exactly as the reference's dense GEMM does (src/kernels.cpp:566-596 with its microkernel
// src/kernels.cpp:78-121): in chunks of 32, each a sequential FMA chain from zero, chunk partials added left to right;
// then bias (src/kernels.cpp:212-241 finish_tile), then the activation. Every step is an fp32 FMA or add, so the
// result is bit-identical to the reference for the activations it shares (none, erf-GELU through erff aside).
// Built for the narrow heads of the decoders' per-point MLPs (e.g. 64 -> 14): memory-bound, n <= 32, n * k <= 16384.
#include "common.h"

namespace idolq {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxWeights = 16384;  // n * k fp32 in LDS (64 KiB)
constexpr int kMaxOut = 32;

__global__ __launch_bounds__(kThreads) void linear_f32_kernel(const void* x, int xdt, int64_t m, int k, int64_t ldx,
                                                              const float* __restrict__ w, int n,
                                                              const float* __restrict__ bias, int act, void* y,
                                                              int ydt, int64_t ldy) {
    __shared__ float ws[kMaxWeights];
    for (int i = threadIdx.x; i < n * k; i += kThreads) ws[i] = w[i];
    __syncthreads();
    const int64_t row = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (row >= m) return;
    // the output arrays are indexed by unrolled loops only, so they stay in registers
    float acc[kMaxOut];
#pragma unroll
    for (int o = 0; o < kMaxOut; ++o) acc[o] = 0.0f;
    for (int k0 = 0; k0 < k; k0 += 32) {
        const int kc = min(32, k - k0);
        float part[kMaxOut];
#pragma unroll
        for (int o = 0; o < kMaxOut; ++o) part[o] = 0.0f;
        for (int kk = 0; kk < kc; ++kk) {
            const float a = load_as_float(x, xdt, row * ldx + k0 + kk);
#pragma unroll
            for (int o = 0; o < kMaxOut; ++o)
                if (o < n) part[o] = fmaf(a, ws[o * k + k0 + kk], part[o]);
        }
#pragma unroll
        for (int o = 0; o < kMaxOut; ++o) acc[o] = k0 == 0 ? part[o] : acc[o] + part[o];
    }
#pragma unroll
    for (int o = 0; o < kMaxOut; ++o) {
        if (o < n) {
            float v = acc[o];
            if (bias) v += bias[o];
            store_from_float(y, ydt, row * ldy + o, apply_act(act, v));
        }
    }
}

// The same sums with each row's depth read 8 elements at a time (k % 8 == 0, 16-byte aligned rows).
template <int XDT>
__global__ __launch_bounds__(kThreads) void linear_f32_vec_kernel(const void* x, int64_t m, int k, int64_t ldx,
                                                                  const float* __restrict__ w, int n,
                                                                  const float* __restrict__ bias, int act, void* y,
                                                                  int ydt, int64_t ldy) {
    __shared__ __attribute__((aligned(16))) float ws[kMaxWeights];
    for (int i = threadIdx.x; i < n * k; i += kThreads) ws[i] = w[i];
    __syncthreads();
    const int64_t row = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (row >= m) return;
    float acc[kMaxOut];
#pragma unroll
    for (int o = 0; o < kMaxOut; ++o) acc[o] = 0.0f;
    for (int k0 = 0; k0 < k; k0 += 32) {
        const int kc = min(32, k - k0);
        float part[kMaxOut];
#pragma unroll
        for (int o = 0; o < kMaxOut; ++o) part[o] = 0.0f;
        for (int g = 0; g < kc; g += 8) {
            float a[8];
            load8<XDT>(x, row * ldx + k0 + g, a);
            // each output's 8 weights in two 16-byte LDS reads (the same address in every lane)
#pragma unroll
            for (int o = 0; o < kMaxOut; ++o)
                if (o < n) {
                    const float4 w0 = *reinterpret_cast<const float4*>(ws + o * k + k0 + g);
                    const float4 w1 = *reinterpret_cast<const float4*>(ws + o * k + k0 + g + 4);
                    const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
                    for (int e = 0; e < 8; ++e) part[o] = fmaf(a[e], wv[e], part[o]);
                }
        }
#pragma unroll
        for (int o = 0; o < kMaxOut; ++o) acc[o] = k0 == 0 ? part[o] : acc[o] + part[o];
    }
#pragma unroll
    for (int o = 0; o < kMaxOut; ++o) {
        if (o < n) {
            float v = acc[o];
            if (bias) v += bias[o];
            store_from_float(y, ydt, row * ldy + o, apply_act(act, v));
        }
    }
}

}  // namespace
}  // namespace idolq

using namespace idolq;

extern "C" int idolq_linear_f32(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const float* w,
                                int64_t n, const float* bias, int act, void* y, int y_dtype, int64_t ldy,
                                void* stream) {
    if (!dtype_ok(x_dtype) || !dtype_ok(y_dtype)) return fail(IDOLQ_EINVAL, "unknown dtype code");
    if (m < 0 || k <= 0 || n <= 0) return fail(IDOLQ_EINVAL, "need m >= 0, k > 0 and n > 0");
    if (n > kMaxOut || n * k > kMaxWeights)
        return fail(IDOLQ_ENOSUPPORT, "dense linear: n <= 32 and n * k <= 16384 (weights held in LDS)");
    if (ldx < k || ldy < n) return fail(IDOLQ_EINVAL, "row stride smaller than the row");
    if (act < IDOLQ_ACT_NONE || act > IDOLQ_ACT_SILU) return fail(IDOLQ_EINVAL, "unknown activation");
    if (m == 0) return IDOLQ_OK;
    if (!x || !w || !y) return fail(IDOLQ_EINVAL, "x, w and y must be non-null");
    const int64_t blocks = (m + kThreads - 1) / kThreads;
    if (blocks > INT32_MAX) return fail(IDOLQ_EINVAL, "too many rows");
    if (k % 8 == 0 && vec8_ok(x, x_dtype, ldx)) {
        hipStream_t s = static_cast<hipStream_t>(stream);
#define IDOLQ_LIN(DT)                                                                                               \
    hipLaunchKernelGGL(linear_f32_vec_kernel<DT>, dim3((unsigned)blocks), dim3(kThreads), 0, s, x, m, (int)k, ldx, w, \
                       (int)n, bias, act, y, y_dtype, ldy)
        if (x_dtype == IDOLQ_F32) IDOLQ_LIN(IDOLQ_F32);
        else if (x_dtype == IDOLQ_BF16) IDOLQ_LIN(IDOLQ_BF16);
        else IDOLQ_LIN(IDOLQ_F16);
#undef IDOLQ_LIN
        return check_launch("linear_f32_vec_kernel");
    }
    hipLaunchKernelGGL(linear_f32_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                       x, x_dtype, m, (int)k, ldx, w, (int)n, bias, act, y, y_dtype, ldy);
    return check_launch("linear_f32_kernel");
}
