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

// Sum of v over the wave's 64 lanes, in every lane: within each row of 16 lanes by four DPP steps (lanes i ^ 1,
// i ^ 2 within quads, then the mirrored lanes of each half row and of the row: after each step every lane of a group
// holds the group's sum, the same value, since the additions are commutative), then the four row sums read from
// lanes 0, 16, 32, 48 and added as (r0 + r1) + (r2 + r3). A fixed order, so every kernel that reduces with it gets
// the same bits; no LDS round trip (a shuffle of a double is two ds_bpermute).
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, 0xf, 0xf, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, 0xf, 0xf, false);
    return __builtin_bit_cast(double, ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}
__device__ __forceinline__ double lane_f64(double v, int lane) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)u, lane);
    const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), lane);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ double wave_sum_f64(double v) {
    v += dpp_f64<0xB1>(v);   // quad_perm(1, 0, 3, 2)
    v += dpp_f64<0x4E>(v);   // quad_perm(2, 3, 0, 1)
    v += dpp_f64<0x141>(v);  // row_half_mirror
    v += dpp_f64<0x140>(v);  // row_mirror
    return (lane_f64(v, 0) + lane_f64(v, 16)) + (lane_f64(v, 32) + lane_f64(v, 48));
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
    sum = wave_sum_f64(sum);
    const float mean = (float)(sum / (double)dim);
    double sq = 0.0;
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const double t = (double)(v[j][e] - mean);
            sq = fma(t, t, sq);
        }
    sq = wave_sum_f64(sq);
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
                o[e + q] = fp32_value(t);
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

// Streaming rows (the HBM-bound form for many rows): each wave takes RPW consecutive rows, all in one adaLN batch,
// and requests every 16-byte chunk of all of them, and its lanes' gamma / beta / shift / scale values, before it
// computes anything; then it normalizes and stores the rows one after another, so the stores of the first rows go
// out while the later rows' loads are still arriving, and the modulation vectors are read once per wave (not once
// per row, after the reductions). Same per-row arithmetic as layernorm_rows_kernel: the same bits.
template <typename T, int NV, int RPW, bool AFF, bool ADA>
__global__ __launch_bounds__(256) void layernorm_stream_kernel(const T* x, int64_t rows, int64_t ldx, float eps,
                                                                const float* __restrict__ gamma,
                                                                const float* __restrict__ beta,
                                                                const float* __restrict__ shift,
                                                                const float* __restrict__ scale,
                                                                int64_t rows_per_batch, T* y, int64_t ldy) {
    // x may be y (in place): a wave requests all of its rows before it writes any of them
    constexpr int E = 16 / sizeof(T);
    constexpr int dim = 64 * NV * E;
    const int lane = threadIdx.x & 63;
    const int64_t r0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW;
    if (r0 >= rows) return;
    // the lane's columns (j * 64 + lane) * E .. + E - 1 of each parameter vector (the wave's rows share a batch),
    // requested first: the row loads complete after them, so the first row's wait does not include them
    const int64_t b = rows_per_batch > 0 ? r0 / rows_per_batch : 0;
    const float* sh = shift ? shift + b * dim : nullptr;
    const float* sc = scale ? scale + b * dim : nullptr;
    float4 pg[NV][E / 4], pb[NV][E / 4], ps[NV][E / 4], ph[NV][E / 4];
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int q = 0; q < E / 4; ++q) {
            const int c = (j * 64 + lane) * E + 4 * q;
            if constexpr (AFF) {
                pg[j][q] = *reinterpret_cast<const float4*>(gamma + c);
                pb[j][q] = beta ? *reinterpret_cast<const float4*>(beta + c) : make_float4(0, 0, 0, 0);
            }
            if constexpr (ADA) {
                ps[j][q] = *reinterpret_cast<const float4*>(sc + c);
                ph[j][q] = *reinterpret_cast<const float4*>(sh + c);
            }
        }
    // rows past the end read the last row (their results are not stored)
    uint4 raw[RPW][NV];
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
        const int64_t r = r0 + i < rows ? r0 + i : rows - 1;
#pragma unroll
        for (int j = 0; j < NV; ++j) raw[i][j] = *reinterpret_cast<const uint4*>(x + r * ldx + (j * 64 + lane) * E);
    }
    float v[RPW][NV][E];
#pragma unroll
    for (int i = 0; i < RPW; ++i)
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const uint32_t w[4] = {raw[i][j].x, raw[i][j].y, raw[i][j].z, raw[i][j].w};
#pragma unroll
            for (int e = 0; e < E; ++e) {
                if (sizeof(T) == 4) v[i][j][e] = __uint_as_float(w[e]);
                else {
                    const uint16_t bits = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
                    v[i][j][e] = std::is_same<T, __bf16>::value ? bf16_bits_to_float(bits) : half_bits_to_float(bits);
                }
            }
        }
    // each row is summed in the one-row-per-wave kernel's order; the RPW rows' sums and cross-lane steps are
    // interleaved, so their latencies overlap
    double sum[RPW], sq[RPW];
    float mean[RPW], inv[RPW];
#pragma unroll
    for (int i = 0; i < RPW; ++i) sum[i] = 0.0;
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int e = 0; e < E; ++e)
#pragma unroll
            for (int i = 0; i < RPW; ++i) sum[i] += (double)v[i][j][e];
#pragma unroll
    for (int i = 0; i < RPW; ++i) sum[i] = wave_sum_f64(sum[i]);
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
        mean[i] = (float)(sum[i] / (double)dim);
        sq[i] = 0.0;
    }
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int e = 0; e < E; ++e)
#pragma unroll
            for (int i = 0; i < RPW; ++i) {
                const double t = (double)(v[i][j][e] - mean[i]);
                sq[i] = fma(t, t, sq[i]);
            }
#pragma unroll
    for (int i = 0; i < RPW; ++i) sq[i] = wave_sum_f64(sq[i]);
#pragma unroll
    for (int i = 0; i < RPW; ++i) inv[i] = 1.0f / sqrtf((float)(sq[i] / (double)dim) + eps);
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
        const int64_t r = r0 + i;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            float o[E];
#pragma unroll
            for (int e = 0; e < E; ++e) {
                const float4& g4 = pg[j][e / 4];
                const float4& b4 = pb[j][e / 4];
                const float4& s4 = ps[j][e / 4];
                const float4& h4 = ph[j][e / 4];
                const float gg = (&g4.x)[e % 4], bb = (&b4.x)[e % 4], ss = (&s4.x)[e % 4], hh = (&h4.x)[e % 4];
                float t = (v[i][j][e] - mean[i]) * inv[i];
                if constexpr (AFF) t = fmaf(t, gg, bb);
                if constexpr (ADA) t = fmaf(t, 1.0f + ss, hh);
                o[e] = fp32_value(t);
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
            if (r < rows) *reinterpret_cast<uint4*>(y + r * ldy + (j * 64 + lane) * E) = make_uint4(w[0], w[1], w[2], w[3]);
        }
    }
}

// Rows per wave of the streaming form, and the smallest row count it takes (below that, one row per wave spreads a
// small call over more CUs).
constexpr int kStreamRows = 4;
constexpr int64_t kStreamMinRows = 4096;

template <typename T>
int launch_stream(const void* x, int64_t rows, int64_t dim, int64_t ldx, float eps, const float* gamma,
                  const float* beta, const float* shift, const float* scale, int64_t rows_per_batch, void* y,
                  int64_t ldy, hipStream_t s) {
    constexpr int E = 16 / sizeof(T);
    const int64_t per_wg = 4 * kStreamRows;
    const dim3 grid((unsigned)((rows + per_wg - 1) / per_wg)), block(256);
    const T* xt = static_cast<const T*>(x);
    T* yt = static_cast<T*>(y);
    auto go = [&](auto nv) {
        constexpr int NV = decltype(nv)::value;
        if (gamma && scale)
            hipLaunchKernelGGL((layernorm_stream_kernel<T, NV, kStreamRows, true, true>), grid, block, 0, s, xt, rows,
                               ldx, eps, gamma, beta, shift, scale, rows_per_batch, yt, ldy);
        else if (gamma)
            hipLaunchKernelGGL((layernorm_stream_kernel<T, NV, kStreamRows, true, false>), grid, block, 0, s, xt, rows,
                               ldx, eps, gamma, beta, shift, scale, rows_per_batch, yt, ldy);
        else if (scale)
            hipLaunchKernelGGL((layernorm_stream_kernel<T, NV, kStreamRows, false, true>), grid, block, 0, s, xt, rows,
                               ldx, eps, gamma, beta, shift, scale, rows_per_batch, yt, ldy);
        else
            hipLaunchKernelGGL((layernorm_stream_kernel<T, NV, kStreamRows, false, false>), grid, block, 0, s, xt, rows,
                               ldx, eps, gamma, beta, shift, scale, rows_per_batch, yt, ldy);
    };
    switch (dim / (64 * E)) {
        case 1: go(std::integral_constant<int, 1>{}); break;
        case 2: go(std::integral_constant<int, 2>{}); break;
        case 3: go(std::integral_constant<int, 3>{}); break;
        case 4: go(std::integral_constant<int, 4>{}); break;
        default: return -1;
    }
    return check_launch("layernorm_stream_kernel");
}

template <typename T>
int launch_rows(const void* x, int64_t rows, int64_t dim, int64_t ldx, float eps, const float* gamma, const float* beta,
                const float* shift, const float* scale, int64_t rows_per_batch, void* y, int64_t ldy, hipStream_t s) {
    constexpr int E = 16 / sizeof(T);
    // many rows whose adaLN batches hold whole groups of kStreamRows rows: the streaming form
    if (rows >= kStreamMinRows && (rows_per_batch <= 0 || rows_per_batch % kStreamRows == 0) && dim / (64 * E) <= 4) {
        const int rc = launch_stream<T>(x, rows, dim, ldx, eps, gamma, beta, shift, scale, rows_per_batch, y, ldy, s);
        if (rc != -1) return rc;
    }
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
