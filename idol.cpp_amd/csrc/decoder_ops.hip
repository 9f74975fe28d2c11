// Small kernels of the real decoders (src/decoders.cpp) that sit between the Q8_0 linears, the layer norms and the
// attention: per-head RMS normalisation, the gated residual add, the octree level embedding and the dense fp32
// linears (the 3-D point input projections, the latent key/value projections and unquantized layers). Each restates the reference loop's fp32 arithmetic step by step (the same
// order of FMAs and adds), so for fp32 inputs they give the reference's floats up to the libm of sin/cos/sqrt.
#include "common.h"

namespace idolq {
namespace {

// One thread per (row, head): ss = sum of squares in order (FMA chain), mult = sqrt(hd) / max(sqrt(ss), 1e-12),
// p = p * mult * gamma (src/decoders.cpp:74-86 rms_heads).
__global__ __launch_bounds__(256) void rms_heads_kernel(void* x, int dt, int64_t rows, int64_t ld, int heads, int hd,
                                                        const float* __restrict__ gamma) {
    const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= rows * heads) return;
    const int64_t r = id / heads;
    const int h = (int)(id - r * heads);
    const int64_t base = r * ld + (int64_t)h * hd;
    float ss = 0.0f;
    for (int d = 0; d < hd; ++d) {
        const float v = load_as_float(x, dt, base + d);
        ss = fmaf(v, v, ss);
    }
    const float mult = sqrtf((float)hd) / fmaxf(sqrtf(ss), 1e-12f);
    const float* g = gamma + (int64_t)h * hd;
    for (int d = 0; d < hd; ++d) store_from_float(x, dt, base + d, load_as_float(x, dt, base + d) * mult * g[d]);
}

// The same for fp32 rows with 16-byte aligned heads of HD values: the head held in registers, read and written with
// 16-byte accesses; the sum of squares is still taken in order, so the result is that of rms_heads_kernel.
template <int HD>
__global__ __launch_bounds__(256) void rms_heads_vec_kernel(float* x, int64_t rows, int64_t ld, int heads,
                                                            const float* __restrict__ gamma) {
    const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= rows * heads) return;
    const int64_t r = id / heads;
    const int h = (int)(id - r * heads);
    f32x4* p = reinterpret_cast<f32x4*>(x + r * ld + (int64_t)h * HD);
    const f32x4* g = reinterpret_cast<const f32x4*>(gamma + (int64_t)h * HD);
    f32x4 v[HD / 4];
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < HD / 4; ++i) {
        v[i] = p[i];
#pragma unroll
        for (int e = 0; e < 4; ++e) ss = fmaf(v[i][e], v[i][e], ss);
    }
    const float mult = sqrtf((float)HD) / fmaxf(sqrtf(ss), 1e-12f);
#pragma unroll
    for (int i = 0; i < HD / 4; ++i) {
        const f32x4 gi = g[i];
        f32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = v[i][e] * mult * gi[e];
        p[i] = o;
    }
}

// x[r, c] += h[r, c] * gate[c] (src/decoders.cpp:45-52 add_gated; the multiply-add is one FMA, as GCC contracts it).
__global__ __launch_bounds__(256) void add_gated_kernel(void* x, int xdt, int64_t ldx, const void* h, int hdt,
                                                        int64_t ldh, int64_t rows, int64_t dim,
                                                        const float* __restrict__ gate) {
    const int64_t total = rows * dim, stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
        const int64_t r = i / dim, c = i - r * dim;
        const float v = fmaf(load_as_float(h, hdt, r * ldh + c), gate[c], load_as_float(x, xdt, r * ldx + c));
        store_from_float(x, xdt, r * ldx + c, v);
    }
}

// emb[i] = cos(((resolution * freqs[i]) * 2) * pi), emb[half + i] = sin(...) (src/decoders.cpp:262-266).
__global__ __launch_bounds__(256) void level_embed_kernel(float resolution, const float* __restrict__ freqs, int half,
                                                          float* __restrict__ out) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= half) return;
    const float kPi = 3.14159265358979323846f;
    const float ang = ((resolution * freqs[i]) * 2.0f) * kPi;
    out[i] = cosf(ang);
    out[half + i] = sinf(ang);
}

// Dense fp32 GEMM y = act(x * W^T + bias + residual) in the reference's summation order (src/kernels.cpp:566-596
// with its microkernel src/kernels.cpp:78-121 and epilogue src/kernels.cpp:212-241): the depth in chunks of 32, each
// an FMA chain from zero, the chunk partials added left to right (the first one taken as is), then bias, residual and
// the activation, each one fp32 operation, so every output is bit-identical to the reference's.
// Workgroup: 256 threads own a 64 x 64 output tile, 4 x 4 outputs per thread (rows ty*4+i, columns tx*4+j); each
// 32-deep chunk of x and W is staged in LDS depth-major, so the 4 operands a thread needs per step are one 16-byte
// read each. VEC (y, and the bias and residual when given, 16-byte aligned with row strides a multiple of 4): a
// thread's 4 columns of a row go out as one 16-byte store (the small-k products, such as the latent K/V projections
// at k = 16, are bound by their output writes), the bias and residual come in as 16-byte loads; the arithmetic per
// element is the same.
constexpr int kGT = 64, kGK = 32, kGPitch = kGT + 4;

template <bool VEC>
__global__ __launch_bounds__(256) void gemm_f32_kernel(const float* __restrict__ x, int m, int k, int64_t ldx,
                                                       const float* __restrict__ w, int n,
                                                       const float* __restrict__ bias, const float* res, int64_t ldr,
                                                       int act, float* y, int64_t ldy) {
    __shared__ __align__(16) float xs[kGK][kGPitch];
    __shared__ __align__(16) float ws[kGK][kGPitch];
    const int tid = threadIdx.x, tx = tid % 16, ty = tid / 16;
    const int m0 = blockIdx.y * kGT, n0 = blockIdx.x * kGT;
    float acc[4][4];
    for (int k0 = 0; k0 < k; k0 += kGK) {
        const int kc = min(kGK, k - k0);
        __syncthreads();
#pragma unroll
        for (int e = 0; e < kGT * kGK / 256; ++e) {
            const int idx = tid + 256 * e, r = idx / kGK, kk = idx % kGK;
            const bool kin = kk < kc;
            xs[kk][r] = (kin && m0 + r < m) ? x[(int64_t)(m0 + r) * ldx + k0 + kk] : 0.0f;
            ws[kk][r] = (kin && n0 + r < n) ? w[(int64_t)(n0 + r) * k + k0 + kk] : 0.0f;
        }
        __syncthreads();
        float part[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) part[i][j] = 0.0f;
        for (int kk = 0; kk < kc; ++kk) {
            const float4 a = *reinterpret_cast<const float4*>(&xs[kk][ty * 4]);
            const float4 b = *reinterpret_cast<const float4*>(&ws[kk][tx * 4]);
            const float av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) part[i][j] = fmaf(av[i], bv[j], part[i][j]);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = k0 == 0 ? part[i][j] : acc[i][j] + part[i][j];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = m0 + ty * 4 + i;
        if (row >= m) continue;
        if constexpr (VEC) {
            const int col = n0 + tx * 4;
            if (col + 3 < n) {
                float4 v = make_float4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]);
                if (bias) {
                    const float4 b = *reinterpret_cast<const float4*>(bias + col);
                    v.x += b.x, v.y += b.y, v.z += b.z, v.w += b.w;
                }
                if (res) {
                    const float4 r = *reinterpret_cast<const float4*>(res + (int64_t)row * ldr + col);
                    v.x += r.x, v.y += r.y, v.z += r.z, v.w += r.w;
                }
                v = make_float4(apply_act(act, v.x), apply_act(act, v.y), apply_act(act, v.z), apply_act(act, v.w));
                *reinterpret_cast<float4*>(y + (int64_t)row * ldy + col) = v;
                continue;
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int col = n0 + tx * 4 + j;
            if (col >= n) continue;
            float v = acc[i][j];
            if (bias) v += bias[col];
            if (res) v += res[(int64_t)row * ldr + col];
            y[(int64_t)row * ldy + col] = apply_act(act, v);
        }
    }
}

// Raw Gaussian features -> activated Gaussians, one thread per (anchor, Gaussian) (src/decoders.cpp:393-431
// to_gaussians). rep: perturbe, kernel, lr_xyz, lr_dc, lr_opacity, lr_scaling, lr_rotation, scale_offset (inverse
// softplus of the scaling bias), opacity_offset (inverse sigmoid of the opacity bias), base_offset_scale.
__device__ __forceinline__ float softplus(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

__global__ __launch_bounds__(256) void to_gaussians_kernel(const float* __restrict__ anchors, int64_t rows,
                                                           const float* __restrict__ features, int G,
                                                           const float* __restrict__ pert, const float* __restrict__ rep,
                                                           float* __restrict__ xyz, float* __restrict__ f_dc,
                                                           float* __restrict__ scale, float* __restrict__ rotation,
                                                           float* __restrict__ opacity) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * G) return;
    const int64_t a = i / G;
    const int g = (int)(i - a * G);
    const float perturbe = rep[0], kernel = rep[1], lr_xyz = rep[2], lr_dc = rep[3], lr_opacity = rep[4],
                lr_scaling = rep[5], lr_rotation = rep[6], scale_offset = rep[7], opacity_offset = rep[8],
                base_offset_scale = rep[9];
    const float* f = features + a * (int64_t)G * 15;
    const int xyz0 = 0, dc0 = G * 3, sc0 = G * 6, rot0 = G * 9, op0 = G * 13, os0 = G * 14;
    const float offset_scale = softplus(f[os0 + g] + base_offset_scale);
    for (int c = 0; c < 3; ++c) {
        const float o = tanhf(f[xyz0 + g * 3 + c] * lr_xyz + pert[g * 3 + c]) * 0.5f * perturbe * offset_scale;
        xyz[i * 3 + c] = (o + anchors[a * 3 + c]) - 0.5f;
        f_dc[i * 3 + c] = f[dc0 + g * 3 + c] * lr_dc;
        const float sv = softplus(f[sc0 + g * 3 + c] * lr_scaling + scale_offset);
        scale[i * 3 + c] = sqrtf(sv * sv + kernel * kernel);
    }
    float q[4], norm = 0.0f;
    for (int c = 0; c < 4; ++c) {
        q[c] = f[rot0 + g * 4 + c] * lr_rotation + (c == 0 ? 1.0f : 0.0f);
        norm += q[c] * q[c];
    }
    norm = fmaxf(sqrtf(norm), 1e-12f);
    for (int c = 0; c < 4; ++c) rotation[i * 4 + c] = q[c] / norm;
    opacity[i] = 1.0f / (1.0f + expf(-(f[op0 + g] * lr_opacity + opacity_offset)));
}

unsigned grid_of(int64_t items) {
    const int64_t g = (items + 255) / 256;
    return (unsigned)(g < 1 ? 1 : g > 1048576 ? 1048576 : g);
}

}  // namespace
}  // namespace idolq

using namespace idolq;

extern "C" int idolq_rms_heads(void* x, int dtype, int64_t rows, int64_t ld, int64_t heads, int64_t head_dim,
                               const float* gamma, void* stream) {
    if (!dtype_ok(dtype)) return fail(IDOLQ_EINVAL, "unknown dtype code");
    if (rows < 0 || heads <= 0 || head_dim <= 0 || ld < heads * head_dim)
        return fail(IDOLQ_EINVAL, "rms_heads: need rows >= 0, heads > 0, head_dim > 0 and ld >= heads * head_dim");
    if (rows == 0) return IDOLQ_OK;
    if (!x || !gamma) return fail(IDOLQ_EINVAL, "x and gamma must be non-null");
    const bool al = reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(gamma) % 16 == 0 &&
                    ld % 4 == 0;
    if (dtype == IDOLQ_F32 && al && (head_dim == 32 || head_dim == 64 || head_dim == 128)) {
        const dim3 grid((unsigned)((rows * heads + 255) / 256));
        hipStream_t s = static_cast<hipStream_t>(stream);
        float* xf = static_cast<float*>(x);
        if (head_dim == 32) hipLaunchKernelGGL(rms_heads_vec_kernel<32>, grid, dim3(256), 0, s, xf, rows, ld, (int)heads, gamma);
        else if (head_dim == 64) hipLaunchKernelGGL(rms_heads_vec_kernel<64>, grid, dim3(256), 0, s, xf, rows, ld, (int)heads, gamma);
        else hipLaunchKernelGGL(rms_heads_vec_kernel<128>, grid, dim3(256), 0, s, xf, rows, ld, (int)heads, gamma);
        return check_launch("rms_heads_vec_kernel");
    }
    hipLaunchKernelGGL(rms_heads_kernel, dim3((unsigned)((rows * heads + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), x, dtype, rows, ld, (int)heads, (int)head_dim, gamma);
    return check_launch("rms_heads_kernel");
}

extern "C" int idolq_add_gated(void* x, int x_dtype, int64_t ldx, const void* h, int h_dtype, int64_t ldh,
                               int64_t rows, int64_t dim, const float* gate, void* stream) {
    if (!dtype_ok(x_dtype) || !dtype_ok(h_dtype)) return fail(IDOLQ_EINVAL, "unknown dtype code");
    if (rows < 0 || dim < 0 || ldx < dim || ldh < dim) return fail(IDOLQ_EINVAL, "add_gated: bad rows, dim or stride");
    if (rows == 0 || dim == 0) return IDOLQ_OK;
    if (!x || !h || !gate) return fail(IDOLQ_EINVAL, "x, h and gate must be non-null");
    hipLaunchKernelGGL(add_gated_kernel, dim3(grid_of(rows * dim)), dim3(256), 0, static_cast<hipStream_t>(stream), x,
                       x_dtype, ldx, h, h_dtype, ldh, rows, dim, gate);
    return check_launch("add_gated_kernel");
}

extern "C" int idolq_level_embed(float resolution, const float* freqs, int64_t half, float* out, void* stream) {
    if (half <= 0 || half > 65536) return fail(IDOLQ_EINVAL, "level_embed: need 0 < half <= 65536");
    if (!freqs || !out) return fail(IDOLQ_EINVAL, "freqs and out must be non-null");
    hipLaunchKernelGGL(level_embed_kernel, dim3((unsigned)((half + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), resolution, freqs, (int)half, out);
    return check_launch("level_embed_kernel");
}

extern "C" int idolq_gemm_f32(const float* x, int64_t m, int64_t k, int64_t ldx, const float* w, int64_t n,
                              const float* bias, const float* residual, int64_t ldr, int act, float* y, int64_t ldy,
                              void* stream) {
    if (m < 0 || k <= 0 || n <= 0) return fail(IDOLQ_EINVAL, "gemm_f32: need m >= 0, k > 0 and n > 0");
    if (m > 0x7fffffffLL - kGT || n > 0x7fffffffLL - kGT || k > 0x7fffffffLL) return fail(IDOLQ_EINVAL, "gemm_f32: shape too large");
    if (ldx < k || ldy < n || (residual && ldr < n)) return fail(IDOLQ_EINVAL, "row stride smaller than the row");
    if (act < IDOLQ_ACT_NONE || act > IDOLQ_ACT_SILU) return fail(IDOLQ_EINVAL, "unknown activation");
    if (residual && residual == y && ldr != ldy) return fail(IDOLQ_EINVAL, "a residual aliasing y needs ldr == ldy");
    if (m == 0) return IDOLQ_OK;
    if (!x || !w || !y) return fail(IDOLQ_EINVAL, "x, w and y must be non-null");
    const int64_t gy = (m + kGT - 1) / kGT;
    if (gy > 65535) return fail(IDOLQ_EINVAL, "gemm_f32: more than 65535 * 64 rows");
    const dim3 grid((unsigned)((n + kGT - 1) / kGT), (unsigned)gy);
    auto a16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    const bool vec = a16(y) && ldy % 4 == 0 && (!bias || a16(bias)) && (!residual || (a16(residual) && ldr % 4 == 0));
    if (vec)
        hipLaunchKernelGGL(gemm_f32_kernel<true>, grid, dim3(256), 0, static_cast<hipStream_t>(stream), x, (int)m,
                           (int)k, ldx, w, (int)n, bias, residual, ldr, act, y, ldy);
    else
        hipLaunchKernelGGL(gemm_f32_kernel<false>, grid, dim3(256), 0, static_cast<hipStream_t>(stream), x, (int)m,
                           (int)k, ldx, w, (int)n, bias, residual, ldr, act, y, ldy);
    return check_launch("gemm_f32_kernel");
}

extern "C" int idolq_to_gaussians(const float* anchors, int64_t rows, const float* features, int64_t per_anchor,
                                  const float* perturbation, const float* rep, float* xyz, float* f_dc, float* scale,
                                  float* rotation, float* opacity, void* stream) {
    if (rows < 0 || per_anchor <= 0 || per_anchor > 4096) return fail(IDOLQ_EINVAL, "to_gaussians: bad rows or per_anchor");
    if (rows == 0) return IDOLQ_OK;
    if (!anchors || !features || !perturbation || !rep || !xyz || !f_dc || !scale || !rotation || !opacity)
        return fail(IDOLQ_EINVAL, "to_gaussians: null pointer");
    hipLaunchKernelGGL(to_gaussians_kernel, dim3((unsigned)((rows * per_anchor + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), anchors, rows, features, (int)per_anchor, perturbation, rep,
                       xyz, f_dc, scale, rotation, opacity);
    return check_launch("to_gaussians_kernel");
}
