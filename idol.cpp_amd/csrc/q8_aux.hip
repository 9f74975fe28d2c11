// Entry points around the Q8_0 GEMM: the C ABI's error slot and version, Q8_0 expansion, the int8 activation
// quantizer, activations, the sine/cosine position embedding and a strided copy.
#include "common.h"

#include <cstdio>
#include <type_traits>

namespace idolq {

namespace {
thread_local std::string g_error;
}

void set_error(const std::string& msg) { g_error = msg; }

int fail(int code, const std::string& msg) {
    g_error = msg;
    return code;
}

int check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(IDOLQ_ELAUNCH, std::string(what) + ": " + hipGetErrorString(e));
    return IDOLQ_OK;
}

namespace {

// ------------------------------------------------------------------------------------------------ Q8_0 expansion
// One thread per Q8_0 block: 32 outputs fp32(d) * q rounded to the output dtype, written as 16-byte stores.
__global__ __launch_bounds__(256) void q8_dequant_kernel(const uint8_t* __restrict__ w, int64_t blocks, void* out,
                                                         int out_dt) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= blocks) return;
    const uint8_t* blk = w + b * kQ8Bytes;
    const float d = half_bits_to_float((uint16_t)(blk[0] | (blk[1] << 8)));
    if (out_dt == IDOLQ_F32) {
        float* o = static_cast<float*>(out) + b * kQ8Block;
        for (int t = 0; t < kQ8Block; t += 4) {
            float4 v;
            v.x = (float)(int8_t)blk[2 + t] * d;
            v.y = (float)(int8_t)blk[3 + t] * d;
            v.z = (float)(int8_t)blk[4 + t] * d;
            v.w = (float)(int8_t)blk[5 + t] * d;
            *reinterpret_cast<float4*>(o + t) = v;
        }
    } else {
        uint16_t* o = static_cast<uint16_t*>(out) + b * kQ8Block;
        for (int t = 0; t < kQ8Block; t += 8) {
            uint32_t packed[4];
            for (int e = 0; e < 4; ++e) {
                const float lo = (float)(int8_t)blk[2 + t + 2 * e] * d, hi = (float)(int8_t)blk[3 + t + 2 * e] * d;
                const uint16_t l = out_dt == IDOLQ_BF16 ? float_to_bf16_bits(lo) : float_to_half_bits(lo);
                const uint16_t h = out_dt == IDOLQ_BF16 ? float_to_bf16_bits(hi) : float_to_half_bits(hi);
                packed[e] = (uint32_t)l | ((uint32_t)h << 16);
            }
            *reinterpret_cast<uint4*>(o + t) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
        }
    }
}

// ------------------------------------------------------------------------------------------------ Q8_0 quantizer
// One thread per 32-value block of an fp32 [n x k] matrix: d = amax / 127, id = d ? 1 / d : 0,
// q = round-half-away-from-zero(x * id), d stored as fp16 (ggml's quantize_row_q8_0_ref, the rule gguf-py's
// Q8_0.quantize_blocks restates). The quotient and the product are IEEE fp32, so the codes match a CPU run of the
// same rule bit for bit.
__global__ __launch_bounds__(256) void q8_quantize_kernel(const float* __restrict__ w, int64_t nb, int64_t blocks,
                                                          int64_t ldw, uint8_t* __restrict__ out) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= blocks) return;
    const int64_t r = b / nb, g = b - r * nb;
    const float* x = w + r * ldw + g * kQ8Block;
    float v[kQ8Block];
    float amax = 0.0f;
    for (int t = 0; t < kQ8Block; ++t) {
        v[t] = x[t];
        amax = fmaxf(amax, fabsf(v[t]));
    }
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint8_t* o = out + b * kQ8Bytes;
    const uint16_t dh = float_to_half_bits(d);
    o[0] = (uint8_t)(dh & 0xff);
    o[1] = (uint8_t)(dh >> 8);
    for (int t = 0; t < kQ8Block; ++t) o[2 + t] = (uint8_t)(int8_t)roundf(v[t] * id);
}

// ------------------------------------------------------------------------------------------------ int8 activations
// One thread per (row, 32-block): amax, s = amax / 127, inv = 127 / amax, q = rint(x * inv). Division and the
// product are IEEE fp32 (correctly rounded), rint rounds ties to even: the same operations, in the same order, as
// the reference's quantize_activations, so qa, s and qsum are bit-identical.
__global__ __launch_bounds__(256) void quantize_act_kernel(const void* __restrict__ x, int x_dt, int64_t m,
                                                           int64_t nb, int64_t ldx, int8_t* __restrict__ qa,
                                                           float* __restrict__ scale, int32_t* __restrict__ qsum) {
    const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= m * nb) return;
    const int64_t r = id / nb, g = id - r * nb;
    float v[kQ8Block];
    const int64_t base = r * ldx + g * kQ8Block;
    for (int t = 0; t < kQ8Block; ++t) v[t] = load_as_float(x, x_dt, base + t);
    float amax = 0.0f;
    for (int t = 0; t < kQ8Block; ++t) amax = fmaxf(amax, fabsf(v[t]));
    const float s = amax / 127.0f;
    const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
    int32_t sum = 0;
    uint32_t words[8];
    for (int t = 0; t < kQ8Block; t += 4) {
        uint32_t word = 0;
        for (int e = 0; e < 4; ++e) {
            const int32_t q = (int32_t)rintf(v[t + e] * inv);
            sum += q;
            word |= (uint32_t)(uint8_t)(int8_t)q << (8 * e);
        }
        words[t / 4] = word;
    }
    int8_t* dst = qa + r * (nb * kQ8Block) + g * kQ8Block;
    *reinterpret_cast<uint4*>(dst) = make_uint4(words[0], words[1], words[2], words[3]);
    *reinterpret_cast<uint4*>(dst + 16) = make_uint4(words[4], words[5], words[6], words[7]);
    scale[id] = s;
    if (qsum) qsum[id] = sum;
}

// The same rule for activations with 16-byte aligned rows, four threads per (row, 32-block): each loads its 8 values
// with 16-byte loads (consecutive lanes read consecutive bytes), the block's maximum comes from two exchanges inside
// the group of four, and each thread writes its 8 codes (the first one the scale). No code sums.
// TILED (the layout of the GEMM on tiled weights): each block's codes in the order 0..7, 16..23, 8..15, 24..31 (the
// k order of the tiled weights' MFMA fragments), and the scales stage-major: block g of row r at
// (g / 2) * 2 m + 2 r + g % 2 (the two blocks of a 64-deep stage of consecutive rows are contiguous).
// zero (TILED): nzero ints cleared on the side (the GEMM's tile counters).
template <typename T, bool TILED>
__global__ __launch_bounds__(256) void quantize_act16_kernel(const T* __restrict__ x, int64_t m, int64_t nb,
                                                             int64_t ldx, int8_t* __restrict__ qa,
                                                             float* __restrict__ scale, int* __restrict__ zero,
                                                             int nzero) {
    const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (TILED && zero)
        for (int64_t i = id; i < nzero; i += (int64_t)gridDim.x * blockDim.x) zero[i] = 0;
    const int64_t blocks = m * nb;
    const bool ok = (id >> 2) < blocks;
    const int64_t b = ok ? id >> 2 : blocks - 1;  // every lane takes part in the exchanges
    const int qt = (int)(id & 3);
    const int64_t r = b / nb, g = b - r * nb;
    float v[8];
    if constexpr (std::is_same<T, float>::value) {
        const float4 lo = *reinterpret_cast<const float4*>(x + r * ldx + g * kQ8Block + 8 * qt);
        const float4 hi = *reinterpret_cast<const float4*>(x + r * ldx + g * kQ8Block + 8 * qt + 4);
        v[0] = lo.x, v[1] = lo.y, v[2] = lo.z, v[3] = lo.w, v[4] = hi.x, v[5] = hi.y, v[6] = hi.z, v[7] = hi.w;
    } else {
        const uint4 raw = *reinterpret_cast<const uint4*>(x + r * ldx + g * kQ8Block + 8 * qt);
        const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint16_t h = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
            v[e] = std::is_same<T, __bf16>::value ? bf16_bits_to_float(h) : half_bits_to_float(h);
        }
    }
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[e]));
    amax = fmaxf(amax, __shfl_xor(amax, 1));
    amax = fmaxf(amax, __shfl_xor(amax, 2));
    const float s = amax / 127.0f;
    const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
    uint32_t word[2] = {0, 0};
#pragma unroll
    for (int e = 0; e < 8; ++e) word[e >> 2] |= (uint32_t)(uint8_t)(int8_t)(int32_t)rintf(v[e] * inv) << (8 * (e & 3));
    if (ok) {
        const int pos = TILED ? 8 * (2 * (qt & 1) + (qt >> 1)) : 8 * qt;
        *reinterpret_cast<uint2*>(qa + r * (nb * kQ8Block) + g * kQ8Block + pos) = make_uint2(word[0], word[1]);
        if (qt == 0) scale[TILED ? (g >> 1) * 2 * m + 2 * r + (g & 1) : b] = s;
    }
}

// The EXACT mode on tiled weights: activations (fp32, bf16 or fp16, 16-byte aligned rows) to bf16 high parts
// hi = bf16(x) and low parts lo = bf16(x - hi), [m, k] each with row stride k (the split of the row-major EXACT
// kernel), eight values per thread; zero: nzero ints cleared on the side (the GEMM's tile counters).
template <typename T>
__global__ __launch_bounds__(256) void split_bf16_kernel(const T* __restrict__ x, int64_t m, int64_t k, int64_t ldx,
                                                         uint16_t* __restrict__ hi, uint16_t* __restrict__ lo,
                                                         int* __restrict__ zero, int nzero) {
    const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (zero)
        for (int64_t i = id; i < nzero; i += (int64_t)gridDim.x * blockDim.x) zero[i] = 0;
    const int64_t per_row = k / 8;
    if (id >= m * per_row) return;
    const int64_t r = id / per_row, c = (id - r * per_row) * 8;
    float v[8];
    if constexpr (std::is_same<T, float>::value) {
        const float4 a = *reinterpret_cast<const float4*>(x + r * ldx + c);
        const float4 b = *reinterpret_cast<const float4*>(x + r * ldx + c + 4);
        v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
    } else {
        const uint4 raw = *reinterpret_cast<const uint4*>(x + r * ldx + c);
        const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint16_t h = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
            v[e] = std::is_same<T, __bf16>::value ? bf16_bits_to_float(h) : half_bits_to_float(h);
        }
    }
    uint32_t h2[4], l2[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const uint16_t h0 = float_to_bf16_bits(v[2 * e]), h1 = float_to_bf16_bits(v[2 * e + 1]);
        const uint16_t l0 = float_to_bf16_bits(v[2 * e] - bf16_bits_to_float(h0));
        const uint16_t l1 = float_to_bf16_bits(v[2 * e + 1] - bf16_bits_to_float(h1));
        h2[e] = (uint32_t)h0 | ((uint32_t)h1 << 16);
        l2[e] = (uint32_t)l0 | ((uint32_t)l1 << 16);
    }
    *reinterpret_cast<uint4*>(hi + r * k + c) = make_uint4(h2[0], h2[1], h2[2], h2[3]);
    *reinterpret_cast<uint4*>(lo + r * k + c) = make_uint4(l2[0], l2[1], l2[2], l2[3]);
}

// ------------------------------------------------------------------------------------------------ elementwise
__global__ __launch_bounds__(256) void activation_kernel(void* x, int dt, int64_t count, int act) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += stride)
        store_from_float(x, dt, i, apply_act(act, load_as_float(x, dt, i)));
}

__global__ __launch_bounds__(256) void pos_embed_kernel(const float* __restrict__ coords, int64_t rows,
                                                        const float* __restrict__ freqs, int nfreq, void* out,
                                                        int out_dt, int64_t ldo) {
    const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t per_row = 3 * (int64_t)nfreq;
    if (id >= rows * per_row) return;
    const int64_t r = id / per_row;
    const int rem = (int)(id - r * per_row);
    const int c = rem / nfreq, j = rem - c * nfreq;
    const float kPi = 3.14159265358979323846f;
    const float ang = (coords[r * 3 + c] * freqs[j]) * kPi;
    const int64_t o = r * ldo + (int64_t)c * 2 * nfreq + j;
    store_from_float(out, out_dt, o, sinf(ang));
    store_from_float(out, out_dt, o + nfreq, cosf(ang));
}

__global__ __launch_bounds__(256) void copy2d_kernel(const void* src, int sdt, int64_t lds, void* dst, int ddt,
                                                     int64_t ldd, int64_t rows, int64_t cols) {
    const int64_t total = rows * cols, stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
        const int64_t r = i / cols, c = i - r * cols;
        store_from_float(dst, ddt, r * ldd + c, load_as_float(src, sdt, r * lds + c));
    }
}

// 16-byte copies of 8-element groups: cols % 8 == 0 and both buffers vector-aligned.
template <int SDT, int DDT>
__global__ __launch_bounds__(256) void copy2d_vec_kernel(const void* src, int64_t lds, void* dst, int64_t ldd,
                                                         int64_t rows, int64_t groups_per_row) {
    const int64_t total = rows * groups_per_row, stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
        const int64_t r = i / groups_per_row, c = (i - r * groups_per_row) * 8;
        float f[8];
        load8<SDT>(src, r * lds + c, f);
        store8<DDT>(dst, r * ldd + c, f);
    }
}

// One thread per (row, coordinate): nfreq sines then nfreq cosines as 16-bit values, stored 8 at a time.
template <int DT>
__global__ __launch_bounds__(256) void pos_embed_vec_kernel(const float* __restrict__ coords, int64_t rows,
                                                            const float* __restrict__ freqs, int nfreq, void* out,
                                                            int64_t ldo) {
    const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= rows * 3) return;
    const int64_t r = id / 3;
    const int c = (int)(id - r * 3);
    const float kPi = 3.14159265358979323846f;
    const float v = coords[r * 3 + c];
    const int64_t o = r * ldo + (int64_t)c * 2 * nfreq;
    for (int j0 = 0; j0 < nfreq; j0 += 8) {
        float sn[8], cs[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float ang = (v * freqs[j0 + e]) * kPi;
            sn[e] = sinf(ang);
            cs[e] = cosf(ang);
        }
        store8<DT>(out, o + j0, sn);
        store8<DT>(out, o + nfreq + j0, cs);
    }
}

unsigned grid_for(int64_t items, int threads = 256) {
    const int64_t g = (items + threads - 1) / threads;
    return (unsigned)(g < 1 ? 1 : g > 1048576 ? 1048576 : g);
}

}  // namespace

// The high / low split of the EXACT mode on tiled weights (split_bf16_kernel); k % 8 == 0, aligned rows.
int split_bf16_launch(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, uint16_t* hi, uint16_t* lo,
                      int* zero, int nzero, hipStream_t stream) {
    const int64_t n = m * (k / 8);
    if (n == 0) return IDOLQ_OK;
    const dim3 grid((unsigned)((n + 255) / 256));
    if (x_dtype == IDOLQ_BF16)
        hipLaunchKernelGGL(split_bf16_kernel<__bf16>, grid, dim3(256), 0, stream, static_cast<const __bf16*>(x), m, k,
                           ldx, hi, lo, zero, nzero);
    else if (x_dtype == IDOLQ_F16)
        hipLaunchKernelGGL(split_bf16_kernel<_Float16>, grid, dim3(256), 0, stream, static_cast<const _Float16*>(x), m,
                           k, ldx, hi, lo, zero, nzero);
    else
        hipLaunchKernelGGL(split_bf16_kernel<float>, grid, dim3(256), 0, stream, static_cast<const float*>(x), m, k, ldx,
                           hi, lo, zero, nzero);
    return check_launch("split_bf16_kernel");
}

// The tiled-GEMM layout of the INT8 mode (quantize_act16_kernel<T, true>): x rows 16-byte aligned, k a multiple of 64.
int quantize_act_tiled_launch(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, int8_t* qa, float* scale,
                              int* zero, int nzero, hipStream_t stream) {
    const int64_t nb = k / kQ8Block;
    if (m * nb == 0) return IDOLQ_OK;
    const dim3 grid((unsigned)((4 * m * nb + 255) / 256));
    if (x_dtype == IDOLQ_BF16)
        hipLaunchKernelGGL((quantize_act16_kernel<__bf16, true>), grid, dim3(256), 0, stream,
                           static_cast<const __bf16*>(x), m, nb, ldx, qa, scale, zero, nzero);
    else if (x_dtype == IDOLQ_F16)
        hipLaunchKernelGGL((quantize_act16_kernel<_Float16, true>), grid, dim3(256), 0, stream,
                           static_cast<const _Float16*>(x), m, nb, ldx, qa, scale, zero, nzero);
    else
        hipLaunchKernelGGL((quantize_act16_kernel<float, true>), grid, dim3(256), 0, stream, static_cast<const float*>(x),
                           m, nb, ldx, qa, scale, zero, nzero);
    return check_launch("quantize_act16_kernel");
}


int quantize_act_launch(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, int8_t* qa, float* scale,
                        int32_t* qsum, hipStream_t stream) {
    const int64_t nb = k / kQ8Block;
    if (m * nb == 0) return IDOLQ_OK;
    const bool vec16 = !qsum && (x_dtype == IDOLQ_BF16 || x_dtype == IDOLQ_F16) &&
                       reinterpret_cast<uintptr_t>(x) % 16 == 0 && (ldx * 2) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(qa) % 8 == 0;
    if (vec16) {
        const dim3 grid((unsigned)((4 * m * nb + 255) / 256));
        if (x_dtype == IDOLQ_BF16)
            hipLaunchKernelGGL((quantize_act16_kernel<__bf16, false>), grid, dim3(256), 0, stream,
                               static_cast<const __bf16*>(x), m, nb, ldx, qa, scale, nullptr, 0);
        else
            hipLaunchKernelGGL((quantize_act16_kernel<_Float16, false>), grid, dim3(256), 0, stream,
                               static_cast<const _Float16*>(x), m, nb, ldx, qa, scale, nullptr, 0);
        return check_launch("quantize_act16_kernel");
    }
    hipLaunchKernelGGL(quantize_act_kernel, dim3((unsigned)((m * nb + 255) / 256)), dim3(256), 0, stream, x, x_dtype, m,
                       nb, ldx, qa, scale, qsum);
    return check_launch("quantize_act_kernel");
}

}  // namespace idolq

using namespace idolq;

extern "C" const char* idolq_last_error(void) { return g_error.c_str(); }

extern "C" const char* idolq_version(void) { return "libidolq 0.1 gfx950"; }

extern "C" int64_t idolq_q8_0_bytes(int64_t n, int64_t k) {
    if (n < 0 || k < 0 || k % kQ8Block) return 0;
    return n * (k / kQ8Block) * kQ8Bytes;
}

extern "C" int idolq_q8_0_dequant(const uint8_t* w, int64_t n, int64_t k, void* out, int out_dtype, void* stream) {
    if (!dtype_ok(out_dtype)) return fail(IDOLQ_EINVAL, "unknown dtype code");
    if (n < 0 || k <= 0 || k % kQ8Block) return fail(IDOLQ_EINVAL, "need n >= 0 and k a positive multiple of 32");
    const int64_t blocks = n * (k / kQ8Block);
    if (blocks == 0) return IDOLQ_OK;
    if (!w || !out) return fail(IDOLQ_EINVAL, "w and out must be non-null");
    if (reinterpret_cast<uintptr_t>(out) % 16 != 0) return fail(IDOLQ_EINVAL, "out must be 16-byte aligned");
    hipLaunchKernelGGL(q8_dequant_kernel, dim3((unsigned)((blocks + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), w, blocks, out, out_dtype);
    return check_launch("q8_dequant_kernel");
}

// One dword of the grouped layout per thread. Dword u of chunk (g, s) (544 dwords):
//   u < 512: byte 4 u of the codes: block b = u / 256, lane l = (u / 4) % 64, dword e = u % 4 of the lane's 16 bytes:
//            codes 16 (e / 2) + 8 (l / 32) + 4 (e % 2) .. + 3 of block 2 s + b of row 32 g + l % 32;
//   u >= 512: the two fp16 scales (blocks 2 s, 2 s + 1) of row 32 g + u - 512.
// Rows past n are zero. A row's codes start 2 bytes into each 34-byte block, so they are read bytewise.
__global__ __launch_bounds__(256) void q8_group_kernel(const uint8_t* __restrict__ w, int64_t n, int64_t row_bytes,
                                                       int stages, int64_t total, uint32_t* __restrict__ out) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t chunk = i / 544;
        const int u = (int)(i - chunk * 544);
        const int64_t g = chunk / stages;
        const int s = (int)(chunk - g * stages);
        const int r = u < 512 ? ((u >> 2) & 63) & 31 : u - 512;
        const int64_t row = g * 32 + r;
        uint32_t v = 0;
        if (row < n) {
            const uint8_t* rp = w + row * row_bytes;
            if (u < 512) {
                const int b = u >> 8, l = (u >> 2) & 63, e = u & 3;
                const uint8_t* q = rp + (int64_t)(2 * s + b) * kQ8Bytes + 2 + 16 * (e >> 1) + 8 * (l >> 5) + 4 * (e & 1);
                v = (uint32_t)q[0] | ((uint32_t)q[1] << 8) | ((uint32_t)q[2] << 16) | ((uint32_t)q[3] << 24);
            } else {
                const uint8_t* d0 = rp + (int64_t)(2 * s) * kQ8Bytes;
                v = (uint32_t)d0[0] | ((uint32_t)d0[1] << 8) | ((uint32_t)d0[kQ8Bytes] << 16) |
                    ((uint32_t)d0[kQ8Bytes + 1] << 24);
            }
        }
        out[i] = v;
    }
}

extern "C" int64_t idolq_q8_0_tiled_bytes(int64_t n, int64_t k) {
    if (n < 0 || k <= 0 || k % 64) return 0;
    return (n + 31) / 32 * (k / 64) * 2176;
}

extern "C" int idolq_q8_0_tile(const uint8_t* w, int64_t n, int64_t k, uint8_t* out, void* stream) {
    if (n < 0 || k <= 0 || k % 64) return fail(IDOLQ_EINVAL, "tiled Q8_0 needs n >= 0 and k a positive multiple of 64");
    if (n == 0) return IDOLQ_OK;
    if (!w || !out) return fail(IDOLQ_EINVAL, "w and out must be non-null");
    if (reinterpret_cast<uintptr_t>(out) & 3) return fail(IDOLQ_EINVAL, "out must be 4-byte aligned");
    const int64_t total = idolq_q8_0_tiled_bytes(n, k) / 4;
    hipLaunchKernelGGL(q8_group_kernel, dim3(grid_for(total)), dim3(256), 0, static_cast<hipStream_t>(stream), w, n,
                       (k / kQ8Block) * kQ8Bytes, (int)(k / 64), total, reinterpret_cast<uint32_t*>(out));
    return check_launch("q8_group_kernel");
}

extern "C" int idolq_q8_0_quantize(const float* w, int64_t n, int64_t k, int64_t ldw, uint8_t* out, void* stream) {
    if (n < 0 || k <= 0 || k % kQ8Block || ldw < k) return fail(IDOLQ_EINVAL, "need n >= 0, k a positive multiple of 32, ldw >= k");
    const int64_t nb = k / kQ8Block, blocks = n * nb;
    if (blocks == 0) return IDOLQ_OK;
    if (!w || !out) return fail(IDOLQ_EINVAL, "w and out must be non-null");
    hipLaunchKernelGGL(q8_quantize_kernel, dim3((unsigned)((blocks + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), w, nb, blocks, ldw, out);
    return check_launch("q8_quantize_kernel");
}

extern "C" int idolq_quantize_act_q8(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, int8_t* qa,
                                     float* scale, int32_t* qsum, void* stream) {
    if (!dtype_ok(x_dtype)) return fail(IDOLQ_EINVAL, "unknown dtype code");
    if (m < 0 || k <= 0 || k % kQ8Block || ldx < k) return fail(IDOLQ_EINVAL, "need m >= 0, k a positive multiple of 32, ldx >= k");
    if (m == 0) return IDOLQ_OK;
    if (!x || !qa || !scale) return fail(IDOLQ_EINVAL, "x, qa and scale must be non-null");
    if (reinterpret_cast<uintptr_t>(qa) % 16 != 0) return fail(IDOLQ_EINVAL, "qa must be 16-byte aligned");
    return quantize_act_launch(x, x_dtype, m, k, ldx, qa, scale, qsum, static_cast<hipStream_t>(stream));
}

extern "C" int idolq_activation(void* x, int dtype, int64_t count, int act, void* stream) {
    if (!x && count > 0) return fail(IDOLQ_EINVAL, "x must be non-null");
    if (!dtype_ok(dtype)) return fail(IDOLQ_EINVAL, "unknown dtype code");
    if (act < IDOLQ_ACT_NONE || act > IDOLQ_ACT_SILU) return fail(IDOLQ_EINVAL, "unknown activation");
    if (count <= 0 || act == IDOLQ_ACT_NONE) return IDOLQ_OK;
    hipLaunchKernelGGL(activation_kernel, dim3(grid_for(count)), dim3(256), 0, static_cast<hipStream_t>(stream), x,
                       dtype, count, act);
    return check_launch("activation_kernel");
}

extern "C" int idolq_pos_embed(const float* coords, int64_t rows, const float* freqs, int64_t nfreq, void* out,
                               int out_dtype, int64_t ldo, void* stream) {
    if (!dtype_ok(out_dtype)) return fail(IDOLQ_EINVAL, "unknown dtype code");
    if (rows < 0 || nfreq <= 0 || nfreq > 65536 || ldo < 6 * nfreq) return fail(IDOLQ_EINVAL, "bad pos_embed shape");
    if (rows == 0) return IDOLQ_OK;
    if (!coords || !freqs || !out) return fail(IDOLQ_EINVAL, "coords, freqs and out must be non-null");
    if (out_dtype != IDOLQ_F32 && nfreq % 8 == 0 && vec8_ok(out, out_dtype, ldo)) {
        const unsigned blocks = (unsigned)((rows * 3 + 255) / 256);
        if (out_dtype == IDOLQ_BF16)
            hipLaunchKernelGGL(pos_embed_vec_kernel<IDOLQ_BF16>, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                               coords, rows, freqs, (int)nfreq, out, ldo);
        else
            hipLaunchKernelGGL(pos_embed_vec_kernel<IDOLQ_F16>, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                               coords, rows, freqs, (int)nfreq, out, ldo);
        return check_launch("pos_embed_vec_kernel");
    }
    const int64_t items = rows * 3 * nfreq;
    hipLaunchKernelGGL(pos_embed_kernel, dim3((unsigned)((items + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), coords, rows, freqs, (int)nfreq, out, out_dtype, ldo);
    return check_launch("pos_embed_kernel");
}

extern "C" int idolq_copy2d(const void* src, int src_dtype, int64_t lds, void* dst, int dst_dtype, int64_t ldd,
                            int64_t rows, int64_t cols, void* stream) {
    if (!dtype_ok(src_dtype) || !dtype_ok(dst_dtype)) return fail(IDOLQ_EINVAL, "unknown dtype code");
    if (rows < 0 || cols < 0 || lds < cols || ldd < cols) return fail(IDOLQ_EINVAL, "bad copy shape");
    if (rows * cols == 0) return IDOLQ_OK;
    if (!src || !dst) return fail(IDOLQ_EINVAL, "src and dst must be non-null");
    if (cols % 8 == 0 && vec8_ok(src, src_dtype, lds) && vec8_ok(dst, dst_dtype, ldd)) {
        hipStream_t s = static_cast<hipStream_t>(stream);
        const int64_t g = cols / 8;
        const dim3 grid(grid_for(rows * g)), block(256);
#define IDOLQ_COPY(S, D) hipLaunchKernelGGL((copy2d_vec_kernel<S, D>), grid, block, 0, s, src, lds, dst, ldd, rows, g)
#define IDOLQ_COPY_TO(S)                                             \
        if (dst_dtype == IDOLQ_F32) IDOLQ_COPY(S, IDOLQ_F32);        \
        else if (dst_dtype == IDOLQ_BF16) IDOLQ_COPY(S, IDOLQ_BF16); \
        else IDOLQ_COPY(S, IDOLQ_F16)
        if (src_dtype == IDOLQ_F32) { IDOLQ_COPY_TO(IDOLQ_F32); }
        else if (src_dtype == IDOLQ_BF16) { IDOLQ_COPY_TO(IDOLQ_BF16); }
        else { IDOLQ_COPY_TO(IDOLQ_F16); }
#undef IDOLQ_COPY_TO
#undef IDOLQ_COPY
        return check_launch("copy2d_vec_kernel");
    }
    hipLaunchKernelGGL(copy2d_kernel, dim3(grid_for(rows * cols)), dim3(256), 0, static_cast<hipStream_t>(stream), src,
                       src_dtype, lds, dst, dst_dtype, ldd, rows, cols);
    return check_launch("copy2d_kernel");
}
