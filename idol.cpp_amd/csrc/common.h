// Shared definitions for the gfx950 kernels of libidolq: vector types for the MFMA builtins, dtype conversion,
// error reporting for the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>
#include <type_traits>
#include <utility>

#include "../../include/idolq.h"

namespace idolq {

// Operand and accumulator vectors of the gfx950 MFMA builtins.
typedef __bf16 bf16x8 __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef _Float16 f16x8 __attribute__((__vector_size__(8 * sizeof(_Float16))));
typedef int i32x4 __attribute__((__vector_size__(4 * sizeof(int))));
typedef float f32x4 __attribute__((__vector_size__(4 * sizeof(float))));
typedef float f32x16 __attribute__((__vector_size__(16 * sizeof(float))));
typedef int i32x16 __attribute__((__vector_size__(16 * sizeof(int))));

// f(std::integral_constant<int, I>) for I = 0 .. N - 1, expanded at compile time (register-array indices stay constant)
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

constexpr int kQ8Block = 32;  // k values per Q8_0 block
constexpr int kQ8Bytes = 34;  // fp16 scale + 32 int8 codes

// ------------------------------------------------------------------------------------------------ host: errors
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int check_launch(const char* what);
inline bool dtype_ok(int dt) { return dt == IDOLQ_F32 || dt == IDOLQ_F16 || dt == IDOLQ_BF16; }
inline size_t dtype_size(int dt) { return dt == IDOLQ_F32 ? 4 : 2; }

// ------------------------------------------------------------------------------------------------ device: dtypes
__device__ __forceinline__ float half_bits_to_float(uint16_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

__device__ __forceinline__ float bf16_bits_to_float(uint16_t b) {
    return __builtin_bit_cast(float, static_cast<uint32_t>(b) << 16);
}

// Round-to-nearest-even conversions (the hardware's default conversion mode).
__device__ __forceinline__ uint16_t float_to_bf16_bits(float f) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f)); }
__device__ __forceinline__ uint16_t float_to_half_bits(float f) { return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f)); }

// Load element i of a buffer of the given dtype as fp32.
__device__ __forceinline__ float load_as_float(const void* p, int dt, int64_t i) {
    if (dt == IDOLQ_F32) return static_cast<const float*>(p)[i];
    const uint16_t b = static_cast<const uint16_t*>(p)[i];
    return dt == IDOLQ_BF16 ? bf16_bits_to_float(b) : half_bits_to_float(b);
}

__device__ __forceinline__ void store_from_float(void* p, int dt, int64_t i, float v) {
    if (dt == IDOLQ_F32) {
        static_cast<float*>(p)[i] = v;
    } else {
        static_cast<uint16_t*>(p)[i] = dt == IDOLQ_BF16 ? float_to_bf16_bits(v) : float_to_half_bits(v);
    }
}

// Eight consecutive elements of a dtype as fp32, through 16-byte accesses (the address must be 16-byte aligned).
template <int DT>
__device__ __forceinline__ void load8(const void* base, int64_t i, float (&f)[8]) {
    if (DT == IDOLQ_F32) {
        const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(base) + i);
        const float4 b = *reinterpret_cast<const float4*>(static_cast<const float*>(base) + i + 4);
        f[0] = a.x, f[1] = a.y, f[2] = a.z, f[3] = a.w, f[4] = b.x, f[5] = b.y, f[6] = b.z, f[7] = b.w;
    } else {
        const uint4 r = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + i);
        const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint16_t b = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
            f[e] = DT == IDOLQ_BF16 ? bf16_bits_to_float(b) : half_bits_to_float(b);
        }
    }
}

template <int DT>
__device__ __forceinline__ void store8(void* base, int64_t i, const float (&f)[8]) {
    if (DT == IDOLQ_F32) {
        *reinterpret_cast<float4*>(static_cast<float*>(base) + i) = make_float4(f[0], f[1], f[2], f[3]);
        *reinterpret_cast<float4*>(static_cast<float*>(base) + i + 4) = make_float4(f[4], f[5], f[6], f[7]);
    } else {
        uint32_t w[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint16_t lo = DT == IDOLQ_BF16 ? float_to_bf16_bits(f[2 * q]) : float_to_half_bits(f[2 * q]);
            const uint16_t hi = DT == IDOLQ_BF16 ? float_to_bf16_bits(f[2 * q + 1]) : float_to_half_bits(f[2 * q + 1]);
            w[q] = (uint32_t)lo | ((uint32_t)hi << 16);
        }
        *reinterpret_cast<uint4*>(static_cast<uint16_t*>(base) + i) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

// The pointer and the row stride (elements of the dtype) allow 16-byte accesses to 8-element groups.
inline bool vec8_ok(const void* p, int dt, int64_t ld) {
    return reinterpret_cast<uintptr_t>(p) % 16 == 0 && (ld * (int64_t)dtype_size(dt)) % 16 == 0;
}

// v as an fp32 register value: the compiler may not fuse the operation that produced it with what consumes it (a
// multiply followed by a 16-bit conversion would otherwise become one v_fma_mix with a single rounding, where the
// fp32 result rounded to the output dtype is two).
__device__ __forceinline__ float fp32_value(float v) {
    asm("" : "+v"(v));
    return v;
}

// Round a float through a dtype and back (identity for fp32).
__device__ __forceinline__ float round_through(int dt, float v) {
    if (dt == IDOLQ_BF16) return bf16_bits_to_float(float_to_bf16_bits(v));
    if (dt == IDOLQ_F16) return half_bits_to_float(float_to_half_bits(v));
    return v;
}

// ------------------------------------------------------------------------------------------------ activations
__device__ __forceinline__ float apply_act(int act, float v) {
    switch (act) {
        case IDOLQ_ACT_GELU_ERF: return 0.5f * v * (1.0f + erff(v * 0.70710678118654752f));
        case IDOLQ_ACT_GELU_TANH: {
            // 0.5 v (1 + tanh(u)) = v / (1 + exp(-2u)), u = sqrt(2/pi) (v + 0.044715 v^3): one exp2 and one
            // reciprocal (a few ulp, far below the 16-bit output rounding); exp2 -> inf gives -0 for large negative v.
            // The exponent -2u log2(e) = v (-0.10294324 v^2 - 2.3022082): 2 sqrt(2/pi) (1, 0.044715) times -log2(e).
            const float t = v * fmaf(-1.0294324160e-01f, v * v, -2.3022081852e+00f);
            return v * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(t));
        }
        case IDOLQ_ACT_RELU: return v > 0.0f ? v : 0.0f;
        case IDOLQ_ACT_SILU: return v / (1.0f + expf(-v));
        default: return v;
    }
}

}  // namespace idolq
