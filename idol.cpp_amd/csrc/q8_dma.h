// Device helpers shared by the DEQUANT GEMM kernels that stage operands with direct global -> LDS loads
// (q8_gemm_pipe.hip, q8_gemm_wide.hip): the 16-bit MFMA wrapper, Q8_0 code -> operand conversion, the LDS-DMA
// instructions and explicit vector-memory waits.
#pragma once

#include "q8_gemm.h"

namespace idolq {

typedef __attribute__((address_space(3))) char lds_char;
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef int i32x2 __attribute__((ext_vector_type(2)));

template <typename T>
struct PipeMfma;
template <>
struct PipeMfma<__bf16> {
    typedef bf16x8 vec;
    typedef bf16x2 pair;
    static __device__ __forceinline__ f32x16 run(vec a, vec b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
};
template <>
struct PipeMfma<_Float16> {
    typedef f16x8 vec;
    typedef f16x2 pair;
    static __device__ __forceinline__ f32x16 run(vec a, vec b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
};

// Eight int8 codes (in a uint2) to eight operands T(fp32(d) * q), pairs rounded by one packed conversion.
template <typename T>
__device__ __forceinline__ uint4 dequant8(uint2 raw, float d) {
    typedef typename PipeMfma<T>::pair T2;
    uint32_t out[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const uint32_t word = e < 2 ? raw.x : raw.y;
        const int sh = 16 * (e & 1);
        f32x2 f;
        f.x = (float)(int)(int8_t)(uint8_t)(word >> sh);
        f.y = (float)(int)(int8_t)(uint8_t)(word >> (sh + 8));
        out[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f * d, T2));
    }
    return make_uint4(out[0], out[1], out[2], out[3]);
}

// Four int8 codes (one dword) to four operands T(fp32(d) * q) (two packed pairs).
template <typename T>
__device__ __forceinline__ uint2 dequant4(uint32_t word, float d) {
    typedef typename PipeMfma<T>::pair T2;
    f32x2 lo, hi;
    lo.x = (float)(int)(int8_t)(uint8_t)word;
    lo.y = (float)(int)(int8_t)(uint8_t)(word >> 8);
    hi.x = (float)(int)(int8_t)(uint8_t)(word >> 16);
    hi.y = (float)(int)(int8_t)(uint8_t)(word >> 24);
    return make_uint2(__builtin_bit_cast(uint32_t, __builtin_convertvector(lo * d, T2)),
                      __builtin_bit_cast(uint32_t, __builtin_convertvector(hi * d, T2)));
}

// A wave-uniform pointer in scalar registers (the value must be the same in every lane).
__device__ __forceinline__ const char* uniform_ptr(const char* ptr) {
    const uint64_t v = reinterpret_cast<uint64_t>(ptr);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return reinterpret_cast<const char*>(((uint64_t)hi << 32) | lo);
}

// Direct global -> LDS loads (16 or 4 bytes per lane): lane i's bytes from base + off land at LDS address lds + 16 i
// (4 i). Written as inline assembly so that the compiler, which cannot tell which LDS bytes such a load writes, does
// not wait for every one of them before each LDS access; the kernels' explicit vmcnt waits and barriers order them.
// base and lds are wave-uniform. The compiler does not see the vector-memory instruction inside the assembly, so
// the assembly supplies the wait states itself: five, enough for an M0 or SGPR operand written just before by a
// scalar or vector instruction (a vector write of an SGPR read by a vector-memory instruction needs five).
__device__ __forceinline__ void lds_dma16(const char* base, uint32_t off, uint32_t lds) {
    asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "{m0}"(lds) : "memory");
}
__device__ __forceinline__ void lds_dma4(const char* base, uint32_t off, uint32_t lds) {
    asm volatile("s_nop 4\n\tglobal_load_lds_dword %0, %1" ::"v"(off), "s"(base), "{m0}"(lds) : "memory");
}

// s_waitcnt on the vector-memory counter only (expcnt and lgkmcnt left at their maximum).
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// One output element through the whole epilogue, any dtype and activation (general paths run it in a loop that is
// not unrolled, so its code exists once).
__device__ __forceinline__ void epilogue_element(const GemmParams& p, int row, int col, float v) {
    if ((p.flags & IDOLQ_FLAG_ROUND_BEFORE_BIAS) != 0) v = round_through(p.y_dt, v);
    if (p.bias) v += load_as_float(p.bias, p.bias_dt, col);
    if (p.res) v += load_as_float(p.res, p.res_dt, (int64_t)row * p.ldr + col);
    store_from_float(p.y, p.y_dt, (int64_t)row * p.ldy + col, apply_act(p.act, v));
}

template <int ACT>
__device__ __forceinline__ float act_fast(float v) {
    if (ACT == IDOLQ_ACT_GELU_TANH) return apply_act(IDOLQ_ACT_GELU_TANH, v);
    if (ACT == IDOLQ_ACT_RELU) return v > 0.0f ? v : 0.0f;
    return v;
}

// Cached multiprocessor count of the current device.
int cu_count();

}  // namespace idolq
