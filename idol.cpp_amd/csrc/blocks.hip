// The other GGUF block formats of the packed-linear surface (tools/idol_packed.py:25-71, tools/idol_triton.py:48-82):
// expansion of Q4_0, Q8_0, Q2_K, Q4_K, Q6_K and F16 weights to a dense dtype, and the exact re-encoding of Q4_0
// blocks as Q8_0 blocks (same scale, codes q - 8), which lets Q4_0 layers run on the Q8_0 GEMMs unchanged.
//
// Block layouts (ggml; values per block / bytes per block):
//   Q4_0   32 / 18:  fp16 d | 16 bytes: element i < 16 is the low nibble of byte i, element 16 + i its high nibble;
//                    w = d * (q - 8)
//   Q8_0   32 / 34:  fp16 d | 32 int8 q;  w = d * q
//   Q2_K  256 / 84:  16 bytes of 4-bit (scale, min) pairs, low nibble scale | 64 bytes of 2-bit codes | fp16 d |
//                    fp16 dmin. Element e = 128 h + 32 s + l takes bits 2 s of byte 32 h + l; 16-element group
//                    g = e / 16 uses pair g;  w = (d * sc_g) * q - dmin * m_g
//   Q4_K  256 / 144: fp16 d | fp16 dmin | 12 bytes of 6-bit scales and mins | 128 bytes of 4-bit codes. Element
//                    e = 64 c + 32 t + l takes nibble t of byte 32 c + l; 32-element group j = e / 32:
//                    sc_j = a_j & 63, m_j = b_j & 63 for j < 4, with a = bytes 0..3, b = bytes 4..7, c = bytes 8..11
//                    of the 12; for j >= 4: sc_j = (c_{j-4} & 15) | ((a_{j-4} >> 6) << 4),
//                    m_j = (c_{j-4} >> 4) | ((b_{j-4} >> 6) << 4);  w = (d * sc_j) * q - dmin * m_j
//   Q6_K  256 / 210: 128 bytes of low nibbles | 64 bytes of high 2-bit pairs | 16 int8 scales | fp16 d. Element
//                    e = 128 h + 32 t + l: low nibble (t & 1 ? byte 32 + l : byte l of half h's 64, high nibble when
//                    t >= 2), high bits 2 t of byte l of half h's 32; 16-element group g = e / 16:
//                    w = (d * sc_g) * (q - 32)
// Each value is computed with the operations the reference's expansion uses (products and differences in fp32, no
// fused multiply-add), then rounded once to the output dtype.
#include "common.h"

namespace idolq {
namespace {

#pragma clang fp contract(off)

__device__ __forceinline__ float f16_at(const uint8_t* p) { return half_bits_to_float((uint16_t)(p[0] | (p[1] << 8))); }

// The 32 values of chunk c (elements 32 c .. 32 c + 31) of one row, into v.
template <int KIND>
__device__ __forceinline__ void decode32(const uint8_t* __restrict__ row, int64_t c, float (&v)[32]) {
    if (KIND == IDOLQ_KIND_Q8_0) {
        const uint8_t* b = row + c * 34;
        const float d = f16_at(b);
#pragma unroll
        for (int i = 0; i < 32; ++i) v[i] = d * (float)(int8_t)b[2 + i];
    } else if (KIND == IDOLQ_KIND_Q4_0) {
        const uint8_t* b = row + c * 18;
        const float d = f16_at(b);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            v[i] = d * (float)((int)(b[2 + i] & 15) - 8);
            v[16 + i] = d * (float)((int)(b[2 + i] >> 4) - 8);
        }
    } else if (KIND == IDOLQ_KIND_F16) {
        const uint8_t* b = row + c * 64;
#pragma unroll
        for (int i = 0; i < 32; ++i) v[i] = f16_at(b + 2 * i);
    } else if (KIND == IDOLQ_KIND_Q2_K) {
        const uint8_t* b = row + (c / 8) * 84;
        const int e0 = (int)(c % 8) * 32, h = e0 / 128, s = (e0 % 128) / 32;
        const float d = f16_at(b + 80), dmin = f16_at(b + 82);
#pragma unroll
        for (int half16 = 0; half16 < 2; ++half16) {
            const int g = e0 / 16 + half16;
            const float sd = d * (float)(b[g] & 15), sm = dmin * (float)(b[g] >> 4);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int l = 16 * half16 + i;
                const int q = (b[16 + 32 * h + l] >> (2 * s)) & 3;
                v[l] = sd * (float)q - sm;
            }
        }
    } else if (KIND == IDOLQ_KIND_Q4_K) {
        const uint8_t* b = row + (c / 8) * 144;
        const int j = (int)(c % 8);
        const float d = f16_at(b), dmin = f16_at(b + 2);
        const uint8_t* s = b + 4;
        int sc, mn;
        if (j < 4) {
            sc = s[j] & 63;
            mn = s[4 + j] & 63;
        } else {
            sc = (s[8 + j - 4] & 15) | ((s[j - 4] >> 6) << 4);
            mn = (s[8 + j - 4] >> 4) | ((s[4 + j - 4] >> 6) << 4);
        }
        const float sd = d * (float)sc, sm = dmin * (float)mn;
        const uint8_t* q = b + 16 + 32 * (j / 2);
        const int shift = 4 * (j % 2);
#pragma unroll
        for (int l = 0; l < 32; ++l) v[l] = sd * (float)((q[l] >> shift) & 15) - sm;
    } else {  // Q6_K
        const uint8_t* b = row + (c / 8) * 210;
        const int e0 = (int)(c % 8) * 32, h = e0 / 128, t = (e0 % 128) / 32;
        const uint8_t* ql = b + 64 * h + 32 * (t & 1);
        const uint8_t* qh = b + 128 + 32 * h;
        const int8_t* sc = reinterpret_cast<const int8_t*>(b + 192);
        const float d = f16_at(b + 208);
#pragma unroll
        for (int half16 = 0; half16 < 2; ++half16) {
            const float sd = d * (float)sc[e0 / 16 + half16];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int l = 16 * half16 + i;
                const int lo = t >= 2 ? ql[l] >> 4 : ql[l] & 15;
                const int q = lo | (((qh[l] >> (2 * t)) & 3) << 4);
                v[l] = sd * (float)(q - 32);
            }
        }
    }
}

// One thread per (row, 32-value chunk): decode, then four 8-value stores.
template <int KIND, int DT>
__global__ __launch_bounds__(256) void blocks_dequant_kernel(const uint8_t* __restrict__ w, int64_t n, int64_t k,
                                                             int64_t row_bytes, void* out) {
    const int64_t chunks = k / 32;
    const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= n * chunks) return;
    const int64_t r = id / chunks, c = id - r * chunks;
    float v[32];
    decode32<KIND>(w + r * row_bytes, c, v);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        float f[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = v[8 * q + e];
        store8<DT>(out, r * k + 32 * c + 8 * q, f);
    }
}

// Q4_0 block -> Q8_0 block: the same fp16 scale, codes q - 8 as int8 (exact). One thread per block.
__global__ __launch_bounds__(256) void q4_0_to_q8_0_kernel(const uint8_t* __restrict__ w, int64_t blocks,
                                                           uint8_t* __restrict__ out) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= blocks) return;
    const uint8_t* s = w + b * 18;
    uint8_t* o = out + b * 34;
    o[0] = s[0];
    o[1] = s[1];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        o[2 + i] = (uint8_t)(int8_t)((int)(s[2 + i] & 15) - 8);
        o[18 + i] = (uint8_t)(int8_t)((int)(s[2 + i] >> 4) - 8);
    }
}

int block_shape(int kind, int& values, int& bytes) {
    switch (kind) {
        case IDOLQ_KIND_F16: values = 32, bytes = 64; return 0;  // handled as 32-value chunks
        case IDOLQ_KIND_Q4_0: values = 32, bytes = 18; return 0;
        case IDOLQ_KIND_Q8_0: values = 32, bytes = 34; return 0;
        case IDOLQ_KIND_Q2_K: values = 256, bytes = 84; return 0;
        case IDOLQ_KIND_Q4_K: values = 256, bytes = 144; return 0;
        case IDOLQ_KIND_Q6_K: values = 256, bytes = 210; return 0;
        default: return -1;
    }
}

template <int KIND>
int launch_dequant(const uint8_t* w, int64_t n, int64_t k, int64_t row_bytes, void* out, int dt, hipStream_t s) {
    const int64_t items = n * (k / 32);
    const dim3 grid((unsigned)((items + 255) / 256));
    if (dt == IDOLQ_F32) hipLaunchKernelGGL((blocks_dequant_kernel<KIND, IDOLQ_F32>), grid, dim3(256), 0, s, w, n, k, row_bytes, out);
    else if (dt == IDOLQ_BF16) hipLaunchKernelGGL((blocks_dequant_kernel<KIND, IDOLQ_BF16>), grid, dim3(256), 0, s, w, n, k, row_bytes, out);
    else hipLaunchKernelGGL((blocks_dequant_kernel<KIND, IDOLQ_F16>), grid, dim3(256), 0, s, w, n, k, row_bytes, out);
    return check_launch("blocks_dequant_kernel");
}

}  // namespace
}  // namespace idolq

using namespace idolq;

extern "C" int64_t idolq_blocks_bytes(int kind, int64_t n, int64_t k) {
    int values, bytes;
    if (block_shape(kind, values, bytes) != 0 || n < 0 || k <= 0 || k % values != 0) return 0;
    if (kind == IDOLQ_KIND_F16) return n * k * 2;
    return n * (k / values) * bytes;
}

extern "C" int idolq_blocks_dequant(const uint8_t* w, int kind, int64_t n, int64_t k, void* out, int out_dtype,
                                    void* stream) {
    int values, bytes;
    if (block_shape(kind, values, bytes) != 0) return fail(IDOLQ_EINVAL, "unsupported block format");
    if (!dtype_ok(out_dtype)) return fail(IDOLQ_EINVAL, "unknown dtype code");
    if (n < 0 || k <= 0 || k % values != 0)
        return fail(IDOLQ_EINVAL, "k must be a positive multiple of the block's value count");
    if (n == 0) return IDOLQ_OK;
    if (!w || !out) return fail(IDOLQ_EINVAL, "w and out must be non-null");
    if (reinterpret_cast<uintptr_t>(out) % 16 != 0) return fail(IDOLQ_EINVAL, "out must be 16-byte aligned");
    if (n * (k / 32) > (int64_t)0xffffffffLL * 256 / 2) return fail(IDOLQ_EINVAL, "matrix too large");
    const int64_t row_bytes = kind == IDOLQ_KIND_F16 ? k * 2 : (k / values) * bytes;
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (kind) {
        case IDOLQ_KIND_F16: return launch_dequant<IDOLQ_KIND_F16>(w, n, k, row_bytes, out, out_dtype, s);
        case IDOLQ_KIND_Q4_0: return launch_dequant<IDOLQ_KIND_Q4_0>(w, n, k, row_bytes, out, out_dtype, s);
        case IDOLQ_KIND_Q8_0: return launch_dequant<IDOLQ_KIND_Q8_0>(w, n, k, row_bytes, out, out_dtype, s);
        case IDOLQ_KIND_Q2_K: return launch_dequant<IDOLQ_KIND_Q2_K>(w, n, k, row_bytes, out, out_dtype, s);
        case IDOLQ_KIND_Q4_K: return launch_dequant<IDOLQ_KIND_Q4_K>(w, n, k, row_bytes, out, out_dtype, s);
        default: return launch_dequant<IDOLQ_KIND_Q6_K>(w, n, k, row_bytes, out, out_dtype, s);
    }
}

extern "C" int idolq_q4_0_to_q8_0(const uint8_t* w, int64_t n, int64_t k, uint8_t* out, void* stream) {
    if (n < 0 || k <= 0 || k % 32 != 0) return fail(IDOLQ_EINVAL, "k must be a positive multiple of 32");
    if (n == 0) return IDOLQ_OK;
    if (!w || !out) return fail(IDOLQ_EINVAL, "w and out must be non-null");
    const int64_t blocks = n * (k / 32);
    hipLaunchKernelGGL(q4_0_to_q8_0_kernel, dim3((unsigned)((blocks + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), w, blocks, out);
    return check_launch("q4_0_to_q8_0_kernel");
}
