// The reference's native quantized panels (src/kernels.hpp:33-51) on the device: validation and size
// (src/kernels.cpp:512-533), lossless conversion of symmetric panels to GGUF Q8_0 blocks for the Q8_0 GEMM, and the
// expansion of any panel to the fp32 values of the reference's dequantizer (src/kernels.cpp:167-209,535-550).
//
// Panel layout. Output rows in panels of 16 columns (the last padded); per panel, per group of `group` k values:
// 16 fp16 scales, 16 fp16 minimums (64 bytes), then for every 8 k values `bits` byte rows of 16 bytes (one byte per
// column) holding bit planes, low bits first: widths {2}, {2,1}, {4}, {4,1}, {4,2}, {8} for bits 2, 3, 4, 5, 6, 8. A
// plane of width w occupies w byte rows; k value r of the 8 sits in byte row r / (8 / w) at bit w * (r % (8 / w)).
// The value is fma(code, scale, min) in fp32.
//
// One thread per (output row, 8 k values).
#include "common.h"

namespace idolq {
namespace {

constexpr int kCols = 16;
constexpr int kHeader = 64;

bool bits_ok(int bits) { return bits == 2 || bits == 3 || bits == 4 || bits == 5 || bits == 6 || bits == 8; }

int64_t group_bytes(int bits, int group) { return kHeader + 2 * (int64_t)group * bits; }

struct PanelArgs {
    const uint8_t* blob;
    int64_t out, in;
    int bits, group;
    int64_t gbytes;  // bytes per (panel, group)
};

// The 8 codes of k values 8 j .. 8 j + 7 of row n (within their group), and the row's scale and minimum.
template <int W0, int W1>
__device__ __forceinline__ void decode8(const PanelArgs& a, int64_t n, int64_t kc, uint32_t codes[8], float& s,
                                        float& m, uint16_t& s_bits) {
    const int64_t panel = n / kCols, c = n % kCols;
    const int64_t k0 = 8 * kc, g = k0 / a.group, j = (k0 % a.group) / 8;
    const uint8_t* base = a.blob + (panel * (a.in / a.group) + g) * a.gbytes;
    s_bits = (uint16_t)(base[2 * c] | (base[2 * c + 1] << 8));
    const uint16_t m_bits = (uint16_t)(base[32 + 2 * c] | (base[33 + 2 * c] << 8));
    s = half_bits_to_float(s_bits);
    m = half_bits_to_float(m_bits);
    const uint8_t* body = base + kHeader + j * 16 * (W0 + W1) + c;
    constexpr int R0 = 8 / W0;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        uint32_t v = (body[16 * (r / R0)] >> (W0 * (r % R0))) & ((1u << W0) - 1);
        if constexpr (W1 > 0) {
            constexpr int R1 = 8 / W1;
            v |= ((body[16 * (W0 + r / R1)] >> (W1 * (r % R1))) & ((1u << W1) - 1)) << W0;
        }
        codes[r] = v;
    }
}

template <int W0, int W1>
__global__ void panel_expand_kernel(PanelArgs a, float* w, int64_t ldw) {
    const int64_t chunks = a.in / 8, total = a.out * chunks;
    for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t n = t / chunks, kc = t % chunks;
        uint32_t codes[8];
        float s, m;
        uint16_t sb;
        decode8<W0, W1>(a, n, kc, codes, s, m, sb);
        float* dst = w + n * ldw + 8 * kc;
#pragma unroll
        for (int r = 0; r < 8; ++r) dst[r] = fmaf((float)codes[r], s, m);
    }
}

// Q8_0 row n: k / 32 blocks of 34 bytes (fp16 d, then 32 int8 q); q = code - 2^(bits - 1), d = the group's scale.
// The first chunk of every (row, group) counts the group in *inexact when its minimum is not -2^(bits-1) * scale.
template <int W0, int W1>
__global__ void panel_to_q8_kernel(PanelArgs a, uint8_t* q8, int32_t* inexact) {
    const int64_t chunks = a.in / 8, total = a.out * chunks, nb = a.in / 32;
    const int half = 1 << (a.bits - 1);
    for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t n = t / chunks, kc = t % chunks;
        uint32_t codes[8];
        float s, m;
        uint16_t sb;
        decode8<W0, W1>(a, n, kc, codes, s, m, sb);
        if ((8 * kc) % a.group == 0 && !(m == -(float)half * s)) atomicAdd(inexact, 1);
        uint8_t* blk = q8 + (n * nb + kc / 4) * 34;
        uint16_t* dst = reinterpret_cast<uint16_t*>(blk + 2 + 8 * (kc % 4));  // blocks are 2-byte aligned
#pragma unroll
        for (int r = 0; r < 8; r += 2) {
            const uint32_t lo = (uint8_t)(int8_t)((int)codes[r] - half), hi = (uint8_t)(int8_t)((int)codes[r + 1] - half);
            dst[r / 2] = (uint16_t)(lo | (hi << 8));
        }
        if (kc % 4 == 0) *reinterpret_cast<uint16_t*>(blk) = sb;
    }
}

int check_panel(const uint8_t* blob, int64_t blob_bytes, int64_t out, int64_t in, int bits, int group) {
    if (!bits_ok(bits)) return fail(IDOLQ_EINVAL, "quantized layers use 2, 3, 4, 5, 6 or 8 bits");
    if (group <= 0 || group % 32 != 0 || in <= 0 || in % group != 0)
        return fail(IDOLQ_EINVAL, "the quantization group must be a multiple of 32 that divides the input size");
    if (out < 0) return fail(IDOLQ_EINVAL, "negative output size");
    if (blob_bytes != (out + kCols - 1) / kCols * (in / group) * group_bytes(bits, group))
        return fail(IDOLQ_EINVAL, "a quantized blob has the wrong size for its shape");
    if (out > 0 && !blob) return fail(IDOLQ_EINVAL, "blob must be non-null");
    return IDOLQ_OK;
}

dim3 grid_for(int64_t total) {
    const int64_t blocks = (total + 255) / 256;
    return dim3((unsigned)(blocks < 65536 ? (blocks > 0 ? blocks : 1) : 65536));
}

#define IDOLQ_PANEL_DISPATCH(KERNEL, ...)                                                                       \
    switch (a.bits) {                                                                                           \
        case 2: hipLaunchKernelGGL((KERNEL<2, 0>), grid, dim3(256), 0, s, __VA_ARGS__); break;                  \
        case 3: hipLaunchKernelGGL((KERNEL<2, 1>), grid, dim3(256), 0, s, __VA_ARGS__); break;                  \
        case 4: hipLaunchKernelGGL((KERNEL<4, 0>), grid, dim3(256), 0, s, __VA_ARGS__); break;                  \
        case 5: hipLaunchKernelGGL((KERNEL<4, 1>), grid, dim3(256), 0, s, __VA_ARGS__); break;                  \
        case 6: hipLaunchKernelGGL((KERNEL<4, 2>), grid, dim3(256), 0, s, __VA_ARGS__); break;                  \
        default: hipLaunchKernelGGL((KERNEL<8, 0>), grid, dim3(256), 0, s, __VA_ARGS__); break;                 \
    }

}  // namespace
}  // namespace idolq

using namespace idolq;

extern "C" int64_t idolq_panel_bytes(int64_t out, int64_t in, int bits, int group) {
    if (!bits_ok(bits) || group <= 0 || group % 32 != 0 || in <= 0 || in % group != 0 || out < 0) return 0;
    return (out + kCols - 1) / kCols * (in / group) * group_bytes(bits, group);
}

extern "C" int idolq_panel_expand_f32(const uint8_t* blob, int64_t blob_bytes, int64_t out, int64_t in, int bits,
                                      int group, float* w, int64_t ldw, void* stream) {
    int rc = check_panel(blob, blob_bytes, out, in, bits, group);
    if (rc) return rc;
    if (ldw < in) return fail(IDOLQ_EINVAL, "row stride smaller than the row");
    if (out == 0) return IDOLQ_OK;
    if (!w) return fail(IDOLQ_EINVAL, "w must be non-null");
    const PanelArgs a{blob, out, in, bits, group, group_bytes(bits, group)};
    const dim3 grid = grid_for(out * (in / 8));
    hipStream_t s = static_cast<hipStream_t>(stream);
    IDOLQ_PANEL_DISPATCH(panel_expand_kernel, a, w, ldw)
    return check_launch("panel_expand_kernel");
}

extern "C" int idolq_panel_to_q8_0(const uint8_t* blob, int64_t blob_bytes, int64_t out, int64_t in, int bits,
                                   int group, uint8_t* q8, int32_t* inexact, void* stream) {
    int rc = check_panel(blob, blob_bytes, out, in, bits, group);
    if (rc) return rc;
    if (out == 0) return IDOLQ_OK;
    if (!q8 || !inexact) return fail(IDOLQ_EINVAL, "q8 and inexact must be non-null");
    if ((reinterpret_cast<uintptr_t>(q8) & 1) != 0) return fail(IDOLQ_EINVAL, "q8 must be 2-byte aligned");
    if ((reinterpret_cast<uintptr_t>(inexact) & 3) != 0) return fail(IDOLQ_EINVAL, "inexact must be 4-byte aligned");
    const PanelArgs a{blob, out, in, bits, group, group_bytes(bits, group)};
    const dim3 grid = grid_for(out * (in / 8));
    hipStream_t s = static_cast<hipStream_t>(stream);
    IDOLQ_PANEL_DISPATCH(panel_to_q8_kernel, a, q8, inexact)
    return check_launch("panel_to_q8_kernel");
}
