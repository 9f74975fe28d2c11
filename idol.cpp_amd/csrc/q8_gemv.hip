// Small-m Q8_0 GEMM (the GEMV form) for gfx950: y = epilogue(x * W^T) for m <= 16 rows of activations on GGUF
// row-major Q8_0 weights, the shape of the decoders' single-row level-embedding MLP (src/decoders.cpp:260-264) and of
// one-token serving through the packed-linear surface. At m <= 16 the weight bytes are the whole cost (1.0625 bytes
// per weight against 2 m FLOP), so the kernel is built to keep the weight loads in flight and to touch each code once:
//
//   workgroup = 16 weight rows, 8 waves; wave w takes a contiguous run of the rows' quads (256 k: eight Q8_0 blocks,
//   272 bytes per row, 16-byte aligned when k % 256 == 0), loads each quad with coalesced 16-byte loads (consecutive
//   lanes, consecutive bytes of a row) into its own LDS stage, together with the quad's activations, while the
//   previous quad is multiplied;
//   v_mfma_f32_16x16x32 computes C = X W^T for one 32-deep block: the A rows are the m <= 16 activation rows (the
//   last row repeated up to 16), the B columns the 16 weight rows; lane l dequantizes codes 8 (l / 16) .. + 7 of
//   weight row l % 16 (block 0 of a pair starts two bytes before its codes' dword boundary and is realigned with
//   alignbyte), and its 4 accumulators all belong to that weight row, so the lane's own block scale applies to them;
//   the 8 waves' partial tiles are added through LDS in wave order (a fixed order: results are deterministic), then
//   bias, residual and the activation as in every mode.
//
// Arithmetic per mode, as the tiled GEMM kernels: DEQUANT multiplies T(fp32(d) * q) by the 16-bit activations with
// fp32 accumulation over the whole depth; EXACT feeds the codes exactly (fp32 activations split into bf16 high and
// low parts), sums each 32-deep block in fp32 and adds d times that sum to the accumulator.
#include "q8_gemm.h"

#include <type_traits>

namespace idolq {

namespace {

constexpr int kGemvWaves = 8;
constexpr int kGemvThreads = 64 * kGemvWaves;
constexpr int kGemvRows = 16;

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// v_mfma_f32_16x16x32: A [16 x 32] (lane l: row l % 16, k = 8 (l / 16) .. + 7), B [32 x 16] (lane l: column l % 16,
// the same k), D [16 x 16] (lane l: column l % 16, rows 4 (l / 16) .. + 3).
template <typename T>
struct GemvMfma;
template <>
struct GemvMfma<__bf16> {
    typedef bf16x8 vec;
    typedef bf16x2 pair;
    static __device__ __forceinline__ f32x4 run(uint4 a, uint4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(vec, a), __builtin_bit_cast(vec, b), c, 0, 0, 0);
    }
};
template <>
struct GemvMfma<_Float16> {
    typedef f16x8 vec;
    typedef f16x2 pair;
    static __device__ __forceinline__ f32x4 run(uint4 a, uint4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(vec, a), __builtin_bit_cast(vec, b), c, 0, 0, 0);
    }
};

// Eight int8 codes (two dwords) to a 16-bit weight operand: the codes themselves (exact in bf16 and fp16) or T(d * q).
template <typename T, bool DEQ>
__device__ __forceinline__ uint4 operand_of(uint32_t lo, uint32_t hi, float d) {
    typedef typename GemvMfma<T>::pair T2;
    uint32_t out[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const uint32_t word = e < 2 ? lo : hi;
        const int sh = 16 * (e & 1);
        f32x2 f = {(float)(int)(int8_t)(uint8_t)(word >> sh), (float)(int)(int8_t)(uint8_t)(word >> (sh + 8))};
        if (DEQ) f = f * d;
        out[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f, T2));
    }
    return make_uint4(out[0], out[1], out[2], out[3]);
}

// Eight fp32 activations to the bf16 high part (and the bf16 low part x - high).
__device__ __forceinline__ void split_f32(const float4& a, const float4& b, uint4& hi, uint4& lo) {
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    uint32_t h[4], l[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const f32x2 f = {v[2 * e], v[2 * e + 1]};
        const bf16x2 fh = __builtin_convertvector(f, bf16x2);
        const f32x2 r = f - __builtin_convertvector(fh, f32x2);
        h[e] = __builtin_bit_cast(uint32_t, fh);
        l[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector(r, bf16x2));
    }
    hi = make_uint4(h[0], h[1], h[2], h[3]);
    lo = make_uint4(l[0], l[1], l[2], l[3]);
}

// XT: activation type; T: the MFMA operand type (bf16 for fp32 activations); DEQ: DEQUANT (else EXACT).
template <int XT, bool DEQ>
__global__ __launch_bounds__(kGemvThreads) void q8_gemv_kernel(GemmParams p) {
    typedef typename std::conditional<XT == XT_F16, _Float16, __bf16>::type T;
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    constexpr int R = kGemvRows;
    constexpr int kChunks = R * 17;              // 16-byte chunks of one quad (4 pairs, 272 bytes) of R rows
    constexpr int kPer = (kChunks + 63) / 64;    // chunk loads per lane
    constexpr int kXv = XT == XT_F32 ? 2 : 1;    // 16-byte activation loads per lane and block
    __shared__ __attribute__((aligned(16))) uint32_t stage[kGemvWaves][R * 68];
    __shared__ float red[kGemvWaves][R][R + 1];

    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c16 = lane & 15, g4 = lane >> 4;  // MFMA column (weight row) / A row, and k group of 8
    const int n0 = blockIdx.x * R;
    const int quads = p.k / 256;
    const int per = quads / kGemvWaves, extra = quads % kGemvWaves;
    const int g_begin = wave * per + min(wave, extra), g_end = g_begin + per + (wave < extra ? 1 : 0);

    // chunk i of this lane: c = lane + 64 i, row c / 17 (rows past n read the last row; their outputs are never
    // stored), 16-byte piece c % 17 of the row's quad; its LDS place is the same (row, piece) of the wave's stage.
    // Every lane loads all kPer pieces (addresses past the quad are clamped to its last piece); the quad buffers are
    // native vectors, so they stay in registers.
    const char* wbase = reinterpret_cast<const char*>(p.w);
    uint32_t goff[kPer], loff[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int c = min(lane + 64 * i, kChunks - 1), row = c / 17, part = c - row * 17;
        goff[i] = (uint32_t)((int64_t)min(n0 + row, p.n - 1) * p.row_bytes + part * 16);
        loff[i] = (uint32_t)(row * 68 + part * 4);
    }
    const char* xrow = static_cast<const char*>(p.x) + (int64_t)min(c16, p.m - 1) * p.ldx * (XT == XT_F32 ? 4 : 2);
    // weights and activations of quad g: block b = 2 u + v of the quad takes k = 256 g + 32 b + 8 g4 .. + 7
    struct Buf {
        u32x4 w[kPer];
        u32x4 x[8][kXv];
    };
    auto load_quad = [&](int g, Buf& buf) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < kPer; ++i) buf.w[i] = *reinterpret_cast<const u32x4*>(wbase + goff[i] + (size_t)g * 272);
#pragma unroll
        for (int b = 0; b < 8; ++b)
#pragma unroll
            for (int v = 0; v < kXv; ++v)
                buf.x[b][v] = *reinterpret_cast<const u32x4*>(
                    xrow + ((int64_t)(256 * g + 32 * b + 8 * g4) * (kXv == 2 ? 4 : 2) + 16 * v));
    };
    uint32_t* const st = stage[wave];
    const uint32_t* const frag = st + c16 * 68;

    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};

    auto quad = [&](const Buf& buf) __attribute__((always_inline)) {
        // the wave's LDS operations run in order: the previous quad's reads are done before these writes
#pragma unroll
        for (int i = 0; i < kPer; ++i)
            if (kChunks % 64 == 0 || i + 1 < kPer || lane + 64 * i < kChunks)
                *reinterpret_cast<u32x4*>(st + loff[i]) = buf.w[i];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            // pair u of row c16: block 0's scale in dword 0 (low half), its codes 2 + 8 g4 .. 9 + 8 g4 in dwords
            // 2 g4 .. 2 g4 + 2; block 1's scale in dword 8 (high half), its codes 36 + 8 g4 .. in dwords 9 + 2 g4, 10 + 2 g4
            const uint32_t* pw = frag + 17 * u;
            const uint32_t d0 = pw[0], d8 = pw[8];
            const uint32_t a0 = pw[2 * g4], a1 = pw[2 * g4 + 1], a2 = pw[2 * g4 + 2];
            const uint32_t b0 = pw[9 + 2 * g4], b1 = pw[10 + 2 * g4];
            const float s[2] = {half_bits_to_float((uint16_t)(d0 & 0xffff)), half_bits_to_float((uint16_t)(d8 >> 16))};
            const uint32_t c[2][2] = {{__builtin_amdgcn_alignbyte(a1, a0, 2), __builtin_amdgcn_alignbyte(a2, a1, 2)},
                                      {b0, b1}};
#pragma unroll
            for (int v = 0; v < 2; ++v) {
                const u32x4 xa = buf.x[2 * u + v][0];
                if constexpr (DEQ) {
                    acc = GemvMfma<T>::run(make_uint4(xa.x, xa.y, xa.z, xa.w), operand_of<T, true>(c[v][0], c[v][1], s[v]), acc);
                } else {
                    const uint4 wq = operand_of<T, false>(c[v][0], c[v][1], 0.0f);
                    f32x4 blk = {0.0f, 0.0f, 0.0f, 0.0f};
                    if constexpr (XT == XT_F32) {
                        const u32x4 xb = buf.x[2 * u + v][kXv - 1];
                        uint4 hi, lo;
                        split_f32(__builtin_bit_cast(float4, xa), __builtin_bit_cast(float4, xb), hi, lo);
                        blk = GemvMfma<T>::run(hi, wq, blk);
                        blk = GemvMfma<T>::run(lo, wq, blk);
                    } else {
                        blk = GemvMfma<T>::run(make_uint4(xa.x, xa.y, xa.z, xa.w), wq, blk);
                    }
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[e] = fmaf(s[v], blk[e], acc[e]);
                }
            }
        }
        // the stage is rewritten by the next quad only after this quad's reads
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };

    // two register buffers: the next quad's weights and activations fly while the current one is multiplied
    Buf bufA, bufB;
    if (g_begin < g_end) load_quad(g_begin, bufA);
    for (int g = g_begin; g < g_end; g += 2) {
        if (g + 1 < g_end) load_quad(g + 1, bufB);
        quad(bufA);
        if (g + 1 >= g_end) break;
        if (g + 2 < g_end) load_quad(g + 2, bufA);
        quad(bufB);
    }

    // ---- the waves' partial tiles, added in wave order; element e of lane l is activation row 4 (l / 16) + e,
    // weight row l % 16
#pragma unroll
    for (int e = 0; e < 4; ++e) red[wave][c16][4 * g4 + e] = acc[e];
    __syncthreads();
    const bool round_first = (p.flags & IDOLQ_FLAG_ROUND_BEFORE_BIAS) != 0;
    for (int o = threadIdx.x; o < R * R; o += kGemvThreads) {
        const int row = o / R, m = o % R;  // weight row (output column), activation row
        const int col = n0 + row;
        if (m >= p.m || col >= p.n) continue;
        float v = red[0][row][m];
#pragma unroll
        for (int w = 1; w < kGemvWaves; ++w) v += red[w][row][m];
        if (round_first) v = round_through(p.y_dt, v);
        if (p.bias) v += load_as_float(p.bias, p.bias_dt, col);
        if (p.res) v += load_as_float(p.res, p.res_dt, (int64_t)m * p.ldr + col);
        store_from_float(p.y, p.y_dt, (int64_t)m * p.ldy + col, apply_act(p.act, v));
    }
}

}  // namespace

bool gemv_eligible(const GemmParams& p, int xt, int mode) {
    return p.m >= 1 && p.m <= kGemvMaxRows && !p.w_tiled && p.k % 256 == 0 &&
           (reinterpret_cast<uintptr_t>(p.w) & 15) == 0 && p.x_aligned &&
           ((mode == MODE_DEQUANT && xt != XT_F32) || mode == MODE_EXACT);
}

int launch_gemv(GemmParams p, int xt, int mode, hipStream_t stream) {
    const dim3 grid((p.n + kGemvRows - 1) / kGemvRows), block(kGemvThreads);
    if (mode == MODE_DEQUANT) {
        if (xt == XT_BF16)
            hipLaunchKernelGGL((q8_gemv_kernel<XT_BF16, true>), grid, block, 0, stream, p);
        else
            hipLaunchKernelGGL((q8_gemv_kernel<XT_F16, true>), grid, block, 0, stream, p);
    } else {
        if (xt == XT_BF16)
            hipLaunchKernelGGL((q8_gemv_kernel<XT_BF16, false>), grid, block, 0, stream, p);
        else if (xt == XT_F16)
            hipLaunchKernelGGL((q8_gemv_kernel<XT_F16, false>), grid, block, 0, stream, p);
        else
            hipLaunchKernelGGL((q8_gemv_kernel<XT_F32, false>), grid, block, 0, stream, p);
    }
    return check_launch("q8_gemv_kernel");
}

}  // namespace idolq
