// Q8_0 GEMM for gfx950: y = epilogue(x * W^T) with W kept as raw GGUF Q8_0 blocks.
//
// Workgroup: 256 threads = 4 waves in a 2 x 2 grid, each wave owning a (BM/2) x (BN/2) tile of 32 x 32 MFMA tiles.
// Each stage covers 64 of k (two Q8_0 blocks):
//   1. global -> registers: the activation tile with 16-byte loads, and the weight tile as a flat run of dwords
//      (or halfwords when a row of blocks is not 4-byte aligned), consecutive lanes reading consecutive bytes of a
//      row, so each row's 68 bytes are fetched as one coalesced span;
//   2. registers -> LDS: activations as 16-bit MFMA operands (fp32 split into bf16 high + low parts), and the weight
//      bytes de-interleaved into a code array (byte-aligned rows of 64 codes) and an fp32 scale array;
//   3. MFMA over the two blocks. The next stage's global loads are in flight meanwhile.
// Arithmetic (see idolq.h): DEQUANT converts codes to T(fp32(d) * q) and chains the MFMA accumulators over k;
// EXACT feeds the codes exactly and folds each block's fp32 sum with its d; INT8 multiplies int8 activations by the
// codes with v_mfma_i32_32x32x32_i8 and folds s_a * d per block.
//
// MFMA operand layout (32 x 32 tiles): lane l supplies row (or column) l % 32 and the 8 (bf16/fp16, 16-deep
// instruction) or 16 (int8, 32-deep) consecutive k starting at (l / 32) * 8 (resp. 16); accumulator element r of
// lane l is row 8 * (r / 4) + 4 * (l / 32) + r % 4, column l % 32.
#include "common.h"

#include <type_traits>

namespace idolq {
namespace {

constexpr int kThreads = 256;
constexpr int kKStep = 64;                // depth per stage: two Q8_0 blocks
constexpr int kAPitch = kKStep + 8;       // 16-bit elements per activation row in LDS (144 bytes)
constexpr int kCodePitch = kKStep + 8;    // bytes per weight row of codes in LDS for 8-byte reads (72)
constexpr int kCodePitch8 = kKStep + 16;  // bytes per row of int8 operands for 16-byte reads (80)

enum { XT_BF16 = 0, XT_F16 = 1, XT_F32 = 2 };
enum { MODE_DEQUANT = 1, MODE_EXACT = 2 };

struct GemmParams {
    const void* x;
    int64_t ldx;
    const uint8_t* w;  // row 0 of the column window
    int64_t row_bytes;
    int m, n, k;
    const void* bias;  // entry 0 of the column window
    int bias_dt;
    const void* res;
    int res_dt;
    int64_t ldr;
    void* y;
    int y_dt;
    int64_t ldy;
    int act, flags;
    int tiles_m, tiles_n;
    int x_aligned;  // x rows are 16-byte aligned
    // INT8 mode
    const int8_t* qa;
    const float* sa;
    int32_t* dots;
};

// ------------------------------------------------------------------------------------------------ tile order
// Workgroup b runs on XCD b % 8. Consecutive logical tiles are given to the same XCD, and logical tiles walk
// groups of 8 row-tiles column by column, so workgroups resident together on one XCD share weight rows and
// activation rows in that XCD's L2.
__device__ __forceinline__ void tile_coords(int tiles_m, int tiles_n, int& tm, int& tn) {
    const int total = tiles_m * tiles_n;
    int b = blockIdx.x;
    if (total % 8 == 0) b = (b % 8) * (total / 8) + b / 8;
    constexpr int G = 8;
    const int per_group = G * tiles_n;
    const int group = b / per_group;
    const int first = group * G;
    const int gm = min(tiles_m - first, G);
    const int in_group = b - group * per_group;
    tm = first + in_group % gm;
    tn = in_group / gm;
}

// ------------------------------------------------------------------------------------------------ weight staging
// Flat loader for the 68 bytes (two blocks) of each of BN weight rows per stage.
template <int BN, bool W4>
struct WeightStage {
    static constexpr int kUnits = W4 ? BN * 17 : BN * 34;  // dwords or halfwords
    static constexpr int kPer = (kUnits + kThreads - 1) / kThreads;
    uint32_t v[kPer];

    __device__ __forceinline__ void load(const GemmParams& p, int n0, int blk0, int nblocks) {
        const int tid = threadIdx.x;
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int u = tid + i * kThreads;
            v[i] = 0;
            if (u < kUnits) {
                const int row = W4 ? u / 17 : u / 34;
                const int part = W4 ? u - row * 17 : u - row * 34;
                const bool second = W4 ? part >= 9 : part >= 17;  // unit touches the second block only
                if (n0 + row < p.n && (!second || blk0 + 1 < nblocks)) {
                    const uint8_t* src = p.w + (int64_t)(n0 + row) * p.row_bytes + (int64_t)blk0 * kQ8Bytes;
                    if (W4)
                        v[i] = reinterpret_cast<const uint32_t*>(src)[part];
                    else
                        v[i] = reinterpret_cast<const uint16_t*>(src)[part];
                }
            }
        }
    }

    // De-interleave into codes [BN][pitch] (int8) and scales [BN][2] (fp32).
    template <int PITCH>
    __device__ __forceinline__ void store(uint8_t* codes, float* scales) const {
        const int tid = threadIdx.x;
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int u = tid + i * kThreads;
            if (u >= kUnits) continue;
            const uint32_t x = v[i];
            if (W4) {
                const int row = u / 17, part = u - row * 17;
                uint8_t* c = codes + row * PITCH;
                if (part == 0) {
                    scales[row * 2] = half_bits_to_float((uint16_t)(x & 0xffff));
                    *reinterpret_cast<uint16_t*>(c) = (uint16_t)(x >> 16);
                } else if (part < 8) {
                    *reinterpret_cast<uint16_t*>(c + 4 * part - 2) = (uint16_t)(x & 0xffff);
                    *reinterpret_cast<uint16_t*>(c + 4 * part) = (uint16_t)(x >> 16);
                } else if (part == 8) {
                    *reinterpret_cast<uint16_t*>(c + 30) = (uint16_t)(x & 0xffff);
                    scales[row * 2 + 1] = half_bits_to_float((uint16_t)(x >> 16));
                } else {
                    *reinterpret_cast<uint32_t*>(c + 4 * part - 4) = x;
                }
            } else {
                const int row = u / 34, part = u - row * 34;
                uint8_t* c = codes + row * PITCH;
                const uint16_t h = (uint16_t)x;
                if (part == 0)
                    scales[row * 2] = half_bits_to_float(h);
                else if (part < 17)
                    *reinterpret_cast<uint16_t*>(c + 2 * part - 2) = h;
                else if (part == 17)
                    scales[row * 2 + 1] = half_bits_to_float(h);
                else
                    *reinterpret_cast<uint16_t*>(c + 2 * part - 4) = h;
            }
        }
    }
};

// ------------------------------------------------------------------------------------------------ activation staging
// BM rows x 64 k of x per stage, 16 bytes per unit.
template <int BM, int XT>
struct ActStage {
    static constexpr int kEsz = XT == XT_F32 ? 4 : 2;
    static constexpr int kUnitsPerRow = kKStep * kEsz / 16;  // 8 (16-bit) or 16 (fp32)
    static constexpr int kUnits = BM * kUnitsPerRow;
    static constexpr int kPer = kUnits / kThreads;
    static_assert(kUnits % kThreads == 0, "tile size");
    uint4 v[kPer];

    __device__ __forceinline__ void load(const GemmParams& p, int m0, int k0) {
        const int tid = threadIdx.x;
        constexpr int kElems = 16 / kEsz;
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int u = tid + i * kThreads;
            const int row = u / kUnitsPerRow, cu = u - row * kUnitsPerRow;
            const int kk = k0 + cu * kElems;
            v[i] = make_uint4(0, 0, 0, 0);
            if (m0 + row < p.m && kk < p.k) {
                const char* src = static_cast<const char*>(p.x) + ((int64_t)(m0 + row) * p.ldx + kk) * kEsz;
                if (p.x_aligned) {
                    v[i] = *reinterpret_cast<const uint4*>(src);
                } else {
                    uint32_t t[4];
                    if (kEsz == 4) {
#pragma unroll
                        for (int e = 0; e < 4; ++e) t[e] = reinterpret_cast<const uint32_t*>(src)[e];
                    } else {
                        const uint16_t* s16 = reinterpret_cast<const uint16_t*>(src);
#pragma unroll
                        for (int e = 0; e < 4; ++e) t[e] = (uint32_t)s16[2 * e] | ((uint32_t)s16[2 * e + 1] << 16);
                    }
                    v[i] = make_uint4(t[0], t[1], t[2], t[3]);
                }
            }
        }
    }

    // hi (and, for fp32 input, lo) tiles [BM][kAPitch] of 16-bit MFMA operands.
    __device__ __forceinline__ void store(uint16_t* hi, uint16_t* lo) const {
        const int tid = threadIdx.x;
        constexpr int kElems = 16 / kEsz;
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int u = tid + i * kThreads;
            const int row = u / kUnitsPerRow, cu = u - row * kUnitsPerRow;
            const int off = row * kAPitch + cu * kElems;
            if (XT != XT_F32) {
                *reinterpret_cast<uint4*>(hi + off) = v[i];
            } else {
                const float f[4] = {__builtin_bit_cast(float, v[i].x), __builtin_bit_cast(float, v[i].y),
                                    __builtin_bit_cast(float, v[i].z), __builtin_bit_cast(float, v[i].w)};
                uint32_t h[2], l[2];
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const uint16_t h0 = float_to_bf16_bits(f[2 * e]), h1 = float_to_bf16_bits(f[2 * e + 1]);
                    const uint16_t l0 = float_to_bf16_bits(f[2 * e] - bf16_bits_to_float(h0));
                    const uint16_t l1 = float_to_bf16_bits(f[2 * e + 1] - bf16_bits_to_float(h1));
                    h[e] = (uint32_t)h0 | ((uint32_t)h1 << 16);
                    l[e] = (uint32_t)l0 | ((uint32_t)l1 << 16);
                }
                *reinterpret_cast<uint2*>(hi + off) = make_uint2(h[0], h[1]);
                *reinterpret_cast<uint2*>(lo + off) = make_uint2(l[0], l[1]);
            }
        }
    }
};

// ------------------------------------------------------------------------------------------------ operand helpers
template <typename T>
struct Mfma;

template <>
struct Mfma<__bf16> {
    typedef bf16x8 vec;
    static __device__ __forceinline__ f32x16 run(vec a, vec b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
};

template <>
struct Mfma<_Float16> {
    typedef f16x8 vec;
    static __device__ __forceinline__ f32x16 run(vec a, vec b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
};

// Eight int8 codes (in a uint2) to an MFMA operand: exact codes, or T(fp32(d) * q).
template <typename T, int MODE>
__device__ __forceinline__ typename Mfma<T>::vec codes_to_operand(uint2 raw, float d) {
    typename Mfma<T>::vec out;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint32_t word = e < 4 ? raw.x : raw.y;
        const int q = (int)(int8_t)(uint8_t)(word >> (8 * (e & 3)));
        const float f = MODE == MODE_DEQUANT ? (float)q * d : (float)q;
        out[e] = static_cast<T>(f);
    }
    return out;
}

// ------------------------------------------------------------------------------------------------ epilogue
__device__ __forceinline__ void epilogue_store(const GemmParams& p, int row, int col, float v, float bias) {
    if ((p.flags & IDOLQ_FLAG_ROUND_BEFORE_BIAS) != 0) v = round_through(p.y_dt, v);
    v += bias;
    if (p.res) v += load_as_float(p.res, p.res_dt, (int64_t)row * p.ldr + col);
    v = apply_act(p.act, v);
    store_from_float(p.y, p.y_dt, (int64_t)row * p.ldy + col, v);
}

template <int TM, int TN, int WM, int WN>
__device__ __forceinline__ void write_tile(const GemmParams& p, const f32x16 (&acc)[TM][TN], int m0, int n0) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
        const int col = n0 + wn * WN + tn * 32 + (lane & 31);
        if (col >= p.n) continue;
        const float bias = p.bias ? load_as_float(p.bias, p.bias_dt, col) : 0.0f;
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm * WM + tm * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (row < p.m) epilogue_store(p, row, col, acc[tm][tn][r], bias);
            }
    }
}

// ------------------------------------------------------------------------------------------------ 16-bit MFMA kernel
template <int BM, int BN, int XT, int MODE, bool W4>
__global__ __launch_bounds__(kThreads) void q8_gemm_kernel(GemmParams p) {
    typedef typename std::conditional<XT == XT_F16, _Float16, __bf16>::type T;
    typedef typename Mfma<T>::vec Vec;
    constexpr int NT = XT == XT_F32 ? 2 : 1;  // activation terms: bf16 high and low parts of fp32 input
    constexpr int WM = BM / 2, WN = BN / 2, TM = WM / 32, TN = WN / 32;

    __shared__ __attribute__((aligned(16))) uint16_t a_lds[NT][BM * kAPitch];
    __shared__ __attribute__((aligned(16))) uint8_t code_lds[BN * kCodePitch];
    __shared__ float scale_lds[BN * 2];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    int tile_m, tile_n;
    tile_coords(p.tiles_m, p.tiles_n, tile_m, tile_n);
    const int m0 = tile_m * BM, n0 = tile_n * BN;
    const int nblocks = p.k / kQ8Block;
    const int nsteps = (nblocks + 1) / 2;

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    ActStage<BM, XT> as;
    WeightStage<BN, W4> ws;
    as.load(p, m0, 0);
    ws.load(p, n0, 0, nblocks);

    for (int s = 0; s < nsteps; ++s) {
        __syncthreads();
        as.store(a_lds[0], a_lds[NT - 1]);
        ws.template store<kCodePitch>(code_lds, scale_lds);
        __syncthreads();
        if (s + 1 < nsteps) {
            as.load(p, m0, (s + 1) * kKStep);
            ws.load(p, n0, 2 * (s + 1), nblocks);
        }
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
            Vec b[TN][2];
            float d[TN];
#pragma unroll
            for (int tn = 0; tn < TN; ++tn) {
                const int col = wn * WN + tn * 32 + (lane & 31);
                d[tn] = scale_lds[col * 2 + blk];
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const uint2 raw = *reinterpret_cast<const uint2*>(code_lds + col * kCodePitch + blk * 32 + h * 16 +
                                                                      (lane >> 5) * 8);
                    b[tn][h] = codes_to_operand<T, MODE>(raw, d[tn]);
                }
            }
#pragma unroll
            for (int tm = 0; tm < TM; ++tm) {
                const int row = wm * WM + tm * 32 + (lane & 31);
                Vec a[NT][2];
#pragma unroll
                for (int t = 0; t < NT; ++t)
#pragma unroll
                    for (int h = 0; h < 2; ++h)
                        a[t][h] = *reinterpret_cast<const Vec*>(a_lds[t] + row * kAPitch + blk * 32 + h * 16 +
                                                                (lane >> 5) * 8);
#pragma unroll
                for (int tn = 0; tn < TN; ++tn) {
                    if (MODE == MODE_DEQUANT) {
                        acc[tm][tn] = Mfma<T>::run(a[0][0], b[tn][0], acc[tm][tn]);
                        acc[tm][tn] = Mfma<T>::run(a[0][1], b[tn][1], acc[tm][tn]);
                    } else {
                        f32x16 part;
#pragma unroll
                        for (int r = 0; r < 16; ++r) part[r] = 0.0f;
#pragma unroll
                        for (int t = 0; t < NT; ++t) {
                            part = Mfma<T>::run(a[t][0], b[tn][0], part);
                            part = Mfma<T>::run(a[t][1], b[tn][1], part);
                        }
#pragma unroll
                        for (int r = 0; r < 16; ++r) acc[tm][tn][r] = fmaf(part[r], d[tn], acc[tm][tn][r]);
                    }
                }
            }
        }
    }
    write_tile<TM, TN, WM, WN>(p, acc, m0, n0);
}

// ------------------------------------------------------------------------------------------------ int8 MFMA kernel
// A = int8 activations (quantized per row and block by quantize_act_kernel) with fp32 scales per row and block.
// DOTS stores the raw int32 block sums instead of folding them (the bit-exact test entry point).
template <int BM, int BN, bool W4, bool DOTS>
__global__ __launch_bounds__(kThreads) void q8_gemm_int8_kernel(GemmParams p) {
    constexpr int WM = BM / 2, WN = BN / 2, TM = WM / 32, TN = WN / 32;
    constexpr int kAUnitsPerRow = kKStep / 16;  // 4 x 16 bytes of int8 per row per stage
    constexpr int kAPer = BM * kAUnitsPerRow / kThreads;
    static_assert(BM * kAUnitsPerRow % kThreads == 0, "tile size");

    __shared__ __attribute__((aligned(16))) uint8_t a_lds[BM * kCodePitch8];
    __shared__ __attribute__((aligned(16))) uint8_t code_lds[BN * kCodePitch8];
    __shared__ float scale_lds[BN * 2];
    __shared__ __attribute__((aligned(16))) float sa_lds[2][BM];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    int tile_m, tile_n;
    tile_coords(p.tiles_m, p.tiles_n, tile_m, tile_n);
    const int m0 = tile_m * BM, n0 = tile_n * BN;
    const int nblocks = p.k / kQ8Block;
    const int nsteps = (nblocks + 1) / 2;

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    WeightStage<BN, W4> ws;
    uint4 av[kAPer];
    float sav = 0.0f;
    auto load_a = [&](int s) {
        const int k0 = s * kKStep;
#pragma unroll
        for (int i = 0; i < kAPer; ++i) {
            const int u = threadIdx.x + i * kThreads;
            const int row = u / kAUnitsPerRow, cu = u - row * kAUnitsPerRow;
            const int kk = k0 + cu * 16;
            av[i] = make_uint4(0, 0, 0, 0);
            if (m0 + row < p.m && kk < p.k) av[i] = *reinterpret_cast<const uint4*>(p.qa + (int64_t)(m0 + row) * p.k + kk);
        }
        sav = 0.0f;
        if (!DOTS && threadIdx.x < 2 * BM) {
            const int row = threadIdx.x >> 1, b = 2 * s + (threadIdx.x & 1);
            if (m0 + row < p.m && b < nblocks) sav = p.sa[(int64_t)(m0 + row) * nblocks + b];
        }
    };
    load_a(0);
    ws.load(p, n0, 0, nblocks);

    for (int s = 0; s < nsteps; ++s) {
        __syncthreads();
#pragma unroll
        for (int i = 0; i < kAPer; ++i) {
            const int u = threadIdx.x + i * kThreads;
            const int row = u / kAUnitsPerRow, cu = u - row * kAUnitsPerRow;
            *reinterpret_cast<uint4*>(a_lds + row * kCodePitch8 + cu * 16) = av[i];
        }
        if (threadIdx.x < 2 * BM) sa_lds[threadIdx.x & 1][threadIdx.x >> 1] = sav;
        ws.template store<kCodePitch8>(code_lds, scale_lds);
        __syncthreads();
        if (s + 1 < nsteps) {
            load_a(s + 1);
            ws.load(p, n0, 2 * (s + 1), nblocks);
        }
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
            if (2 * s + blk >= nblocks) break;
            i32x4 b[TN];
            float dw[TN];
#pragma unroll
            for (int tn = 0; tn < TN; ++tn) {
                const int col = wn * WN + tn * 32 + (lane & 31);
                dw[tn] = scale_lds[col * 2 + blk];
                b[tn] = *reinterpret_cast<const i32x4*>(code_lds + col * kCodePitch8 + blk * 32 + (lane >> 5) * 16);
            }
#pragma unroll
            for (int tm = 0; tm < TM; ++tm) {
                const int row = wm * WM + tm * 32 + (lane & 31);
                const i32x4 a = *reinterpret_cast<const i32x4*>(a_lds + row * kCodePitch8 + blk * 32 + (lane >> 5) * 16);
                f32x4 sa4[4];
                if (!DOTS) {
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        sa4[q] = *reinterpret_cast<const f32x4*>(&sa_lds[blk][wm * WM + tm * 32 + 8 * q + 4 * (lane >> 5)]);
                }
#pragma unroll
                for (int tn = 0; tn < TN; ++tn) {
                    i32x16 zero;
#pragma unroll
                    for (int r = 0; r < 16; ++r) zero[r] = 0;
                    const i32x16 dots = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b[tn], zero, 0, 0, 0);
                    if (DOTS) {
                        const int col = n0 + wn * WN + tn * 32 + (lane & 31);
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            const int grow = m0 + wm * WM + tm * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                            if (grow < p.m && col < p.n)
                                p.dots[((int64_t)grow * p.n + col) * nblocks + 2 * s + blk] = dots[r];
                        }
                    } else {
#pragma unroll
                        for (int r = 0; r < 16; ++r)
                            acc[tm][tn][r] = fmaf((float)dots[r], sa4[r >> 2][r & 3] * dw[tn], acc[tm][tn][r]);
                    }
                }
            }
        }
    }
    if (!DOTS) write_tile<TM, TN, WM, WN>(p, acc, m0, n0);
}

// ------------------------------------------------------------------------------------------------ launch
template <int BM, int BN>
int launch_16bit(GemmParams p, int xt, int mode, bool w4, hipStream_t stream) {
    p.tiles_m = (p.m + BM - 1) / BM;
    p.tiles_n = (p.n + BN - 1) / BN;
    const dim3 grid(p.tiles_m * p.tiles_n), block(kThreads);
#define IDOLQ_LAUNCH(XT, MODE, W4) \
    hipLaunchKernelGGL((q8_gemm_kernel<BM, BN, XT, MODE, W4>), grid, block, 0, stream, p)
    if (xt == XT_BF16 && mode == MODE_DEQUANT) { if (w4) IDOLQ_LAUNCH(XT_BF16, MODE_DEQUANT, true); else IDOLQ_LAUNCH(XT_BF16, MODE_DEQUANT, false); }
    else if (xt == XT_BF16 && mode == MODE_EXACT) { if (w4) IDOLQ_LAUNCH(XT_BF16, MODE_EXACT, true); else IDOLQ_LAUNCH(XT_BF16, MODE_EXACT, false); }
    else if (xt == XT_F16 && mode == MODE_DEQUANT) { if (w4) IDOLQ_LAUNCH(XT_F16, MODE_DEQUANT, true); else IDOLQ_LAUNCH(XT_F16, MODE_DEQUANT, false); }
    else if (xt == XT_F16 && mode == MODE_EXACT) { if (w4) IDOLQ_LAUNCH(XT_F16, MODE_EXACT, true); else IDOLQ_LAUNCH(XT_F16, MODE_EXACT, false); }
    else if (xt == XT_F32 && mode == MODE_EXACT) { if (w4) IDOLQ_LAUNCH(XT_F32, MODE_EXACT, true); else IDOLQ_LAUNCH(XT_F32, MODE_EXACT, false); }
    else return fail(IDOLQ_ENOSUPPORT, "this activation dtype does not support the requested GEMM mode");
#undef IDOLQ_LAUNCH
    return check_launch("q8_gemm_kernel");
}

template <int BM, int BN, bool DOTS>
int launch_int8(GemmParams p, bool w4, hipStream_t stream) {
    p.tiles_m = (p.m + BM - 1) / BM;
    p.tiles_n = (p.n + BN - 1) / BN;
    const dim3 grid(p.tiles_m * p.tiles_n), block(kThreads);
    if (w4)
        hipLaunchKernelGGL((q8_gemm_int8_kernel<BM, BN, true, DOTS>), grid, block, 0, stream, p);
    else
        hipLaunchKernelGGL((q8_gemm_int8_kernel<BM, BN, false, DOTS>), grid, block, 0, stream, p);
    return check_launch("q8_gemm_int8_kernel");
}

}  // namespace

// Quantizes activations for the int8 path (q8_aux.hip).
int quantize_act_launch(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, int8_t* qa, float* scale,
                        int32_t* qsum, hipStream_t stream);

}  // namespace idolq

using namespace idolq;

extern "C" size_t idolq_q8_0_gemm_workspace(int64_t m, int64_t k, int mode) {
    if (mode != IDOLQ_MODE_INT8 || m <= 0 || k <= 0 || k % kQ8Block) return 0;
    const size_t qa = ((size_t)m * (size_t)k + 255) / 256 * 256;
    return qa + (size_t)m * (size_t)(k / kQ8Block) * sizeof(float);
}

extern "C" int idolq_q8_0_gemm(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const uint8_t* w,
                               int64_t n_total, int64_t n_offset, int64_t n, const void* bias, int bias_dtype,
                               const void* residual, int residual_dtype, int64_t ldr, int act, int mode, int flags,
                               void* y, int y_dtype, int64_t ldy, void* workspace, size_t workspace_bytes,
                               void* stream) {
    if (!dtype_ok(x_dtype) || !dtype_ok(y_dtype) || (bias && !dtype_ok(bias_dtype)) ||
        (residual && !dtype_ok(residual_dtype)))
        return fail(IDOLQ_EINVAL, "unknown dtype code");
    if (m < 0 || n < 0 || k <= 0 || k % kQ8Block) return fail(IDOLQ_EINVAL, "need m >= 0, n >= 0 and k a positive multiple of 32");
    if (n_offset < 0 || n_offset + n > n_total) return fail(IDOLQ_EINVAL, "column window outside the weight rows");
    if (ldx < k || ldy < n || (residual && ldr < n)) return fail(IDOLQ_EINVAL, "row stride smaller than the row");
    if (m > INT32_MAX / 2 || n > INT32_MAX / 2 || k > INT32_MAX / 2) return fail(IDOLQ_EINVAL, "dimension too large");
    if (act < IDOLQ_ACT_NONE || act > IDOLQ_ACT_RELU) return fail(IDOLQ_EINVAL, "unknown activation");
    if (residual == y && residual && (residual_dtype != y_dtype || ldr != ldy))
        return fail(IDOLQ_EINVAL, "a residual that aliases y must have y's dtype and stride");
    if ((reinterpret_cast<uintptr_t>(w) & 1) != 0) return fail(IDOLQ_EINVAL, "Q8_0 weights must be 2-byte aligned");
    if (mode == IDOLQ_MODE_AUTO) mode = x_dtype == IDOLQ_F32 ? IDOLQ_MODE_EXACT : IDOLQ_MODE_DEQUANT;
    if (mode < IDOLQ_MODE_DEQUANT || mode > IDOLQ_MODE_INT8) return fail(IDOLQ_EINVAL, "unknown GEMM mode");
    if (mode == IDOLQ_MODE_DEQUANT && x_dtype == IDOLQ_F32)
        return fail(IDOLQ_EINVAL, "DEQUANT mode takes bf16 or fp16 activations");
    if (m == 0 || n == 0) return IDOLQ_OK;  // empty input: nothing to read or write (pointers may be null)
    if (!x || !w || !y) return fail(IDOLQ_EINVAL, "x, w and y must be non-null");
    hipStream_t s = static_cast<hipStream_t>(stream);

    GemmParams p{};
    p.x = x;
    p.ldx = ldx;
    p.row_bytes = (k / kQ8Block) * kQ8Bytes;
    p.w = w + n_offset * p.row_bytes;
    p.m = (int)m;
    p.n = (int)n;
    p.k = (int)k;
    p.bias = bias ? static_cast<const char*>(bias) + n_offset * dtype_size(bias_dtype) : nullptr;
    p.bias_dt = bias_dtype;
    p.res = residual;
    p.res_dt = residual_dtype;
    p.ldr = ldr;
    p.y = y;
    p.y_dt = y_dtype;
    p.ldy = ldy;
    p.act = act;
    p.flags = flags;
    const size_t esz = dtype_size(x_dtype);
    p.x_aligned = (reinterpret_cast<uintptr_t>(x) % 16 == 0) && ((size_t)ldx * esz) % 16 == 0;
    const bool w4 = p.row_bytes % 4 == 0 && (reinterpret_cast<uintptr_t>(p.w) & 3) == 0;

    if (mode == IDOLQ_MODE_INT8) {
        const size_t need = idolq_q8_0_gemm_workspace(m, k, mode);
        if (!workspace || workspace_bytes < need)
            return fail(IDOLQ_EINVAL, "INT8 mode needs a workspace of idolq_q8_0_gemm_workspace() bytes");
        if (reinterpret_cast<uintptr_t>(workspace) % 16 != 0) return fail(IDOLQ_EINVAL, "workspace must be 16-byte aligned");
        int8_t* qa = static_cast<int8_t*>(workspace);
        float* sa = reinterpret_cast<float*>(static_cast<char*>(workspace) + ((size_t)m * (size_t)k + 255) / 256 * 256);
        int rc = quantize_act_launch(x, x_dtype, m, k, ldx, qa, sa, nullptr, s);
        if (rc) return rc;
        p.qa = qa;
        p.sa = sa;
        return launch_int8<128, 128, false>(p, w4, s);
    }
    const int xt = x_dtype == IDOLQ_BF16 ? XT_BF16 : x_dtype == IDOLQ_F16 ? XT_F16 : XT_F32;
    return launch_16bit<128, 128>(p, xt, mode == IDOLQ_MODE_DEQUANT ? MODE_DEQUANT : MODE_EXACT, w4, s);
}

extern "C" int idolq_q8_0_block_dots(const int8_t* qa, int64_t m, int64_t k, const uint8_t* w, int64_t n_total,
                                     int64_t n_offset, int64_t n, int32_t* dots, void* stream) {
    if (m < 0 || n < 0 || k <= 0 || k % kQ8Block) return fail(IDOLQ_EINVAL, "need m >= 0, n >= 0 and k a positive multiple of 32");
    if (n_offset < 0 || n_offset + n > n_total) return fail(IDOLQ_EINVAL, "column window outside the weight rows");
    if (m == 0 || n == 0) return IDOLQ_OK;
    if (!qa || !w || !dots) return fail(IDOLQ_EINVAL, "qa, w and dots must be non-null");
    if (reinterpret_cast<uintptr_t>(qa) % 16 != 0 || k % 16 != 0) return fail(IDOLQ_EINVAL, "qa must be 16-byte aligned");
    if ((reinterpret_cast<uintptr_t>(w) & 1) != 0) return fail(IDOLQ_EINVAL, "Q8_0 weights must be 2-byte aligned");
    if (m == 0 || n == 0) return IDOLQ_OK;
    GemmParams p{};
    p.row_bytes = (k / kQ8Block) * kQ8Bytes;
    p.w = w + n_offset * p.row_bytes;
    p.m = (int)m;
    p.n = (int)n;
    p.k = (int)k;
    p.qa = qa;
    p.dots = dots;
    const bool w4 = p.row_bytes % 4 == 0 && (reinterpret_cast<uintptr_t>(p.w) & 3) == 0;
    return launch_int8<128, 128, true>(p, w4, static_cast<hipStream_t>(stream));
}
