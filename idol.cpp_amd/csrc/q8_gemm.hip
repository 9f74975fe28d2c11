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
#include "q8_gemm.h"

#include <algorithm>
#include <mutex>
#include <type_traits>

namespace idolq {
namespace {

constexpr int kThreads = 256;
constexpr int kKStep = 64;                // depth per stage: two Q8_0 blocks
constexpr int kAPitch = kKStep + 8;       // 16-bit elements per activation row in LDS (144 bytes)
constexpr int kCodePitch8 = kKStep + 16;  // bytes per row of int8 operands for 16-byte reads (80)

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
// BM rows x 64 k of x per stage in 16-byte units. The per-thread row offsets (in 16-byte units, ~0u for rows
// outside m) are computed once; a stage only adds its k offset. Unit u = tid + 256 i covers row u / kUnitsPerRow,
// column unit tid % kUnitsPerRow (the same for every i).
// XA: x is known to be 16-byte aligned (no runtime test, so the load sequence has no branch for the compiler's
// wait counts to merge over).
template <int BM, int XT, int THREADS, bool XA = false>
struct ActStage {
    static constexpr int kEsz = XT == XT_F32 ? 4 : 2;
    static constexpr int kUnitsPerRow = kKStep * kEsz / 16;  // 8 (16-bit) or 16 (fp32)
    static constexpr int kRowsPerPass = THREADS / kUnitsPerRow;
    static constexpr int kPer = BM / kRowsPerPass;
    static constexpr int kElems = 16 / kEsz;
    static_assert(BM % kRowsPerPass == 0, "tile size");
    uint32_t off[kPer];  // element offset of the unit's row start + column unit, ~0u when the row is outside m
    uint4 v[kPer];
    bool ok[kPer];  // the unit holds x (else it is stored as zeros)

    __device__ __forceinline__ void init(const GemmParams& p, int m0) {
        const int cu = threadIdx.x % kUnitsPerRow, r0 = threadIdx.x / kUnitsPerRow;
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int row = m0 + r0 + i * kRowsPerPass;
            off[i] = row < p.m ? (uint32_t)((int64_t)row * p.ldx + cu * kElems) : ~0u;
        }
    }

    // Invalid units (rows outside m, depth beyond k) read the first element of x and are zeroed when stored (not
    // when loaded, which would make the load's consumer wait for it), so the loads need no branches.
    __device__ __forceinline__ void load(const GemmParams& p, int k0) {
        const int kk = k0 + (threadIdx.x % kUnitsPerRow) * kElems;
        const bool kin = kk < p.k;
        if (XA || p.x_aligned) {
#pragma unroll
            for (int i = 0; i < kPer; ++i) {
                ok[i] = off[i] != ~0u && kin;
                const char* src = static_cast<const char*>(p.x) + (ok[i] ? ((size_t)off[i] + k0) * kEsz : 0);
                v[i] = *reinterpret_cast<const uint4*>(src);
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            v[i] = make_uint4(0, 0, 0, 0);
            ok[i] = true;
            if (off[i] != ~0u && kin) {
                const char* src = static_cast<const char*>(p.x) + ((size_t)off[i] + k0) * kEsz;
                {
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
        const int cu = threadIdx.x % kUnitsPerRow, r0 = threadIdx.x / kUnitsPerRow;
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int off_lds = (r0 + i * kRowsPerPass) * kAPitch + cu * kElems;
            // a mask, not a select: a select of the loaded value lets the compiler branch around the use, and the
            // joins make its wait counts fall back to waiting for every outstanding load
            const uint32_t mk = 0u - (uint32_t)ok[i];
            const uint4 vi = make_uint4(v[i].x & mk, v[i].y & mk, v[i].z & mk, v[i].w & mk);
            if (XT != XT_F32) {
                *reinterpret_cast<uint4*>(hi + off_lds) = vi;
            } else {
                const float f[4] = {__builtin_bit_cast(float, vi.x), __builtin_bit_cast(float, vi.y),
                                    __builtin_bit_cast(float, vi.z), __builtin_bit_cast(float, vi.w)};
                uint32_t h[2], l[2];
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const uint16_t h0 = float_to_bf16_bits(f[2 * e]), h1 = float_to_bf16_bits(f[2 * e + 1]);
                    const uint16_t l0 = float_to_bf16_bits(f[2 * e] - bf16_bits_to_float(h0));
                    const uint16_t l1 = float_to_bf16_bits(f[2 * e + 1] - bf16_bits_to_float(h1));
                    h[e] = (uint32_t)h0 | ((uint32_t)h1 << 16);
                    l[e] = (uint32_t)l0 | ((uint32_t)l1 << 16);
                }
                *reinterpret_cast<uint2*>(hi + off_lds) = make_uint2(h[0], h[1]);
                *reinterpret_cast<uint2*>(lo + off_lds) = make_uint2(l[0], l[1]);
            }
        }
    }
};

// ------------------------------------------------------------------------------------------------ raw weight staging
// The 68 bytes (two Q8_0 blocks) of each of BN weight rows per stage, copied unchanged into LDS as a [BN][68-byte]
// array: dword (W4) or halfword unit u of the flat run is row u / 17 (u / 34), and it lands at LDS unit u, so the
// global reads are one coalesced run per row and the LDS writes one contiguous run per wave.
template <int BN, bool W4, int THREADS>
struct RawStage {
    static constexpr int kUnitsPerRow = W4 ? 17 : 34;
    static constexpr int kUnits = BN * kUnitsPerRow;
    static constexpr int kPer = (kUnits + THREADS - 1) / THREADS;
    // dwords of one LDS stage: every thread's kPer units have a slot (units past the rows land in padding, so the
    // stores need no branch, which would make the compiler wait for every outstanding load before them)
    static constexpr int kWords = W4 ? kPer * THREADS : (kPer * THREADS + 1) / 2;
    uint32_t off[kPer];  // byte offset of the unit within the window (row * row_bytes + part * size), ~0u if unused
    bool second[kPer];   // the unit belongs to the second block of the stage
    uint32_t v[kPer];
    bool ok[kPer];  // the unit holds weight bytes (else it is stored as zero)

    __device__ __forceinline__ void init(const GemmParams& p, int n0) {
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int u = threadIdx.x + i * THREADS;
            const int row = u / kUnitsPerRow, part = u - row * kUnitsPerRow;
            off[i] = (u < kUnits && n0 + row < p.n) ? (uint32_t)((int64_t)(n0 + row) * p.row_bytes + part * (W4 ? 4 : 2))
                                                    : ~0u;
            second[i] = W4 ? part >= 9 : part >= 17;
        }
    }

    // Units outside the window (or in a missing second block) read the window's first bytes and are zeroed when
    // stored.
    __device__ __forceinline__ void load(const GemmParams& p, int blk0, int nblocks) {
        const bool has_second = blk0 + 1 < nblocks;
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            ok[i] = off[i] != ~0u && (has_second || !second[i]);
            const uint8_t* src = p.w + (ok[i] ? off[i] + (size_t)blk0 * kQ8Bytes : 0);
            v[i] = W4 ? *reinterpret_cast<const uint32_t*>(src) : (uint32_t) * reinterpret_cast<const uint16_t*>(src);
        }
    }

    __device__ __forceinline__ void store(uint32_t* raw) const {
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int u = threadIdx.x + i * THREADS;
            const uint32_t vi = v[i] & (0u - (uint32_t)ok[i]);  // a mask, not a select (as in ActStage::store)
            if (W4)
                raw[u] = vi;
            else
                reinterpret_cast<uint16_t*>(raw)[u] = (uint16_t)vi;
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

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Eight int8 codes (in a uint2) to eight 16-bit operand values: exact codes, or T(fp32(d) * q). Pairs are rounded
// together (one v_cvt_pk_bf16_f32 for bf16).
template <typename T, int MODE>
__device__ __forceinline__ uint4 codes_to_operand(uint2 raw, float d) {
    typedef typename std::conditional<std::is_same<T, __bf16>::value, bf16x2, f16x2>::type T2;
    uint32_t out[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const uint32_t word = e < 2 ? raw.x : raw.y;
        const int sh = 16 * (e & 1);
        f32x2 f;
        f.x = (float)(int)(int8_t)(uint8_t)(word >> sh);
        f.y = (float)(int)(int8_t)(uint8_t)(word >> (sh + 8));
        if (MODE == MODE_DEQUANT) f = f * d;
        out[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f, T2));
    }
    return make_uint4(out[0], out[1], out[2], out[3]);
}

// Converts the raw [BN][68-byte] stage into 16-bit B operands [BN][kAPitch] (and, for EXACT, fp32 scales [BN][2]).
// Thread t handles row t / 2 (+128 per pass) and the four 8-code chunks (blk, jj = 2 q + t % 2): block 0's codes sit
// at byte 2 + 8 jj (two bytes off dword alignment, realigned with alignbyte), block 1's at byte 36 + 8 jj.
// All LDS reads of a pass are issued before any of its arithmetic, so their latency is paid once.
template <typename T, int BN, int MODE, int THREADS>
__device__ __forceinline__ void convert_stage(const uint32_t* raw, uint16_t* b, float* bscale) {
    constexpr int kRows = THREADS / 2;  // rows per pass: two threads per row
    const int half = threadIdx.x & 1;
#pragma unroll
    for (int rp = 0; rp < (BN + kRows - 1) / kRows; ++rp) {
        const int row = rp * kRows + (threadIdx.x >> 1);
        if (BN % kRows != 0 && row >= BN) break;
        const uint32_t* rw = raw + row * 17;
        // dwords 2jj..2jj+2 (block 0) and 9+2jj, 10+2jj (block 1) for jj = half and 2 + half; dword 0 and 8 scales
        uint32_t w[12];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int jj = 2 * q + half;
            w[6 * q + 0] = rw[2 * jj];
            w[6 * q + 1] = rw[2 * jj + 1];
            w[6 * q + 2] = rw[2 * jj + 2];
            w[6 * q + 3] = rw[9 + 2 * jj];
            w[6 * q + 4] = rw[10 + 2 * jj];
        }
        const uint32_t s0 = rw[0], s8 = rw[8];
        const float d0 = half_bits_to_float((uint16_t)(s0 & 0xffff));
        const float d1 = half_bits_to_float((uint16_t)(s8 >> 16));
        if (MODE == MODE_EXACT && half == 0) {
            bscale[row * 2] = d0;
            bscale[row * 2 + 1] = d1;
        }
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int jj = 2 * q + half;
            const uint2 c0 = make_uint2(__builtin_amdgcn_alignbyte(w[6 * q + 1], w[6 * q + 0], 2),
                                        __builtin_amdgcn_alignbyte(w[6 * q + 2], w[6 * q + 1], 2));
            const uint4 o0 = codes_to_operand<T, MODE>(c0, d0);
            const uint4 o1 = codes_to_operand<T, MODE>(make_uint2(w[6 * q + 3], w[6 * q + 4]), d1);
            *reinterpret_cast<uint4*>(b + row * kAPitch + 8 * jj) = o0;
            *reinterpret_cast<uint4*>(b + row * kAPitch + 32 + 8 * jj) = o1;
        }
    }
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


// Epilogue through LDS: the accumulator tile is written to LDS as fp32 ([BM][BN + 4]), then each thread takes runs of
// 8 consecutive columns of one row and applies the epilogue with vector loads of bias and residual and one 16-byte
// (32-byte for fp32) store per run, so each wave writes whole row segments instead of 2-byte scattered stores.
// KS == 2: the workgroup's waves form two depth groups and only the first group's accumulators (which already hold
// the second group's sums) are written.
template <int BM, int BN, int TM, int TN, int WM, int WN, int THREADS, int KS = 1>
__device__ __forceinline__ void write_tile_staged(const GemmParams& p, const f32x16 (&acc)[TM][TN], int m0, int n0,
                                                  float* stage) {
    constexpr int kPitch = BN + 4;
    constexpr int kRuns = BN / 8;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wq = wave % (THREADS / 64 / KS);
    const int wm = wq >> 1, wn = wq & 1;
    const bool round_first = (p.flags & IDOLQ_FLAG_ROUND_BEFORE_BIAS) != 0;
    __syncthreads();
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
        if (KS == 2 && wave >= THREADS / 128) break;
        const int col = wn * WN + tn * 32 + (lane & 31);
        const float bias = p.bias && n0 + col < p.n ? load_as_float(p.bias, p.bias_dt, n0 + col) : 0.0f;
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = wm * WM + tm * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                float v = acc[tm][tn][r];
                if (round_first) v = round_through(p.y_dt, v);
                stage[row * kPitch + col] = v + bias;
            }
    }
    __syncthreads();
    for (int c = threadIdx.x; c < BM * kRuns; c += THREADS) {
        const int row = c / kRuns, col = (c % kRuns) * 8;
        const int grow = m0 + row, gcol = n0 + col;
        if (grow >= p.m || gcol >= p.n) continue;
        float v[8];
        const float4 lo = *reinterpret_cast<const float4*>(stage + row * kPitch + col);
        const float4 hi = *reinterpret_cast<const float4*>(stage + row * kPitch + col + 4);
        v[0] = lo.x, v[1] = lo.y, v[2] = lo.z, v[3] = lo.w, v[4] = hi.x, v[5] = hi.y, v[6] = hi.z, v[7] = hi.w;
        const int cnt = min(8, p.n - gcol);
        if (cnt == 8 && p.y_vec) {
            float r[8];
            if (p.res) {
                const char* rp = static_cast<const char*>(p.res) + ((int64_t)grow * p.ldr + gcol) * (p.res_dt == IDOLQ_F32 ? 4 : 2);
                if (p.res_dt == IDOLQ_F32) {
                    const float4 a = reinterpret_cast<const float4*>(rp)[0], b = reinterpret_cast<const float4*>(rp)[1];
                    r[0] = a.x, r[1] = a.y, r[2] = a.z, r[3] = a.w, r[4] = b.x, r[5] = b.y, r[6] = b.z, r[7] = b.w;
                } else {
                    const uint4 u = *reinterpret_cast<const uint4*>(rp);
                    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const uint16_t bits = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
                        r[e] = p.res_dt == IDOLQ_BF16 ? bf16_bits_to_float(bits) : half_bits_to_float(bits);
                    }
                }
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = apply_act(p.act, p.res ? v[e] + r[e] : v[e]);
            char* yp = static_cast<char*>(p.y) + ((int64_t)grow * p.ldy + gcol) * (p.y_dt == IDOLQ_F32 ? 4 : 2);
            if (p.y_dt == IDOLQ_F32) {
                reinterpret_cast<float4*>(yp)[0] = make_float4(v[0], v[1], v[2], v[3]);
                reinterpret_cast<float4*>(yp)[1] = make_float4(v[4], v[5], v[6], v[7]);
            } else {
                uint32_t w[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint16_t a = p.y_dt == IDOLQ_BF16 ? float_to_bf16_bits(v[2 * e]) : float_to_half_bits(v[2 * e]);
                    const uint16_t b = p.y_dt == IDOLQ_BF16 ? float_to_bf16_bits(v[2 * e + 1]) : float_to_half_bits(v[2 * e + 1]);
                    w[e] = (uint32_t)a | ((uint32_t)b << 16);
                }
                *reinterpret_cast<uint4*>(yp) = make_uint4(w[0], w[1], w[2], w[3]);
            }
        } else {
            for (int e = 0; e < cnt; ++e) {
                float x = v[e];
                if (p.res) x += load_as_float(p.res, p.res_dt, (int64_t)grow * p.ldr + gcol + e);
                store_from_float(p.y, p.y_dt, (int64_t)grow * p.ldy + gcol + e, apply_act(p.act, x));
            }
        }
    }
}

// ------------------------------------------------------------------------------------------------ 16-bit MFMA kernel
// Software pipeline with one barrier per stage. At the start of stage s: A[s%2] and B[s%2] hold stage s, raw[(s+1)%2]
// holds stage s+1's weight bytes, one activation register set holds stage s+1 and one weight register set stage s+2.
// During stage s each wave stores those registers (A[(s+1)%2], raw[s%2]), reloads them with activations s+3 and
// weights s+4, converts raw[(s+1)%2] into B[(s+1)%2] and runs the MFMAs of stage s; every buffer it writes was last
// read in stage s-1, before the barrier that ends it.
// KS == 2 (EXACT): the waves form two depth groups of (THREADS / 256) x 2; group g multiplies block g of every
// two-block stage into its own accumulators, and the second group's sums are added to the first's at the end (twice
// the waves per workgroup for the latency of the per-block MFMA chains, the same loads and conversion).
template <int BM, int BN, int XT, int MODE, bool W4, int THREADS, int KS = 1, bool XA = false>
__global__ __launch_bounds__(THREADS) void q8_gemm_kernel(GemmParams p) {
    typedef typename std::conditional<XT == XT_F16, _Float16, __bf16>::type T;
    typedef typename Mfma<T>::vec Vec;
    constexpr int NT = XT == XT_F32 ? 2 : 1;  // activation terms: bf16 high and low parts of fp32 input
    static_assert(KS == 1 || (KS == 2 && MODE == MODE_EXACT), "depth groups are for the EXACT fold");
    // waves in a (THREADS / KS / 128) x 2 grid per depth group, each owning a WM x WN tile of 32 x 32 MFMA tiles
    constexpr int WAVES_M = THREADS / KS / 128;
    constexpr int NB = 2 / KS;  // blocks of a stage each wave multiplies
    constexpr int WM = BM / WAVES_M, WN = BN / 2, TM = WM / 32, TN = WN / 32;

    constexpr int kRawWords = RawStage<BN, W4, THREADS>::kWords;
    constexpr int kABytes = 2 * NT * BM * kAPitch * 2, kBBytes = 2 * BN * kAPitch * 2, kRawBytes = 2 * kRawWords * 4;
    constexpr int kScaleBytes = MODE == MODE_EXACT ? 2 * BN * 2 * 4 : 16;
    constexpr int kLoopBytes = kABytes + kBBytes + kRawBytes + kScaleBytes;
    constexpr int kStageBytes = BM * (BN + 4) * 4;
    __shared__ __attribute__((aligned(16))) char smem[kLoopBytes > kStageBytes ? kLoopBytes : kStageBytes];
    typedef uint16_t ATile[NT][BM * kAPitch];
    typedef uint16_t BTile[BN * kAPitch];
    typedef uint32_t RawTile[kRawWords];
    typedef float ScaleTile[MODE == MODE_EXACT ? BN * 2 : 4];
    ATile* a_lds = reinterpret_cast<ATile*>(smem);
    BTile* b_lds = reinterpret_cast<BTile*>(smem + kABytes);
    RawTile* raw_lds = reinterpret_cast<RawTile*>(smem + kABytes + kBBytes);
    ScaleTile* bscale = reinterpret_cast<ScaleTile*>(smem + kABytes + kBBytes + kRawBytes);

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int kg = KS == 2 ? wave / (THREADS / 128) : 0;  // depth group
    const int wq = wave % (THREADS / 64 / KS);
    const int wm = wq >> 1, wn = wq & 1;
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

    // Two register sets for the activation and weight loads, used alternately, so every load is issued two stages
    // before its registers are stored to LDS: set (s + 1) % 2 of activations holds stage s + 1 at the start of
    // stage s, set s % 2 of weights holds stage s + 2.
    ActStage<BM, XT, THREADS, XA> as0, as1;
    RawStage<BN, W4, THREADS> ws0, ws1;
    as0.init(p, m0);
    as1.init(p, m0);
    ws0.init(p, n0);
    ws1.init(p, n0);

    // prologue: A(0) and raw(0) into LDS, B(0) converted, raw(1) into LDS; then activations 1, 2 and weights 2, 3
    // are in the registers
    as0.load(p, 0);
    ws0.load(p, 0, nblocks);
    if (nsteps > 1) {
        as1.load(p, kKStep);
        ws1.load(p, 2, nblocks);
    }
    as0.store(a_lds[0][0], a_lds[0][NT - 1]);
    ws0.store(raw_lds[0]);
    if (nsteps > 2) {
        as0.load(p, 2 * kKStep);
        ws0.load(p, 4, nblocks);
    }
    __syncthreads();
    convert_stage<T, BN, MODE, THREADS>(raw_lds[0], b_lds[0], bscale[0]);
    if (nsteps > 1) ws1.store(raw_lds[1]);
    if (nsteps > 3) ws1.load(p, 6, nblocks);
    __syncthreads();

    auto stage = [&](int s, auto& ra, auto& rw) {
        // The body has no branches: past the last stage the prefetch indices are clamped and the stores and the
        // conversion fill buffers that are never read again, so the whole stage is one scheduling region.
        const int cur = s & 1, nxt = cur ^ 1;
        ra.store(a_lds[nxt][0], a_lds[nxt][NT - 1]);
        ra.load(p, min(s + 3, nsteps - 1) * kKStep);
        rw.store(raw_lds[cur]);
        rw.load(p, 2 * min(s + 4, nsteps - 1), nblocks);
        convert_stage<T, BN, MODE, THREADS>(raw_lds[nxt], b_lds[nxt], bscale[nxt]);

        const uint16_t* bc = b_lds[cur];
        // Operands of the wave's blocks of the stage are read before the first MFMA (the second block's reads
        // complete under the first block's MFMAs).
        Vec a[NB][NT][TM][2], b[NB][TN][2];
#pragma unroll
        for (int bi = 0; bi < NB; ++bi)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int koff = (KS == 2 ? kg : bi) * 32 + h * 16 + (lane >> 5) * 8;
#pragma unroll
                for (int t = 0; t < NT; ++t)
#pragma unroll
                    for (int tm = 0; tm < TM; ++tm)
                        a[bi][t][tm][h] = *reinterpret_cast<const Vec*>(a_lds[cur][t] + (wm * WM + tm * 32 + (lane & 31)) * kAPitch + koff);
#pragma unroll
                for (int tn = 0; tn < TN; ++tn)
                    b[bi][tn][h] = *reinterpret_cast<const Vec*>(bc + (wn * WN + tn * 32 + (lane & 31)) * kAPitch + koff);
            }
#pragma unroll
        for (int bi = 0; bi < NB; ++bi) {
            const int blk = KS == 2 ? kg : bi;
#pragma unroll
            for (int tm = 0; tm < TM; ++tm)
#pragma unroll
                for (int tn = 0; tn < TN; ++tn) {
                    if (MODE == MODE_DEQUANT) {
                        acc[tm][tn] = Mfma<T>::run(a[bi][0][tm][0], b[bi][tn][0], acc[tm][tn]);
                        acc[tm][tn] = Mfma<T>::run(a[bi][0][tm][1], b[bi][tn][1], acc[tm][tn]);
                    } else {
                        const float d = bscale[cur][(wn * WN + tn * 32 + (lane & 31)) * 2 + blk];
                        f32x16 part;
#pragma unroll
                        for (int r = 0; r < 16; ++r) part[r] = 0.0f;
#pragma unroll
                        for (int t = 0; t < NT; ++t) {
                            part = Mfma<T>::run(a[bi][t][tm][0], b[bi][tn][0], part);
                            part = Mfma<T>::run(a[bi][t][tm][1], b[bi][tn][1], part);
                        }
#pragma unroll
                        for (int r = 0; r < 16; ++r) acc[tm][tn][r] = fmaf(part[r], d, acc[tm][tn][r]);
                    }
                }
        }
        __syncthreads();
    };

    for (int s = 0; s < nsteps; s += 2) {
        stage(s, as1, ws0);
        if (s + 1 < nsteps) stage(s + 1, as0, ws1);
    }
    if constexpr (KS == 2) {
        // the second group's sums (odd blocks) through LDS into the first group's (even blocks): a fixed order
        float* red = reinterpret_cast<float*>(smem);
        constexpr int kPitch = BN + 4;
        __syncthreads();
        if (kg == 1)
#pragma unroll
            for (int tm = 0; tm < TM; ++tm)
#pragma unroll
                for (int tn = 0; tn < TN; ++tn)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        red[(wm * WM + tm * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * kPitch + wn * WN + tn * 32 +
                            (lane & 31)] = acc[tm][tn][r];
        __syncthreads();
        if (kg == 0)
#pragma unroll
            for (int tm = 0; tm < TM; ++tm)
#pragma unroll
                for (int tn = 0; tn < TN; ++tn)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        acc[tm][tn][r] += red[(wm * WM + tm * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * kPitch +
                                              wn * WN + tn * 32 + (lane & 31)];
    }
    write_tile_staged<BM, BN, TM, TN, WM, WN, THREADS, KS>(p, acc, m0, n0, reinterpret_cast<float*>(smem));
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
template <int BM, int BN, int THREADS>
int launch_16bit_tile(GemmParams p, int xt, int mode, bool w4, hipStream_t stream) {
    p.tiles_m = (p.m + BM - 1) / BM;
    p.tiles_n = (p.n + BN - 1) / BN;
    const dim3 grid(p.tiles_m * p.tiles_n), block(THREADS);
#define IDOLQ_LAUNCH(XT, MODE, W4) \
    hipLaunchKernelGGL((q8_gemm_kernel<BM, BN, XT, MODE, W4, THREADS>), grid, block, 0, stream, p)
    if (xt == XT_BF16 && mode == MODE_DEQUANT) { if (w4) IDOLQ_LAUNCH(XT_BF16, MODE_DEQUANT, true); else IDOLQ_LAUNCH(XT_BF16, MODE_DEQUANT, false); }
    else if (xt == XT_BF16 && mode == MODE_EXACT) { if (w4) IDOLQ_LAUNCH(XT_BF16, MODE_EXACT, true); else IDOLQ_LAUNCH(XT_BF16, MODE_EXACT, false); }
    else if (xt == XT_F16 && mode == MODE_DEQUANT) { if (w4) IDOLQ_LAUNCH(XT_F16, MODE_DEQUANT, true); else IDOLQ_LAUNCH(XT_F16, MODE_DEQUANT, false); }
    else if (xt == XT_F16 && mode == MODE_EXACT) { if (w4) IDOLQ_LAUNCH(XT_F16, MODE_EXACT, true); else IDOLQ_LAUNCH(XT_F16, MODE_EXACT, false); }
    else return fail(IDOLQ_ENOSUPPORT, "this activation dtype does not support the requested GEMM mode");
#undef IDOLQ_LAUNCH
    return check_launch("q8_gemm_kernel");
}

// fp32 activations (EXACT): eight waves in two depth groups (the even and the odd block of each stage)
template <int BM, int BN>
int launch_f32_tile(GemmParams p, bool w4, hipStream_t stream) {
    p.tiles_m = (p.m + BM - 1) / BM;
    p.tiles_n = (p.n + BN - 1) / BN;
    const dim3 grid(p.tiles_m * p.tiles_n), block(2 * kThreads);
    if (w4 && p.x_aligned)
        hipLaunchKernelGGL((q8_gemm_kernel<BM, BN, XT_F32, MODE_EXACT, true, 2 * kThreads, 2, true>), grid, block, 0, stream, p);
    else if (w4)
        hipLaunchKernelGGL((q8_gemm_kernel<BM, BN, XT_F32, MODE_EXACT, true, 2 * kThreads, 2>), grid, block, 0, stream, p);
    else
        hipLaunchKernelGGL((q8_gemm_kernel<BM, BN, XT_F32, MODE_EXACT, false, 2 * kThreads, 2>), grid, block, 0, stream, p);
    return check_launch("q8_gemm_kernel");
}

// Tile choice: one workgroup per CU fits in LDS, so a launch runs in ceil(tiles / 256) rounds on the 256 CUs; pick
// the tile with the smallest rounds * tile area / efficiency (the per-CU critical path). `eff` is the tile's measured
// throughput relative to the 256 x 128 eight-wave tile on a large GEMM (4096 x 6144 x 1536).
struct TileChoice {
    int bm, bn;
    float eff;
};

TileChoice choose_tile(int m, int n, const TileChoice* cands, int count) {
    constexpr long kCUs = 256;
    TileChoice best = cands[0];
    float best_cost = -1.0f;
    for (int i = 0; i < count; ++i) {
        const long tiles = (long)((m + cands[i].bm - 1) / cands[i].bm) * ((n + cands[i].bn - 1) / cands[i].bn);
        const float cost = (float)((tiles + kCUs - 1) / kCUs * cands[i].bm * cands[i].bn) / cands[i].eff;
        if (best_cost < 0.0f || cost < best_cost) {
            best = cands[i];
            best_cost = cost;
        }
    }
    return best;
}

int launch_16bit(GemmParams p, int xt, int mode, bool w4, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    if (xt == XT_F32) {
        static const TileChoice cands[] = {{128, 128, 1.0f}, {128, 64, 1.0f}, {64, 64, 0.75f}};
        const TileChoice t = choose_tile(p.m, p.n, cands, 3);
        if (t.bn == 128) return launch_f32_tile<128, 128>(p, w4, stream);
        if (t.bm == 128) return launch_f32_tile<128, 64>(p, w4, stream);
        return launch_f32_tile<64, 64>(p, w4, stream);
    }
    static const TileChoice cands[] = {{256, 128, 1.0f}, {128, 128, 0.5f}, {128, 64, 0.6f}};
    const TileChoice t = choose_tile(p.m, p.n, cands, 3);
    if (p.w_tiled) {
        if (!wide_eligible(p, xt, mode))
            return fail(IDOLQ_EINVAL, "tiled weights need bf16/fp16 activations with 16-byte aligned rows and 16-byte "
                                      "aligned weights");
        return launch_wide(p, xt, workspace, workspace_bytes, stream);
    }
    if (t.bm == 256 && pipe_eligible(p, xt, mode)) return launch_pipe(p, xt, stream);
    if (t.bm == 256) return launch_16bit_tile<256, 128, 512>(p, xt, mode, w4, stream);
    if (t.bn == 128) return launch_16bit_tile<128, 128, kThreads>(p, xt, mode, w4, stream);
    return launch_16bit_tile<128, 64, kThreads>(p, xt, mode, w4, stream);
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

// Quantizes activations for the int8 path (q8_aux.hip); the tiled variant writes the layout of the tiled INT8 GEMM.
int quantize_act_launch(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, int8_t* qa, float* scale,
                        int32_t* qsum, hipStream_t stream);
int quantize_act_tiled_launch(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, int8_t* qa, float* scale,
                              int* zero, int nzero, hipStream_t stream);
// Splits activations into bf16 high and low parts for the EXACT mode on tiled weights (q8_aux.hip).
int split_bf16_launch(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, uint16_t* hi, uint16_t* lo,
                      int* zero, int nzero, hipStream_t stream);

// INT8 scratch: the activation codes (m x k bytes), then the scales (m x k / 32 fp32, 16 bytes of padding), each
// rounded up to 256 bytes; the tiled path may use the rest as the stream-K workspace.
size_t int8_prefix_bytes(int64_t m, int64_t k) {
    const size_t qa = ((size_t)m * (size_t)k + 255) / 256 * 256;
    const size_t sa = ((size_t)m * (size_t)(k / kQ8Block) * sizeof(float) + 16 + 255) / 256 * 256;
    return qa + sa;
}

// Scratch of the EXACT mode on tiled weights: the bf16 high parts, then the low parts (m x k x 2 bytes each, rounded
// up to 256 bytes); the rest may be the stream-K workspace.
size_t exact_prefix_bytes(int64_t m, int64_t k) { return 2 * (((size_t)m * (size_t)k * 2 + 255) / 256 * 256); }

}  // namespace idolq

using namespace idolq;

extern "C" size_t idolq_q8_0_gemm_workspace(int64_t m, int64_t k, int mode) {
    if (mode == IDOLQ_MODE_DEQUANT) return wide_workspace_bytes();
    if (m <= 0 || k <= 0 || k % kQ8Block) return 0;
    // EXACT: the scratch of the tiled path (the row-major EXACT kernel needs none), INT8: the scratch of either
    // path; each plus the stream-K workspace the tiled path can use after it
    if (mode == IDOLQ_MODE_EXACT) return exact_prefix_bytes(m, k) + wide_workspace_bytes();
    if (mode != IDOLQ_MODE_INT8) return 0;
    return int8_prefix_bytes(m, k) + wide_workspace_bytes();
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
    if (act < IDOLQ_ACT_NONE || act > IDOLQ_ACT_SILU) return fail(IDOLQ_EINVAL, "unknown activation");
    if (residual == y && residual && (residual_dtype != y_dtype || ldr != ldy))
        return fail(IDOLQ_EINVAL, "a residual that aliases y must have y's dtype and stride");
    if ((reinterpret_cast<uintptr_t>(w) & 1) != 0) return fail(IDOLQ_EINVAL, "Q8_0 weights must be 2-byte aligned");
    // the kernels address activations and weights with 32-bit element / byte offsets
    if (m * ldx >= (int64_t)UINT32_MAX || n * (k / kQ8Block) * kQ8Bytes >= (int64_t)UINT32_MAX)
        return fail(IDOLQ_EINVAL, "x or the weight window exceeds 2^32 elements / bytes");
    if (mode == IDOLQ_MODE_AUTO) mode = x_dtype == IDOLQ_F32 ? IDOLQ_MODE_EXACT : IDOLQ_MODE_DEQUANT;
    if (mode < IDOLQ_MODE_DEQUANT || mode > IDOLQ_MODE_INT8) return fail(IDOLQ_EINVAL, "unknown GEMM mode");
    if (mode == IDOLQ_MODE_DEQUANT && x_dtype == IDOLQ_F32)
        return fail(IDOLQ_EINVAL, "DEQUANT mode takes bf16 or fp16 activations");
    const bool tiled = (flags & IDOLQ_FLAG_TILED_WEIGHTS) != 0;
    if (tiled && (k % 64 || n_offset % 32))
        return fail(IDOLQ_EINVAL, "tiled weights need k a multiple of 64 and n_offset a multiple of 32");
    if (m == 0 || n == 0) return IDOLQ_OK;  // empty input: nothing to read or write (pointers may be null)
    if (!x || !w || !y) return fail(IDOLQ_EINVAL, "x, w and y must be non-null");
    hipStream_t s = static_cast<hipStream_t>(stream);

    GemmParams p{};
    p.x = x;
    p.ldx = ldx;
    p.row_bytes = (k / kQ8Block) * kQ8Bytes;
    p.w = tiled ? w + (n_offset / 32) * (k / 64) * 2176 : w + n_offset * p.row_bytes;
    p.w_tiled = tiled ? 1 : 0;
    p.groups = tiled ? (int)((n_total + 31) / 32 - n_offset / 32) : 0;
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
    const size_t ysz = dtype_size(y_dtype), rsz = residual ? dtype_size(residual_dtype) : 0;
    p.y_vec = reinterpret_cast<uintptr_t>(y) % 16 == 0 && ((size_t)ldy * ysz) % 16 == 0 &&
              (!residual || (reinterpret_cast<uintptr_t>(residual) % 16 == 0 && ((size_t)ldr * rsz) % 16 == 0));

    if (mode == IDOLQ_MODE_INT8) {
        // at least the codes and scales; beyond them the tiled path may split tiles over the CUs
        const size_t need = int8_prefix_bytes(m, k);
        if (!workspace || workspace_bytes < need)
            return fail(IDOLQ_EINVAL, "INT8 mode needs a workspace of idolq_q8_0_gemm_workspace() bytes");
        if (reinterpret_cast<uintptr_t>(workspace) % 16 != 0) return fail(IDOLQ_EINVAL, "workspace must be 16-byte aligned");
        int8_t* qa = static_cast<int8_t*>(workspace);
        float* sa = reinterpret_cast<float*>(static_cast<char*>(workspace) + ((size_t)m * (size_t)k + 255) / 256 * 256);
        if (tiled) {
            const size_t xsz = dtype_size(x_dtype);
            if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || ((size_t)ldx * xsz) % 16 != 0 ||
                (reinterpret_cast<uintptr_t>(w) & 15) != 0)
                return fail(IDOLQ_EINVAL, "the tiled INT8 GEMM needs 16-byte aligned activation rows and weights");
            if (p.groups <= 0) return fail(IDOLQ_EINVAL, "tiled weights: n_total exceeds the layout");
            // the stream-K workspace after the scratch: its tile counters are cleared by the quantizer (the caller's
            // workspace need not be zero)
            char* rest = static_cast<char*>(workspace) + need;
            const bool has_rest = workspace_bytes >= need + wide_workspace_bytes();
            int rc = quantize_act_tiled_launch(x, x_dtype, m, k, ldx, qa, sa, has_rest ? reinterpret_cast<int*>(rest) : nullptr,
                                               has_rest ? (int)(kWideCountBytes / sizeof(int)) : 0, s);
            if (rc) return rc;
            p.qa = qa;
            p.sa = sa;
            return launch_wide_i8(p, has_rest ? rest : nullptr, has_rest ? workspace_bytes - need : 0, s);
        }
        int rc = quantize_act_launch(x, x_dtype, m, k, ldx, qa, sa, nullptr, s);
        if (rc) return rc;
        p.qa = qa;
        p.sa = sa;
        return launch_int8<128, 128, false>(p, w4, s);
    }
    if (mode == IDOLQ_MODE_EXACT && tiled) {
        // x -> bf16 high and low parts (x - hi rounded to bf16) in the scratch, then two bf16 products per block
        const size_t need = exact_prefix_bytes(m, k);
        if (!workspace || workspace_bytes < need)
            return fail(IDOLQ_EINVAL, "EXACT mode on tiled weights needs a workspace of idolq_q8_0_gemm_workspace() bytes");
        if (reinterpret_cast<uintptr_t>(workspace) % 16 != 0) return fail(IDOLQ_EINVAL, "workspace must be 16-byte aligned");
        const size_t xsz = dtype_size(x_dtype);
        if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || ((size_t)ldx * xsz) % 16 != 0 || (reinterpret_cast<uintptr_t>(w) & 15) != 0)
            return fail(IDOLQ_EINVAL, "the tiled EXACT GEMM needs 16-byte aligned activation rows and weights");
        if (p.groups <= 0) return fail(IDOLQ_EINVAL, "tiled weights: n_total exceeds the layout");
        // the fold kernel addresses the high and low parts (row stride k, 2 bytes each) and the weight groups with
        // 32-bit byte offsets
        if (m * k * 2 >= (int64_t)UINT32_MAX || (int64_t)p.groups * (k / 64) * 2176 >= (int64_t)UINT32_MAX)
            return fail(IDOLQ_EINVAL, "the tiled EXACT GEMM needs m * k * 2 and the weight layout below 2^32 bytes");
        uint16_t* hi = static_cast<uint16_t*>(workspace);
        uint16_t* lo = reinterpret_cast<uint16_t*>(static_cast<char*>(workspace) + need / 2);
        char* rest = static_cast<char*>(workspace) + need;
        const bool has_rest = workspace_bytes >= need + wide_workspace_bytes();
        int rc = split_bf16_launch(x, x_dtype, m, k, ldx, hi, lo, has_rest ? reinterpret_cast<int*>(rest) : nullptr,
                                   has_rest ? (int)(kWideCountBytes / sizeof(int)) : 0, s);
        if (rc) return rc;
        p.x = hi;
        p.x_lo = lo;
        p.ldx = k;
        p.x_aligned = true;
        return launch_wide_exact(p, has_rest ? rest : nullptr, has_rest ? workspace_bytes - need : 0, s);
    }
    const int xt = x_dtype == IDOLQ_BF16 ? XT_BF16 : x_dtype == IDOLQ_F16 ? XT_F16 : XT_F32;
    const int kmode = mode == IDOLQ_MODE_DEQUANT ? MODE_DEQUANT : MODE_EXACT;
    if (gemv_eligible(p, xt, kmode)) return launch_gemv(p, xt, kmode, s);
    return launch_16bit(p, xt, kmode, w4, workspace, workspace_bytes, s);
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

// ------------------------------------------------------------------------------------------------ no-allocation GEMM
// idolq_q8_0_gemm_noalloc takes its scratch (the INT8 mode's quantized activations and scales) from this array. Each
// device holds its own copy for the life of the process; host code reaches it only through the address
// hipGetSymbolAddress returns on that device (kept in noalloc_scratch below), never through the array's name.
namespace {

constexpr size_t kNoAllocScratchBytes = (size_t)32 << 20;
__device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;

// The device address of `scratch` on the current device, looked up once per device (with that device current).
void* noalloc_scratch(int* rc) {
    static std::mutex mu;
    static void* addr[kMaxDevices] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        *rc = fail(IDOLQ_ELAUNCH, "no current HIP device (or more than 64 devices)");
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[dev]) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) {
            *rc = fail(IDOLQ_ELAUNCH, std::string("hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(e));
            return nullptr;
        }
        addr[dev] = ptr;
    }
    *rc = IDOLQ_OK;
    return addr[dev];
}

}  // namespace

extern "C" size_t idolq_q8_0_gemm_noalloc_max_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int idolq_q8_0_gemm_noalloc(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const uint8_t* w,
                                       int64_t n_total, int64_t n_offset, int64_t n, const void* bias, int bias_dtype,
                                       const void* residual, int residual_dtype, int64_t ldr, int act, int mode,
                                       int flags, void* y, int y_dtype, int64_t ldy, void* stream) {
    const int eff = mode == IDOLQ_MODE_AUTO ? (x_dtype == IDOLQ_F32 ? IDOLQ_MODE_EXACT : IDOLQ_MODE_DEQUANT) : mode;
    const bool tiled = (flags & IDOLQ_FLAG_TILED_WEIGHTS) != 0;
    if (!(eff == IDOLQ_MODE_INT8 || (eff == IDOLQ_MODE_EXACT && tiled)) || m <= 0 || n <= 0 || k <= 0 || k % kQ8Block)
        // DEQUANT without a workspace runs whole tiles and row-major EXACT needs none: nothing to take from the
        // scratch (the GEMM's own checks handle bad shapes and empty inputs)
        return idolq_q8_0_gemm(x, x_dtype, m, k, ldx, w, n_total, n_offset, n, bias, bias_dtype, residual,
                               residual_dtype, ldr, act, mode, flags, y, y_dtype, ldy, nullptr, 0, stream);
    // INT8: the codes and scales, EXACT on tiled weights: the high and low parts (tiled weights then run whole tiles)
    const size_t need = eff == IDOLQ_MODE_INT8 ? int8_prefix_bytes(m, k) : exact_prefix_bytes(m, k);
    if (need > kNoAllocScratchBytes)
        return fail(IDOLQ_EINVAL, std::string(eff == IDOLQ_MODE_INT8 ? "INT8" : "EXACT") + " GEMM of m x k = " +
                                      std::to_string(m) + " x " + std::to_string(k) + " needs " + std::to_string(need) +
                                      " bytes of scratch; idolq_q8_0_gemm_noalloc holds " +
                                      std::to_string(kNoAllocScratchBytes) +
                                      " (INT8: m * k * 9 / 8 bytes at most, EXACT on tiled weights: m * k * 4)");
    int rc = IDOLQ_OK;
    void* ptr = noalloc_scratch(&rc);
    if (!ptr) return rc;
    // exactly the scratch: no stream-K room, so every call runs whole tiles
    return idolq_q8_0_gemm(x, x_dtype, m, k, ldx, w, n_total, n_offset, n, bias, bias_dtype, residual, residual_dtype,
                           ldr, act, mode, flags, y, y_dtype, ldy, ptr, need, stream);
}
