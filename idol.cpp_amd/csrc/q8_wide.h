#pragma once
// The grouped-layout Q8_0 GEMM kernel template shared by q8_gemm_wide.hip (DEQUANT and Q4_K on tiled / row-major
// weights) and q8_gemm_wide_fold.hip (INT8 and EXACT modes on tiled weights), with the launch pieces both use. Each source
// file instantiates its own kernels (internal linkage).
//
// Q8_0 GEMM for gfx950 on the grouped weight layout (idolq_q8_0_tile), DEQUANT arithmetic: y = epilogue(x * W^T),
// the MFMA operands being x (bf16 or fp16) and T(fp32(d) * q) for the Q8_0 weights, accumulated in fp32.
//
// Grouped layout. Weight rows in groups of 32 (the last group padded with zero rows), k in stages of 64 (two Q8_0
// blocks); chunk (g, s) of 2176 bytes (32 rows x 68) at byte (g * S + s) * 2176, S = k / 64:
//   [1024 b, 1024 b + 1024), b = 0, 1: the 32 codes of block b of each row in MFMA lane order: lane l's 16 bytes at
//       16 l are, for row l % 32 and h = l / 32, codes 8 h .. 8 h + 7 of the block, then codes 16 + 8 h .. 16 + 8 h + 7
//   [2048, 2176): 4 bytes per row r at 2048 + 4 r: the fp16 scale of block 0 (low half) and of block 1 (high half).
// So one 16-byte load per lane fetches a block's MFMA operands for two 16-deep MFMA steps, and every load of a wave
// reads 1 KB of contiguous bytes.
//
// Workgroup: 4 waves, one per SIMD, each owning all BM = 32 RT rows of the x tile and 32 CT weight rows (output
// columns): RT x CT tiles of v_mfma_f32_32x32x16 accumulators (the transposed product C^T = W X^T, weights as the MFMA
// rows, so accumulator element e of lane l is output row l % 32 and output column 8 (e / 4) + 4 (l / 32) + e % 4: four
// consecutive columns per lane, stored as one vector). Tile BM x BN, BN = 128 CT. With RT = 8, CT = 2 a wave reads
// 256 + 64 operand rows from LDS per 16 MFMAs: half the LDS bytes per MFMA of a 64 x 64 wave tile, which is what keeps
// the LDS port (128 bytes per clock per CU) below the MFMA rate.
//
// Stage s covers k [64 s, 64 s + 64). Global memory reaches LDS without passing through registers
// (global_load_lds_dwordx4):
//   activations: BM rows x 128 bytes into one of three buffers, the eight 16-byte chunks of row r stored at chunk
//       position c ^ ((r >> 1) & 7) (conflict-free MFMA operand reads); each wave loads a quarter of the rows;
//   weights: each wave loads only its own CT groups (CT x 2 KB of codes + CT x 128 bytes of scales) into its own
//       region of one of three buffers; no other wave reads them, so they need no barrier.
// Each wave converts its weight codes in registers (T(fp32(d) * q), one MFMA step ahead) and reads its x operands
// from LDS one MFMA step ahead. Stage s:
//   issue weight loads of stage s + 2;
//   steps 0..2: 16 MFMAs each, interleaved with the next step's x reads and weight conversion;
//   wait until this wave's weight loads of stage s + 1 (and everything issued before them, which includes its
//   activation loads of stage s + 1) have landed; barrier (every wave's share of activations s + 1 is in LDS and every
//   wave has finished reading activation buffer s % 3); issue activation loads of stage s + 3 into buffer s % 3;
//   step 3: 16 MFMAs, interleaved with the reads of stage s + 1's first x operands and weight bytes, then the
//   conversion of its first weight operands.
// Loads complete in issue order (A = activation loads of a stage, W = weight loads):
//   prologue A0 W0 A1 W1 A2, then stage s issues W(s + 2) and A(s + 3),
// so at the wait of stage s the loads issued after W(s + 1) are A(s + 2) and W(s + 2). Rows of x beyond m and weight
// groups beyond the layout read the last valid row / group (they only feed outputs that are never stored).
#include "q8_dma.h"

#include <algorithm>
#include <numeric>
#include <cstdlib>
#include <string>
#include <type_traits>
#include <utility>

namespace idolq {
namespace {


constexpr int kGroupBytes = 2176;  // one group (32 rows) x one stage (64 k)
constexpr int kWideThreads = 256;  // 4 waves

// Stream-K. The first dp tiles (a multiple of the G workgroups) are taken whole, round-robin. The k stages of the
// other tiles, in tile-major order, are split into G contiguous ranges of L (the first R ranges L + 1) stages, one per
// workgroup. A tile whose stages fall into several ranges is finished by the part that arrives last: a part that
// finds the others already counted keeps its sum in registers; otherwise it stores its fp32 partial tile in its slot
// of `part` (device-coherent stores) and counts itself in count[first range of the tile]. The part that sees the
// count complete sums the parts in range order, left to right, its own registers taking its range's place (so the
// result is the same whichever part finishes), runs the epilogue and clears the count for the next launch. Nobody
// waits for anybody, so the workgroups need not be resident together.
struct WideSplit {
    int G;        // workgroups
    int dp;       // tiles taken whole
    int L, R;     // stream-K ranges over the remaining tiles' stages; null part: whole tiles only
    float* part;  // 2 G partial tiles: slot 2 r + f holds range r's first (f = 0) or last (f = 1) part
    int* count;   // G counters, zero between launches (the workspace's first bytes)
    // Order of the split tiles. Ranges whose starts differ by a multiple of the tile depth run at the same k offset
    // (with all ranges of L stages, ranges r and r + S / gcd(L, S) are ph = L / gcd(L, S) tiles apart): split tile
    // tl is walked as tile (tl % ph) * (nsplit / ph) + tl / ph, so that the in-phase ranges of one XCD take
    // neighbouring tiles, in groups of gh row tiles walked column by column (gh = 4: blocks of 4 x 2 tiles), and read
    // the same activation and weight rows at the same time (0 / 1: tiles in range order, groups of 8).
    int ph, gh;
};

// Q4K: the weights are GGUF Q4_K super-blocks, row-major (one row: k / 256 blocks of 144 bytes: fp16 d, fp16 dmin,
// 12 bytes of 6-bit scales and minimums, 128 bytes of nibbles); a 64-deep stage is the 32-groups 2 j and 2 j + 1 of a
// super-block (j = stage % 4), whose codes are the low and the high nibbles of the same 32 bytes 16 + 32 j .. of the
// block. Per 32-row group and stage a wave loads those 32 bytes of each row (1 KB, lane l: row l % 32, bytes
// 16 (l / 32) .. + 15) and the rows' 16-byte headers (512 bytes), straight from the row-major bytes.
// FOLD: 0 (DEQUANT: one accumulation over the whole depth), kFoldI8 (the INT8 mode: a stage of activations is BM
// rows x 64 int8 codes, then the rows' two fp32 block scales), kFoldExact (the EXACT mode: BM rows x 64 bf16 high
// parts, then BM rows x 64 bf16 low parts of fp32 activations).
constexpr int kFoldI8 = 1, kFoldExact = 2;
// workgroups per CU of each mode's kernel (its launch bounds; the INT8 fold runs two, see q8_gemm_wide_fold.hip)
template <int FOLD>
constexpr int kWideFoldSlots = FOLD == kFoldI8 ? 2 : 1;
template <int RT, int CT, bool Q4K = false, int FOLD = 0>
struct WideCfg {
    static constexpr bool I8 = FOLD == kFoldI8, EX = FOLD == kFoldExact;
    static constexpr int BM = 32 * RT, BN = 128 * CT;
    // one stage of activations: BM rows x 64 16-bit values
    static constexpr int ABuf = I8 ? BM * 72 : EX ? BM * 256 : BM * 128;
    static constexpr int WCode = Q4K ? 1024 : 2048;  // one 32-row group's codes per stage
    static constexpr int WScale = Q4K ? 512 : 128;   // and its scales (Q4_K: the super-block headers)
    static constexpr int WWave = CT * (WCode + WScale);  // one stage of one wave's weight groups: codes, then scales
    static constexpr int WBuf = 4 * WWave;
    static constexpr int WBase = 3 * ABuf;
    static constexpr int Lds = WBase + 3 * WBuf;
    // activation loads per wave per stage: 1 KB each; I8: BM / 64 of 1 KB and one of the rows' scales (256 bytes);
    // EX: BM / 32 of the high parts, then as many of the low parts
    static constexpr int DA = I8 ? BM / 64 + 1 : EX ? BM / 16 : BM / 32;
    static constexpr int DW = Q4K ? 2 * CT : 2 * CT + 1;  // weight loads per wave per stage
    static_assert(Lds <= 163840, "LDS budget");
};

// (d * sc, dmin * m) of the 32-groups 2 pair and 2 pair + 1 of a Q4_K super-block from its 16-byte header (bytes 0-1
// d, 2-3 dmin, 4-15 the 6-bit scales and minimums s[0..11]): for group j < 4, sc = s[j] & 63, m = s[4 + j] & 63; for
// j >= 4, sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4), m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4). The products are
// exact in fp32 (11-bit by 6-bit).
__device__ __forceinline__ void q4k_header(uint4 hd, int pair, float (&ab)[4]) {
    const float d = half_bits_to_float((uint16_t)(hd.x & 0xffff)), dmin = half_bits_to_float((uint16_t)(hd.x >> 16));
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int j = 2 * pair + t;
        uint32_t sc, mn;
        if (j < 4) {
            sc = (hd.y >> (8 * j)) & 63;
            mn = (hd.z >> (8 * j)) & 63;
        } else {
            const int jj = j - 4;
            const uint32_t c = (hd.w >> (8 * jj)) & 0xff;
            sc = (c & 15) | (((hd.y >> (8 * jj + 6)) & 3) << 4);
            mn = (c >> 4) | (((hd.z >> (8 * jj + 6)) & 3) << 4);
        }
        ab[2 * t] = d * (float)sc;
        ab[2 * t + 1] = dmin * (float)mn;
    }
}

// The tiles of one launch shape (RT, CT), with this workgroup's share of them; smem: the kernel's LDS (C::Lds bytes).
// FAST selects the register epilogue (activation ACT, a residual iff RES), otherwise the general one.
// FOLD: the INT8 or EXACT mode (see run_segment_fold); T then only names the output type of the register epilogue.
template <typename T, int RT, int CT, int ACT, bool FAST, bool RES, bool SPLIT, bool Q4K, int FOLD = 0>
__device__ __forceinline__ void wide_tiles(const GemmParams& p, const WideSplit& sp, char* smem) {
    typedef WideCfg<RT, CT, Q4K, FOLD> C;
    constexpr bool I8 = C::I8, EX = C::EX;
    typedef typename PipeMfma<T>::vec Vec;
    typedef typename PipeMfma<T>::pair T2;
    constexpr int DA = C::DA, DW = C::DW;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int S = p.k / 64;  // stages of the whole depth
    const int64_t gstride = (int64_t)S * kGroupBytes;
    const uint32_t lds0 = (uint32_t)(size_t)(lds_char*)smem;
    const char* xg;  // activations and weights of the segment's first stage
    const char* wg;
    const char* sag = nullptr;  // I8: the activation scales of the segment's first stage; EX: the low parts

    // ---- per-tile load offsets (bytes, 32-bit)
    // activations: load j of this wave fills LDS 16-byte chunks u = 64 (DA wave + j) + lane of the stage buffer:
    // row u / 8, position u % 8, holding chunk (u % 8) ^ ((row >> 1) & 7) of the row
    uint32_t a_off[DA], w_off[CT], ws_off, wh_off[CT];
    int seg_k0 = 0;  // Q4K: the segment's first stage (the stage's super-block and 32-group pair follow from it)
    auto start_tile = [&](int m0, int n0, int k0) __attribute__((always_inline)) {
        wg = uniform_ptr(reinterpret_cast<const char*>(p.w) + (Q4K ? 0 : (size_t)k0 * kGroupBytes));
        seg_k0 = k0;
        if constexpr (I8) {
            // codes: row stride k bytes, stage s at byte 64 s; LDS chunk u = 64 (DA' wave + j) + lane (DA' = DA - 1)
            // is row u / 4, position u % 4, holding chunk (u % 4) ^ ((row >> 2) & 3) of the row's 64 bytes
            xg = uniform_ptr(reinterpret_cast<const char*>(p.qa) + (size_t)k0 * 64);
            sag = uniform_ptr(reinterpret_cast<const char*>(p.sa) + (size_t)k0 * p.m * 8);
#pragma unroll
            for (int j = 0; j < DA - 1; ++j) {
                const int u = (wave * (DA - 1) + j) * 64 + lane, row = u >> 2, c = (u & 3) ^ ((row >> 2) & 3);
                a_off[j] = (uint32_t)((int64_t)min(m0 + row, p.m - 1) * p.k + c * 16);
            }
            // scales (stage-major: the stage's (block 2 s, 2 s + 1) pair of row r at 8 r): lane l < 16 of wave w takes
            // rows 32 w + 2 l and + 1 with one 16-byte load from the first; rows from m on read row m - 1's bytes
            // onward (the scale buffer is padded by 16 bytes), feeding only outputs that are never stored
            a_off[DA - 1] = (uint32_t)min(m0 + 32 * wave + 2 * lane, p.m - 1) * 8u;
        } else {
            // EX: the low parts share the high parts' layout (row stride k), so their loads use the same offsets
            constexpr int DX = EX ? DA / 2 : DA;
            xg = uniform_ptr(static_cast<const char*>(p.x) + (size_t)k0 * 128);
            if constexpr (EX) sag = uniform_ptr(static_cast<const char*>(p.x_lo) + (size_t)k0 * 128);
#pragma unroll
            for (int j = 0; j < DX; ++j) {
                const int u = (wave * DX + j) * 64 + lane, row = u >> 3, c = (u & 7) ^ ((row >> 1) & 7);
                a_off[j] = (uint32_t)((int64_t)min(m0 + row, p.m - 1) * p.ldx * 2 + c * 16);
            }
        }
        if constexpr (Q4K) {
            // rows past the window read its last row (their outputs are never stored)
#pragma unroll
            for (int c = 0; c < CT; ++c) {
                const int row0 = n0 + 32 * (wave * CT + c);
                w_off[c] = (uint32_t)((int64_t)min(row0 + (lane & 31), p.groups - 1) * p.row_bytes + 16 * (lane >> 5));
                wh_off[c] = (uint32_t)((int64_t)min(row0 + (lane & 31), p.groups - 1) * p.row_bytes);
            }
        } else {
            const int g0 = n0 / 32 + wave * CT;
#pragma unroll
            for (int c = 0; c < CT; ++c) w_off[c] = (uint32_t)(min(g0 + c, p.groups - 1) * gstride + 16 * lane);
            // scales: lanes 8 c .. 8 c + 7 fetch the 128 bytes of group c
            ws_off = (uint32_t)(min(g0 + min(lane >> 3, CT - 1), p.groups - 1) * gstride + 2048 + 16 * (lane & 7));
        }
    };
    // load j < DA of this wave's share of activation stage s
    auto issue_a_piece = [&](int s, int j) __attribute__((always_inline)) {
        if constexpr (I8) {
            if (j < DA - 1)
                lds_dma16(xg + (size_t)s * 64, a_off[j], lds0 + (s % 3) * C::ABuf + (wave * (DA - 1) + j) * 1024);
            else if (lane < 16)
                lds_dma16(sag + (size_t)s * p.m * 8, a_off[j], lds0 + (s % 3) * C::ABuf + C::BM * 64 + wave * 256);
        } else if constexpr (EX) {
            constexpr int DX = DA / 2;
            if (j < DX)
                lds_dma16(xg + (size_t)s * 128, a_off[j], lds0 + (s % 3) * C::ABuf + (wave * DX + j) * 1024);
            else
                lds_dma16(sag + (size_t)s * 128, a_off[j - DX], lds0 + (s % 3) * C::ABuf + C::BM * 128 + (wave * DX + j - DX) * 1024);
        } else {
            lds_dma16(xg + (size_t)s * 128, a_off[j], lds0 + (s % 3) * C::ABuf + (wave * DA + j) * 1024);
        }
    };
    auto issue_a = [&](int s) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < DA; ++j) issue_a_piece(s, j);
    };
    // load i < DW of this wave's weight stage s: block i % 2 of group i / 2, then (i = 2 CT) the scales
    auto issue_w_piece = [&](int s, int i) __attribute__((always_inline)) {
        const uint32_t dst = lds0 + C::WBase + (s % 3) * C::WBuf + wave * C::WWave;
        if constexpr (Q4K) {
            // stage seg_k0 + s: super-block (seg_k0 + s) / 4, nibble bytes 16 + 32 ((seg_k0 + s) % 4) .. + 31
            const int as = seg_k0 + s;
            const char* sb = wg + (size_t)(as >> 2) * 144;
            if (i < CT)
                lds_dma16(sb + 16 + 32 * (as & 3), w_off[i], dst + i * 1024);
            else if (lane < 32)
                lds_dma16(sb, wh_off[i - CT], dst + CT * 1024 + (i - CT) * 512);
        } else {
            const char* base = wg + (size_t)s * kGroupBytes;
            if (i < 2 * CT)
                lds_dma16(base + (i & 1) * 1024, w_off[i >> 1], dst + (i >> 1) * 2048 + (i & 1) * 1024);
            else if (lane < 8 * CT)
                lds_dma16(base, ws_off, dst + CT * 2048);
        }
    };
    auto issue_w = [&](int s) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < DW; ++i) issue_w_piece(s, i);
    };

    // ---- MFMA operands
    // x (MFMA columns): output row 32 rt + lane % 32, k = 16 j + 8 (lane / 32) .. + 7: chunk 2 j + lane / 32 of the row
    uint32_t x_lane[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) x_lane[j] = (lane & 31) * 128 + (((2 * j + (lane >> 5)) ^ ((lane >> 1) & 7)) * 16);
    Vec xo[2][RT];     // x operands of two steps
    uint4 wq[2][CT];   // weight operands of two steps (bits of Vec)
    uint4 rc[CT][2];   // this stage's codes: group c, block b (two MFMA steps each); Q4K: rc[c][0] only
    uint32_t rs[CT];   // this stage's scales: group c, block 0 low / block 1 high
    float rab[CT][4];  // Q4K: (d * sc, dmin * m) of the stage's two 32-groups, for group c
    f32x16 acc[RT][CT];

    auto read_x1 = [&](int buf, int j, int set, int rt) __attribute__((always_inline)) {
        xo[set][rt] = *reinterpret_cast<const Vec*>(smem + buf * C::ABuf + x_lane[j] + rt * 4096);
    };
    // piece c < CT: the codes of group c; piece CT: the scales of every group
    // stage: the segment stage whose bytes buffer buf holds (Q4K: its 32-group pair is (seg_k0 + stage) % 4)
    auto read_raw_piece = [&](int buf, int c, int stage) __attribute__((always_inline)) {
        const char* wb = smem + C::WBase + buf * C::WBuf + wave * C::WWave;
        if constexpr (Q4K) {
            if (c < CT) {
                // row lane % 32: nibble bytes 8 h .. 8 h + 7 (steps 0 and 2) and 16 + 8 h .. (steps 1 and 3)
                const int r = lane & 31, h = lane >> 5;
                const uint2 lo = *reinterpret_cast<const uint2*>(wb + c * 1024 + 16 * r + 8 * h);
                const uint2 hi = *reinterpret_cast<const uint2*>(wb + c * 1024 + 16 * (32 + r) + 8 * h);
                rc[c][0] = make_uint4(lo.x, lo.y, hi.x, hi.y);
            } else {
#pragma unroll
                for (int g = 0; g < CT; ++g) {
                    const uint4 hd = *reinterpret_cast<const uint4*>(wb + CT * 1024 + g * 512 + 16 * (lane & 31));
                    q4k_header(hd, (seg_k0 + stage) & 3, rab[g]);
                }
            }
        } else {
            if (c < CT) {
#pragma unroll
                for (int b = 0; b < 2; ++b) rc[c][b] = *reinterpret_cast<const uint4*>(wb + c * 2048 + b * 1024 + 16 * lane);
            } else {
#pragma unroll
                for (int g = 0; g < CT; ++g) rs[g] = *reinterpret_cast<const uint32_t*>(wb + CT * 2048 + g * 128 + 4 * (lane & 31));
            }
        }
    };
    // piece q < 4 CT of step j's weight operands: two codes to T(fp32(d) * q) (Q4K: T(a * q - b)), dword q % 4 of
    // group q / 4's operand. Dwords 0, 1 come from the first code word of the step (x for even steps, z for odd
    // ones), dwords 2, 3 from the second (y, w); each dword is the pair of codes at bytes 2 (q % 2), 2 (q % 2) + 1.
    auto convert_piece = [&](int j, int set, int q) __attribute__((always_inline)) {
        const int c = q >> 2, e = q & 3, b = j >> 1, sh = 16 * (e & 1);
        uint32_t o;
        if constexpr (Q4K) {
            // step j: 32-group b = j / 2 of the pair (low nibbles for b = 0, high for b = 1), bytes of piece j % 2
            const uint4 w = rc[c][0];
            const uint32_t word = (j & 1) ? ((e >> 1) ? w.w : w.z) : ((e >> 1) ? w.y : w.x);
            const uint32_t nib = b ? (word >> 4) & 0x0f0f0f0fu : word & 0x0f0f0f0fu;
            const f32x2 f = {(float)((nib >> sh) & 0xff), (float)((nib >> (sh + 8)) & 0xff)};
            o = __builtin_bit_cast(uint32_t, __builtin_convertvector(f * rab[c][2 * b] - rab[c][2 * b + 1], T2));
        } else {
            const float d = half_bits_to_float((uint16_t)(rs[c] >> (16 * b)));
            const uint4 w = rc[c][b];
            const uint32_t word = (j & 1) ? ((e >> 1) ? w.w : w.z) : ((e >> 1) ? w.y : w.x);
            const f32x2 f = {(float)(int)(int8_t)(uint8_t)(word >> sh), (float)(int)(int8_t)(uint8_t)(word >> (sh + 8))};
            o = __builtin_bit_cast(uint32_t, __builtin_convertvector(f * d, T2));
        }
        if (e == 0) wq[set][c].x = o;
        else if (e == 1) wq[set][c].y = o;
        else if (e == 2) wq[set][c].z = o;
        else wq[set][c].w = o;
    };
    constexpr int NM = RT * CT;         // MFMAs per 16-deep step
    constexpr int NP = 4 * CT;          // conversion pieces per step
    // The conversion (2.5 VALU instructions per code) is spread evenly over a step's MFMA slots, so that each slot's
    // VALU work stays within the 32 cycles of its MFMA: in steps 0..2 piece q goes after MFMA PS q + PS - 1; in step 3,
    // whose pieces convert the next stage's codes read from LDS in its first slots, the pieces fill the second half
    // (FC on), PF per slot.
    constexpr int PS = NM / NP;
    constexpr int FC = NM / 2, PF = NP / (NM - FC);
    static_assert(NM % NP == 0 && NP % (NM - FC) == 0, "conversion slots");
    // One 16-deep step: MFMA i on operand set `cur`, then slot(i) -- the other work of the stage (loads, the next
    // step's LDS reads and conversion) -- each slot pinned after its MFMA by a scheduling barrier, so that this work
    // is issued while the matrix core runs the step instead of being moved next to its first use.
    auto run_step = [&](int cur, auto slot) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < NM; ++i) {
            acc[i / CT][i % CT] = PipeMfma<T>::run(__builtin_bit_cast(Vec, wq[cur][i % CT]), xo[cur][i / CT], acc[i / CT][i % CT]);
            slot(i);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // steps 0..2 of the stage in buffer buf (operands of step 0 in set 0); with ISSUE_W the weight loads of stage ws
    // go out in the first slots
    auto steps012 = [&](int buf, auto issue_w_tag, int ws) __attribute__((always_inline)) {
        run_step(0, [&](int i) __attribute__((always_inline)) {
            if constexpr (decltype(issue_w_tag)::value) {
                if (i < DW) issue_w_piece(ws, i);
            }
            if (i < RT) read_x1(buf, 1, 1, i);
            if (i % PS == PS - 1) convert_piece(1, 1, i / PS);
        });
        run_step(1, [&](int i) __attribute__((always_inline)) {
            if (i < RT) read_x1(buf, 2, 0, i);
            if (i % PS == PS - 1) convert_piece(2, 0, i / PS);
        });
        run_step(0, [&](int i) __attribute__((always_inline)) {
            if (i < RT) read_x1(buf, 3, 1, i);
            if (i % PS == PS - 1) convert_piece(3, 1, i / PS);
        });
    };
    // step 3 and the first operands of the next stage (buffers nb): its weight bytes, x operands and the conversion
    // of its first weight operands; with ISSUE_A the activation loads of stage as go out in the first slots
    auto step3_next = [&](int nb, auto issue_a_tag, int as, int next) __attribute__((always_inline)) {
        run_step(1, [&](int i) __attribute__((always_inline)) {
            if constexpr (decltype(issue_a_tag)::value) {
                if (i < DA) issue_a_piece(as, i);
            }
            if (i <= CT)
                read_raw_piece(nb, i, next);
            else if (i <= CT + RT)
                read_x1(nb, 0, 0, i - CT - 1);
            if (i >= FC) {
#pragma unroll
                for (int q = 0; q < PF; ++q) convert_piece(0, 0, (i - FC) * PF + q);
            }
        });
    };

    // ---- epilogue
    // Each wave's fp32 accumulators go through LDS, CH row tiles at a time (rows of 32 CT columns, pitch EP floats, in
    // the activation buffers, free once every wave has finished the last stage), and come back row-major: LPR lanes
    // per row, 4 columns each, so that the residual loads and the output stores move whole rows of the wave's 32 CT
    // columns (every cache line written whole) instead of 8-byte pieces of 32 rows.
    // FAST (chosen by the host): y and the residual have the activation dtype, the bias is fp32, n is a multiple of 4
    // with vector-aligned 4-column groups, and the activation is ACT; rows and 4-column groups outside y are skipped.
    // Otherwise the general path: per element bounds checks and dtype conversions.
    const bool round_first = (p.flags & IDOLQ_FLAG_ROUND_BEFORE_BIAS) != 0;
    constexpr int CH = RT >= 8 ? 2 : 1;   // row tiles per chunk
    constexpr int EP = 32 * CT + 4;       // floats per staged row (the 4-float pad spreads the 16-byte writes of 16
                                          // consecutive rows over distinct banks)
    constexpr int ER = 32 * CH;           // rows per chunk
    constexpr int LPR = 8 * CT;           // read-back lanes per row
    constexpr int RPI = 64 / LPR;         // rows per read-back instruction (CT = 3: 2 rows of 24 lanes, lanes 48..63
                                          // sit out: lane_ok)
    constexpr int NR = ER / RPI;          // read-back instructions per chunk
    static_assert(ER % RPI == 0, "read-back rows");
    constexpr int NQ = RT / CH;           // chunks
    static_assert(4 * ER * EP * 4 <= C::Lds, "epilogue staging fits in LDS");
    // chunk q of the accumulators to the wave's staging rows; the reads that follow take values other lanes wrote:
    // the wave's LDS operations run in order, and the fences keep the compiler from moving the reads above the writes
    auto stage_chunk = [&](float* st, auto qtag) __attribute__((always_inline)) {
        constexpr int q = decltype(qtag)::value;
#pragma unroll
        for (int h = 0; h < CH; ++h)
#pragma unroll
            for (int c = 0; c < CT; ++c)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const f32x16& a = acc[CH * q + h][c];
                    *reinterpret_cast<float4*>(st + (32 * h + (lane & 31)) * EP + 32 * c + 8 * g + 4 * (lane >> 5)) =
                        make_float4(a[4 * g], a[4 * g + 1], a[4 * g + 2], a[4 * g + 3]);
                }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    // Without a residual (FAST), chunk q is staged finished: each accumulator rounded to T (when asked), plus its
    // column's bias (bacc[c][g]: the 4 columns 32 c + 8 g + 4 (lane / 32) .. of the wave's range), through the
    // activation -- the operations and order of the read-back path below, applied to a whole chunk's outputs at once
    // so that their vector work (tanh-GELU: an exp2 and a reciprocal per output) is not interleaved with the output
    // stores; the read-back then only converts to T.
    auto stage_chunk_act = [&](float* st, auto qtag, const f32x4 (&bacc)[CT][4]) __attribute__((always_inline)) {
        constexpr int q = decltype(qtag)::value;
#pragma unroll
        for (int h = 0; h < CH; ++h)
#pragma unroll
            for (int c = 0; c < CT; ++c)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const f32x16& a = acc[CH * q + h][c];
                    f32x2 lo = {a[4 * g], a[4 * g + 1]}, hi = {a[4 * g + 2], a[4 * g + 3]};
                    if (round_first) {
                        lo = __builtin_convertvector(__builtin_convertvector(lo, T2), f32x2);
                        hi = __builtin_convertvector(__builtin_convertvector(hi, T2), f32x2);
                    }
                    lo = lo + f32x2{bacc[c][g][0], bacc[c][g][1]};
                    hi = hi + f32x2{bacc[c][g][2], bacc[c][g][3]};
                    lo = f32x2{act_fast<ACT>(lo.x), act_fast<ACT>(lo.y)};
                    hi = f32x2{act_fast<ACT>(hi.x), act_fast<ACT>(hi.y)};
                    *reinterpret_cast<float4*>(st + (32 * h + (lane & 31)) * EP + 32 * c + 8 * g + 4 * (lane >> 5)) =
                        make_float4(lo.x, lo.y, hi.x, hi.y);
                }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    auto chunk_done = [&]() __attribute__((always_inline)) {  // the next chunk reuses the staging rows just read
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    auto fast_epilogue = [&](int m0, int n0) __attribute__((always_inline)) {
        float* const st = reinterpret_cast<float*>(smem) + wave * ER * EP;
        const int rl = lane / LPR, cl = lane % LPR;
        const int col = n0 + wave * 32 * CT + 4 * cl;
        // Every global access here is a buffer access whose offset is moved past the end of the buffer (kOff) when
        // the element is outside y: such a load reads 0 and such a store is dropped. A missing bias or residual is a
        // buffer of no bytes, so its loads read 0. The epilogue then has no branches around memory instructions,
        // and the compiler's waits cover exactly the loads an instruction uses; around a branch they fall back to
        // waiting for every earlier memory operation, the stores included, which serialized the output writes.
        // The host keeps y and the residual below 2 GB for this path (byte offsets fit in 31 bits).
        constexpr uint32_t kOff = 0x80000000u;
        constexpr int kRaw = 0x00020000;  // raw buffer, 32-bit data format
        const bool col_ok = (col < p.n) & (lane < RPI * LPR);
        const __amdgpu_buffer_rsrc_t ry = __builtin_amdgcn_make_buffer_rsrc(p.y, 0, 0x7fffffff, kRaw);
        const __amdgpu_buffer_rsrc_t rr =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.res ? p.res : p.y), 0, p.res ? 0x7fffffff : 0, kRaw);
        const __amdgpu_buffer_rsrc_t rb =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.bias ? p.bias : p.y), 0, p.bias ? 0x7fffffff : 0, kRaw);
        const f32x4 b = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rb, col_ok ? (uint32_t)col * 4 : kOff, 0, 0));
        f32x4 bacc[CT][4];  // !RES: the biases in the accumulator layout (stage_chunk_act)
        if constexpr (!RES) {
#pragma unroll
            for (int c = 0; c < CT; ++c)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int ca = n0 + wave * 32 * CT + 32 * c + 8 * g + 4 * (lane >> 5);
                    bacc[c][g] = __builtin_bit_cast(
                        f32x4, __builtin_amdgcn_raw_buffer_load_b128(rb, ca < p.n ? (uint32_t)ca * 4 : kOff, 0, 0));
                }
        }
        auto out_off = [&](int row, int64_t ld) __attribute__((always_inline)) {
            const bool ok = col_ok & (row < p.m);  // no short-circuit: a select, not a branch
            return ok ? (uint32_t)(row * (uint32_t)ld + col) * 2u : kOff;
        };
        // RES: the residual loads of the first PD chunks go out first, those of chunk q + PD before chunk q's stores;
        // PD = every chunk where the registers allow
        constexpr int PD = !RES ? 1 : NQ * NR <= 32 ? NQ : 2;
        uint2 r2[PD][NR];
        auto load_res = [&](int q) __attribute__((always_inline)) {
            if constexpr (RES) {
#pragma unroll
                for (int i = 0; i < NR; ++i) {
                    // (elements taken by index: a bit cast of an ext-vector element accessor (.y) read the wrong half)
                    const auto w = __builtin_amdgcn_raw_buffer_load_b64(rr, out_off(m0 + ER * q + RPI * i + rl, p.ldr), 0, 0);
                    r2[q % PD][i] = make_uint2(w[0], w[1]);
                }
            }
        };
#pragma unroll
        for (int q = 0; q < PD; ++q) load_res(q);
        __syncthreads();  // every wave has finished reading the activation buffers
        static_for<NQ>([&](auto qtag) __attribute__((always_inline)) {
            constexpr int q = decltype(qtag)::value;
            if (q >= 1 && q - 1 + PD < NQ) load_res(q - 1 + PD);
            if constexpr (RES)
                stage_chunk(st, qtag);
            else
                stage_chunk_act(st, qtag, bacc);
#pragma unroll
            for (int i = 0; i < NR; ++i) {
                const int lrow = RPI * i + rl, row = m0 + ER * q + lrow;
                const float4 v4 = *reinterpret_cast<const float4*>(st + lrow * EP + 4 * cl);
                f32x2 lo = {v4.x, v4.y}, hi = {v4.z, v4.w};
                if constexpr (RES) {
                    if (round_first) {
                        lo = __builtin_convertvector(__builtin_convertvector(lo, T2), f32x2);
                        hi = __builtin_convertvector(__builtin_convertvector(hi, T2), f32x2);
                    }
                    const uint2 rr2 = r2[q % PD][i];
                    lo = lo + f32x2{b[0], b[1]} + __builtin_convertvector(__builtin_bit_cast(T2, rr2.x), f32x2);
                    hi = hi + f32x2{b[2], b[3]} + __builtin_convertvector(__builtin_bit_cast(T2, rr2.y), f32x2);
                    lo = f32x2{act_fast<ACT>(lo.x), act_fast<ACT>(lo.y)};
                    hi = f32x2{act_fast<ACT>(hi.x), act_fast<ACT>(hi.y)};
                }
                const i32x2 o = {__builtin_bit_cast(int, __builtin_convertvector(lo, T2)),
                                 __builtin_bit_cast(int, __builtin_convertvector(hi, T2))};
                __builtin_amdgcn_raw_buffer_store_b64(o, ry, out_off(row, p.ldy), 0, 0);
            }
            chunk_done();
        });
    };
    auto general_epilogue = [&](int m0, int n0) __attribute__((always_inline)) {
        float* const st = reinterpret_cast<float*>(smem) + wave * ER * EP;
        const int rl = lane / LPR, cl = lane % LPR;
        const int col = n0 + wave * 32 * CT + 4 * cl;
        __syncthreads();  // every wave has finished reading the activation buffers
        static_for<NQ>([&](auto qtag) __attribute__((always_inline)) {
            constexpr int q = decltype(qtag)::value;
            stage_chunk(st, qtag);
#pragma unroll 1
            for (int i = 0; i < NR * 4; ++i) {
                const int lrow = RPI * (i >> 2) + rl, row = m0 + ER * q + lrow, cc = col + (i & 3);
                if (row < p.m && cc < p.n && lane < RPI * LPR) {
                    float x = st[lrow * EP + 4 * cl + (i & 3)];
                    if (round_first) x = round_through(p.y_dt, x);
                    if (p.bias) x += load_as_float(p.bias, p.bias_dt, cc);
                    if (p.res) x += load_as_float(p.res, p.res_dt, (int64_t)row * p.ldr + cc);
                    store_from_float(p.y, p.y_dt, (int64_t)row * p.ldy + cc, apply_act(p.act, x));
                }
            }
            chunk_done();
        });
    };
    auto epilogue = [&](int m0, int n0) __attribute__((always_inline)) {
        if constexpr (FAST)
            fast_epilogue(m0, n0);
        else
            general_epilogue(m0, n0);
    };

    // ---- I8 (the INT8 mode): the reference's integer kernel, y = sum over 32-blocks b of (sa * d) * dot_b, with dot_b
    // the exact int32 dot product of the block's int8 activation codes and weight codes. One v_mfma_i32_32x32x32_i8
    // per block and accumulator tile takes the weight codes straight from the tiled layout (a lane's 16 bytes are
    // codes 8 h .. 8 h + 7 and 16 + 8 h .. of row l % 32, h = l / 32) and the activation codes in the same order (the
    // quantizer stores each block as codes 0..7, 16..23, 8..15, 24..31, so a lane reads 16 consecutive bytes); the
    // int32 result is folded into the fp32 accumulator as fmaf(dot, sa * d, acc), block after block in k order (the
    // order and the roundings of the row-major INT8 kernel). Stage s of three LDS buffers: wait for A(s), W(s);
    // barrier; issue A(s + 2), W(s + 2) into the buffer stage s - 1 used; compute stage s. The fold (three VALU
    // instructions per accumulator element and block) bounds the kernel, not the matrix cores.
    auto compute_i8 = [&](int buf) __attribute__((always_inline)) {
        const char* ab = smem + buf * C::ABuf;
        const char* wb = smem + C::WBase + buf * C::WBuf + wave * C::WWave;
        const int half = lane >> 5;
        uint4 wc[CT][2];
        float2 sv[RT];
#pragma unroll
        for (int c = 0; c < CT; ++c)
#pragma unroll
            for (int b = 0; b < 2; ++b) wc[c][b] = *reinterpret_cast<const uint4*>(wb + c * 2048 + b * 1024 + 16 * lane);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) sv[rt] = *reinterpret_cast<const float2*>(ab + C::BM * 64 + (32 * rt + (lane & 31)) * 8);
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            i32x4 xv[RT];
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                const int row = 32 * rt + (lane & 31), chunk = (2 * b + half) ^ ((row >> 2) & 3);
                xv[rt] = *reinterpret_cast<const i32x4*>(ab + row * 64 + 16 * chunk);
            }
            // group by group (registers): the fp16 scales of block b of accumulator rows 8 q + 4 h .. + 3 (block 0 in
            // the low half of each row's dword, block 1 in the high half), as fp32, then the group's products
#pragma unroll
            for (int c = 0; c < CT; ++c) {
                float dw[16];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const uint4 r4 = *reinterpret_cast<const uint4*>(wb + CT * 2048 + c * 128 + 32 * q + 16 * half);
                    const uint32_t w4[4] = {r4.x, r4.y, r4.z, r4.w};
#pragma unroll
                    for (int j = 0; j < 4; ++j) dw[4 * q + j] = half_bits_to_float((uint16_t)(w4[j] >> (16 * b)));
                }
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) {
                    const float sa = b == 0 ? sv[rt].x : sv[rt].y;
                    i32x16 zero;
#pragma unroll
                    for (int e = 0; e < 16; ++e) zero[e] = 0;
                    const i32x16 dot = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, wc[c][b]), xv[rt],
                                                                              zero, 0, 0, 0);
#pragma unroll
                    for (int e = 0; e < 16; ++e) acc[rt][c][e] = fmaf((float)dot[e], sa * dw[e], acc[rt][c][e]);
                }
            }
        }
    };
    // ---- EX (the EXACT mode): the reference's float kernel, y = sum over 32-blocks b of d * s_b, with s_b the fp32
    // sum of the block's products of fp32 activations and exact codes. The activations come as bf16 high and low
    // parts (x = hi + lo to within 2^-16 relative); per block and accumulator tile four v_mfma_f32_32x32x16_bf16
    // (the high parts' two 16-deep steps, then the low parts') sum into a fresh fp32 tile that is folded as
    // fmaf(s, d, acc), block after block. The row-major EXACT kernel computes the same block sums and folds but
    // adds even and odd blocks in two depth groups merged at the end, so the two paths agree to fp32 reassociation.
    auto codes_bf16 = [&](uint32_t lo, uint32_t hi) __attribute__((always_inline)) {
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t word = e < 2 ? lo : hi;
            const int sh = 16 * (e & 1);
            const f32x2 f = {(float)(int)(int8_t)(uint8_t)(word >> sh), (float)(int)(int8_t)(uint8_t)(word >> (sh + 8))};
            o[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2));
        }
        return __builtin_bit_cast(bf16x8, make_uint4(o[0], o[1], o[2], o[3]));
    };
    auto compute_ex = [&](int buf) __attribute__((always_inline)) {
        const char* ab = smem + buf * C::ABuf;
        const char* wb = smem + C::WBase + buf * C::WBuf + wave * C::WWave;
        const int half = lane >> 5;
        uint4 wc[CT][2];
#pragma unroll
        for (int c = 0; c < CT; ++c)
#pragma unroll
            for (int b = 0; b < 2; ++b) wc[c][b] = *reinterpret_cast<const uint4*>(wb + c * 2048 + b * 1024 + 16 * lane);
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            // the block's codes of each group as the bf16 operands of its two 16-deep steps, and the fp16 scales of
            // the lane's accumulator rows 8 q + 4 h .. + 3 as fp32
            bf16x8 wop[CT][2];
            float dw[CT][16];
#pragma unroll
            for (int c = 0; c < CT; ++c) {
                wop[c][0] = codes_bf16(wc[c][b].x, wc[c][b].y);
                wop[c][1] = codes_bf16(wc[c][b].z, wc[c][b].w);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const uint4 r4 = *reinterpret_cast<const uint4*>(wb + CT * 2048 + c * 128 + 32 * q + 16 * half);
                    const uint32_t w4[4] = {r4.x, r4.y, r4.z, r4.w};
#pragma unroll
                    for (int j = 0; j < 4; ++j) dw[c][4 * q + j] = half_bits_to_float((uint16_t)(w4[j] >> (16 * b)));
                }
            }
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                // high and low parts of the row's k-steps 2 b and 2 b + 1 (chunk 2 step + h of the row, swizzled)
                const int row = 32 * rt + (lane & 31);
                bf16x8 xh[2], xl[2];
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) {
                    const int chunk = (2 * (2 * b + kk) + half) ^ ((row >> 1) & 7);
                    xh[kk] = *reinterpret_cast<const bf16x8*>(ab + row * 128 + 16 * chunk);
                    xl[kk] = *reinterpret_cast<const bf16x8*>(ab + C::BM * 128 + row * 128 + 16 * chunk);
                }
#pragma unroll
                for (int c = 0; c < CT; ++c) {
                    f32x16 s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wop[c][0], xh[0], f32x16{}, 0, 0, 0);
                    s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wop[c][1], xh[1], s, 0, 0, 0);
                    s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wop[c][0], xl[0], s, 0, 0, 0);
                    s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wop[c][1], xl[1], s, 0, 0, 0);
#pragma unroll
                    for (int e = 0; e < 16; ++e) acc[rt][c][e] = fmaf(s[e], dw[c][e], acc[rt][c][e]);
                }
            }
        }
    };
    // the segment's pipeline in the fold modes (INT8, EXACT)
    auto run_segment_fold = [&](int m0, int n0, int k0, int S) __attribute__((always_inline)) {
        start_tile(m0, n0, k0);
        __syncthreads();  // every wave is done with the previous segment's LDS
        issue_a(0);
        issue_w(0);
        if (S > 1) {
            issue_a(1);
            issue_w(1);
        }
#pragma unroll
        for (int i = 0; i < RT; ++i)
#pragma unroll
            for (int j = 0; j < CT; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
        for (int s = 0; s < S; ++s) {
            if (s + 1 < S)
                wait_vm<DA + DW>();  // A(s), W(s) landed: A(s + 1), W(s + 1) may remain
            else
                wait_vm<0>();
            __syncthreads();  // every wave's share of stage s is in LDS; every wave is done with stage s - 1
            if (s + 2 < S) {
                issue_a(s + 2);
                issue_w(s + 2);
            }
            if constexpr (I8)
                compute_i8(s % 3);
            else
                compute_ex(s % 3);
        }
    };

    // ---- one segment: stages k0 .. k0 + S - 1 of the tile at (m0, n0), accumulated from zero into acc
    auto run_segment = [&](int m0, int n0, int k0, int S) __attribute__((always_inline)) {
        if constexpr (I8 || EX) {
            run_segment_fold(m0, n0, k0, S);
            return;
        }
        start_tile(m0, n0, k0);
        __syncthreads();  // every wave is done with the previous segment's LDS
        issue_a(0);
        issue_w(0);
        if (S > 1) {
            issue_a(1);
            issue_w(1);
        }
        if (S > 2) issue_a(2);
#pragma unroll
        for (int i = 0; i < RT; ++i)
#pragma unroll
            for (int j = 0; j < CT; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
        // W0 (and A0 before it) landed: A1, W1, A2 may remain
        if (S > 2)
            wait_vm<2 * DA + DW>();
        else if (S > 1)
            wait_vm<DA + DW>();
        else
            wait_vm<0>();
        __syncthreads();
#pragma unroll
        for (int c = 0; c <= CT; ++c) read_raw_piece(0, c, 0);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) read_x1(0, 0, 0, rt);
#pragma unroll
        for (int q = 0; q < NP; ++q) convert_piece(0, 0, q);

        const std::true_type issue;
        const std::false_type no_issue;
        int s = 0;
        for (; s + 3 < S; ++s) {
            steps012(s % 3, issue, s + 2);
            wait_vm<DA + DW>();  // W(s + 1): A(s + 2), W(s + 2) may remain
            __syncthreads();
            step3_next((s + 1) % 3, issue, s + 3, s + 1);
        }
        if (s + 3 == S) {  // W(s + 2) is the last weight stage; no more activation loads
            steps012(s % 3, issue, s + 2);
            wait_vm<DA + DW>();
            __syncthreads();
            step3_next((s + 1) % 3, no_issue, 0, s + 1);
            ++s;
        }
        if (s + 2 == S) {  // nothing issued after W(s + 1)
            steps012(s % 3, no_issue, 0);
            wait_vm<0>();
            __syncthreads();
            step3_next((s + 1) % 3, no_issue, 0, s + 1);
            ++s;
        }
        // last stage
        steps012(s % 3, no_issue, 0);
        run_step(1, [](int) {});
        __builtin_amdgcn_sched_barrier(0);
    };
    // tile t: groups of gh row tiles walked column by column
    auto tile_at = [&](int t, int& m0, int& n0, int gh = 8) __attribute__((always_inline)) {
        const int per_group = gh * p.tiles_n, group = t / per_group, first = group * gh;
        const int gm = min(p.tiles_m - first, gh), in_group = t - group * per_group;
        m0 = __builtin_amdgcn_readfirstlane((first + in_group % gm) * C::BM);
        n0 = __builtin_amdgcn_readfirstlane((in_group / gm) * C::BN);
    };

    // ---- the workgroups on one XCD (b % 8) take consecutive tiles / ranges, so those running together share
    // activation and weight rows in that XCD's L2
    const int G = gridDim.x;
    int r = blockIdx.x;
    if (G % 8 == 0) r = (r % 8) * (G / 8) + r / 8;
    const int ntiles = p.tiles_m * p.tiles_n;
    if constexpr (!SPLIT) {
        for (int t = r; t < ntiles; t += G) {
            int m0, n0;
            tile_at(t, m0, n0);
            run_segment(m0, n0, 0, S);
            epilogue(m0, n0);
        }
    } else {
        for (int t = r; t < sp.dp; t += G) {
            int m0, n0;
            tile_at(t, m0, n0);
            run_segment(m0, n0, 0, S);
            epilogue(m0, n0);
        }
        // partial tiles: uint4 q (floats 4 (q % 4) .. of accumulator tile q / 4) of thread tid at byte
        // (q * 256 + tid) * 16 of the slot
        constexpr int kQ = RT * CT * 4;
        constexpr int kSlot = C::BM * C::BN * 4;
        const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(sp.part, 0, 2 * G * kSlot, 0x00020000);
        constexpr int kCoherent = 16;  // sc1: device scope, through to the coherence point shared by all XCDs
        const int64_t big = (int64_t)sp.R * (sp.L + 1);
        auto begin_of = [&](int c) __attribute__((always_inline)) { return (int64_t)c * sp.L + min(c, sp.R); };
        auto owner = [&](int64_t i) __attribute__((always_inline)) {
            return (int)(i < big ? i / (sp.L + 1) : sp.R + (i - big) / sp.L);
        };
        __shared__ int arrivals;
        const int64_t begin = begin_of(r), end = begin + sp.L + (r < sp.R ? 1 : 0);
        for (int64_t i = begin; i < end;) {
            const int tl = (int)(i / S), k0 = (int)(i - (int64_t)tl * S);
            const int n = (int)min((int64_t)(S - k0), end - i);
            int m0, n0;
            const int nsplit = ntiles - sp.dp;
            const int v = sp.ph > 1 ? (tl % sp.ph) * (nsplit / sp.ph) + tl / sp.ph : tl;
            tile_at(sp.dp + v, m0, n0, sp.gh > 0 ? sp.gh : 8);
            run_segment(m0, n0, k0, n);
            if (n < S) {
                const int64_t t0 = (int64_t)tl * S;
                const int first = owner(t0), last = owner(t0 + S - 1);
                if (tid == 0) arrivals = __hip_atomic_load(sp.count + first, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __syncthreads();
                bool finish = arrivals == last - first;
                __syncthreads();
                if (!finish) {
                    const int off = (2 * r + (i > begin ? 1 : 0)) * kSlot + tid * 16;
#pragma unroll
                    for (int q = 0; q < kQ; ++q) {
                        const f32x16& a = acc[(q >> 2) / CT][(q >> 2) % CT];
                        const f32x4 v = {a[4 * (q & 3)], a[4 * (q & 3) + 1], a[4 * (q & 3) + 2], a[4 * (q & 3) + 3]};
                        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, v), prs, off + q * 4096, 0, kCoherent);
                    }
                    // the stores have reached the coherence point before the count moves
                    __builtin_amdgcn_s_waitcnt(0);
                    __syncthreads();
                    if (tid == 0)
                        arrivals = __hip_atomic_fetch_add(sp.count + first, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __syncthreads();
                    finish = arrivals == last - first;
                }
                if (finish) {
                    // every other part is stored: the tile's sum is part first + part first + 1 + ... + part last,
                    // added left to right whichever part finishes (this part's own sum enters at its range's
                    // position), so the result does not depend on the order of arrival. The accumulators are taken
                    // in kH passes of kP uint4 pieces (register budget); in a pass every stored part is read with
                    // one batch of loads (one round trip per part): the parts before this one are summed into t,
                    // then this part's own pieces are added to t, then the parts after it.
                    constexpr int kH = RT >= 8 || FOLD ? 4 : 2, kP = kQ / kH;  // fold modes: within 256 VGPRs
                    auto slot_off = [&](int c) __attribute__((always_inline)) {
                        return (2 * c + (t0 > begin_of(c) ? 1 : 0)) * kSlot + tid * 16;
                    };
#pragma unroll
                    for (int hp = 0; hp < kH; ++hp) {
                        auto piece = [&](int q) __attribute__((always_inline)) -> f32x16& {
                            return acc[((hp * kP + q) >> 2) / CT][((hp * kP + q) >> 2) % CT];
                        };
                        auto load_part = [&](int c, f32x4 (&v)[kP]) __attribute__((always_inline)) {
                            const int off = slot_off(c);
#pragma unroll
                            for (int q = 0; q < kP; ++q)
                                v[q] = __builtin_bit_cast(
                                    f32x4, __builtin_amdgcn_raw_buffer_load_b128(prs, off + (hp * kP + q) * 4096, 0, kCoherent));
                        };
                        f32x4 t[kP];
                        if (first < r) {
                            load_part(first, t);
                            for (int c = first + 1; c < r; ++c) {
                                f32x4 v[kP];
                                load_part(c, v);
#pragma unroll
                                for (int q = 0; q < kP; ++q) t[q] = t[q] + v[q];
                            }
#pragma unroll
                            for (int q = 0; q < kP; ++q) {
                                f32x16& a = piece(q);
                                const int e0 = 4 * ((hp * kP + q) & 3);
                                const f32x4 own = {a[e0], a[e0 + 1], a[e0 + 2], a[e0 + 3]};
                                const f32x4 sum = t[q] + own;
#pragma unroll
                                for (int e = 0; e < 4; ++e) a[e0 + e] = sum[e];
                            }
                        }
                        for (int c = r + 1; c <= last; ++c) {
                            f32x4 v[kP];
                            load_part(c, v);
#pragma unroll
                            for (int q = 0; q < kP; ++q) {
                                f32x16& a = piece(q);
                                const int e0 = 4 * ((hp * kP + q) & 3);
#pragma unroll
                                for (int e = 0; e < 4; ++e) a[e0 + e] = a[e0 + e] + v[q][e];
                            }
                        }
                    }
                    if (tid == 0) __hip_atomic_store(sp.count + first, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    epilogue(m0, n0);
                }
            } else {
                epilogue(m0, n0);
            }
            i += n;
        }
    }
}

template <typename T, int RT, int CT, int ACT, bool FAST, bool RES, bool SPLIT, bool Q4K = false, int FOLD = 0>
__global__ __launch_bounds__(kWideThreads, kWideFoldSlots<FOLD>) void q8_wide_kernel(GemmParams p, WideSplit sp) {
    __shared__ __attribute__((aligned(1024))) char smem[WideCfg<RT, CT, Q4K, FOLD>::Lds];
    wide_tiles<T, RT, CT, ACT, FAST, RES, SPLIT, Q4K, FOLD>(p, sp, smem);
}

// f(activation, residual present) as compile-time constants, for the register epilogue's activations (the others
// take the general epilogue)
template <typename F>
void with_fast_epilogue(const GemmParams& p, F&& f) {
    auto with_act = [&](auto act) {
        if (p.res)
            f(act, std::true_type{});
        else
            f(act, std::false_type{});
    };
    if (p.act == IDOLQ_ACT_GELU_TANH)
        with_act(std::integral_constant<int, IDOLQ_ACT_GELU_TANH>{});
    else if (p.act == IDOLQ_ACT_RELU)
        with_act(std::integral_constant<int, IDOLQ_ACT_RELU>{});
    else
        with_act(std::integral_constant<int, IDOLQ_ACT_NONE>{});
}

// The register epilogue addresses y and the residual with 31-bit byte offsets (buffer accesses).
bool below_2gb(const GemmParams& p) {
    const int64_t y_end = ((int64_t)(p.m - 1) * p.ldy + p.n) * 2, r_end = ((int64_t)(p.m - 1) * p.ldr + p.n) * 2;
    return y_end < INT32_MAX && (!p.res || r_end < INT32_MAX);
}

template <typename T, int RT, int CT, bool SPLIT, bool Q4K, int FOLD = 0>
int launch_wide_s(GemmParams p, const WideSplit& sp, hipStream_t stream) {
    const dim3 grid(sp.G), block(kWideThreads);
    p.tiles_m = (p.m + 32 * RT - 1) / (32 * RT);
    p.tiles_n = (p.n + 128 * CT - 1) / (128 * CT);
    constexpr int kYdt = std::is_same<T, __bf16>::value ? IDOLQ_BF16 : IDOLQ_F16;
    const bool fast = p.y_vec4 && p.n % 4 == 0 && below_2gb(p) && p.y_dt == kYdt && (!p.res || p.res_dt == kYdt) &&
                      (!p.bias || p.bias_dt == IDOLQ_F32) &&
                      (p.act == IDOLQ_ACT_NONE || p.act == IDOLQ_ACT_GELU_TANH || p.act == IDOLQ_ACT_RELU);
    if (!fast)
        hipLaunchKernelGGL((q8_wide_kernel<T, RT, CT, IDOLQ_ACT_NONE, false, false, SPLIT, Q4K, FOLD>), grid, block, 0, stream,
                           p, sp);
    else
        with_fast_epilogue(p, [&](auto act, auto res) {
            hipLaunchKernelGGL((q8_wide_kernel<T, RT, CT, decltype(act)::value, true, decltype(res)::value, SPLIT, Q4K, FOLD>),
                               grid, block, 0, stream, p, sp);
        });
    return check_launch("q8_wide_kernel");
}

// Workspace: tile counters in the first kCountBytes, then the partial tiles.
constexpr size_t kCountBytes = kWideCountBytes;

// The stream-K split of the tiles left after whole rounds (tiles, S stages each, over cus workgroups; workspace: the
// counters, then the partial tiles).
WideSplit split_plan(long tiles, long S, long cus, void* workspace) {
    const long dp = tiles / cus * cus, units = (tiles - dp) * S;
    WideSplit sp{(int)cus, (int)dp, (int)(units / cus), (int)(units % cus),
                 reinterpret_cast<float*>(static_cast<char*>(workspace) + kCountBytes), static_cast<int*>(workspace), 1, 8};
    // in-phase ranges (all of L stages) on neighbouring tiles; groups of 4 row tiles when every tile is split (the
    // walk of the whole tiles is then not involved)
    const long g = std::gcd((long)sp.L, S), nsplit = tiles - dp;
    if (sp.R == 0 && sp.L > 0 && sp.L / g > 1 && nsplit % (sp.L / g) == 0) sp.ph = (int)(sp.L / g);
    if (dp == 0) sp.gh = 4;
    return sp;
}

// 4-element groups of y, the residual and the bias are vector-accessible
inline void set_y_vec4(GemmParams& p) {
    int vec4 = reinterpret_cast<uintptr_t>(p.y) % (4 * dtype_size(p.y_dt)) == 0 && p.ldy % 4 == 0;
    if (p.res) vec4 = vec4 && reinterpret_cast<uintptr_t>(p.res) % (4 * dtype_size(p.res_dt)) == 0 && p.ldr % 4 == 0;
    if (p.bias) vec4 = vec4 && reinterpret_cast<uintptr_t>(p.bias) % (4 * dtype_size(p.bias_dt)) == 0;
    p.y_vec4 = vec4;
}

}  // namespace
}  // namespace idolq
