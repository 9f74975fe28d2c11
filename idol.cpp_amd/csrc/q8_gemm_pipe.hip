// Pipelined Q8_0 GEMM for gfx950 in DEQUANT arithmetic: y = epilogue(x * W^T), the MFMA operands being x (bf16 or
// fp16) and T(fp32(d) * q) for the Q8_0 weights, accumulated in fp32.
//
// Output tile 256 (rows of x) x 128 (weight rows); 512 threads = 8 waves in a 4 x 2 grid, each wave owning 64 x 64
// as 2 x 2 tiles of v_mfma_f32_32x32x16. The MFMA computes the transposed tile C^T = W * X^T: the weights supply the
// 32 MFMA rows (output columns) and x the 32 MFMA columns (output rows), so accumulator element r of lane l is output
// row l % 32 and output column 8 (r / 4) + 4 (l / 32) + r % 4 -- four consecutive columns per lane, written by the
// epilogue as one vector straight from the registers.
//
// Stage s covers k [64 s, 64 s + 64): two Q8_0 blocks. Global memory reaches LDS without passing through registers
// (global_load_lds): the activation tile goes to one of three 32 KiB buffers (256 rows x 128 bytes; the eight
// 16-byte chunks of row r are stored at chunk position c ^ ((r >> 1) & 7), which makes the MFMA operand reads free of
// bank conflicts), and the 68 weight bytes of each of the 128 weight rows, unchanged, to one of three 8.5 KiB
// buffers. During stage s each wave
//   1. issues the loads of activations s + 3 and of weight bytes s + 4,
//   2. reads stage s + 1's MFMA operands from LDS into its second register set,
//   3. converts the weight bytes of stage s + 2 into MFMA operands (one of two 18 KiB buffers, rows padded to 144 B),
//   4. runs the 16 MFMAs of stage s on the operands read during stage s - 1,
//   5. waits until its loads of activations s + 2 and weight bytes s + 3 have landed, then meets the barrier.
// Every buffer written in a stage was last read before the barrier that ended the previous stage. Rows of x beyond m
// and weight rows beyond n read the last valid row instead (they only feed outputs that are never stored), so the
// loads need no masks; k is a multiple of 64, so there is no partial stage.
#include "q8_dma.h"

#include <string>
#include <type_traits>

namespace idolq {
namespace {

constexpr int kThreads = 512;
constexpr int kABuf = kPipeBM * 128;                  // 32768 bytes: 256 rows x 64 16-bit activations
constexpr int kRawUnits = kPipeBN * 17;               // 2176 dwords: 68 bytes for each of 128 weight rows
constexpr int kRawBuf = kRawUnits * 4;                // 8704 bytes
constexpr int kBPitch = 144;                          // bytes per converted weight row (64 operands + 16 B pad)
constexpr int kBBuf = kPipeBN * kBPitch;              // 18432 bytes
constexpr int kRawBase = 3 * kABuf;                   // 98304
constexpr int kBBase = kRawBase + 3 * kRawBuf;        // 124416
constexpr int kJunk = kBBase + 2 * kBBuf;             // 161280: 256 bytes that absorb the unused weight loads
constexpr int kLdsBytes = kJunk + 256;                // 161536 (of 163840)
static_assert(kLdsBytes <= 163840, "LDS budget");

// The common epilogue: y and the residual (if any) of the activation dtype T, fp32 bias (if any), n a multiple of 4
// and 4-element groups vector-aligned. All loads are issued (epilogue_loads) before the first store
// (epilogue_stores): a wait for a load also waits for every store issued before it.
struct EpilogueLoads {
    float4 b4[2][4];
    uint2 r2[2][2][4];
};

__device__ __forceinline__ void epilogue_loads(const GemmParams& p, int row0, int col0, EpilogueLoads& L) {
#pragma unroll
    for (int tn = 0; tn < 2; ++tn)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int col = col0 + tn * 32 + 8 * g;
            const bool full = col < p.n;
            L.b4[tn][g] = p.bias && full ? *reinterpret_cast<const float4*>(static_cast<const float*>(p.bias) + col)
                                         : make_float4(0, 0, 0, 0);
#pragma unroll
            for (int tm = 0; tm < 2; ++tm) {
                const int row = row0 + tm * 32;
                L.r2[tm][tn][g] = p.res && full && row < p.m
                                      ? *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p.res) + (int64_t)row * p.ldr + col)
                                      : make_uint2(0, 0);
            }
        }
}

template <typename T, int ACT>
__device__ __forceinline__ void epilogue_stores(const GemmParams& p, const f32x16 (&acc)[2][2], int row0, int col0,
                                                const EpilogueLoads& L) {
    typedef typename PipeMfma<T>::pair T2;
    const bool round_first = (p.flags & IDOLQ_FLAG_ROUND_BEFORE_BIAS) != 0;
#pragma unroll
    for (int tm = 0; tm < 2; ++tm) {
        const int row = row0 + tm * 32;
        if (row >= p.m) continue;
#pragma unroll
        for (int tn = 0; tn < 2; ++tn)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int col = col0 + tn * 32 + 8 * g;
                if (col >= p.n) continue;
                f32x2 lo = {acc[tm][tn][4 * g], acc[tm][tn][4 * g + 1]}, hi = {acc[tm][tn][4 * g + 2], acc[tm][tn][4 * g + 3]};
                if (round_first) {
                    lo = __builtin_convertvector(__builtin_convertvector(lo, T2), f32x2);
                    hi = __builtin_convertvector(__builtin_convertvector(hi, T2), f32x2);
                }
                const float4 b = L.b4[tn][g];
                const T2 rlo = __builtin_bit_cast(T2, L.r2[tm][tn][g].x), rhi = __builtin_bit_cast(T2, L.r2[tm][tn][g].y);
                lo = lo + f32x2{b.x, b.y} + __builtin_convertvector(rlo, f32x2);
                hi = hi + f32x2{b.z, b.w} + __builtin_convertvector(rhi, f32x2);
                lo = f32x2{act_fast<ACT>(lo.x), act_fast<ACT>(lo.y)};
                hi = f32x2{act_fast<ACT>(hi.x), act_fast<ACT>(hi.y)};
                *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p.y) + (int64_t)row * p.ldy + col) =
                    make_uint2(__builtin_bit_cast(uint32_t, __builtin_convertvector(lo, T2)),
                               __builtin_bit_cast(uint32_t, __builtin_convertvector(hi, T2)));
            }
    }
}

template <typename T>
__global__ __launch_bounds__(kThreads) void q8_gemm_pipe_kernel(GemmParams p, int vec4, int S) {
    typedef typename PipeMfma<T>::vec Vec;
    __shared__ __attribute__((aligned(1024))) char smem[kLdsBytes];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    // ---- global -> LDS load offsets (bytes, 32-bit) of the current tile, set by start_segment
    // activations: unit u = 512 j + tid (16 bytes) is LDS chunk u of the buffer: row u / 8, position u % 8, which
    // holds chunk (u % 8) ^ ((row >> 1) & 7) of the row's 128 bytes
    // weights: dword unit u = 512 j + tid of the [128 rows][17 dwords] stage is LDS dword u
    uint32_t a_off[4], w_off[5];
    const char* xg;  // activations / weight bytes of the segment's first stage
    const char* wg;
    int nsteps;      // stages in the segment
    auto start_segment = [&](int m0, int n0, int k0, int n) __attribute__((always_inline)) {
        const int r = tid >> 3, c = (tid & 7) ^ ((r >> 1) & 7);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int row = min(m0 + 64 * j + r, p.m - 1);
            a_off[j] = (uint32_t)((int64_t)row * p.ldx * 2 + c * 16);
        }
#pragma unroll
        for (int j = 0; j < 5; ++j) {
            const int u = min(512 * j + tid, kRawUnits - 1);
            const int row = min(n0 + u / 17, p.n - 1);
            w_off[j] = (uint32_t)((int64_t)row * p.row_bytes + (u % 17) * 4);
        }
        xg = uniform_ptr(static_cast<const char*>(p.x) + (size_t)k0 * 128);
        wg = uniform_ptr(reinterpret_cast<const char*>(p.w) + (size_t)k0 * 68);
        nsteps = n;
    };

    const uint32_t lds0 = (uint32_t)(size_t)(lds_char*)smem;
    auto issue_a = [&](int s) __attribute__((always_inline)) {
        const char* base = xg + (size_t)s * 128;
        const uint32_t dst = lds0 + (s % 3) * kABuf + wave * 1024;
#pragma unroll
        for (int j = 0; j < 4; ++j) lds_dma16(base, a_off[j], dst + j * 8192);
    };
    // 2176 dwords are 4.25 loads per wave: the fifth load of waves 2..7 reads a valid address into a junk area, so
    // every wave issues the same five loads (no branch, and the same vmcnt on every wave)
    const uint32_t w_dst4 = wave < (kRawUnits - 2048) / 64 ? kRawBase + 4 * 2048 + wave * 256 : kJunk;
    auto issue_w = [&](int s) __attribute__((always_inline)) {
        const char* base = wg + (size_t)s * 68;
        const uint32_t dst = lds0 + kRawBase + (s % 3) * kRawBuf + wave * 256;
#pragma unroll
        for (int j = 0; j < 4; ++j) lds_dma4(base, w_off[j], dst + j * 2048);
        lds_dma4(base, w_off[4], lds0 + w_dst4 + (w_dst4 == kJunk ? 0 : (s % 3) * kRawBuf));
    };

    // ---- weight conversion: thread -> row tid % 128, chunk q = tid / 128 of each block (8 codes per block).
    // Consecutive lanes take consecutive rows, so each 4-byte read (row stride 17 dwords, odd) hits 64 distinct banks
    // and each 16-byte write (row stride 144 bytes) 16 distinct 4-bank groups per cycle.
    const int cv_row = tid & (kPipeBN - 1), cv_q = tid >> 7;
    struct RawIn {
        uint32_t w0, w8, a0, a1, a2, b0, b1;
    };
    auto convert_load = [&](int s) __attribute__((always_inline)) {
        const uint32_t* rw = reinterpret_cast<const uint32_t*>(smem + kRawBase + (s % 3) * kRawBuf + cv_row * 68);
        return RawIn{rw[0], rw[8], rw[2 * cv_q], rw[2 * cv_q + 1], rw[2 * cv_q + 2], rw[9 + 2 * cv_q], rw[10 + 2 * cv_q]};
    };
    auto convert_store = [&](int s, const RawIn& r) __attribute__((always_inline)) {
        const float d0 = half_bits_to_float((uint16_t)(r.w0 & 0xffff));
        const float d1 = half_bits_to_float((uint16_t)(r.w8 >> 16));
        // block 0's codes start at byte 2 of the row (two bytes off dword alignment), block 1's at byte 36
        const uint2 c0 = make_uint2(__builtin_amdgcn_alignbyte(r.a1, r.a0, 2), __builtin_amdgcn_alignbyte(r.a2, r.a1, 2));
        char* bdst = smem + kBBase + (s & 1) * kBBuf + cv_row * kBPitch + cv_q * 16;
        *reinterpret_cast<uint4*>(bdst) = dequant8<T>(c0, d0);
        *reinterpret_cast<uint4*>(bdst + 64) = dequant8<T>(make_uint2(r.b0, r.b1), d1);
    };
    auto convert = [&](int s) __attribute__((always_inline)) { convert_store(s, convert_load(s)); };

    // ---- MFMA operand addresses (bytes within a buffer)
    // weights (MFMA rows): output column wn*64 + tn*32 + lane%32, k = 32 blk + 16 h + 8 (lane/32) + e
    const uint32_t b_lane = (uint32_t)((wn * 64 + (lane & 31)) * kBPitch + (lane >> 5) * 16);
    // activations (MFMA columns): output row wm*64 + tm*32 + lane%32, chunk c = 4 blk + 2 h + lane/32 swizzled
    uint32_t x_lane[2][2];
    {
        const int r = lane & 31, sw = (r >> 1) & 7;
#pragma unroll
        for (int blk = 0; blk < 2; ++blk)
#pragma unroll
            for (int h = 0; h < 2; ++h)
                x_lane[blk][h] = (uint32_t)((wm * 64 + r) * 128 + (((4 * blk + 2 * h + (lane >> 5)) ^ sw) * 16));
    }

    f32x16 acc[2][2];

    // MFMA operands of one stage in registers, in four groups g = 2 blk + h (16 deep each): w[g][tn], x[g][tm]
    Vec ow[4][2], ox[4][2];
    auto read_group = [&](int s, int g) __attribute__((always_inline)) {
        const char* ab = smem + (s % 3) * kABuf;
        const char* bb = smem + kBBase + (s & 1) * kBBuf + b_lane;
        const int blk = g >> 1, h = g & 1;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            ow[g][t] = *reinterpret_cast<const Vec*>(bb + t * 32 * kBPitch + blk * 64 + h * 32);
            ox[g][t] = *reinterpret_cast<const Vec*>(ab + x_lane[blk][h] + t * 32 * 128);
        }
    };
    auto read_operands = [&](int s) __attribute__((always_inline)) {
#pragma unroll
        for (int g = 0; g < 4; ++g) read_group(s, g);
    };
    auto mfma_group = [&](int g) __attribute__((always_inline)) {
#pragma unroll
        for (int tm = 0; tm < 2; ++tm)
#pragma unroll
            for (int tn = 0; tn < 2; ++tn) acc[tm][tn] = PipeMfma<T>::run(ow[g][tn], ox[g][tm], acc[tm][tn]);
    };

    // the segment's first loads: activations 0 and 1, weight bytes 0..2 (LDS must no longer be read by the previous
    // segment)
    auto prologue_issue = [&]() __attribute__((always_inline)) {
        issue_a(0);
        issue_w(0);
        if (nsteps > 1) issue_w(1);
        if (nsteps > 1) issue_a(1);
        if (nsteps > 2) issue_w(2);
    };
    auto run_segment = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // ---- prologue (its first loads were issued by prologue_issue). At the start of stage s, stage s's operands are
    // in registers, activations s + 1 and weights s + 1 (converted) are in LDS, weight bytes s + 2 have landed,
    // activations s + 2 and weight bytes s + 3 are in flight.
    wait_vm<0>();
    __syncthreads();
    convert(0);
    if (nsteps > 1) convert(1);
    __syncthreads();
    read_operands(0);
    if (nsteps > 2) issue_a(2);
    if (nsteps > 3) issue_w(3);
    __syncthreads();

    // Stage s: the MFMAs run on operands read during stage s - 1 while the wave issues the loads of activations
    // s + 3 and weight bytes s + 4, converts weight bytes s + 2 and reads stage s + 1's operands into the registers
    // of each group as soon as that group's MFMAs have been issued. Every buffer written in stage s was last read in
    // stage s - 1 (activations s, weight bytes s + 1, weights s).
    //
    // Steady stages (s + 4 < nsteps) are one basic block, scheduled so that the MFMAs are spread over the stage
    // with the LDS reads and the conversion arithmetic issued between them (the matrix core runs an MFMA while the
    // wave issues the following independent instructions).
    auto stage_steady = [&](int s) __attribute__((always_inline)) {
        const RawIn raw = convert_load(s + 2);
        __builtin_amdgcn_sched_barrier(0);
        // four segments, one per operand group: a quarter of the global loads (one activation load, one or two
        // weight loads), the group's 4 MFMAs, the reads of stage s + 1's operands of the group and a quarter of the
        // conversion (4 codes). Spreading the loads over the stage keeps the vector-memory queue from filling up and
        // stalling the wave in front of its MFMAs.
        const float d0 = half_bits_to_float((uint16_t)(raw.w0 & 0xffff));
        const float d1 = half_bits_to_float((uint16_t)(raw.w8 >> 16));
        char* bdst = smem + kBBase + (s & 1) * kBBuf + cv_row * kBPitch + cv_q * 16;
        const char* abase = xg + (size_t)(s + 3) * 128;
        const uint32_t adst = lds0 + ((s + 3) % 3) * kABuf + wave * 1024;
        const char* wbase = wg + (size_t)(s + 4) * 68;
        const int wslot = (s + 4) % 3;
        const uint32_t wdst = lds0 + kRawBase + wslot * kRawBuf + wave * 256;
        uint2 q0, q1, q2, q3;
#define IDOLQ_SEGMENT(G, WORK)                                     \
        lds_dma16(abase, a_off[G], adst + G * 8192);               \
        lds_dma4(wbase, w_off[G], wdst + G * 2048);                \
        mfma_group(G);                                             \
        read_group(s + 1, G);                                      \
        WORK;                                                      \
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);         \
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);         \
        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);         \
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);         \
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);         \
        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);         \
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);         \
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);         \
        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);         \
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);         \
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);         \
        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);         \
        __builtin_amdgcn_sched_barrier(0)
        // block 0's codes start at byte 2 of the row (two bytes off dword alignment), block 1's at byte 36
        IDOLQ_SEGMENT(0, q0 = dequant4<T>(__builtin_amdgcn_alignbyte(raw.a1, raw.a0, 2), d0));
        IDOLQ_SEGMENT(1, q1 = dequant4<T>(__builtin_amdgcn_alignbyte(raw.a2, raw.a1, 2), d0);
                         *reinterpret_cast<uint4*>(bdst) = make_uint4(q0.x, q0.y, q1.x, q1.y));
        IDOLQ_SEGMENT(2, q2 = dequant4<T>(raw.b0, d1));
        IDOLQ_SEGMENT(3, q3 = dequant4<T>(raw.b1, d1);
                         *reinterpret_cast<uint4*>(bdst + 64) = make_uint4(q2.x, q2.y, q3.x, q3.y));
#undef IDOLQ_SEGMENT
        lds_dma4(wbase, w_off[4], lds0 + w_dst4 + (w_dst4 == kJunk ? 0 : wslot * kRawBuf));
        // activations s + 2 and weight bytes s + 3 (issued in stage s - 1) have landed once at most the loads issued
        // in this stage remain outstanding: 4 + 5
        wait_vm<9>();
        __syncthreads();
    };
    auto stage_tail = [&](int s) __attribute__((always_inline)) {
        if (s + 3 < nsteps) issue_a(s + 3);
        if (s + 2 < nsteps) convert(s + 2);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            mfma_group(g);
            if (s + 1 < nsteps) read_group(s + 1, g);
        }
        if (s + 3 < nsteps)
            wait_vm<4>();
        else
            wait_vm<0>();
        __syncthreads();
    };
    const int steady = nsteps > 4 ? nsteps - 4 : 0;
    int s = 0;
    for (; s < steady; ++s) stage_steady(s);
    for (; s < nsteps; ++s) stage_tail(s);
    };

    // ---- epilogue from the registers
    constexpr int kYdt = std::is_same<T, __bf16>::value ? IDOLQ_BF16 : IDOLQ_F16;
    // the register epilogue applies (the same for every tile of the launch)
    const bool fast_epilogue = vec4 && p.n % 4 == 0 && p.y_dt == kYdt && (!p.res || p.res_dt == kYdt) &&
                               (!p.bias || p.bias_dt == IDOLQ_F32) &&
                               (p.act == IDOLQ_ACT_NONE || p.act == IDOLQ_ACT_GELU_TANH || p.act == IDOLQ_ACT_RELU);
    auto fast_stores = [&](int row0, int col0, const EpilogueLoads& L) __attribute__((always_inline)) {
        if (p.act == IDOLQ_ACT_NONE) return epilogue_stores<T, IDOLQ_ACT_NONE>(p, acc, row0, col0, L);
        if (p.act == IDOLQ_ACT_GELU_TANH) return epilogue_stores<T, IDOLQ_ACT_GELU_TANH>(p, acc, row0, col0, L);
        return epilogue_stores<T, IDOLQ_ACT_RELU>(p, acc, row0, col0, L);
    };
    auto epilogue = [&](int m0, int n0) __attribute__((always_inline)) {
    const int row0 = m0 + wm * 64 + (lane & 31);
    const int col0 = n0 + wn * 64 + 4 * (lane >> 5);
    if (fast_epilogue) {
        EpilogueLoads L;
        epilogue_loads(p, row0, col0, L);
        return fast_stores(row0, col0, L);
    }
    // General path: the accumulators go to LDS (element i of thread t at float i * 512 + t; LDS is no longer read by
    // the main loop after its last barrier) and one loop that is not unrolled runs them through the epilogue.
    float* stash = reinterpret_cast<float*>(smem);
#pragma unroll
    for (int i = 0; i < 64; ++i) stash[i * kThreads + tid] = acc[i >> 5][(i >> 4) & 1][i & 15];
#pragma unroll 1
    for (int i = 0; i < 64; ++i) {
        const int row = row0 + (i >> 5) * 32, r = i & 15;
        const int col = col0 + ((i >> 4) & 1) * 32 + 8 * (r >> 2) + (r & 3);
        if (row < p.m && col < p.n) epilogue_element(p, row, col, stash[i * kThreads + tid]);
    }
    };

    // ---- work: whole tiles r, r + G, ... (groups of 8 row tiles walked column by column; the workgroups of one XCD
    // take consecutive tiles, so those running together share weight and activation rows in that XCD's L2)
    const int G = gridDim.x;
    int r = blockIdx.x;
    if (G % 8 == 0) r = (r % 8) * (G / 8) + r / 8;
    const int ntiles = p.tiles_m * p.tiles_n;
    auto tile_at = [&](int t, int& m0, int& n0) __attribute__((always_inline)) {
        constexpr int G8 = 8;
        const int per_group = G8 * p.tiles_n, group = t / per_group, first = group * G8;
        const int gm = min(p.tiles_m - first, G8), in_group = t - group * per_group;
        // integer division runs on the vector unit: bring the (uniform) results back to scalar registers
        m0 = __builtin_amdgcn_readfirstlane((first + in_group % gm) * kPipeBM);
        n0 = __builtin_amdgcn_readfirstlane((in_group / gm) * kPipeBN);
    };
    // With the register epilogue, the next tile's first loads are issued between the epilogue's loads and its
    // arithmetic and stores, which hide their latency (the epilogue does not use LDS).
    int m0 = 0, n0 = 0;
    if (r < ntiles) {
        tile_at(r, m0, n0);
        start_segment(m0, n0, 0, S);
        prologue_issue();
    }
    for (int t = r; t < ntiles; t += G) {
        run_segment();
        const int tn = t + G, cm0 = m0, cn0 = n0;
        if (fast_epilogue) {
            const int row0 = cm0 + wm * 64 + (lane & 31), col0 = cn0 + wn * 64 + 4 * (lane >> 5);
            EpilogueLoads L;
            epilogue_loads(p, row0, col0, L);
            // the epilogue's loads complete first: a compiler wait for one of them would otherwise also wait for
            // the later loads issued below, which it cannot see
            wait_vm<0>();
            if (tn < ntiles) {
                tile_at(tn, m0, n0);
                start_segment(m0, n0, 0, S);
                prologue_issue();
            }
            fast_stores(row0, col0, L);
        } else {
            epilogue(cm0, cn0);
            __syncthreads();
            if (tn < ntiles) {
                tile_at(tn, m0, n0);
                start_segment(m0, n0, 0, S);
                prologue_issue();
            }
        }
    }
}

}  // namespace

bool pipe_eligible(const GemmParams& p, int xt, int mode) {
    return mode == MODE_DEQUANT && (xt == XT_BF16 || xt == XT_F16) && p.x_aligned && p.k % 64 == 0 &&
           !p.w_tiled && p.row_bytes % 4 == 0 && (reinterpret_cast<uintptr_t>(p.w) & 3) == 0 &&
           (int64_t)p.m * p.ldx * 2 < (int64_t)UINT32_MAX && (int64_t)p.n * p.row_bytes < (int64_t)UINT32_MAX;
}

int cu_count() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cached[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

int launch_pipe(GemmParams p, int xt, hipStream_t stream) {
    p.tiles_m = (p.m + kPipeBM - 1) / kPipeBM;
    p.tiles_n = (p.n + kPipeBN - 1) / kPipeBN;
    // 4-element groups of y, the residual and the bias are vector-accessible
    int vec4 = reinterpret_cast<uintptr_t>(p.y) % (4 * dtype_size(p.y_dt)) == 0 && p.ldy % 4 == 0;
    if (p.res) vec4 = vec4 && reinterpret_cast<uintptr_t>(p.res) % (4 * dtype_size(p.res_dt)) == 0 && p.ldr % 4 == 0;
    if (p.bias) vec4 = vec4 && reinterpret_cast<uintptr_t>(p.bias) % (4 * dtype_size(p.bias_dt)) == 0;
    const int cus = cu_count(), tiles = p.tiles_m * p.tiles_n, S = p.k / 64;
    const dim3 grid(tiles < cus ? tiles : cus), block(kThreads);
    if (xt == XT_BF16)
        hipLaunchKernelGGL((q8_gemm_pipe_kernel<__bf16>), grid, block, 0, stream, p, vec4, S);
    else
        hipLaunchKernelGGL((q8_gemm_pipe_kernel<_Float16>), grid, block, 0, stream, p, vec4, S);
    return check_launch("q8_gemm_pipe_kernel");
}

}  // namespace idolq
