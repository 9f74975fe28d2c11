// Q8_0 GEMM on the grouped weight layout, DEQUANT arithmetic (and Q4_K super-blocks decoded in the weight loader):
// the split-column pair kernel, the launch plans and the entry points. The kernel template (layout, pipeline,
// epilogue, stream-K) is in q8_wide.h.
#include "q8_wide.h"

#include <algorithm>
#include <cstdlib>
#include <string>
#include <type_traits>
#include <utility>

namespace idolq {
namespace {

// Two column ranges in one launch: 256 x 256 tiles on pa's columns, 128 x 256 tiles on pb's (the column split of
// the launch plans). A workgroup takes its share of both ranges, the second range's first loads following the first
// range's epilogue without a kernel boundary between them. The workgroups with (blockIdx.x & swap) != 0 take pb's
// share first, so that their first epilogue (and its burst of output writes) falls in the others' main loop instead
// of every workgroup writing its first tile at once.
template <typename T, int ACT, bool FAST, bool RES, bool Q4K>
__global__ __launch_bounds__(kWideThreads) void q8_wide_pair_kernel(GemmParams pa, GemmParams pb, unsigned swap) {
    constexpr int kLds = WideCfg<8, 2, Q4K>::Lds > WideCfg<4, 2, Q4K>::Lds ? WideCfg<8, 2, Q4K>::Lds : WideCfg<4, 2, Q4K>::Lds;
    __shared__ __attribute__((aligned(1024))) char smem[kLds];
    const WideSplit whole{0, 0, 0, 0, nullptr, nullptr};
    const int first = (blockIdx.x & swap) != 0 ? 1 : 0;
    for (int pass = 0; pass < 2; ++pass) {
        if ((pass ^ first) == 0)
            wide_tiles<T, 8, 2, ACT, FAST, RES, false, Q4K>(pa, whole, smem);
        else
            wide_tiles<T, 4, 2, ACT, FAST, RES, false, Q4K>(pb, whole, smem);
    }
}

// swap: see q8_wide_pair_kernel (1: the workgroups on every other XCD start with the 128-row range)
template <typename T, bool Q4K>
int launch_wide_pair(GemmParams pa, GemmParams pb, int grid, hipStream_t stream, unsigned swap = 1) {
    pa.tiles_m = (pa.m + 255) / 256;
    pa.tiles_n = (pa.n + 255) / 256;
    pb.tiles_m = (pb.m + 127) / 128;
    pb.tiles_n = (pb.n + 255) / 256;
    constexpr int kYdt = std::is_same<T, __bf16>::value ? IDOLQ_BF16 : IDOLQ_F16;
    const GemmParams& p = pa;  // both ranges share dtypes, activation and alignment
    const bool fast = p.y_vec4 && pa.n % 4 == 0 && pb.n % 4 == 0 && below_2gb(pa) && below_2gb(pb) && p.y_dt == kYdt &&
                      (!p.res || p.res_dt == kYdt) &&
                      (!p.bias || p.bias_dt == IDOLQ_F32) &&
                      (p.act == IDOLQ_ACT_NONE || p.act == IDOLQ_ACT_GELU_TANH || p.act == IDOLQ_ACT_RELU);
    const dim3 g(grid), block(kWideThreads);
    if (!fast)
        hipLaunchKernelGGL((q8_wide_pair_kernel<T, IDOLQ_ACT_NONE, false, false, Q4K>), g, block, 0, stream, pa, pb, swap);
    else
        with_fast_epilogue(p, [&](auto act, auto res) {
            hipLaunchKernelGGL((q8_wide_pair_kernel<T, decltype(act)::value, true, decltype(res)::value, Q4K>), g, block, 0,
                               stream, pa, pb, swap);
        });
    return check_launch("q8_wide_pair_kernel");
}

// The columns [n0, n0 + n) of a launch (multiples of 32). Q4K: p.groups counts weight rows (row-major blocks).
template <bool Q4K>
GemmParams column_window(GemmParams p, int n0, int n) {
    const int S = p.k / 64;
    if (Q4K) {
        p.w += (size_t)n0 * p.row_bytes;
        p.groups -= n0;
    } else {
        p.w += (size_t)(n0 / 32) * S * kGroupBytes;
        p.groups -= n0 / 32;
    }
    if (p.bias) p.bias = static_cast<const char*>(p.bias) + (size_t)n0 * dtype_size(p.bias_dt);
    if (p.res) p.res = static_cast<const char*>(p.res) + (size_t)n0 * dtype_size(p.res_dt);
    p.y = static_cast<char*>(p.y) + (size_t)n0 * dtype_size(p.y_dt);
    p.n = n;
    return p;
}


// Launch plans, costed in microseconds from MI355X measurements: a 64-deep stage of a round of tiles takes STAGE, a
// tile's fixed part (first loads; the epilogue, where the whole round's outputs are written at once, at the memory's
// write rate) FIXED. Tiles: 256 x 256 (RT 8, CT 2), 128 x 256 (4, 2) and 128 x 384 (4, 3; whole tiles only, Q8_0 only).
// 128 x 384 runs its main loop at about the 256 x 256 tile's time per MFMA (48 MFMAs per wave per stage against 64),
// and makes n = 1536 at 8192 rows exactly one round (64 x 4 = 256 tiles, where 256 x 256 tiles leave 64 CUs idle);
// split over k its finisher needs more registers than the 128 x 256 one, and it is not split. Plans:
//   whole tiles of one shape;
//   columns split in two ranges (one launch, q8_wide_pair_kernel): whole rounds of 256-row tiles on the first
//     columns, 128-row tiles on the rest;
//   128-row tiles with stream-K over the tiles left after the whole rounds (a workspace is needed; about 6 more for
//     the partial tiles). 256-row tiles are not split: on the MLP block's down projection (4096 x 6144 -> 1536) their
//     stream-K plan took 134 us against 105 us for 128-row stream-K; the split ranges lose the L2 sharing of
//     neighbouring workgroups.
struct WideShape {
    int rt, ct;
    double stage, fixed;
};
constexpr WideShape kShapes[3] = {{8, 2, 1.42, 16.0}, {4, 2, 0.85, 9.0}, {4, 3, 1.16, 12.0}};
constexpr int kNumShapes = sizeof(kShapes) / sizeof(kShapes[0]);

template <typename T, bool Q4K, int RT, int CT>
int launch_shape(GemmParams p, const WideSplit& sp, bool split, hipStream_t stream) {
    return split ? launch_wide_s<T, RT, CT, true, Q4K>(p, sp, stream) : launch_wide_s<T, RT, CT, false, Q4K>(p, sp, stream);
}

template <typename T, bool Q4K>
int launch_wide_dtype(GemmParams p, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    const long cus = cu_count(), S = p.k / 64;
    auto rounds = [&](long tiles) { return (tiles + cus - 1) / cus; };
    auto tiles_of = [&](const WideShape& c) {
        return (long)((p.m + 32 * c.rt - 1) / (32 * c.rt)) * ((p.n + 128 * c.ct - 1) / (128 * c.ct));
    };
    double best = -1.0;
    int best_shape = 0;
    bool best_split = false;
    for (int i = 0; i < kNumShapes; ++i) {
        const WideShape& c = kShapes[i];
        if (Q4K && c.ct == 3) continue;
        const long tiles = tiles_of(c);
        const double whole = rounds(tiles) * (S * c.stage + c.fixed);
        if (best < 0 || whole < best) best = whole, best_shape = i, best_split = false;
        if (c.rt == 4 && c.ct == 2) {  // 256-row and 384-column tiles are not split (above)
            const long dp = tiles / cus * cus, units = (tiles - dp) * S;
            const size_t need = kCountBytes + (size_t)2 * cus * (32 * c.rt) * (128 * c.ct) * 4;
            if (workspace && workspace_bytes >= need && units >= cus) {
                const double split = (double)dp / cus * (S * c.stage + c.fixed) + (double)rounds(units) * c.stage +
                                     2 * c.fixed + 6.0;
                if (split < best) best = split, best_shape = i, best_split = true;
            }
        }
    }
    // split columns: as many column blocks as fill whole rounds of 256-row tiles, the rest with 128-row tiles
    const long tm8 = (p.m + 255) / 256, tm4 = (p.m + 127) / 128, tn = (p.n + 255) / 256;
    const long cb8 = (tm8 * tn) / cus * cus / tm8;
    const WideShape &c8 = kShapes[0], &c4 = kShapes[1];
    const double hybrid = cb8 > 0 && cb8 < tn ? rounds(tm8 * cb8) * (S * c8.stage + c8.fixed) +
                                                    rounds(tm4 * (tn - cb8)) * (S * c4.stage + c4.fixed)
                                              : -1.0;
    const WideSplit none{0, 0, 0, 0, nullptr, nullptr};
    auto whole = [&](long tiles) { WideSplit sp = none; sp.G = (int)std::min(tiles, cus); return sp; };
    if (hybrid > 0 && hybrid < best) {
        const int n1 = (int)cb8 * 256;
        const long grid = std::min(std::max(tm8 * cb8, tm4 * (tn - cb8)), cus);
        return launch_wide_pair<T, Q4K>(column_window<Q4K>(p, 0, n1), column_window<Q4K>(p, n1, p.n - n1), (int)grid, stream);
    }
    const WideShape& c = kShapes[best_shape];
    const long tiles = tiles_of(c);
    WideSplit sp = whole(tiles);
    if (best_split) sp = split_plan(tiles, S, cus, workspace);
    if (best_shape == 0) return launch_wide_s<T, 8, 2, false, Q4K>(p, sp, stream);
    if constexpr (!Q4K) {
        if (best_shape == 2) return launch_wide_s<T, 4, 3, false, Q4K>(p, sp, stream);
    }
    return launch_shape<T, Q4K, 4, 2>(p, sp, best_split, stream);
}

}  // namespace

bool wide_eligible(const GemmParams& p, int xt, int mode) {
    return mode == MODE_DEQUANT && (xt == XT_BF16 || xt == XT_F16) && p.w_tiled && p.x_aligned && p.k % 64 == 0 &&
           (reinterpret_cast<uintptr_t>(p.w) & 15) == 0 && p.groups > 0 &&
           (int64_t)p.m * p.ldx * 2 < (int64_t)UINT32_MAX &&
           (int64_t)p.groups * (p.k / 64) * kGroupBytes < (int64_t)UINT32_MAX;
}

// tile counters, then two partial tiles of the split shape (128 x 256 fp32) per workgroup slot: one per CU for
// DEQUANT, two for the INT8 fold
size_t wide_workspace_bytes() { return kCountBytes + (size_t)2 * kWideFoldSlots<kFoldI8> * cu_count() * 128 * 256 * 4; }

namespace {
template <bool Q4K>
int launch_wide_any(GemmParams p, int xt, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    set_y_vec4(p);
    if (workspace && reinterpret_cast<uintptr_t>(workspace) % 256 != 0) workspace = nullptr;
    if (xt == XT_BF16) return launch_wide_dtype<__bf16, Q4K>(p, workspace, workspace_bytes, stream);
    return launch_wide_dtype<_Float16, Q4K>(p, workspace, workspace_bytes, stream);
}
}  // namespace

int launch_wide(GemmParams p, int xt, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    return launch_wide_any<false>(p, xt, workspace, workspace_bytes, stream);
}

}  // namespace idolq

using namespace idolq;

extern "C" int64_t idolq_q4_k_bytes(int64_t n, int64_t k) { return k > 0 && k % 256 == 0 && n >= 0 ? n * (k / 256) * 144 : 0; }

extern "C" int idolq_q4_k_gemm(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const uint8_t* w,
                               int64_t n_total, int64_t n_offset, int64_t n, const void* bias, int bias_dtype,
                               const void* residual, int residual_dtype, int64_t ldr, int act, int flags, void* y,
                               int y_dtype, int64_t ldy, void* workspace, size_t workspace_bytes, void* stream) {
    if (!dtype_ok(x_dtype) || !dtype_ok(y_dtype) || (bias && !dtype_ok(bias_dtype)) ||
        (residual && !dtype_ok(residual_dtype)))
        return fail(IDOLQ_EINVAL, "unknown dtype code");
    if (x_dtype == IDOLQ_F32) return fail(IDOLQ_EINVAL, "the Q4_K GEMM takes bf16 or fp16 activations");
    if (m < 0 || n < 0 || k <= 0 || k % 256) return fail(IDOLQ_EINVAL, "need m >= 0, n >= 0 and k a positive multiple of 256");
    if (n_offset < 0 || n_offset + n > n_total) return fail(IDOLQ_EINVAL, "column window outside the weight rows");
    if (ldx < k || ldy < n || (residual && ldr < n)) return fail(IDOLQ_EINVAL, "row stride smaller than the row");
    if (m > INT32_MAX / 2 || n_total > INT32_MAX / 2 || k > INT32_MAX / 2) return fail(IDOLQ_EINVAL, "dimension too large");
    if (act < IDOLQ_ACT_NONE || act > IDOLQ_ACT_SILU) return fail(IDOLQ_EINVAL, "unknown activation");
    if (flags & ~IDOLQ_FLAG_ROUND_BEFORE_BIAS) return fail(IDOLQ_EINVAL, "unknown flag for the Q4_K GEMM");
    if (residual == y && residual && (residual_dtype != y_dtype || ldr != ldy))
        return fail(IDOLQ_EINVAL, "a residual that aliases y must have y's dtype and stride");
    const int64_t row_bytes = k / 256 * 144;
    if (m * ldx * 2 >= (int64_t)UINT32_MAX || (n_total - n_offset) * row_bytes >= (int64_t)UINT32_MAX)
        return fail(IDOLQ_EINVAL, "x or the weight window exceeds 2^32 elements / bytes");
    if (m == 0 || n == 0) return IDOLQ_OK;
    if (!x || !w || !y) return fail(IDOLQ_EINVAL, "x, w and y must be non-null");
    const uint8_t* wwin = w + n_offset * row_bytes;
    if ((reinterpret_cast<uintptr_t>(wwin) & 15) != 0) return fail(IDOLQ_EINVAL, "Q4_K weights must be 16-byte aligned");
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || (ldx * 2) % 16 != 0)
        return fail(IDOLQ_EINVAL, "the Q4_K GEMM needs 16-byte aligned activation rows");
    GemmParams p{};
    p.x = x;
    p.ldx = ldx;
    p.row_bytes = row_bytes;
    p.w = wwin;
    p.groups = (int)(n_total - n_offset);  // weight rows from p.w on
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
    p.x_aligned = 1;
    return launch_wide_any<true>(p, x_dtype == IDOLQ_BF16 ? XT_BF16 : XT_F16, workspace, workspace_bytes,
                                 static_cast<hipStream_t>(stream));
}
