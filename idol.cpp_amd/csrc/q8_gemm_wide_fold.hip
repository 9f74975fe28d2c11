// The modes that fold 32-block sums on tiled weights (q8_wide.h, FOLD): INT8 (int8 MFMA on the tiled fragments,
// fmaf(dot, sa * d, acc)) and EXACT (exact codes against the bf16 high and low parts of fp32 activations,
// fmaf(sum, d, acc)). Built with MFMA results in VGPRs: the fold reads every result element with the vector ALU, and
// results in AGPRs would cost a copy per element.
#include "q8_wide.h"

#include <algorithm>

namespace idolq {

namespace {

// 128 x 256 tiles (the fold's register budget), whole rounds or stream-K over the tiles left after them, costed like
// the DEQUANT plans with the mode's stage time. The register epilogue takes bf16 outputs; others the general one.
// INT8 runs two workgroups per CU (256 registers per lane and 78 KB of LDS each): its fold is bound by the vector ALU,
// which one wave per SIMD leaves idle while it waits on its MFMA results and loads, and a second wave fills those
// cycles. So a round is 2 x CUs tiles. EXACT (148 KB of LDS) runs one per CU.
template <int FOLD>
int launch_wide_fold(GemmParams p, double stage, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    constexpr double kFixed = 9.0;
    set_y_vec4(p);
    const long slots = (long)kWideFoldSlots<FOLD> * cu_count(), S = p.k / 64;
    const long tiles = (long)((p.m + 127) / 128) * ((p.n + 255) / 256);
    auto rounds = [&](long t) { return (t + slots - 1) / slots; };
    const long dp = tiles / slots * slots, units = (tiles - dp) * S;
    const size_t need = kCountBytes + (size_t)2 * slots * 128 * 256 * 4;
    const double whole = rounds(tiles) * (S * stage + kFixed);
    const double split = (double)dp / slots * (S * stage + kFixed) + (double)rounds(units) * stage + 2 * kFixed + 6.0;
    if (workspace && reinterpret_cast<uintptr_t>(workspace) % 256 == 0 && workspace_bytes >= need && units >= slots &&
        split < whole)
        return launch_wide_s<__bf16, 4, 2, true, false, FOLD>(p, split_plan(tiles, S, slots, workspace), stream);
    const WideSplit sp{(int)std::min(tiles, slots), 0, 0, 0, nullptr, nullptr, 1, 8};
    return launch_wide_s<__bf16, 4, 2, false, false, FOLD>(p, sp, stream);
}

}  // namespace

// p.qa / p.sa: the activation codes and scales in the tiled quantizer's layout (fold-bound: a stage of a round of
// two tiles per CU ~3 us)
int launch_wide_i8(GemmParams p, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    return launch_wide_fold<kFoldI8>(p, 3.0, workspace, workspace_bytes, stream);
}

// p.x / p.x_lo: the bf16 high and low parts of the activations, row stride k (MFMA-bound: twice DEQUANT's products)
int launch_wide_exact(GemmParams p, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    return launch_wide_fold<kFoldExact>(p, 1.9, workspace, workspace_bytes, stream);
}

}  // namespace idolq
