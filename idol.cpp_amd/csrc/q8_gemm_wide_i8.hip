// The INT8 mode on tiled weights (q8_wide.h, I8): int8 MFMA on the tiled fragments with the per-block scale fold.
// Built with MFMA results in VGPRs (the fold reads every result element with the vector ALU; results in AGPRs
// would cost a copy per element).
#include "q8_wide.h"

#include <algorithm>

namespace idolq {

// The INT8 mode on tiled weights: 128 x 256 tiles (register budget of the fold), whole rounds or stream-K over the
// tiles left after them, costed like the DEQUANT plans with the fold-bound stage time. p.qa / p.sa: the activation
// codes and scales in the tiled quantizer's layout. The register epilogue takes bf16 outputs; others the general one.
int launch_wide_i8(GemmParams p, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    constexpr double kStage = 2.0, kFixed = 9.0;
    set_y_vec4(p);
    const long cus = cu_count(), S = p.k / 64;
    const long tiles = (long)((p.m + 127) / 128) * ((p.n + 255) / 256);
    auto rounds = [&](long t) { return (t + cus - 1) / cus; };
    const long dp = tiles / cus * cus, units = (tiles - dp) * S;
    const size_t need = kCountBytes + (size_t)2 * cus * 128 * 256 * 4;
    const double whole = rounds(tiles) * (S * kStage + kFixed);
    const double split = (double)dp / cus * (S * kStage + kFixed) + (double)rounds(units) * kStage + 2 * kFixed + 6.0;
    if (workspace && reinterpret_cast<uintptr_t>(workspace) % 256 == 0 && workspace_bytes >= need && units >= cus &&
        split < whole)
        return launch_wide_s<__bf16, 4, 2, true, false, true>(p, split_plan(tiles, S, cus, workspace), stream);
    const WideSplit sp{(int)std::min(tiles, cus), 0, 0, 0, nullptr, nullptr, 1, 8};
    return launch_wide_s<__bf16, 4, 2, false, false, true>(p, sp, stream);
}

}  // namespace idolq
