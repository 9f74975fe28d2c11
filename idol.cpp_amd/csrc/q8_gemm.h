// Launch parameters and tile order shared by the Q8_0 GEMM kernels (q8_gemm.hip, q8_gemm_pipe.hip).
#pragma once

#include "common.h"

namespace idolq {

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
    int y_vec;      // y (and the residual, when given) rows and base are 16-byte aligned: vector epilogue stores
    int w_tiled;    // w is in the grouped layout (idolq_q8_0_tile), p.w at the window's first 32-row group
    int groups;     // grouped layout: 32-row groups from p.w to the end of the layout
    int y_vec4;     // y, the residual and the bias allow vector access to 4-element groups
    // INT8 mode
    const int8_t* qa;
    const void* x_lo;  // EXACT on tiled weights: the bf16 low parts of fp32 activations (p.x: the high parts)
    const float* sa;
    int32_t* dots;
};

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

// The pipelined DEQUANT kernel (q8_gemm_pipe.hip) on GGUF row-major weights: 256 x 128 tiles, 16-bit activations with
// 16-byte aligned rows, k a multiple of 64 and a 4-byte aligned weight window; one persistent workgroup per CU.
constexpr int kPipeBM = 256, kPipeBN = 128;
bool pipe_eligible(const GemmParams& p, int xt, int mode);
int launch_pipe(GemmParams p, int xt, hipStream_t stream);

// The grouped-layout kernel (q8_gemm_wide.hip): 256 x 256 or 128 x 256 tiles, 4 waves; with a workspace of
// wide_workspace_bytes() (zero-filled before first use) the leftover tiles' k stages may be split over the CUs.
bool wide_eligible(const GemmParams& p, int xt, int mode);
size_t wide_workspace_bytes();
constexpr size_t kWideCountBytes = 4096;  // the tile counters at the start of that workspace (zero between launches)
int launch_wide(GemmParams p, int xt, void* workspace, size_t workspace_bytes, hipStream_t stream);
// The INT8 mode on tiled weights (p.qa, p.sa from the tiled quantizer); workspace as launch_wide's (may be null).
int launch_wide_i8(GemmParams p, void* workspace, size_t workspace_bytes, hipStream_t stream);
// The EXACT mode on tiled weights (p.x, p.x_lo: bf16 high and low parts of the activations, row stride k).
int launch_wide_exact(GemmParams p, void* workspace, size_t workspace_bytes, hipStream_t stream);

// The small-m form (q8_gemv.hip): m <= kGemvMaxRows activation rows on GGUF row-major weights (k % 256 == 0, 16-byte
// aligned), DEQUANT on 16-bit activations or EXACT; 16 weight rows per workgroup, the depth split over 8 waves.
constexpr int kGemvMaxRows = 16;
bool gemv_eligible(const GemmParams& p, int xt, int mode);
int launch_gemv(GemmParams p, int xt, int mode, hipStream_t stream);

}  // namespace idolq
