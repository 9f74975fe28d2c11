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
    int w_tiled;    // w is in the tiled layout (idolq_q8_0_tile), p.w at the window's first tile
    // INT8 mode
    const int8_t* qa;
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

// The pipelined DEQUANT kernel (q8_gemm_pipe.hip): 256 x 128 tiles, 16-bit activations with 16-byte aligned rows,
// k a multiple of 64 and a 4-byte aligned weight window. One persistent workgroup per CU; with a workspace of
// pipe_workspace_bytes() the tiles' k stages are split evenly over the workgroups (stream-K).
constexpr int kPipeBM = 256, kPipeBN = 128;

struct PipeSplit {
    int G;        // workgroups
    int S;        // 64-deep stages per tile
    int L, R;     // stream-K: workgroup r holds L + (r < R) stages
    float* part;  // stream-K: G partial tiles (kPipeBM x kPipeBN fp32); null: whole tiles only
    int* flags;   // G flags: workgroup r stores epoch when its partial tile is ready
    int* error;   // set to 1 if a wait for a partial tile gave up
    int epoch;    // launch number, never 0
};

size_t pipe_workspace_bytes();
bool pipe_eligible(const GemmParams& p, int xt, int mode);
int launch_pipe(GemmParams p, int xt, void* workspace, size_t workspace_bytes, hipStream_t stream);

}  // namespace idolq
