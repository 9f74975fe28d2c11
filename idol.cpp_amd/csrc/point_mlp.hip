// The decoders' per-point MLP in one kernel: fp32 point features and a sine/cosine position embedding of the point
// coordinates, three linears with ReLU on Q8_0 weight values, and a dense fp32 head (the per-point heads of
// src/decoders.cpp:232-316; the embedding of src/decoders.cpp:215-230).
//
//   x  = [features (256) | sin/cos embedding (3 coordinates x 16 frequencies x 2)]     352 values per point
//   h1 = relu(x  W1^T + b1)   256      h2 = relu(h1 W2^T + b2)   256      h3 = relu(h2 W3^T + b3)   64
//   y  = h3 Wh^T + bh         up to 16 fp32 outputs
//
// Arithmetic: the layer-by-layer route's (three DEQUANT Q8_0 GEMMs and the fp32 head): x, h1, h2 and h3 rounded to
// bf16, the weights the bf16 values of their Q8_0 blocks, fp32 accumulation in bf16 MFMAs in ascending depth,
// then bias and ReLU in fp32; the head sums each half of the depth in a sequential fp32 FMA chain and adds the two
// halves, then the bias (the order of idolq_linear_f32).
//
// One workgroup (4 waves) takes 32 points, four workgroups per CU (their loads, embeddings and products overlap;
// measured faster than 64 points with two per CU and 128 with one); nothing but the fp32 inputs and outputs
// touches HBM:
//   LDS X [32 x 352] bf16 (row stride 720 B: 16 B of padding keep the 16-byte operand reads conflict-free)
//   LDS H [32 x 256] bf16 (row stride 528 B); h2 goes back into X's bytes with H's stride
// Layers 1 and 2: wave w computes output features [64w, 64w + 64) of the 32 points, 2 accumulator tiles of
// v_mfma_f32_32x32x16_bf16 in the transposed form D = W X^T (D rows are output features, columns points), point
// operands from LDS, weight operands from global memory (L2-resident) in MFMA fragment order: fragment (n-tile t,
// 16-deep chunk c) is 1 KB at (t K / 16 + c) KB, lane l = 32 h + r holding row 32 t + r, depth 16 c + 8 h .. + 8,
// so one wave's operand load is 1 KB of consecutive bytes.
// Layer 3 and the head: wave 0 takes the 32 points and all 64 features; the weight rows are
// permuted (row 32 b + i is feature 32 ((i / 4) % 2) + 16 b + 4 (i / 8) + i % 4) so that the lane halves of a point
// hold its features 0..31 and 32..63 in ascending order, and the head runs on those registers.
#include <hip/hip_runtime.h>

#include "common.h"
#include "../../include/idolq.h"

using namespace idolq;

namespace {

constexpr int kPoints = 32, kThreads = 256, kTiles = kPoints / 32;
constexpr int kFeat = 256, kFreq = 16, kK1 = kFeat + 6 * kFreq, kHidden = 256, kMid = 64, kMaxOut = 16;
constexpr int kXStride = kK1 * 2 + 16;      // 720 bytes
constexpr int kHStride = kHidden * 2 + 16;  // 528 bytes
constexpr int kXBytes = kPoints * kXStride, kHBytes = kPoints * kHStride;
constexpr int kLds = kXBytes + kHBytes;
static_assert(4 * kLds <= 163840, "LDS budget: four workgroups per CU");
static_assert(kXBytes >= kHBytes, "h2 reuses X's bytes");
static_assert(kHBytes >= kThreads * 16 && kMaxOut * kMid <= kThreads * 4, "the head's weights fit in H's bytes");

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
    return (uint32_t)float_to_bf16_bits(lo) | ((uint32_t)float_to_bf16_bits(hi) << 16);
}

// One 256-wide layer with ReLU for the workgroup's 128 points: in (LDS, `in_stride`) holds KC 16-deep chunks per
// point, w is [256 x 16 KC] bf16 row-major; wave `wave` writes features [64 wave, 64 wave + 64) of out (LDS, H's
// stride) as bf16.
template <int KC>
__device__ __forceinline__ void wide_layer(const char* in, int in_stride, const __bf16* __restrict__ w,
                                           const float* __restrict__ bias, char* out, int wave, int lane) {
    const int r = lane & 31, h = lane >> 5;
    const int n0 = 64 * wave;
    f32x16 acc[2][kTiles];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int t = 0; t < kTiles; ++t)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[b][t][e] = 0.0f;
    // fragment (n-tile 2 wave + b, chunk c): 1 KB at ((2 wave + b) KC + c) KB, lane l's 16 bytes at 16 l
    const char* wf0 = reinterpret_cast<const char*>(w) + (size_t)(2 * wave * KC) * 1024 + 16 * lane;
    const char* wf1 = wf0 + KC * 1024;
    const char* xrow = in + r * in_stride + 16 * h;
#pragma unroll
    for (int c = 0; c < KC; ++c) {
        const bf16x8 a0 = as_bf16x8(*reinterpret_cast<const uint4*>(wf0 + 1024 * c));
        const bf16x8 a1 = as_bf16x8(*reinterpret_cast<const uint4*>(wf1 + 1024 * c));
        bf16x8 bx[kTiles];
#pragma unroll
        for (int t = 0; t < kTiles; ++t) bx[t] = as_bf16x8(*reinterpret_cast<const uint4*>(xrow + 32 * t * in_stride + 32 * c));
#pragma unroll
        for (int t = 0; t < kTiles; ++t) {
            acc[0][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, bx[t], acc[0][t], 0, 0, 0);
            acc[1][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, bx[t], acc[1][t], 0, 0, 0);
        }
    }
    // element e of lane (r, h) in a tile: feature 8 (e / 4) + 4 h + e % 4 of the tile's 32, point r of its 32
#pragma unroll
    for (int b = 0; b < 2; ++b) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int n = n0 + 32 * b + 8 * q + 4 * h;
            const float4 bb = *reinterpret_cast<const float4*>(bias + n);
#pragma unroll
            for (int t = 0; t < kTiles; ++t) {
                const float v0 = fmaxf(acc[b][t][4 * q] + bb.x, 0.0f), v1 = fmaxf(acc[b][t][4 * q + 1] + bb.y, 0.0f);
                const float v2 = fmaxf(acc[b][t][4 * q + 2] + bb.z, 0.0f), v3 = fmaxf(acc[b][t][4 * q + 3] + bb.w, 0.0f);
                *reinterpret_cast<uint2*>(out + (32 * t + r) * kHStride + 2 * n) = make_uint2(pack_bf16(v0, v1), pack_bf16(v2, v3));
            }
        }
    }
}

__global__ __launch_bounds__(kThreads, 3) void point_mlp_kernel(const float* __restrict__ feats, int64_t m, int64_t ldf,
                                                             const float* __restrict__ coords,
                                                             const float* __restrict__ freqs,
                                                             const __bf16* __restrict__ w1, const float* __restrict__ b1,
                                                             const __bf16* __restrict__ w2, const float* __restrict__ b2,
                                                             const __bf16* __restrict__ w3, const float* __restrict__ b3,
                                                             const float* __restrict__ wh, const float* __restrict__ bh,
                                                             int nout, float* __restrict__ y, int64_t ldy) {
    __shared__ __attribute__((aligned(16))) char smem[kLds];
    char* const X = smem;
    char* const H = smem + kXBytes;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t p0 = (int64_t)blockIdx.x * kPoints;

    // Global loads complete in issue order, and a wait for one load waits for every load issued before it: so the
    // embedding's inputs are requested first (their wait then leaves the features in flight), and the head's
    // weights (nout x 64 fp32, one float4 per thread) are fetched now and parked in LDS once layer 2 is done,
    // instead of the head waiting on global loads output by output.
    // ---- the embedding's item (point i / 6, coordinate (i / 2) % 3, frequencies 8 (i % 2) .. + 8), i = tid; the
    // threads past the items load item kPoints * 6 - 1 and do not store
    constexpr int kItems = kPoints * 6;
    static_assert(kItems <= kThreads, "one embedding item per thread");
    const int item = min(tid, kItems - 1);
    const int erow = item / 6, ec = (item >> 1) - 3 * erow, ej0 = 8 * (item & 1);
    const float ev = coords[min(p0 + erow, m - 1) * 3 + ec];
    float ef[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) ef[j] = freqs[ej0 + j];
    const float4 whv = reinterpret_cast<const float4*>(wh)[min(tid, nout * (kMid / 4) - 1)];
    // ---- x: the tile's features (rows past m repeat the last row; their outputs are not stored), 16 pieces of 8
    // values per thread, rounded to bf16 into LDS after the embedding has been computed
    constexpr int kPieces = kPoints * (kFeat / 8) / kThreads;
    float4 fv[kPieces][2];
#pragma unroll
    for (int j = 0; j < kPieces; ++j) {
        const int i = j * kThreads + tid, row = i >> 5, g = i & 31;
        const int64_t src = min(p0 + row, m - 1);
        const float4* f = reinterpret_cast<const float4*>(feats + src * ldf + 8 * g);
        fv[j][0] = f[0];
        fv[j][1] = f[1];
    }
    // ---- the embedding: coordinate c of a point fills values 256 + 32 c + j (sine) and + 16 (cosine), j < 16
    {
        const float kPi = 3.14159265358979323846f;
        uint32_t sn[4], cs[4];
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
            const float a0 = (ev * ef[j]) * kPi, a1 = (ev * ef[j + 1]) * kPi;
            sn[j / 2] = pack_bf16(sinf(a0), sinf(a1));
            cs[j / 2] = pack_bf16(cosf(a0), cosf(a1));
        }
        if (tid < kItems) {
            char* dst = X + erow * kXStride + 2 * (kFeat + 32 * ec + ej0);
            *reinterpret_cast<uint4*>(dst) = make_uint4(sn[0], sn[1], sn[2], sn[3]);
            *reinterpret_cast<uint4*>(dst + 32) = make_uint4(cs[0], cs[1], cs[2], cs[3]);
        }
    }
#pragma unroll
    for (int j = 0; j < kPieces; ++j) {
        const int i = j * kThreads + tid, row = i >> 5, g = i & 31;
        const float4 u = fv[j][0], v = fv[j][1];
        *reinterpret_cast<uint4*>(X + row * kXStride + 16 * g) =
            make_uint4(pack_bf16(u.x, u.y), pack_bf16(u.z, u.w), pack_bf16(v.x, v.y), pack_bf16(v.z, v.w));
    }
    __syncthreads();

    wide_layer<kK1 / 16>(X, kXStride, w1, b1, H, wave, lane);
    __syncthreads();
    wide_layer<kHidden / 16>(H, kHStride, w2, b2, X, wave, lane);
    __syncthreads();
    // h1 is dead: its bytes take the head's weights ([nout][64] fp32, 4 KB at most)
    float* const whs = reinterpret_cast<float*>(H);
    reinterpret_cast<float4*>(whs)[tid] = whv;
    __syncthreads();

    if (wave >= kTiles) return;  // no barrier follows
    // ---- layer 3: points [32 wave, 32 wave + 32), tile b row i = 8 (i / 8) .. holds feature
    // 32 ((i / 4) % 2) + 16 b + 4 (i / 8) + i % 4, so lane half h holds features 32 h + 16 b + e in element e
    const int r = lane & 31, h = lane >> 5;
    f32x16 acc[2];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[b][e] = 0.0f;
    {
        const char* wrow0 = reinterpret_cast<const char*>(w3) + 16 * lane;
        const char* wrow1 = wrow0 + (kHidden / 16) * 1024;
        const char* xrow = X + (32 * wave + r) * kHStride + 16 * h;
#pragma unroll
        for (int c = 0; c < kHidden / 16; ++c) {
            const bf16x8 a0 = as_bf16x8(*reinterpret_cast<const uint4*>(wrow0 + 1024 * c));
            const bf16x8 a1 = as_bf16x8(*reinterpret_cast<const uint4*>(wrow1 + 1024 * c));
            const bf16x8 bx = as_bf16x8(*reinterpret_cast<const uint4*>(xrow + 32 * c));
            acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, bx, acc[0], 0, 0, 0);
            acc[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, bx, acc[1], 0, 0, 0);
        }
    }
    float h3[32], bias3[32];
#pragma unroll
    for (int k = 0; k < 32; ++k) bias3[k] = b3[32 * h + k];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const float v = fmaxf(acc[b][e] + bias3[16 * b + e], 0.0f);
            h3[16 * b + e] = bf16_bits_to_float(float_to_bf16_bits(v));
        }

    // ---- head: each lane half sums its 32 features in order, the halves are added (first half first), then bias
    const int64_t p = p0 + 32 * wave + r;
    float out[kMaxOut];
#pragma unroll
    for (int o = 0; o < kMaxOut; ++o) {
        if (o < nout) {
            const float* wo = whs + o * kMid + 32 * h;
            float part = 0.0f;
#pragma unroll
            for (int k = 0; k < 32; ++k) part = fmaf(h3[k], wo[k], part);
            const float other = __shfl_xor(part, 32);
            const float sum = h == 0 ? part + other : other + part;
            out[o] = bh ? sum + bh[o] : sum;
        }
    }
    if (p < m) {
#pragma unroll
        for (int o = 0; o < kMaxOut; ++o)
            if (o < nout && (o >> 3) == h) y[p * ldy + o] = out[o];
    }
}

}  // namespace

extern "C" int idolq_point_mlp(const float* feats, int64_t m, int64_t ldf, const float* coords, const float* freqs,
                               int64_t nfreq, const void* w1, const float* b1, const void* w2, const float* b2,
                               const void* w3, const float* b3, const float* wh, const float* bh, int64_t nout,
                               float* y, int64_t ldy, void* stream) {
    if (m < 0 || nfreq != kFreq || nout < 1 || nout > kMaxOut)
        return fail(IDOLQ_EINVAL, "the fused per-point MLP takes 16 frequencies and 1..16 outputs");
    if (ldf < kFeat || ldy < nout || ldf % 4) return fail(IDOLQ_EINVAL, "row stride too small or not a multiple of 4");
    if (m == 0) return IDOLQ_OK;
    if (!feats || !coords || !freqs || !w1 || !b1 || !w2 || !b2 || !w3 || !b3 || !wh || !y)
        return fail(IDOLQ_EINVAL, "null pointer");
    auto al = [](const void* q) { return reinterpret_cast<uintptr_t>(q) % 16 == 0; };
    if (!al(feats) || !al(w1) || !al(w2) || !al(w3) || !al(b1) || !al(b2) || !al(wh))
        return fail(IDOLQ_EINVAL, "features, weights, the head and the 256-wide biases must be 16-byte aligned");
    if (m > (int64_t)INT32_MAX * kPoints / 2) return fail(IDOLQ_EINVAL, "too many points");
    const unsigned blocks = (unsigned)((m + kPoints - 1) / kPoints);
    hipLaunchKernelGGL(point_mlp_kernel, dim3(blocks), dim3(kThreads), 0, static_cast<hipStream_t>(stream), feats, m,
                       ldf, coords, freqs, static_cast<const __bf16*>(w1), b1, static_cast<const __bf16*>(w2), b2,
                       static_cast<const __bf16*>(w3), b3, wh, bh, (int)nout, y, ldy);
    return check_launch("point_mlp_kernel");
}
