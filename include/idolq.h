/*
 * libidolq: MI355X (gfx950) kernels for the Q8_0 block-quantized linear path of idol.cpp, behind a plain C ABI.
 *
 * Conventions
 *   - Every pointer is device memory on the current HIP device, except where a comment says otherwise.
 *   - `stream` is a hipStream_t passed as void* (NULL is the default stream). All calls are asynchronous on it and
 *     allocate nothing; scratch that a call needs is passed in by the caller (workspace arguments).
 *   - Return 0 on success or a negative IDOLQ_E* code; idolq_last_error() then describes the failure (the message
 *     slot is thread-local). Argument errors are detected on the host before anything is launched.
 *   - dtype codes: IDOLQ_F32, IDOLQ_F16, IDOLQ_BF16. Strides (ld*) are in elements.
 *   - Q8_0 weights are the raw GGUF blocks: for each output row n, k / 32 blocks of 34 bytes, each a little-endian
 *     fp16 scale d followed by 32 int8 codes q; the weight is w = fp32(d) * q.
 */
#ifndef IDOLQ_H
#define IDOLQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { IDOLQ_F32 = 0, IDOLQ_F16 = 1, IDOLQ_BF16 = 2 };

/* Activations applied after bias and residual. GELU_ERF is the reference's fused epilogue (src/kernels.cpp:826-850),
 * GELU_TANH its decoder MLP activation (src/decoders.cpp:55-71), SILU x / (1 + exp(-x)) its level-embedding MLP
 * activation (src/decoders.cpp:88). */
enum { IDOLQ_ACT_NONE = 0, IDOLQ_ACT_GELU_ERF = 1, IDOLQ_ACT_GELU_TANH = 2, IDOLQ_ACT_RELU = 3, IDOLQ_ACT_SILU = 4 };

/* GGUF block formats (the ggml type codes) of the packed-linear surface. */
enum {
    IDOLQ_KIND_F16 = 1,
    IDOLQ_KIND_Q4_0 = 2,
    IDOLQ_KIND_Q8_0 = 8,
    IDOLQ_KIND_Q2_K = 10,
    IDOLQ_KIND_Q4_K = 12,
    IDOLQ_KIND_Q6_K = 14
};

/* GEMM arithmetic.
 *   DEQUANT  weights dequantized to the activation's 16-bit type (bf16 or fp16 of fp32(d) * q) in LDS, MFMA with fp32
 *            accumulation over the whole depth: the numerics of the reference's fused GPU path.
 *   EXACT    codes fed to bf16/fp16 MFMA exactly, each 32-deep block summed in fp32 and scaled by its fp32 d; fp32
 *            activations are split into bf16 high and low parts. Tracks the reference's CPU float kernel.
 *   INT8     activations quantized per row and 32-block to int8 exactly as the reference's integer kernel does,
 *            int8 MFMA with int32 block sums, scales folded per block in fp32. Needs a workspace. On tiled weights
 *            the same bits as on row-major weights when tiles are not split along k.
 *   AUTO     DEQUANT for bf16/fp16 activations, EXACT for fp32. */
enum { IDOLQ_MODE_AUTO = 0, IDOLQ_MODE_DEQUANT = 1, IDOLQ_MODE_EXACT = 2, IDOLQ_MODE_INT8 = 3 };

/* GEMM flags. ROUND_BEFORE_BIAS rounds the product to the output dtype before the bias is added, as the reference's
 * fused GPU path does (tools/idol_triton.py:84-89). TILED_WEIGHTS: w is in the tiled Q8_0 layout written by
 * idolq_q8_0_tile, in DEQUANT mode (bf16/fp16 activations), INT8 mode, or EXACT mode (fp32, bf16 or fp16 activations;
 * it then needs a workspace of at least 2 * round_up(m * k * 2, 256) bytes for the activations' bf16 high and low
 * parts); activation rows 16-byte aligned, weights 16-byte aligned, k % 64 == 0, n_offset % 32 == 0. */
enum { IDOLQ_FLAG_ROUND_BEFORE_BIAS = 1, IDOLQ_FLAG_TILED_WEIGHTS = 2 };

enum {
    IDOLQ_OK = 0,
    IDOLQ_EINVAL = -1,  /* bad argument: shape, dtype, stride, alignment, size */
    IDOLQ_ELAUNCH = -2, /* a HIP launch failed */
    IDOLQ_ENOSUPPORT = -3
};

/* Message for the last failing call on this thread ("" if none). */
const char* idolq_last_error(void);

/* Library version and the gfx target it was built for. */
const char* idolq_version(void);

/* Bytes of one Q8_0 weight of n rows and k columns: n * (k / 32) * 34 (0 when k % 32 != 0).
 * Replaces the size check of tools/idol_triton.py:103-105 and tools/idol_packed.py:28-31. */
int64_t idolq_q8_0_bytes(int64_t n, int64_t k);

/* y[i, j] = epilogue( sum_k x[i, k] * w[n_offset + j, k] ) for i < m, j < n.
 *   x        [m x k] in x_dtype, row stride ldx (>= k)
 *   w        Q8_0 weight with n_total rows of k; only rows [n_offset, n_offset + n) are read
 *   bias     NULL or n_total values in bias_dtype, indexed n_offset + j
 *   residual NULL or [m x n] in residual_dtype, row stride ldr; may alias y (same dtype and stride)
 *   act      IDOLQ_ACT_*, applied after bias and residual
 *   y        [m x n] in y_dtype, row stride ldy
 *   workspace / workspace_bytes  scratch of idolq_q8_0_gemm_workspace bytes: required by IDOLQ_MODE_INT8 (quantized
 *            activations and scales, m * k * 9 / 8 bytes and some padding at the start; with tiled weights the
 *            rest, when present, is used like the DEQUANT workspace and needs no zero-fill: the call clears its
 *            counters); required by IDOLQ_MODE_EXACT with tiled weights (the activations split into bf16 high and
 *            low parts, m * k * 4 bytes at the start, the rest used the same way); optional for
 *            IDOLQ_MODE_DEQUANT with tiled weights, where it lets the k stages of the
 *            tiles left after whole rounds of the CUs be split over the CUs (tile counters, then partial tiles). A
 *            DEQUANT workspace must be zero-filled before its first use and used by one stream at a time; calls
 *            leave its counters at zero, ready for the next call.
 * Replaces src/kernels.hpp:73-76 gemm_packed (fp32 x, residual before GELU, column window n_offset / n) and
 * tools/idol_triton.py:94-126 fused_linear (bf16/fp16 x, bias after rounding: IDOLQ_FLAG_ROUND_BEFORE_BIAS). */
int idolq_q8_0_gemm(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const uint8_t* w, int64_t n_total,
                    int64_t n_offset, int64_t n, const void* bias, int bias_dtype, const void* residual,
                    int residual_dtype, int64_t ldr, int act, int mode, int flags, void* y, int y_dtype, int64_t ldy,
                    void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes idolq_q8_0_gemm uses for m rows of depth k in the given mode: the quantized activations and
 * scales, then room for the tiled path's split, for IDOLQ_MODE_INT8; the tile counters and partial tiles of the
 * current device's CUs for IDOLQ_MODE_DEQUANT; the high and low parts, then the same split room, for
 * IDOLQ_MODE_EXACT (used with tiled weights only: the row-major EXACT kernel takes no workspace).
 * This is the most a call can use. The minimum a call requires is smaller, and a caller that sizes its buffer for
 * row-major weights only may pass just that: INT8 round_up(m * k, 256) + round_up(m * (k / 32) * 4 + 16, 256) bytes
 * (the split room, about 64 MiB on 256 CUs, serves tiled weights only); EXACT 0 on row-major weights and
 * 2 * round_up(m * k * 2, 256) on tiled weights; DEQUANT 0 (without a workspace every tile is taken whole). */
size_t idolq_q8_0_gemm_workspace(int64_t m, int64_t k, int mode);

/* idolq_q8_0_gemm for callers that cannot allocate (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc): no workspace argument, and the call allocates nothing. No counterpart in the reference.
 * IDOLQ_MODE_INT8 takes its quantized activations and scales, IDOLQ_MODE_EXACT on tiled weights its bf16 high and
 * low parts, from a static device array of idolq_q8_0_gemm_noalloc_max_bytes() bytes (32 MiB; INT8 uses
 * m * k * 9 / 8 bytes, EXACT m * k * 4, a larger need is IDOLQ_EINVAL); every call runs whole tiles (no stream-K
 * split) and row-major EXACT needs no scratch. Each device has its own array, shared by
 * every call on that device: calls that overlap on one device (several streams or threads at once) race on it. */
int idolq_q8_0_gemm_noalloc(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const uint8_t* w,
                            int64_t n_total, int64_t n_offset, int64_t n, const void* bias, int bias_dtype,
                            const void* residual, int residual_dtype, int64_t ldr, int act, int mode, int flags,
                            void* y, int y_dtype, int64_t ldy, void* stream);
size_t idolq_q8_0_gemm_noalloc_max_bytes(void);

/* Quantizes an fp32 [n x k] matrix (row stride ldw) to Q8_0 blocks: per 32 values d = amax / 127,
 * q = round-half-away-from-zero(x * (1 / d)), d stored as fp16. The rule of ggml's quantize_row_q8_0_ref, which
 * gguf-py's quantize(..., Q8_0) restates (tools/export_full_gguf.py:332-335, tests/python/test_fused_packed.py:40). */
int idolq_q8_0_quantize(const float* w, int64_t n, int64_t k, int64_t ldw, uint8_t* out, void* stream);

/* Tiled (grouped) Q8_0: the same 34-byte blocks, reordered once (at load time) so that each GEMM load reads contiguous
 * bytes already in MFMA operand order. Rows are grouped by 32 (the last group padded with zero rows) and k in stages
 * of 64 (two blocks); chunk (g, s) of 2176 bytes at byte (g * (k / 64) + s) * 2176 holds, for b = 0, 1, the 32 codes
 * of block 2 s + b of each row at [1024 b, 1024 b + 1024) -- lane l's 16 bytes at 16 l are codes 8 h .. 8 h + 7 then
 * 16 + 8 h .. 16 + 8 h + 7 of row 32 g + l % 32, h = l / 32 -- and at [2048, 2176) per row r the fp16 scales of blocks
 * 2 s (low half) and 2 s + 1 (high half) at 2048 + 4 r. Size = 34 bytes per 32 weights of the padded rows. Needs
 * k % 64 == 0 (else the size is 0 / EINVAL). Layout of this library only: the reference keeps GGUF blocks row-major
 * (tools/idol_packed.py:28-31) and its CPU kernels use 16-column panels (src/kernels.hpp:33-51). */
int64_t idolq_q8_0_tiled_bytes(int64_t n, int64_t k);
int idolq_q8_0_tile(const uint8_t* w, int64_t n, int64_t k, uint8_t* out, void* stream);

/* out[r, c] = out_dtype(fp32(d) * q) for the whole [n x k] weight, out row stride k.
 * Replaces tools/idol_triton.py:24-33 _unpack_q8 and tools/idol_packed.py:25-31,71 PackedLinear.dequantize. */
int idolq_q8_0_dequant(const uint8_t* w, int64_t n, int64_t k, void* out, int out_dtype, void* stream);

/* Per row and 32-block of x [m x k]: amax, scale = amax / 127, inv = 127 / amax (0 when amax == 0),
 * qa = round-to-nearest-even(x * inv) as int8, qsum = sum of qa. qa is [m x k], scale and qsum [m x k / 32].
 * qsum may be NULL. Replaces src/kernels.cpp:368-404 quantize_activations (bit-exact). */
int idolq_quantize_act_q8(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, int8_t* qa, float* scale,
                          int32_t* qsum, void* stream);

/* The int32 block dot products the INT8 GEMM computes with int8 MFMA, before any scaling:
 * dots[(i * n + j) * (k / 32) + b] = sum_{t < 32} qa[i, 32 b + t] * q[n_offset + j, 32 b + t].
 * A test entry point for the integer path of src/kernels.cpp:407-452 (vnni_task), whose sums are
 * sum qa * (q + 128) = dots + 128 * qsum. */
int idolq_q8_0_block_dots(const int8_t* qa, int64_t m, int64_t k, const uint8_t* w, int64_t n_total,
                          int64_t n_offset, int64_t n, int32_t* dots, void* stream);

/* Row-wise layer norm: y = (x - mean) / sqrt(var + eps), then * gamma + beta when gamma is given, then
 * * (1 + scale[b]) + shift[b] when scale is given (adaLN), b = row / rows_per_batch (0 when rows_per_batch <= 0).
 * Mean and variance are accumulated in fp64. gamma/beta are [dim] fp32; shift/scale are [batches x dim] fp32.
 * y may alias x when the dtypes and strides match.
 * Replaces src/decoders.cpp:23-42 norm_rows and src/kernels.cpp:599-618 layer_norm (eps 1e-5, gamma and beta). */
int idolq_layernorm(const void* x, int x_dtype, int64_t rows, int64_t dim, int64_t ldx, float eps, const float* gamma,
                    const float* beta, const float* shift, const float* scale, int64_t rows_per_batch, void* y,
                    int y_dtype, int64_t ldy, void* stream);

/* Non-causal multi-head attention, softmax(q k^T / sqrt(head_dim)) v per head and batch.
 *   q  [batch][lq rows of stride ldq], head h at columns [h * head_dim, (h + 1) * head_dim), batch stride q_bs
 *   k, v [batch][lk rows of stride ldkv], batch stride kv_bs
 *   out  [batch][lq rows of stride ldo], batch stride o_bs
 * q, k, v share `dtype`; out has out_dtype. bf16/fp16 inputs use MFMA (QK^T in the input type, fp32 online softmax,
 * P and V in fp16 for P*V); fp32 inputs and head_dim other than 64 use an fp32 kernel.
 * Replaces src/kernels.hpp:81-84 attention (batch 1, out stride dim). */
int idolq_attention(const void* q, const void* k, const void* v, int dtype, int64_t batch, int64_t lq, int64_t lk,
                    int64_t heads, int64_t head_dim, int64_t ldq, int64_t ldkv, int64_t q_bs, int64_t kv_bs, void* out,
                    int out_dtype, int64_t ldo, int64_t o_bs, void* stream);

/* idolq_attention with a workspace of idolq_attention_workspace() bytes (256-byte aligned; the call writes it
 * before reading it, so it needs no zero-fill): bf16 inputs with head_dim 64 then convert V once per call into
 * fp16 V^T tiles (scaled per tile where |v| exceeds fp16, by the same rule as without the workspace) instead of
 * once per query workgroup; the operands and the arithmetic are those of idolq_attention, so are the output bits.
 * A null or short workspace runs idolq_attention's path. Calls sharing a workspace must not overlap.
 * Same reference interface as idolq_attention (src/kernels.hpp:81-84). */
int idolq_attention_ws(const void* q, const void* k, const void* v, int dtype, int64_t batch, int64_t lq, int64_t lk,
                       int64_t heads, int64_t head_dim, int64_t ldq, int64_t ldkv, int64_t q_bs, int64_t kv_bs,
                       void* out, int out_dtype, int64_t ldo, int64_t o_bs, void* workspace, size_t workspace_bytes,
                       void* stream);
/* Workspace bytes idolq_attention_ws uses for these shapes: the fp16 V^T tiles (batch x heads x ceil(lk / 64) tiles
 * of 8 KiB) and their exponents for bf16 inputs with head_dim 64; 0 for every other call. */
size_t idolq_attention_workspace(int dtype, int64_t batch, int64_t lk, int64_t heads, int64_t head_dim);

/* In-place activation over count values: tanh-GELU (src/decoders.cpp:55-71 gelu_tanh), erf-GELU
 * (src/kernels.cpp:826-850) or ReLU. */
int idolq_activation(void* x, int dtype, int64_t count, int act, void* stream);

/* Sine/cosine position embedding of 3-D coordinates (src/decoders.cpp:215-230 pos_embed, without the zero padding):
 * out[r * ldo + c * 2 * nfreq + j] = sin((coords[r, c] * freqs[j]) * pi) and at + nfreq the cosine, for c < 3.
 * coords [rows x 3] fp32, freqs [nfreq] fp32, out in out_dtype. */
int idolq_pos_embed(const float* coords, int64_t rows, const float* freqs, int64_t nfreq, void* out, int out_dtype,
                    int64_t ldo, void* stream);

/* Dense fp32 linear y[m x n] = act(x[m x k] * w^T + bias) for narrow layers (n <= 32, n * k <= 16384; else
 * IDOLQ_ENOSUPPORT): the fp32 heads of the decoders' per-point MLPs. w [n x k] fp32 row-major, bias NULL or [n] fp32.
 * Sums the depth in 32-deep FMA chunks added left to right, then adds the bias: bit-identical to the reference's
 * dense gemm_packed (src/kernels.hpp:73-76 with an unquantized PackedLinear, src/kernels.cpp:566-596). */
int idolq_linear_f32(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const float* w, int64_t n,
                     const float* bias, int act, void* y, int y_dtype, int64_t ldy, void* stream);

/* The decoders' per-point MLP in one launch (the per-point heads of src/decoders.cpp:232-316, the embedding of
 * src/decoders.cpp:215-230): x = [feats (256) | sin/cos embedding of coords (3 x nfreq x 2, nfreq = 16)],
 * h1 = relu(x W1^T + b1) (256), h2 = relu(h1 W2^T + b2) (256), h3 = relu(h2 W3^T + b3) (64), y = h3 Wh^T + bh.
 * feats [m x 256] fp32 (row stride ldf, a multiple of 4), coords [m x 3] fp32, freqs [16] fp32; w1 [256 x 352],
 * w2 [256 x 256], w3 [64 x 256]: the bf16 values of Q8_0 weights (idolq_q8_0_dequant to bf16) in MFMA fragment
 * order -- fragment (row tile t of 32 rows, 16-deep chunk c) is 1 KB at byte (t * k / 16 + c) * 1024, its 16-byte
 * piece l = 32 h + r holding row 32 t + r, depth 16 c + 8 h .. + 8 -- with w3's rows first permuted so that row
 * 32 b + i is feature 32 ((i / 4) % 2) + 16 b + 4 (i / 8) + i % 4 (idolq_lib.point_mlp_pack); biases fp32; wh [nout x 64] fp32 with 1 <= nout <= 16, bh NULL or [nout]; y [m x nout] fp32 (row stride ldy). The same
 * arithmetic as the layer-by-layer route (idolq_pos_embed, three DEQUANT idolq_q8_0_gemm calls with ReLU,
 * idolq_linear_f32): x and the hidden activations rounded to bf16, fp32 accumulation, the head's sums in
 * idolq_linear_f32's order. feats, w1, w2, w3, b1 and b2 16-byte aligned. */
int idolq_point_mlp(const float* feats, int64_t m, int64_t ldf, const float* coords, const float* freqs, int64_t nfreq,
                    const void* w1, const float* b1, const void* w2, const float* b2, const void* w3, const float* b3,
                    const float* wh, const float* bh, int64_t nout, float* y, int64_t ldy, void* stream);

/* Copies a [rows x cols] block between dtypes and strides (a column slice of a wider row is a pointer offset). */
int idolq_copy2d(const void* src, int src_dtype, int64_t lds, void* dst, int dst_dtype, int64_t ldd, int64_t rows,
                 int64_t cols, void* stream);

/* ---- Other block formats (tools/idol_packed.py:25-71, tools/idol_triton.py:48-82). ---- */

/* Bytes of an [n x k] matrix in block format `kind` (0 when k is not a multiple of the block's value count). */
int64_t idolq_blocks_bytes(int kind, int64_t n, int64_t k);

/* out[r, c] = out_dtype(w[r, c]) for the whole [n x k] matrix in block format `kind` (Q4_0, Q8_0, Q2_K, Q4_K, Q6_K,
 * F16), out row stride k, 16-byte aligned. Each value is computed in fp32 with the reference expansion's operations
 * (PackedLinear.dequantize, tools/idol_packed.py:25-71), then rounded once. */
int idolq_blocks_dequant(const uint8_t* w, int kind, int64_t n, int64_t k, void* out, int out_dtype, void* stream);

/* Bytes of a row-major GGUF Q4_K matrix [n x k]: n * (k / 256) * 144 (0 when k % 256 != 0). */
int64_t idolq_q4_k_bytes(int64_t n, int64_t k);

/* y = epilogue(x * W^T) for GGUF Q4_K weights as they are stored (row-major 144-byte super-blocks of 256 values:
 * fp16 d, fp16 dmin, 12 bytes of 6-bit scales and minimums, 128 bytes of 4-bit codes), decoded inside the GEMM's
 * weight loader: each weight enters the MFMA as T((d * sc) * q - dmin * m), the reference's fused decode
 * (tools/idol_triton.py:61-82), with fp32 accumulation (DEQUANT arithmetic). x bf16 or fp16 with 16-byte aligned rows,
 * k % 256 == 0, the weight window 16-byte aligned; every other argument as idolq_q8_0_gemm (DEQUANT workspace optional,
 * IDOLQ_FLAG_ROUND_BEFORE_BIAS for the fused path's bias order, tools/idol_triton.py:84-89). */
int idolq_q4_k_gemm(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const uint8_t* w, int64_t n_total,
                    int64_t n_offset, int64_t n, const void* bias, int bias_dtype, const void* residual,
                    int residual_dtype, int64_t ldr, int act, int flags, void* y, int y_dtype, int64_t ldy,
                    void* workspace, size_t workspace_bytes, void* stream);

/* Re-encodes Q4_0 blocks [n x k] as Q8_0 blocks (same fp16 scale, codes q - 8): exact, so every Q8_0 GEMM mode
 * computes the Q4_0 layer's products (the Q4_0 case of tools/idol_triton.py:48-60). */
int idolq_q4_0_to_q8_0(const uint8_t* w, int64_t n, int64_t k, uint8_t* out, void* stream);

/* ---- Native quantized panels (src/kernels.hpp:33-51), the reference's own weight format for gemm_packed. ---- */

/* Bytes of the panel blob of an [out x in] layer quantized with `bits` in groups of `group` k values:
 * ceil(out / 16) * (in / group) * (64 + 2 * group * bits); 0 when bits is not 2, 3, 4, 5, 6 or 8 or group is not a
 * multiple of 32 dividing in. Replaces src/kernels.cpp:512-514 quant_panel_bytes (times the panel count). */
int64_t idolq_panel_bytes(int64_t out, int64_t in, int bits, int group);

/* w[r * ldw + c] = fma(code, scale, min) in fp32 for every weight of a panel blob (device memory, blob_bytes long):
 * the values of the reference's dequantizer, src/kernels.cpp:167-209 dequant8 / dequant_chunk and :535-550
 * dequantize_linear, bit for bit. The argument checks and messages are those of src/kernels.cpp:516-533
 * quantized_linear (bits, group, blob size). */
int idolq_panel_expand_f32(const uint8_t* blob, int64_t blob_bytes, int64_t out, int64_t in, int bits, int group,
                           float* w, int64_t ldw, void* stream);

/* A panel blob whose every minimum is -2^(bits-1) * scale holds exactly fp32(scale) * (code - 2^(bits-1)); this
 * writes those values as GGUF Q8_0 blocks q8 (out * in / 32 * 34 bytes, 2-byte aligned): d = the group's fp16 scale,
 * q = code - 2^(bits-1), the inverse of tools/gguf_to_decoder.py:16-40 native_blob for any width and group. Groups
 * whose minimum is not exact are counted into the device int32 *inexact (added to, so zero it first); where it ends
 * non-zero the blocks do not hold the panel's values and the layer is expanded with idolq_panel_expand_f32 instead.
 * Same argument checks as idolq_panel_expand_f32. */
int idolq_panel_to_q8_0(const uint8_t* blob, int64_t blob_bytes, int64_t out, int64_t in, int bits, int group,
                        uint8_t* q8, int32_t* inexact, void* stream);

/* ---- The real decoders' operators (src/decoders.cpp), fp32 surface, in the reference's operation order. ---- */

/* Dense fp32 GEMM of any shape: y[m x n] = act(x[m x k] * w^T + bias + residual), w [n x k] row-major, bias NULL or
 * [n], residual NULL or [m x n] with row stride ldr (it may be y itself, with ldr == ldy; y must not overlap x).
 * Replaces the reference's gemm_packed on an unquantized PackedLinear (src/kernels.hpp:73-76,
 * src/kernels.cpp:566-596): the depth summed in 32-deep FMA chains added left to right, then bias, residual and the
 * activation (src/kernels.cpp:212-241), so the result is bit-identical to it. m < 65535 * 64. */
int idolq_gemm_f32(const float* x, int64_t m, int64_t k, int64_t ldx, const float* w, int64_t n, const float* bias,
                   const float* residual, int64_t ldr, int act, float* y, int64_t ldy, void* stream);

/* In place, for each row (row stride ld) and head: p = p * (sqrt(head_dim) / max(|p|, 1e-12)) * gamma[head, :], |p|
 * from the sum of squares taken in order (src/decoders.cpp:74-86 rms_heads). gamma fp32 [heads * head_dim]. */
int idolq_rms_heads(void* x, int dtype, int64_t rows, int64_t ld, int64_t heads, int64_t head_dim, const float* gamma,
                    void* stream);

/* x[r, c] += h[r, c] * gate[c] for r < rows, c < dim, one FMA per element (src/decoders.cpp:45-52 add_gated). */
int idolq_add_gated(void* x, int x_dtype, int64_t ldx, const void* h, int h_dtype, int64_t ldh, int64_t rows,
                    int64_t dim, const float* gate, void* stream);

/* Raw Gaussian features [rows x per_anchor * 15] of anchors [rows x 3] -> activated Gaussians (rows * per_anchor of
 * them): xyz, f_dc, scale [n x 3], rotation [n x 4] (unit quaternion, w first), opacity [n] (src/decoders.cpp:393-431
 * to_gaussians). perturbation [per_anchor x 3]; rep[10] = perturbe, kernel, lr_xyz, lr_dc, lr_opacity, lr_scaling,
 * lr_rotation, scale_offset, opacity_offset, base_offset_scale (all fp32). */
int idolq_to_gaussians(const float* anchors, int64_t rows, const float* features, int64_t per_anchor,
                       const float* perturbation, const float* rep, float* xyz, float* f_dc, float* scale,
                       float* rotation, float* opacity, void* stream);

/* The octree level embedding: out[i] = cos(((resolution * freqs[i]) * 2) * pi), out[half + i] = sin(same), fp32,
 * out [2 * half] (src/decoders.cpp:262-266). */
int idolq_level_embed(float resolution, const float* freqs, int64_t half, float* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* IDOLQ_H */
