/*
 * CPU oracle for the Q8_0 block-quantized linear path: a plain-C restatement of the reference algorithm.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (the HIP library or the Python host modules) may link, load or
 * call this code. It is imported by tests/, by __graft_entry__.smoke() and by bench.py's cpu_baseline leg, and
 * only to check results against, never as the thing measured or shipped.
 *
 * Every function cites the reference file:line it restates (paths relative to the reference checkout). All
 * functions are single-precision IEEE code built with -ffp-contract=off; where the reference build fuses a
 * multiply-add (explicit _mm256_fmadd_ps, or GCC contraction of a*b+c under -mfma), the restatement writes fmaf
 * explicitly, so the results are bit-identical to the reference build (pinned by tests/test_oracle.py).
 *
 * Parity pins (which check fixes each function):
 *   orc_half_to_float / orc_float_to_half   numpy float16 casts over all 65536 half values and 1e6 floats
 *   orc_q8_0_quantize                       closed form of ggml's quantize_row_q8_0_ref (gguf-py Q8_0); the exact
 *                                           codes of gguf-py 0.19.0 are PARITY UNPINNED (gguf is not installed)
 *   orc_q8_0_dequant, orc_q8_0_to_panel     closed form w = fp32(d)*q; reference dequantize_linear on the panel
 *   orc_gemm_q8_float                       reference gemm_packed (float kernel) golden vectors, bit-exact
 *   orc_gemm_dense                          reference gemm_packed on dense fp32 weights (live build), bit-exact
 *   orc_quantize_act, orc_gemm_q8_int8      reference quantize_activations / gemm_packed (int8 kernel), bit-exact
 *   orc_layer_norm, orc_norm_rows           reference layer_norm / norm_rows, bit-exact
 *   orc_attention                           reference attention (blocked and dot paths), bit-exact
 *   orc_exp256, orc_gelu_erf, orc_gelu_scalar, orc_gelu_tanh   reference exp256/gelu256/gelu_scalar/gelu_tanh
 *   orc_pos_embed                           reference Decoders::Impl::pos_embed semantics (libm sinf/cosf)
 */
#ifndef IDOLQ_ORACLE_H
#define IDOLQ_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

float orc_half_to_float(uint16_t h);
uint16_t orc_float_to_half(float f);  /* round to nearest even, like F16C _MM_FROUND_TO_NEAREST_INT */
void orc_half_to_float_n(const uint16_t* h, int64_t count, float* out);
void orc_float_to_half_n(const float* f, int64_t count, uint16_t* out);

/* Q8_0 blocks: 34 bytes per 32 consecutive k of one output row, fp16 d (little endian) then 32 int8 q. */
void orc_q8_0_quantize(const float* w, int64_t n, int64_t k, uint8_t* blocks);
void orc_q8_0_dequant(const uint8_t* blocks, int64_t n, int64_t k, float* w);
/* GGUF Q8_0 -> native 8-bit group-32 panel blob (code = q + 128, scale = d, min = -128 d). Returns 0, or -1 when
 * -128 d is not exact in fp16. */
int orc_q8_0_to_panel(const uint8_t* blocks, int64_t n, int64_t k, uint8_t* blob);
int64_t orc_panel_bytes(int64_t n, int64_t k);

/* Epilogue activations. */
enum { ORC_ACT_NONE = 0, ORC_ACT_GELU_ERF = 1, ORC_ACT_GELU_TANH = 2, ORC_ACT_RELU = 3 };

/* C[m x n] = A[m x k] * W^T + bias for output columns [n_offset, n_offset + n) of a Q8_0 weight with n_total rows.
 * bias has n_total entries (NULL means zero), residual and c have row stride n, residual may alias c. gelu != 0
 * applies the reference's erf-GELU after the residual. Float kernel semantics. */
void orc_gemm_q8_float(const float* a, int64_t m, const uint8_t* w, int64_t n_total, int64_t k, const float* bias,
                       int64_t n_offset, int64_t n, const float* residual, int gelu, float* c);
/* Dense fp32 weights [n_total x k] (an unquantized layer), same chunked summation and epilogue (no residual). */
void orc_gemm_dense(const float* a, int64_t m, const float* w, int64_t n_total, int64_t k, const float* bias,
                    int64_t n_offset, int64_t n, int gelu, float* c);
/* Integer kernel semantics: activations quantized per row and 32-group, int32 block dots, per-group fold. */
void orc_quantize_act(const float* a, int64_t m, int64_t k, int8_t* qa, float* scale, int32_t* qsum);
void orc_gemm_q8_int8(const float* a, int64_t m, const uint8_t* w, int64_t n_total, int64_t k, const float* bias,
                      int64_t n_offset, int64_t n, const float* residual, int gelu, float* c);
/* dots[(i * n + j) * (k / 32) + b] = sum over block b of qa[i, :] * q[n_offset + j, :] (int8 x int8 -> int32). */
void orc_block_dots(const int8_t* qa, int64_t m, const uint8_t* w, int64_t n_offset, int64_t n, int64_t k,
                    int32_t* dots);

void orc_layer_norm(const float* x, int64_t rows, int64_t dim, const float* gamma, const float* beta, float* y);
/* shift/scale (adaLN) are indexed [row / rows_per_batch][dim] when rows_per_batch > 0 (else a single vector). */
void orc_norm_rows(const float* x, float* y, int64_t rows, int64_t dim, float eps, const float* gamma,
                   const float* beta, const float* shift, const float* scale, int64_t rows_per_batch);
void orc_attention(const float* q, int64_t lq, int64_t ldq, const float* k, const float* v, int64_t lk, int64_t ldkv,
                   int64_t heads, int64_t head_dim, float* out, int64_t dim);

void orc_exp256(const float* x, int64_t count, float* y);
void orc_gelu_erf(const float* x, int64_t count, float* y);    /* gelu256, lane by lane */
void orc_gelu_scalar(const float* x, int64_t count, float* y);
void orc_gelu_tanh(float* x, int64_t count);                   /* in place, 8-wide body and scalar tail */
void orc_pos_embed(const float* freqs, int64_t nfreq, const float* coords, int64_t rows, float* out, int64_t ldo);

#ifdef __cplusplus
}
#endif

#endif
