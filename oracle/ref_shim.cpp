// extern "C" entry points over the reference's own CPU kernels, compiled from the reference sources where they lie
// (oracle/Makefile passes their directory with -I). TEST INFRASTRUCTURE ONLY: the result, oracle/_ref/libidolref.so,
// writes golden vectors (tests/golden/make_golden.py), validates the oracle restatement (tests/test_oracle.py) and
// is the timed CPU baseline in bench.py. It is never part of the product.
//
// kernels.cpp and decoders.cpp are included as one translation unit so that the helpers they keep in anonymous
// namespaces (quantize_activations, norm_rows, gelu_tanh) can be called directly; nothing in them is modified.
#include "kernels.cpp"
#include "decoders.cpp"

#include <cstdint>
#include <cstring>
#include <exception>
#include <string>
#include <vector>

namespace {

thread_local int g_status = 0;
thread_local std::string g_message;

template <typename F>
int guarded(F&& f) {
    try {
        f();
        return 0;
    } catch (const std::exception& e) {
        g_message = e.what();
        return -1;
    }
}

}  // namespace

extern "C" {

// 1 when the integer (AVX-VNNI) kernel can run on this CPU.
int ref_quant_int8_supported() { return idol::detail::quant_int8_supported() ? 1 : 0; }

// quantized_linear + gemm_packed. mode: 0 float kernel, 1 integer kernel (as set_quant_kernel).
int ref_gemm_panel(const float* a, int m, const std::uint8_t* blob, std::int64_t blob_bytes, const float* bias,
                   int out, int in, int bits, int group, int n_offset, int n, const float* residual, int gelu,
                   float* c, int mode) {
    return guarded([&] {
        std::vector<std::uint8_t> b(blob, blob + blob_bytes);
        std::vector<float> bv(bias, bias + out);
        const auto w = idol::detail::quantized_linear(std::move(b), bv, out, in, bits, group);
        idol::detail::set_quant_kernel(mode);
        idol::detail::gemm_packed(a, m, w, n_offset, n, residual, gelu != 0, c);
        idol::detail::set_quant_kernel(-1);
    });
}

// pack_linear + gemm_packed on dense fp32 weights [out x in].
int ref_gemm_dense(const float* a, int m, const float* weight, const float* bias, int out, int in, int n_offset,
                   int n, const float* residual, int gelu, float* c) {
    return guarded([&] {
        std::vector<float> wv(weight, weight + (std::size_t)out * in), bv(bias, bias + out);
        const auto w = idol::detail::pack_linear(wv, bv, out, in);
        idol::detail::gemm_packed(a, m, w, n_offset, n, residual, gelu != 0, c);
    });
}

// quantized_linear + dequantize_linear: the weights [out x in] the GEMM sees. Returns -1 when quantized_linear
// rejects the shape or blob.
int ref_dequantize_panel(const std::uint8_t* blob, std::int64_t blob_bytes, int out, int in, int bits, int group,
                         float* weight) {
    return guarded([&] {
        std::vector<std::uint8_t> b(blob, blob + blob_bytes);
        std::vector<float> bias(out, 0.0f);
        const auto w = idol::detail::quantized_linear(std::move(b), bias, out, in, bits, group);
        const auto d = idol::detail::dequantize_linear(w);
        std::copy(d.begin(), d.end(), weight);
    });
}

std::int64_t ref_quant_panel_bytes(int in, int bits, int group) {
    return (std::int64_t)idol::detail::quant_panel_bytes(in, bits, group);
}

// The integer kernel's activation quantization for group 32 (rows [0, m), no padding rows).
int ref_quantize_activations(const float* a, int m, int k, std::int8_t* qa, float* scale, std::int32_t* qsum) {
#ifdef IDOL_VNNI_PATH
    idol::detail::quantize_activations(a, m, m, k, 32, qa, scale, qsum);
    return 0;
#else
    (void)a, (void)m, (void)k, (void)qa, (void)scale, (void)qsum;
    return -1;
#endif
}

void ref_layer_norm(const float* x, int rows, int dim, const float* gamma, const float* beta, float* y) {
    idol::detail::layer_norm(x, rows, dim, gamma, beta, y);
}

void ref_norm_rows(const float* x, float* y, int rows, int dim, float eps, const float* gamma, const float* beta,
                   const float* shift, const float* scale) {
    idol::norm_rows(x, y, rows, dim, eps, gamma, beta, shift, scale);
}

void ref_attention(const float* q, int lq, int ldq, const float* k, const float* v, int lk, int ldkv, int heads,
                   int head_dim, float* out, int dim) {
    idol::detail::attention(q, lq, ldq, k, v, lk, ldkv, heads, head_dim, out, dim);
}

void ref_gelu_tanh(float* x, std::int64_t count) { idol::gelu_tanh(x, (std::size_t)count); }

// exp256 / gelu256 over count values (count a multiple of 8) and gelu_scalar over count values.
void ref_exp256(const float* x, std::int64_t count, float* y) {
    for (std::int64_t i = 0; i + 8 <= count; i += 8) _mm256_storeu_ps(y + i, idol::detail::exp256(_mm256_loadu_ps(x + i)));
}
void ref_gelu256(const float* x, std::int64_t count, float* y) {
    for (std::int64_t i = 0; i + 8 <= count; i += 8) _mm256_storeu_ps(y + i, idol::detail::gelu256(_mm256_loadu_ps(x + i)));
}
void ref_gelu_scalar(const float* x, std::int64_t count, float* y) {
    for (std::int64_t i = 0; i < count; ++i) y[i] = idol::detail::gelu_scalar(x[i]);
}

// set_quant_kernel: -1 decide from IDOL_QUANT_KERNEL and the CPU, 0 float kernel, 1 integer kernel.
void ref_set_quant_kernel(int mode) { idol::detail::set_quant_kernel(mode); }

// The message of the last exception a guarded call caught on this thread.
const char* ref_last_error() { return g_message.c_str(); }

// rms_heads and add_gated of src/decoders.cpp, in place.
void ref_rms_heads(float* x, int rows, int ld, int heads, int hd, const float* gamma) {
    idol::rms_heads(x, rows, ld, heads, hd, gamma);
}
void ref_add_gated(float* x, const float* h, int rows, int dim, const float* gate) {
    idol::add_gated(x, h, rows, dim, gate);
}

// idol::Decoders over an export directory: open (NULL on failure, message in ref_last_error), query, run, close.
void* ref_decoders_open(const char* dir) {
    idol::Decoders* d = nullptr;
    guarded([&] { d = new idol::Decoders(dir); });
    return d;
}
void ref_decoders_close(void* d) { delete static_cast<idol::Decoders*>(d); }
void ref_decoders_config(void* d, int* cfg) {
    const idol::DecoderConfig& c = static_cast<idol::Decoders*>(d)->config();
    const int v[6] = {c.dim, c.heads, c.oct_blocks, c.gs_blocks, c.cond, c.per_anchor};
    std::memcpy(cfg, v, sizeof v);
}
std::int64_t ref_decoders_weight_bytes(void* d) { return (std::int64_t)static_cast<idol::Decoders*>(d)->weight_bytes(); }
int ref_decoders_octree_logits(void* d, const float* x, int rows, float resolution, const float* cond, int cond_rows,
                               float* out) {
    return guarded([&] { static_cast<idol::Decoders*>(d)->octree_logits(x, rows, resolution, cond, cond_rows, out); });
}
int ref_decoders_gaussian_features(void* d, const float* points, int rows, const float* cond, int cond_rows,
                                   float* out) {
    return guarded([&] { static_cast<idol::Decoders*>(d)->gaussian_features(points, rows, cond, cond_rows, out); });
}

// The generator and distribution the reference's sampling uses (src/decoders.cpp:338-339): count uniform floats in
// [0, 1) from std::mt19937_64(seed) through std::uniform_real_distribution<float>, and the raw 64-bit outputs.
void ref_uniform_floats(std::uint64_t seed, std::int64_t count, float* out, std::uint64_t* raw) {
    std::mt19937_64 rng(seed), rng2(seed);
    std::uniform_real_distribution<float> uniform(0.0f, 1.0f);
    for (std::int64_t i = 0; i < count; ++i) {
        out[i] = uniform(rng);
        if (raw) raw[i] = rng2();
    }
}

// Decoders::sample_anchors (num_points x 3 into out), to_gaussians (anchors rows x 3, features rows x G*15 ->
// xyz, f_dc, scale [n x 3], rotation [n x 4], opacity [n]) and write_gaussian_ply of such a cloud.
int ref_decoders_sample_anchors(void* d, const float* cond, int cond_rows, int num_points, int level,
                                std::uint64_t seed, float* out) {
    return guarded([&] {
        const std::vector<float> p = static_cast<idol::Decoders*>(d)->sample_anchors(cond, cond_rows, num_points,
                                                                                     level, seed);
        std::copy(p.begin(), p.end(), out);
    });
}
int ref_decoders_to_gaussians(void* d, const float* anchors, int rows, const float* features, float* xyz,
                              float* f_dc, float* scale, float* rotation, float* opacity) {
    return guarded([&] {
        const idol::GaussianCloud c = static_cast<idol::Decoders*>(d)->to_gaussians(anchors, rows, features);
        std::copy(c.xyz.begin(), c.xyz.end(), xyz);
        std::copy(c.f_dc.begin(), c.f_dc.end(), f_dc);
        std::copy(c.scale.begin(), c.scale.end(), scale);
        std::copy(c.rotation.begin(), c.rotation.end(), rotation);
        std::copy(c.opacity.begin(), c.opacity.end(), opacity);
    });
}
int ref_write_gaussian_ply(const float* xyz, const float* f_dc, const float* scale, const float* rotation,
                           const float* opacity, std::int64_t n, const char* path) {
    return guarded([&] {
        idol::GaussianCloud c;
        c.xyz.assign(xyz, xyz + n * 3);
        c.f_dc.assign(f_dc, f_dc + n * 3);
        c.scale.assign(scale, scale + n * 3);
        c.rotation.assign(rotation, rotation + n * 4);
        c.opacity.assign(opacity, opacity + n);
        idol::write_gaussian_ply(c, path);
    });
}

}  // extern "C"
