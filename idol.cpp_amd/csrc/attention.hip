// Non-causal multi-head attention for gfx950.
//
// attn_mfma_hd64 (bf16/fp16 inputs, head_dim 64): a flash-style kernel. A workgroup of 4 waves owns 128 queries of
// one (batch, head); each wave owns 32 queries. Key/value tiles of 64 rows are staged in LDS (K as [key][d],
// V transposed to [d][key] in fp16) and shared by the 4 waves. Scores are computed transposed, S^T = K * Q^T, so a
// lane holds 32 scores of a single query (its column) and the online softmax (fp32, base-2 exponent with the
// 1/sqrt(64) * log2(e) factor folded in) needs one cross-lane exchange (lanes l and l + 32). The running maximum is
// raised only when a tile exceeds it by more than 2^8 in probability, so most tiles skip rescaling. The probabilities
// stay in registers and become, converted to fp16, the B operand of O^T = V^T * P^T (the row sums are taken from the
// same fp16 values with dot2); the MFMA's k order is permuted to the order in which the score accumulator holds the
// keys, and the V^T operand is read in that same order. bf16 values of V beyond fp16's range (|v| >= 65504) are
// staged scaled by a power of two per tile and the tile's product is scaled back exactly, so the fp16 P * V never
// overflows where the reference's fp32 attention does not. With a workspace (idolq_attention_ws), attn_v_tiles
// converts bf16 V into those fp16 V^T tiles once per call and the workgroups copy them (the same operands, so the
// same bits). 16-bit outputs leave through LDS as 16-byte row pieces.
//
// attn_f32_mfma (fp32 inputs, head_dim 32 or 64, 16-byte aligned rows): fp32 matrix cores for both products, the key
// range split over the 4 waves of a 32-query workgroup; the reference's float attention surface at fp32 accuracy.
//
// attn_f32 (any dtype, head_dim <= 256): one wave per (query, head, batch), 64 keys per step with one key per lane
// for the scores and the head dimension split over lanes for P * V; fp32 throughout. Used for the remaining fp32
// cases (unaligned rows, other head sizes) and 16-bit inputs with head sizes other than 64.
#include "common.h"

#include <type_traits>

namespace idolq {
namespace {

struct AttnParams {
    const void* q;
    const void* k;
    const void* v;
    void* out;
    int dt, out_dt;
    int64_t lq, lk, heads, head_dim;
    int64_t ldq, ldkv, q_bs, kv_bs, ldo, o_bs;
    float scale_log2;  // log2(e) / sqrt(head_dim)
    // V staged ahead of attn_mfma_hd64<bf16, true> by attn_v_tiles: fp16 V^T tiles and their exponents
    const uint16_t* vt;
    const int* vexps;
    int64_t ntiles;
    int out_vec;  // out has the input dtype and 16-byte aligned rows and batches: rows go out as 16-byte stores
};

constexpr int kHD = 64;
constexpr int kBQ = 128;
constexpr int kBKV = 64;
constexpr int kKPitch = kHD + 8;    // elements per key row of K in LDS (144 bytes: conflict-free 16-byte reads)
constexpr int kVPitch = kBKV + 4;   // elements per d row of V^T in LDS (136 bytes: conflict-free 8-byte reads)

template <typename T>
struct AttnMfma;
template <>
struct AttnMfma<__bf16> {
    typedef bf16x8 vec;
    static __device__ __forceinline__ f32x16 run(vec a, vec b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
};
template <>
struct AttnMfma<_Float16> {
    typedef f16x8 vec;
    static __device__ __forceinline__ f32x16 run(vec a, vec b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
};

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));


// VT (bf16 inputs): V comes as the fp16 V^T tiles attn_v_tiles wrote (scaled by 2^-vexps[tile]), so staging a tile
// is a copy instead of each workgroup converting, transposing and range-checking it again.
template <typename T, bool VT = false>
__global__ __launch_bounds__(256, 3) void attn_mfma_hd64(AttnParams p) {
    typedef typename AttnMfma<T>::vec Vec;
    static_assert(!VT || std::is_same<T, __bf16>::value, "staged V^T tiles are for bf16 inputs");
    // two key/value tiles in LDS: tile j is read from buffer j % 2 while tile j + 1 is loaded into registers and then
    // written to the other buffer; one barrier per tile publishes the next tile
    __shared__ __attribute__((aligned(16))) uint16_t k_lds[2][kBKV * kKPitch];
    __shared__ __attribute__((aligned(16))) uint16_t vt_lds[2][kHD * kVPitch];
    __shared__ uint32_t vote[2][4];
    __shared__ uint32_t vexp_vote[4];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t b = blockIdx.z, h = blockIdx.y;
    const int64_t q0 = (int64_t)blockIdx.x * kBQ + wave * 32;
    const int64_t qi = q0 + (lane & 31);
    const int half = lane >> 5;

    const uint16_t* qbase = static_cast<const uint16_t*>(p.q) + b * p.q_bs + h * kHD;
    // K and V rows through buffer loads: keys past lk get an offset past the buffer and read 0 (no branch around the
    // loads); the host keeps lk * ldkv elements below 2^30
    constexpr uint32_t kOff = 0x80000000u;
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(static_cast<const uint16_t*>(p.k) + b * p.kv_bs + h * kHD), 0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(static_cast<const uint16_t*>(p.v) + b * p.kv_bs + h * kHD), 0, 0x7fffffff, 0x00020000);

    // Q^T operand: lane supplies query qi, d = 16 c + 8 half + e.
    Vec qf[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        uint4 raw = make_uint4(0, 0, 0, 0);
        if (qi < p.lq) raw = *reinterpret_cast<const uint4*>(qbase + qi * p.ldq + 16 * c + 8 * half);
        qf[c] = __builtin_bit_cast(Vec, raw);
    }

    f32x16 o[2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[t][r] = 0.0f;

    // The running maximum mc is kept in the scaled (base-2) domain: the first tile's maximum, raised lazily
    // afterwards, only for a tile whose fp16 probabilities sum to 2^15 or more (some score more than 10 above mc),
    // so every probability stays inside fp16 and most tiles neither take a maximum nor rescale o and l. Scores are
    // turned into u = s * c - mc first (a maximum is taken over u: products of an FMA need no NaN canonicalization,
    // MFMA results would). l is summed per lane (half of each query's keys) and combined at the end.
    const float c = p.scale_log2;
    float mc = -INFINITY, l_part = 0.0f;
    const f16x2 ones = {(_Float16)1.0f, (_Float16)1.0f};

    // bf16 V beyond the fp16 range: a tile holding |v| >= 65504 is staged as fp16(v * 2^-e), exactly scaled by the
    // power of two that brings its largest magnitude below 2^15, and its P * V is added as 2^e (2^-e o + P V')
    // (exact scalings); other tiles, and every fp16 input, take the plain fp16 V^T.
    constexpr bool kWideV = std::is_same<T, __bf16>::value;

    // staging: thread t takes keys 2 (t / 8) and 2 (t / 8) + 1, d chunk 8 (t % 8); V^T gets one (key, key + 1) pair
    // per d and dword store
    const int kp = threadIdx.x >> 3, part = threadIdx.x & 7;
    uint4 kr[2], vr[2];
    int vexp_cur = VT ? p.vexps[(b * p.heads + h) * p.ntiles] : 0;  // VT: the exponent of the next step's tile
    // VT: thread t copies 32 bytes of the staged tile, d row t / 4, keys 16 (t % 4) .. + 16
    const uint16_t* vt_bh = VT ? p.vt + ((b * p.heads + h) * p.ntiles) * (kHD * kBKV) : nullptr;
    auto load_tile = [&](int64_t j0) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int64_t key = j0 + 2 * kp + i;
            const uint32_t off = key < p.lk ? (uint32_t)(key * p.ldkv + 8 * part) * 2u : kOff;
            kr[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 0));
            if constexpr (!VT)
                vr[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 0));
            else
                vr[i] = *reinterpret_cast<const uint4*>(vt_bh + (j0 / kBKV) * (kHD * kBKV) + 16 * threadIdx.x + 8 * i);
        }
    };
    // the V values of thread-local element e of key kp2 + i (16-bit bits)
    auto vbits = [&](int i, int e) __attribute__((always_inline)) {
        const uint32_t word = (e >> 1) == 0 ? vr[i].x : (e >> 1) == 1 ? vr[i].y : (e >> 1) == 2 ? vr[i].z : vr[i].w;
        return (uint16_t)(word >> (16 * (e & 1)));
    };
    // registers -> LDS buffer buf; with kWideV, records whether any staged |v| >= 65504 (one vote per wave)
    auto stage_tile = [&](int buf) __attribute__((always_inline)) {
        bool big = false;
#pragma unroll
        for (int i = 0; i < 2; ++i) *reinterpret_cast<uint4*>(&k_lds[buf][(2 * kp + i) * kKPitch + 8 * part]) = kr[i];
        if constexpr (VT) {
            // rows of kVPitch elements are 8-byte aligned: four 8-byte stores
            uint16_t* dst = &vt_lds[buf][(threadIdx.x >> 2) * kVPitch + 16 * (threadIdx.x & 3)];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                *reinterpret_cast<uint2*>(dst + 8 * i) = make_uint2(vr[i].x, vr[i].y);
                *reinterpret_cast<uint2*>(dst + 8 * i + 4) = make_uint2(vr[i].z, vr[i].w);
            }
            return;
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint16_t b0 = vbits(0, e), b1 = vbits(1, e);
            f16x2 pair;
            if constexpr (!kWideV) {
                pair = f16x2{__builtin_bit_cast(_Float16, b0), __builtin_bit_cast(_Float16, b1)};
            } else {
                const f32x2 f = {bf16_bits_to_float(b0), bf16_bits_to_float(b1)};
                big = big || fabsf(f.x) >= 65504.0f || fabsf(f.y) >= 65504.0f;
                pair = __builtin_convertvector(f, f16x2);
            }
            *reinterpret_cast<f16x2*>(&vt_lds[buf][(8 * part + e) * kVPitch + 2 * kp]) = pair;
        }
        if constexpr (kWideV) {
            const uint32_t wave_big = __builtin_amdgcn_ballot_w64(big) != 0 ? 1u : 0u;  // every lane takes part
            if (lane == 0) vote[buf][wave] = wave_big;
        }
    };
    // the rare path for tile buf (after the barrier that published it, while vr still holds its values): every wave
    // saw the same votes, so the whole workgroup re-stages its V^T scaled by 2^-vexp; returns vexp
    auto rescale_tile = [&](int buf) __attribute__((always_inline)) {
        // the largest exponent field among the tile's values (bf16 bits 14..7)
        uint32_t eb = 0;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t w4[4] = {vr[i].x, vr[i].y, vr[i].z, vr[i].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) eb = max(eb, max(w4[e] & 0x7f80u, (w4[e] >> 16) & 0x7f80u));
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) eb = max(eb, (uint32_t)__shfl_xor((int)eb, off));
        if (lane == 0) vexp_vote[wave] = eb;
        __syncthreads();
        eb = max(max(vexp_vote[0], vexp_vote[1]), max(vexp_vote[2], vexp_vote[3]));
        // |v| < 2^(E + 1), E = (eb >> 7) - 127 >= 15: scaled by 2^-(E - 14) every value is below 2^15
        const int vexp = (int)(eb >> 7) - 127 - 14;
        const float down = __builtin_bit_cast(float, (uint32_t)(127 - vexp) << 23);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const f32x2 f = {bf16_bits_to_float(vbits(0, e)) * down, bf16_bits_to_float(vbits(1, e)) * down};
            *reinterpret_cast<f16x2*>(&vt_lds[buf][(8 * part + e) * kVPitch + 2 * kp]) = __builtin_convertvector(f, f16x2);
        }
        __syncthreads();  // the scaled V^T is in place; every wave has read vexp_vote
        return vexp;
    };

    // the scores, softmax and P * V of the tile in buffer buf (keys j0 ..); MASK: the last tile, which holds fewer
    // than 64 keys; FIRST: the first tile, which sets mc
    auto compute = [&](int buf, int64_t j0, int vexp, auto mask_tag, auto first_tag) __attribute__((always_inline)) {
        constexpr bool MASK = decltype(mask_tag)::value, FIRST = decltype(first_tag)::value;
        // S^T for 64 keys: two 32-key sub-tiles, 4 MFMAs each over d.
        f32x16 s[2];
#pragma unroll
        for (int st = 0; st < 2; ++st) {
#pragma unroll
            for (int c4 = 0; c4 < 4; ++c4) {
                const Vec a = *reinterpret_cast<const Vec*>(&k_lds[buf][(st * 32 + (lane & 31)) * kKPitch + 16 * c4 + 8 * half]);
                s[st] = AttnMfma<T>::run(a, qf[c4], c4 == 0 ? f32x16{} : s[st]);
            }
        }
        // The V^T operands of the product (chunk (st, kc), d block t): those of the first 32 keys are read now, so
        // that their LDS latency passes under the softmax's vector work, the others before the product (under the
        // first half's MFMAs), instead of each P * V MFMA waiting for its own read.
        f16x8 va[2][2][2];
        auto read_v = [&](int st) __attribute__((always_inline)) {
#pragma unroll
            for (int kc = 0; kc < 2; ++kc)
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const int d = t * 32 + (lane & 31), key0 = st * 32 + 16 * kc + 4 * half;
                    const uint2 lo = *reinterpret_cast<const uint2*>(&vt_lds[buf][d * kVPitch + key0]);
                    const uint2 hi = *reinterpret_cast<const uint2*>(&vt_lds[buf][d * kVPitch + key0 + 8]);
                    va[st][kc][t] = __builtin_bit_cast(f16x8, make_uint4(lo.x, lo.y, hi.x, hi.y));
                }
        };
        read_v(0);
        if (MASK) {
            // keys past lk get no weight
            const int valid = (int)(p.lk - j0);
#pragma unroll
            for (int st = 0; st < 2; ++st)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (st * 32 + 8 * (r >> 2) + 4 * half + (r & 3) >= valid) s[st][r] = -INFINITY;
        }
        if (FIRST) {
            float mx = -INFINITY;
#pragma unroll
            for (int i = 0; i < 32; ++i) mx = fmaxf(mx, s[i >> 4][i & 15]);
            mc = fmaxf(mx, __shfl_xor(mx, 32)) * c;
        }
#pragma unroll
        for (int i = 0; i < 32; ++i) s[i >> 4][i & 15] = fmaf(s[i >> 4][i & 15], c, -mc);
        // The probabilities as fp16 MFMA operands, chunk (st, kc) holding keys st*32 + 16 kc + ..., and this lane's
        // sum of them as rounded (fp32 dot products with ones).
        f16x8 pf[2][2];
        float lt;
        auto probabilities = [&]() __attribute__((always_inline)) {
            float ls[2] = {0.0f, 0.0f};  // two dependent chains of dot products instead of one
#pragma unroll
            for (int st = 0; st < 2; ++st)
#pragma unroll
                for (int kc = 0; kc < 2; ++kc)
#pragma unroll
                    for (int e = 0; e < 8; e += 2) {
                        const f32x2 pe = {__builtin_amdgcn_exp2f(s[st][8 * kc + e]),
                                          __builtin_amdgcn_exp2f(s[st][8 * kc + e + 1])};
                        const f16x2 hp = __builtin_convertvector(pe, f16x2);
                        pf[st][kc][e] = hp.x;
                        pf[st][kc][e + 1] = hp.y;
                        ls[st] = __builtin_amdgcn_fdot2(hp, ones, ls[st], false);
                    }
            lt = ls[0] + ls[1];
        };
        probabilities();
        if (!FIRST) {
            // The maximum is not taken per tile: a score more than 16 above mc overflows its fp16 probability (inf)
            // and so the sum. A sum that is not below 2^15 (inf or NaN included; every probability below 2^8 keeps
            // it under 2^13) sends the wave through the rare path (a wave-uniform branch): the lanes whose query's
            // maximum (over both lanes of the query, lane ^ 32) exceeds mc by more than 8 raise mc to it, scale o
            // and l by 2^-delta, and the tile's probabilities are recomputed.
            if (__builtin_amdgcn_ballot_w64(!(lt < 32768.0f)) != 0) {
                float mx = -INFINITY;
#pragma unroll
                for (int i = 0; i < 32; i += 2) mx = fmaxf(mx, fmaxf(s[i >> 4][i & 15], s[i >> 4][(i & 15) + 1]));
                mx = fmaxf(mx, __shfl_xor(mx, 32));
                const bool raise = mx > 8.0f;
                const float delta = raise ? mx : 0.0f;
                const float alpha = __builtin_amdgcn_exp2f(-delta);
                l_part *= alpha;
#pragma unroll
                for (int t = 0; t < 2; ++t)
#pragma unroll
                    for (int r = 0; r < 16; ++r) o[t][r] *= alpha;
#pragma unroll
                for (int i = 0; i < 32; ++i) s[i >> 4][i & 15] -= delta;
                mc += delta;
                probabilities();
            }
        }
        l_part += lt;

        // O^T += V^T * P^T over 4 chunks of 16 keys. Chunk (st, kc) uses accumulator elements r = 8 kc + e of
        // sub-tile st; slot 8 * half + e of the MFMA's k holds key st*32 + 16 kc + 8 (e / 4) + 4 half + e % 4.
        if (kWideV && vexp != 0) {
            const float down = __builtin_bit_cast(float, (uint32_t)(127 - vexp) << 23);
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[t][r] *= down;
        }
        read_v(1);
        // raised wave priority while the product issues, so that the SIMD's other waves (in their softmax) do not
        // delay its MFMAs (1-2% on the self-attention shape)
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int st = 0; st < 2; ++st)
#pragma unroll
            for (int kc = 0; kc < 2; ++kc)
#pragma unroll
                for (int t = 0; t < 2; ++t) o[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va[st][kc][t], pf[st][kc], o[t], 0, 0, 0);
        __builtin_amdgcn_s_setprio(0);
        if (kWideV && vexp != 0) {
            const float up = __builtin_bit_cast(float, (uint32_t)(127 + vexp) << 23);
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[t][r] *= up;
        }
    };
    // tile j0 (in buffer buf): the rare rescaling, the next tile's loads, the product, the next tile's staging and
    // the barrier that publishes it
    auto step = [&](int buf, int64_t j0, bool has_next, auto mask_tag, auto first_tag) __attribute__((always_inline)) {
        int vexp = 0;
        if constexpr (VT) {
            vexp = vexp_cur;
            if (has_next) vexp_cur = p.vexps[(b * p.heads + h) * p.ntiles + (j0 + kBKV) / kBKV];
        } else if constexpr (kWideV) {
            if ((vote[buf][0] | vote[buf][1] | vote[buf][2] | vote[buf][3]) != 0) vexp = rescale_tile(buf);  // uniform
        }
        if (has_next) load_tile(j0 + kBKV);
        compute(buf, j0, vexp, mask_tag, first_tag);
        if (has_next) stage_tile(buf ^ 1);
        __syncthreads();
    };

    load_tile(0);
    stage_tile(0);
    __syncthreads();
    const int64_t full_end = p.lk / kBKV * kBKV;
    if (full_end == 0) {
        step(0, 0, false, std::true_type{}, std::true_type{});
    } else {
        const bool tail = full_end < p.lk;
        step(0, 0, kBKV < p.lk, std::false_type{}, std::true_type{});
        int buf = 1;
        for (int64_t j0 = kBKV; j0 < full_end; j0 += kBKV, buf ^= 1)
            step(buf, j0, j0 + kBKV < p.lk, std::false_type{}, std::false_type{});
        if (tail) step(buf, full_end, false, std::true_type{}, std::false_type{});
    }

    const float l_run = l_part + __shfl_xor(l_part, 32);
    const float inv = 1.0f / l_run;
    if (p.out_vec) {
        // the wave's 32 query rows x 64 d in the input type through its part of k_lds (free after the last tile's
        // barrier), then read back as whole 16-byte pieces of rows: four row-contiguous stores per lane instead of
        // 32 scattered 2-byte ones
        uint16_t* ob = &k_lds[0][0] + wave * 32 * kKPitch;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; r += 2) {
                const int d = t * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
                const float v0 = o[t][r] * inv, v1 = o[t][r + 1] * inv;
                const uint32_t w = std::is_same<T, __bf16>::value
                                       ? (uint32_t)float_to_bf16_bits(v0) | ((uint32_t)float_to_bf16_bits(v1) << 16)
                                       : (uint32_t)float_to_half_bits(v0) | ((uint32_t)float_to_half_bits(v1) << 16);
                *reinterpret_cast<uint32_t*>(&ob[(lane & 31) * kKPitch + d]) = w;
            }
        // the wave's LDS operations run in order; the fences keep the compiler from moving the reads above the writes
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = lane + 64 * i, row = c >> 3, cc = c & 7;
            const uint4 v = *reinterpret_cast<const uint4*>(&ob[row * kKPitch + 8 * cc]);
            const int64_t q = q0 + row;
            if (q < p.lq)
                *reinterpret_cast<uint4*>(static_cast<uint16_t*>(p.out) + b * p.o_bs + q * p.ldo + h * kHD + 8 * cc) = v;
        }
        return;
    }
    if (qi >= p.lq) return;
    const int64_t obase = b * p.o_bs + qi * p.ldo + h * kHD;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int d = t * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
            store_from_float(p.out, p.out_dt, obase + d, o[t][r] * inv);
        }
}

// bf16 V -> the fp16 V^T tiles of attn_mfma_hd64<bf16, true>, once per call instead of once per query workgroup:
// tile j of (batch b, head h) is 64 d rows x 64 keys at ((b heads + h) ntiles + j) x 4096 elements (keys past lk are
// 0), scaled by 2^-vexps[...] with the rule of the in-kernel path: a tile holding a finite |v| >= 65504 (no bf16
// value lies in [65504, 65536)) or an infinity takes vexp = E - 14, E its largest exponent, so every scaled value is
// below 2^15; other tiles 0. One workgroup per tile; the transpose goes through LDS so the stores are 16-byte rows.
__global__ __launch_bounds__(256) void attn_v_tiles(AttnParams p, uint16_t* __restrict__ vt, int* __restrict__ vexps) {
    __shared__ __attribute__((aligned(16))) uint16_t tr[kHD * (kBKV + 8)];
    __shared__ uint32_t red[2][4];
    const int64_t j = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kp = tid >> 3, part = tid & 7;
    const uint16_t* vbase = static_cast<const uint16_t*>(p.v) + b * p.kv_bs + h * kHD;
    uint4 vr[2];
    uint32_t ex = 0, fin = 0;  // the largest exponent field (any value) and the largest finite magnitude's bits
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int64_t key = j * kBKV + 2 * kp + i;
        vr[i] = key < p.lk ? *reinterpret_cast<const uint4*>(vbase + key * p.ldkv + 8 * part) : make_uint4(0, 0, 0, 0);
        const uint32_t w4[4] = {vr[i].x, vr[i].y, vr[i].z, vr[i].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t m = (w4[e >> 1] >> (16 * (e & 1))) & 0x7fffu;
            ex = max(ex, m & 0x7f80u);
            fin = max(fin, m <= 0x7f80u ? m : 0u);  // NaN is not counted, as fabsf(NaN) >= 65504 is false
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        ex = max(ex, (uint32_t)__shfl_xor((int)ex, off));
        fin = max(fin, (uint32_t)__shfl_xor((int)fin, off));
    }
    if (lane == 0) red[0][wave] = ex, red[1][wave] = fin;
    __syncthreads();
    ex = max(max(red[0][0], red[0][1]), max(red[0][2], red[0][3]));
    fin = max(max(red[1][0], red[1][1]), max(red[1][2], red[1][3]));
    const int vexp = fin >= 0x4780u ? (int)(ex >> 7) - 127 - 14 : 0;
    const float down = __builtin_bit_cast(float, (uint32_t)(127 - vexp) << 23);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint32_t w0 = e >> 1 == 0 ? vr[0].x : e >> 1 == 1 ? vr[0].y : e >> 1 == 2 ? vr[0].z : vr[0].w;
        const uint32_t w1 = e >> 1 == 0 ? vr[1].x : e >> 1 == 1 ? vr[1].y : e >> 1 == 2 ? vr[1].z : vr[1].w;
        const f32x2 f = {bf16_bits_to_float((uint16_t)(w0 >> (16 * (e & 1)))) * down,
                         bf16_bits_to_float((uint16_t)(w1 >> (16 * (e & 1)))) * down};
        *reinterpret_cast<f16x2*>(&tr[(8 * part + e) * (kBKV + 8) + 2 * kp]) = __builtin_convertvector(f, f16x2);
    }
    __syncthreads();
    // thread t stores 32 bytes: d row t / 4, keys 16 (t % 4) .. + 16
    const int d = tid >> 2, c = tid & 3;
    const uint4 a0 = *reinterpret_cast<const uint4*>(&tr[d * (kBKV + 8) + 16 * c]);
    const uint4 a1 = *reinterpret_cast<const uint4*>(&tr[d * (kBKV + 8) + 16 * c + 8]);
    uint16_t* dst = vt + ((b * p.heads + h) * p.ntiles + j) * (kHD * kBKV) + d * kBKV + 16 * c;
    *reinterpret_cast<uint4*>(dst) = a0;
    *reinterpret_cast<uint4*>(dst + 8) = a1;
    if (tid == 0) vexps[(b * p.heads + h) * p.ntiles + j] = vexp;
}

// ------------------------------------------------------------------------------------------------ fp32 kernel
constexpr int kMaxHD = 256;

__global__ __launch_bounds__(64) void attn_f32(AttnParams p) {
    __shared__ float qs[kMaxHD];
    __shared__ float ps[64];
    const int lane = threadIdx.x;
    const int64_t qi = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int64_t hd = p.head_dim;
    const int64_t qo = b * p.q_bs + qi * p.ldq + h * hd;
    for (int64_t d = lane; d < hd; d += 64) qs[d] = load_as_float(p.q, p.dt, qo + d);
    __syncthreads();
    const float scale = 1.0f / sqrtf((float)hd);
    float acc[kMaxHD / 64];
#pragma unroll
    for (int i = 0; i < kMaxHD / 64; ++i) acc[i] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;
    const int64_t kvo = b * p.kv_bs + h * hd;
    for (int64_t j0 = 0; j0 < p.lk; j0 += 64) {
        const int64_t j = j0 + lane;
        float sc = -INFINITY;
        if (j < p.lk) {
            float dot = 0.0f;
            for (int64_t d = 0; d < hd; ++d) dot = fmaf(qs[d], load_as_float(p.k, p.dt, kvo + j * p.ldkv + d), dot);
            sc = dot * scale;
        }
        float mx = sc;
        for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
        const float m_new = fmaxf(m_run, mx);
        const float alpha = expf(m_run - m_new);
        const float e = j < p.lk ? expf(sc - m_new) : 0.0f;
        float sum = e;
        for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
        l_run = l_run * alpha + sum;
        m_run = m_new;
        __syncthreads();
        ps[lane] = e;
        __syncthreads();
        const int64_t nk = p.lk - j0 < 64 ? p.lk - j0 : 64;
#pragma unroll
        for (int i = 0; i < kMaxHD / 64; ++i) {
            const int64_t d = lane + 64 * i;
            if (d < hd) {
                float a = acc[i] * alpha;
                for (int64_t t = 0; t < nk; ++t) a = fmaf(ps[t], load_as_float(p.v, p.dt, kvo + (j0 + t) * p.ldkv + d), a);
                acc[i] = a;
            }
        }
    }
    const float inv = 1.0f / l_run;
    const int64_t oo = b * p.o_bs + qi * p.ldo + h * hd;
#pragma unroll
    for (int i = 0; i < kMaxHD / 64; ++i) {
        const int64_t d = lane + 64 * i;
        if (d < hd) store_from_float(p.out, p.out_dt, oo + d, acc[i] * inv);
    }
}

// ------------------------------------------------------------------------------------------------ fp32 MFMA kernel
// attn_f32_mfma<HD> (fp32 inputs, head_dim 32 or 64, 16-byte aligned rows): fp32 matrix cores
// (v_mfma_f32_32x32x2_f32: fp32 products, fp32 accumulation) for both products, so the scores and the output keep
// fp32 accuracy. A workgroup owns 32 queries of one (batch, head); its 4 waves split the key range into 4 contiguous
// parts, each running an online softmax over 32-key tiles, and the four partial results (max, sum, unnormalized
// output) are merged through LDS at the end.
//   scores S^T = K Q^T: A = K tile (lane l: key l % 32), B = Q^T (lane l: query l % 32); the depth slot of lane l at
//     step i is d = (l / 32) * HD / 2 + i, so each lane reads HD / 2 contiguous floats of its key and query rows.
//     Accumulator element r of lane l is key 8 (r / 4) + 4 (l / 32) + r % 4 of query l % 32.
//   output O^T += V^T P^T: step j takes the keys the lanes' accumulator element j holds (8 (j / 4) + 4 (l / 32) +
//     j % 4), so P needs no exchange; A = V^T (lane l: d = l % 32 of the 32-wide d block).
constexpr int kF32Waves = 4;

template <int HD>
__global__ __launch_bounds__(256) void attn_f32_mfma(AttnParams p) {
    constexpr int HH = HD / 2;   // depth per lane half
    constexpr int DB = HD / 32;  // 32-wide d blocks of the output
    __shared__ float red_o[kF32Waves][HD][33];
    __shared__ float red_m[kF32Waves][32], red_l[kF32Waves][32];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = lane & 31, half = lane >> 5;
    const int64_t b = blockIdx.z, h = blockIdx.y;
    const int64_t q0 = (int64_t)blockIdx.x * 32;
    const int64_t lq = p.lq, lk = p.lk;
    const float* qbase = static_cast<const float*>(p.q) + b * p.q_bs + h * HD;
    const float* kbase = static_cast<const float*>(p.k) + b * p.kv_bs + h * HD;
    const float* vbase = static_cast<const float*>(p.v) + b * p.kv_bs + h * HD;

    float qv[HH];
    {
        const float* qr = qbase + (q0 + col < lq ? q0 + col : lq - 1) * p.ldq + half * HH;
#pragma unroll
        for (int i = 0; i < HH; i += 4) {
            const f32x4 v = *reinterpret_cast<const f32x4*>(qr + i);
            qv[i] = v[0], qv[i + 1] = v[1], qv[i + 2] = v[2], qv[i + 3] = v[3];
        }
    }

    const int64_t tiles = (lk + 31) / 32, per = (tiles + kF32Waves - 1) / kF32Waves;
    const int64_t t0 = wave * per, t1 = t0 + per < tiles ? t0 + per : tiles;
    const float c = p.scale_log2;
    float m = -INFINITY, l = 0.0f;
    f32x16 o[DB];
#pragma unroll
    for (int t = 0; t < DB; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[t][r] = 0.0f;

    // Software-pipelined over the wave's tiles, three tiles in flight: in the step of tile t the matrix cores take the
    // scores of tile t + 1 and the product of tile t - 1, alternating (two independent chains, so no MFMA waits on the
    // one before it), while the vector ALU runs tile t's softmax between them (each of the 64 slots pinned by a
    // scheduling barrier). K is loaded two tiles ahead and V one, into two register sets each; the probabilities wait
    // one step for their product. Every value is computed as in a plain tile-by-tile loop, in the same order.
    float ks[2][HH], vs[2][DB][16];
    f32x16 ps[2], sc;  // probabilities of tiles awaiting their product; scores of the next tile
    float alpha_p = 1.0f;  // tile t - 1's rescale factor, applied to o before its product
    auto load_k = [&](int set, int64_t k0) __attribute__((always_inline)) {
        const float* kr = kbase + (k0 + col < lk ? k0 + col : lk - 1) * p.ldkv + half * HH;
#pragma unroll
        for (int i = 0; i < HH; i += 4) {
            const f32x4 v = *reinterpret_cast<const f32x4*>(kr + i);
            ks[set][i] = v[0], ks[set][i + 1] = v[1], ks[set][i + 2] = v[2], ks[set][i + 3] = v[3];
        }
    };
    auto load_v = [&](int set, int64_t k0) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int64_t key = k0 + 8 * (j >> 2) + 4 * half + (j & 3);
            const float* vr = vbase + (key < lk ? key : lk - 1) * p.ldkv + col;
#pragma unroll
            for (int t2 = 0; t2 < DB; ++t2) vs[set][t2][j] = vr[t2 * 32];
        }
    };
    // o *= alpha_p (skipped when every lane's factor is 1, which leaves o unchanged)
    auto rescale = [&]() __attribute__((always_inline)) {
        if (__builtin_amdgcn_ballot_w64(alpha_p != 1.0f) != 0) {
#pragma unroll
            for (int t2 = 0; t2 < DB; ++t2)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[t2][r] *= alpha_p;
        }
    };
    // product MFMA q of the tile whose V is in vs[set] and probabilities in ps[set]: d block q % DB, key chunk q / DB
    auto pv = [&](int set, int q) __attribute__((always_inline)) {
        const int t2 = q % DB, j = q / DB;
        o[t2] = __builtin_amdgcn_mfma_f32_32x32x2f32(vs[set][t2][j], ps[set][j], o[t2], 0, 0, 0);
    };
    // the step of tile t (parity P: its K was in ks[P], its V goes to vs[P], its probabilities to ps[P]); NEXT: tile
    // t + 1 exists (its K in ks[P ^ 1]); PREV: tile t - 1 awaits its product (vs[P ^ 1], ps[P ^ 1])
    auto step = [&](int64_t t, auto p_tag, auto next_tag, auto prev_tag) __attribute__((always_inline)) {
        constexpr int P = decltype(p_tag)::value;
        constexpr bool NEXT = decltype(next_tag)::value, PREV = decltype(prev_tag)::value;
        const int64_t k0 = t * 32;
        load_v(P, k0);
        if (NEXT && t + 2 < t1) load_k(P, k0 + 64);
        if constexpr (PREV) rescale();
        __builtin_amdgcn_sched_barrier(0);
        f32x16 s = sc, acc;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
        float mx = -INFINITY, mxo = 0.0f, m_new = 0.0f, alpha = 0.0f, sum = 0.0f;
        static_for<64>([&](auto I) __attribute__((always_inline)) {
            constexpr int i = decltype(I)::value;
            if constexpr (i % 2 == 0) {
                if constexpr (NEXT && i / 2 < HH)
                    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(ks[P ^ 1][i / 2], qv[i / 2], acc, 0, 0, 0);
            } else {
                if constexpr (PREV && i / 2 < 16 * DB) pv(P ^ 1, i / 2);
            }
            if constexpr (i < 16) {  // scale and mask score i, running maximum
                const int64_t key = k0 + 8 * (i >> 2) + 4 * half + (i & 3);
                s[i] = key < lk ? s[i] * c : -INFINITY;
                mx = fmaxf(mx, s[i]);
            } else if constexpr (i == 16) {
                mxo = __shfl_xor(mx, 32);
            } else if constexpr (i == 20) {
                mx = fmaxf(mx, mxo);
                m_new = fmaxf(m, mx);
                alpha = exp2f(m - m_new);
            } else if constexpr (i >= 21 && i < 37) {  // probability i - 21, summed in order
                constexpr int r = i - 21;
                s[r] = exp2f(s[r] - m_new);
                sum += s[r];
            } else if constexpr (i == 37) {
                l = l * alpha + sum;
                m = m_new;
            }
            __builtin_amdgcn_sched_barrier(0);
        });
        ps[P] = s;
        alpha_p = alpha;
        if constexpr (NEXT) sc = acc;
    };
    // the product of the last tile (parity P)
    auto drain = [&](auto p_tag) __attribute__((always_inline)) {
        constexpr int P = decltype(p_tag)::value;
        rescale();
#pragma unroll
        for (int q = 0; q < 16 * DB; ++q) pv(P, q);
    };
    const std::integral_constant<int, 0> p0;
    const std::integral_constant<int, 1> p1;
    const std::true_type yes;
    const std::false_type no;
    if (t0 < t1) {
        load_k(0, t0 * 32);
        if (t0 + 1 < t1) load_k(1, t0 * 32 + 32);
#pragma unroll
        for (int r = 0; r < 16; ++r) sc[r] = 0.0f;
#pragma unroll
        for (int i = 0; i < HH; ++i) sc = __builtin_amdgcn_mfma_f32_32x32x2f32(ks[0][i], qv[i], sc, 0, 0, 0);
        if (t0 + 1 < t1)
            step(t0, p0, yes, no);
        else
            step(t0, p0, no, no);
        int64_t t = t0 + 1;
        for (; t + 2 < t1; t += 2) {
            step(t, p1, yes, yes);
            step(t + 1, p0, yes, yes);
        }
        if (t + 1 < t1) {
            step(t, p1, yes, yes);
            step(t + 1, p0, no, yes);
            drain(p0);
        } else if (t < t1) {
            step(t, p1, no, yes);
            drain(p1);
        } else {
            drain(p0);
        }
    }
    l += __shfl_xor(l, 32);

    // merge the waves' partial results: out = sum_w O_w 2^(m_w - m*) / sum_w l_w 2^(m_w - m*)
#pragma unroll
    for (int t2 = 0; t2 < DB; ++t2)
#pragma unroll
        for (int r = 0; r < 16; ++r) red_o[wave][t2 * 32 + 8 * (r >> 2) + 4 * half + (r & 3)][col] = o[t2][r];
    if (half == 0) {
        red_m[wave][col] = m;
        red_l[wave][col] = l;
    }
    __syncthreads();
    const int qi = threadIdx.x >> 3, part = threadIdx.x & 7;  // 32 queries x 8 column parts
    float mstar = -INFINITY;
#pragma unroll
    for (int w = 0; w < kF32Waves; ++w) mstar = fmaxf(mstar, red_m[w][qi]);
    float wgt[kF32Waves], lsum = 0.0f;
#pragma unroll
    for (int w = 0; w < kF32Waves; ++w) {
        wgt[w] = red_m[w][qi] == -INFINITY ? 0.0f : exp2f(red_m[w][qi] - mstar);
        lsum += red_l[w][qi] * wgt[w];
    }
    const float inv = 1.0f / lsum;
    if (q0 + qi < lq) {
        const int64_t obase = b * p.o_bs + (q0 + qi) * p.ldo + h * HD;
#pragma unroll
        for (int d = part; d < HD; d += 8) {
            float acc = 0.0f;
#pragma unroll
            for (int w = 0; w < kF32Waves; ++w) acc += red_o[w][d][qi] * wgt[w];
            store_from_float(p.out, p.out_dt, obase + d, acc * inv);
        }
    }
}

}  // namespace
}  // namespace idolq

using namespace idolq;

namespace {
// The staged V^T tiles and their exponents of a bf16 call with head_dim 64 (0 bytes for any other call).
size_t attn_workspace_bytes(int dtype, int64_t batch, int64_t lk, int64_t heads, int64_t head_dim) {
    if (dtype != IDOLQ_BF16 || head_dim != kHD || batch <= 0 || lk <= 0 || heads <= 0) return 0;
    const size_t tiles = (size_t)batch * (size_t)heads * (size_t)((lk + kBKV - 1) / kBKV);
    return tiles * kHD * kBKV * 2 + (tiles * 4 + 255) / 256 * 256;
}
}  // namespace

extern "C" size_t idolq_attention_workspace(int dtype, int64_t batch, int64_t lk, int64_t heads, int64_t head_dim) {
    return attn_workspace_bytes(dtype, batch, lk, heads, head_dim);
}

extern "C" int idolq_attention(const void* q, const void* k, const void* v, int dtype, int64_t batch, int64_t lq,
                               int64_t lk, int64_t heads, int64_t head_dim, int64_t ldq, int64_t ldkv, int64_t q_bs,
                               int64_t kv_bs, void* out, int out_dtype, int64_t ldo, int64_t o_bs, void* stream) {
    return idolq_attention_ws(q, k, v, dtype, batch, lq, lk, heads, head_dim, ldq, ldkv, q_bs, kv_bs, out, out_dtype,
                              ldo, o_bs, nullptr, 0, stream);
}

extern "C" int idolq_attention_ws(const void* q, const void* k, const void* v, int dtype, int64_t batch, int64_t lq,
                                  int64_t lk, int64_t heads, int64_t head_dim, int64_t ldq, int64_t ldkv, int64_t q_bs,
                                  int64_t kv_bs, void* out, int out_dtype, int64_t ldo, int64_t o_bs, void* workspace,
                                  size_t workspace_bytes, void* stream) {
    if (!dtype_ok(dtype) || !dtype_ok(out_dtype)) return fail(IDOLQ_EINVAL, "unknown dtype code");
    if (batch < 0 || lq < 0 || lk <= 0 || heads <= 0 || head_dim <= 0 || head_dim > kMaxHD)
        return fail(IDOLQ_EINVAL, "bad attention shape (needs lk > 0 and 0 < head_dim <= 256)");
    const int64_t dim = heads * head_dim;
    if (ldq < dim || ldkv < dim || ldo < dim) return fail(IDOLQ_EINVAL, "row stride smaller than heads * head_dim");
    if (batch > 65535 || heads > 65535 || lq > 0x7fffffff) return fail(IDOLQ_EINVAL, "grid too large");
    if (batch == 0 || lq == 0) return IDOLQ_OK;
    if (!q || !k || !v || !out) return fail(IDOLQ_EINVAL, "q, k, v and out must be non-null");
    AttnParams p{q, k, v, out, dtype, out_dtype, lq, lk, heads, head_dim, ldq, ldkv, q_bs, kv_bs, ldo, o_bs,
                 1.4426950408889634f / sqrtf((float)head_dim)};
    p.out_vec = out_dtype == dtype && dtype != IDOLQ_F32 && reinterpret_cast<uintptr_t>(out) % 16 == 0 &&
                (ldo * 2) % 16 == 0 && (o_bs * 2) % 16 == 0;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const size_t esz = dtype_size(dtype);
    const bool aligned = reinterpret_cast<uintptr_t>(q) % 16 == 0 && reinterpret_cast<uintptr_t>(k) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(v) % 16 == 0 && (ldq * esz) % 16 == 0 &&
                         (ldkv * esz) % 16 == 0 && (q_bs * esz) % 16 == 0 && (kv_bs * esz) % 16 == 0;
    if (dtype != IDOLQ_F32 && head_dim == kHD && aligned && lk * ldkv < ((int64_t)1 << 30)) {
        const dim3 grid((unsigned)((lq + kBQ - 1) / kBQ), (unsigned)heads, (unsigned)batch);
        const size_t need = attn_workspace_bytes(dtype, batch, lk, heads, head_dim);
        if (need && workspace && workspace_bytes >= need && reinterpret_cast<uintptr_t>(workspace) % 256 == 0 &&
            (lk + kBKV - 1) / kBKV <= 0x7fffffff) {
            // bf16: V staged once as fp16 V^T tiles, then the attention copies them
            p.ntiles = (lk + kBKV - 1) / kBKV;
            uint16_t* vt = static_cast<uint16_t*>(workspace);
            int* vexps = reinterpret_cast<int*>(static_cast<char*>(workspace) +
                                                (size_t)batch * heads * p.ntiles * kHD * kBKV * 2);
            hipLaunchKernelGGL(attn_v_tiles, dim3((unsigned)p.ntiles, (unsigned)heads, (unsigned)batch), dim3(256), 0, s,
                               p, vt, vexps);
            int rc = check_launch("attn_v_tiles");
            if (rc) return rc;
            p.vt = vt;
            p.vexps = vexps;
            hipLaunchKernelGGL((attn_mfma_hd64<__bf16, true>), grid, dim3(256), 0, s, p);
            return check_launch("attn_mfma_hd64");
        }
        if (dtype == IDOLQ_BF16)
            hipLaunchKernelGGL(attn_mfma_hd64<__bf16>, grid, dim3(256), 0, s, p);
        else
            hipLaunchKernelGGL(attn_mfma_hd64<_Float16>, grid, dim3(256), 0, s, p);
        return check_launch("attn_mfma_hd64");
    }
    if (dtype == IDOLQ_F32 && (head_dim == 32 || head_dim == 64) && aligned) {
        const dim3 grid((unsigned)((lq + 31) / 32), (unsigned)heads, (unsigned)batch);
        if (head_dim == 64)
            hipLaunchKernelGGL(attn_f32_mfma<64>, grid, dim3(256), 0, s, p);
        else
            hipLaunchKernelGGL(attn_f32_mfma<32>, grid, dim3(256), 0, s, p);
        return check_launch("attn_f32_mfma");
    }
    const dim3 grid((unsigned)lq, (unsigned)heads, (unsigned)batch);
    hipLaunchKernelGGL(attn_f32, grid, dim3(64), 0, s, p);
    return check_launch("attn_f32");
}
