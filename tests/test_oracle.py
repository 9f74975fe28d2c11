"""Pins the CPU oracle (oracle/oracle.c) before the GPU path is checked against it.

Three kinds of pin, chosen so that a plausible slip (a dropped term, a wrong sign, index or rounding rule, a
transposed operand, a changed summation order) fails at least one:
  * golden vectors written by the reference's own kernels (tests/golden/*.npz, tests/golden/make_golden.py),
    compared bit for bit;
  * the reference build itself (oracle/_ref, present where the reference checkout is), on fresh seeds;
  * closed forms and invariants: fp64 products, exact GELU/exp, integer identities, tie-breaking cases.
"""
import math

import numpy as np
import pytest

import oracle as O
from conftest import norm_rel

pytestmark = pytest.mark.filterwarnings("ignore::RuntimeWarning")

needs_ref = pytest.mark.skipif(not O.ref_available(), reason="reference build (oracle/_ref) not present")


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


# ------------------------------------------------------------------------------------------------ fp16
def test_half_to_float_matches_numpy_for_every_half():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = O.half_to_float(h)
    ref = h.view(np.float16).astype(np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(bits(got[finite]), bits(ref[finite]))
    assert np.all(np.isnan(got[np.isnan(ref)]))
    assert np.array_equal(got[np.isinf(ref)], ref[np.isinf(ref)])


def test_float_to_half_rounds_to_nearest_even_like_numpy():
    rng = np.random.default_rng(1)
    f = np.concatenate([rng.normal(0, 1, 200000), rng.normal(0, 1e-5, 100000), rng.normal(0, 3e4, 100000),
                        [65504, 65519.99, 65520, 1e9, -1e9, 2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0001,
                         3 * 2.0 ** -26, 0.0, -0.0]]).astype(np.float32)
    # halfway cases between adjacent halves, both parities
    base = rng.integers(0, 0x7bff, 20000).astype(np.uint16).view(np.float16).astype(np.float32)
    nxt = (rng.integers(0, 0x7bff, 20000).astype(np.uint16) + 1).astype(np.uint16).view(np.float16)
    f = np.concatenate([f, base, ((base.astype(np.float64) + np.nextafter(base, np.inf).astype(np.float64)) / 2)
                        .astype(np.float32), nxt.astype(np.float32)])
    got = O.float_to_half(f)
    ref = f.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


# ------------------------------------------------------------------------------------------------ Q8_0 format
def test_q8_0_quantize_closed_form_properties():
    rng = np.random.default_rng(2)
    w = rng.normal(0, 0.02, (64, 256)).astype(np.float32)
    blocks = O.q8_0_quantize(w).reshape(64, 8, 34)
    d = blocks[:, :, :2].copy().view(np.float16).astype(np.float32)[..., 0]
    q = blocks[:, :, 2:].view(np.int8).astype(np.int32)
    amax = np.abs(w.reshape(64, 8, 32)).max(-1)
    assert np.array_equal(d, (amax / np.float32(127)).astype(np.float16).astype(np.float32))
    assert np.all(np.abs(q) <= 127)
    # the largest magnitude of every block maps to +-127
    idx = np.abs(w.reshape(64, 8, 32)).argmax(-1)
    assert np.all(np.abs(np.take_along_axis(q, idx[..., None], -1)) == 127)
    # reconstruction error is half a step of the fp32 scale (plus the fp16 rounding of the scale)
    recon = q * d[..., None]
    step = (amax / 127)[..., None]
    assert np.all(np.abs(recon - w.reshape(64, 8, 32)) <= 0.5 * step + 127 * np.abs(d[..., None] - step) + 1e-12)


def test_q8_0_quantize_rounds_half_away_from_zero_with_a_reciprocal_multiply():
    # amax = 127 gives d = 1 exactly: x * id lands on the ties exactly. Half-away gives +-3 and +-1; ties-to-even
    # (numpy.round) would give +-2 and 0.
    block = np.zeros((1, 32), np.float32)
    block[0, :6] = [127.0, 2.5, -2.5, 0.5, -0.5, 126.5]
    q = O.q8_0_quantize(block)[2:].view(np.int8)
    assert list(q[:6]) == [127, 3, -3, 1, -1, 127]
    assert np.all(q[6:] == 0)
    # all-zero block: d = 0, id = 0, codes 0
    z = O.q8_0_quantize(np.zeros((1, 32), np.float32))
    assert np.all(z == 0)
    # The codes come from x * fl(1 / d), not from x / d. Values placed on the k + 0.5 boundaries of random scales
    # (and one ulp either side) expose inputs where the two round differently; the oracle must follow the multiply.
    rng = np.random.default_rng(3)
    amax = rng.uniform(0.5, 2.0, 4000).astype(np.float32)
    d = (amax / np.float32(127)).astype(np.float32)
    inv = (np.float32(1) / d).astype(np.float32)
    kk = rng.integers(0, 126, 4000).astype(np.float32)
    x = ((kk + np.float32(0.5)) * d).astype(np.float32)
    found = 0
    for cand in (x, np.nextafter(x, np.float32(np.inf)), np.nextafter(x, np.float32(-np.inf))):
        mul = (cand * inv).astype(np.float32)
        div = (cand / d).astype(np.float32)
        # round half away from zero, evaluated exactly in fp64 (all values here are positive)
        r_mul = np.floor(mul.astype(np.float64) + 0.5)
        r_div = np.floor(div.astype(np.float64) + 0.5)
        differ = r_mul != r_div
        for j in np.nonzero(differ)[0][:50]:
            block = np.zeros((1, 32), np.float32)
            block[0, 0], block[0, 1] = amax[j], cand[j]
            q = O.q8_0_quantize(block)[2:].view(np.int8)
            assert int(q[1]) == int(r_mul[j])
            assert int(q[1]) != int(r_div[j])
            found += 1
    assert found > 0


def test_q8_0_dequant_is_scale_times_code():
    rng = np.random.default_rng(4)
    blocks = O.q8_0_quantize(rng.normal(0, 0.1, (5, 96)).astype(np.float32))
    w = O.q8_0_dequant(blocks, 5, 96)
    b = blocks.reshape(5, 3, 34)
    d = b[:, :, :2].copy().view(np.float16).astype(np.float64)
    q = b[:, :, 2:].view(np.int8).astype(np.float64)
    assert np.array_equal(w.reshape(5, 3, 32).astype(np.float64), q * d)


def test_panel_bridge_against_golden_reference_dequantization(golden):
    g = golden("gemm_q8")
    for i in range(int(g["cases"])):
        m, n, k, *_ = g[f"c{i}_shape"]
        w = g[f"c{i}_w"]
        # the reference's dequantize_linear over the bridged panel equals q * d exactly (fact: fma(q+128, d, -128d))
        assert np.array_equal(g[f"c{i}_w_dense"], O.q8_0_dequant(w, n, k))
        blob = O.q8_0_to_panel(w, n, k)
        assert blob.size == O.panel_bytes(n, k) == ((n + 15) // 16) * (k // 32) * 576


def test_panel_bridge_rejects_inexact_minimum():
    blocks = np.zeros((1, 34), np.uint8)
    blocks[0, :2] = np.array([np.float16(600.0)]).view(np.uint8)  # -128 * 600 overflows fp16
    with pytest.raises(ValueError):
        O.q8_0_to_panel(blocks.reshape(-1), 1, 32)


# ------------------------------------------------------------------------------------------------ GEMM
def _gemm_case(g, i):
    m, n, k, off, cnt, res, gelu = (int(v) for v in g[f"c{i}_shape"])
    return dict(m=m, n=n, k=k, off=off, cnt=cnt, gelu=bool(gelu), a=g[f"c{i}_a"], w=g[f"c{i}_w"],
                bias=g[f"c{i}_bias"], residual=g.get(f"c{i}_residual"))


def test_float_gemm_matches_reference_golden_bit_for_bit(golden):
    g = golden("gemm_q8")
    for i in range(int(g["cases"])):
        c = _gemm_case(g, i)
        y = O.gemm_q8_float(c["a"], c["w"], c["n"], c["k"], c["bias"], c["off"], c["cnt"], c["residual"], c["gelu"])
        assert np.array_equal(bits(y), bits(g[f"c{i}_y_float"])), f"case {i}"


def test_int8_gemm_matches_reference_golden_bit_for_bit(golden):
    g = golden("gemm_q8")
    for i in range(int(g["cases"])):
        c = _gemm_case(g, i)
        y = O.gemm_q8_int8(c["a"], c["w"], c["n"], c["k"], c["bias"], c["off"], c["cnt"], c["residual"], c["gelu"])
        assert np.array_equal(bits(y), bits(g[f"c{i}_y_int8"])), f"case {i}"


def test_golden_discriminates_plausible_mistakes(golden):
    # Planted mistakes, each a plausible slip in a restatement, must not reproduce the reference's fixture: a single
    # running sum over k instead of 32-deep chunks, the scale of the neighbouring block, unsigned codes without the
    # -128 d minimum, and the bias added after the GELU.
    g = golden("gemm_q8")
    c = _gemm_case(g, 6)  # m=64, n=64, k=1024, window [0, 64), residual and GELU
    m, n, k = c["m"], c["n"], c["k"]
    ref = g["c6_y_float"]
    a, bias, res = c["a"], c["bias"], c["residual"]
    blocks = c["w"].reshape(n, k // 32, 34)
    d = blocks[:, :, :2].copy().view(np.float16).astype(np.float32)[..., 0]
    q = blocks[:, :, 2:].view(np.int8).astype(np.float32)
    w = (q * d[..., None]).reshape(n, k)

    def epilogue(acc, gelu_first=False):
        if gelu_first:
            return O.gelu_erf(acc).reshape(acc.shape) + bias + res
        return O.gelu_erf(acc + bias + res).reshape(acc.shape)

    one_sum = np.zeros((m, n), np.float32)
    for kk in range(k):
        one_sum = (one_sum + a[:, kk:kk + 1] * w[:, kk][None]).astype(np.float32)
    assert not np.array_equal(bits(epilogue(one_sum)), bits(ref))
    neighbour = (q * np.roll(d, 1, axis=1)[..., None]).reshape(n, k)
    assert norm_rel(epilogue(a @ neighbour.T), ref) > 1e-2
    unsigned = ((q + 128) * d[..., None]).reshape(n, k)
    assert norm_rel(epilogue(a @ unsigned.T), ref) > 1e-2
    assert norm_rel(epilogue(a @ w.T, gelu_first=True), ref) > 1e-2
    # the correct arithmetic in numpy lands within fp32 rounding of the fixture
    assert norm_rel(epilogue(a.astype(np.float64) @ w.T.astype(np.float64)), ref) < 1e-6


def test_float_gemm_against_fp64_naive_with_k_tails():
    # tests/test_kernels.cpp:111-136 restated on Q8_0 weights: fp64 dot products, tolerance 1e-4
    rng = np.random.default_rng(5)
    for k in (32, 64, 96, 128, 352, 1024):
        m, n = 5, 20
        w = O.q8_0_quantize(rng.uniform(-0.5, 0.5, (n, k)).astype(np.float32))
        dense = O.q8_0_dequant(w, n, k).astype(np.float64)
        bias = rng.uniform(-0.5, 0.5, n).astype(np.float32)
        a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
        y = O.gemm_q8_float(a, w, n, k, bias)
        assert np.max(np.abs(y - (a.astype(np.float64) @ dense.T + bias))) < 1e-4


def test_float_gemm_column_window_adds_residual_before_exact_gelu():
    # tests/test_kernels.cpp:138-155 on Q8_0 weights
    rng = np.random.default_rng(6)
    m, k, out, first, n = 6, 64, 37, 16, 21
    w = O.q8_0_quantize(rng.uniform(-0.5, 0.5, (out, k)).astype(np.float32))
    dense = O.q8_0_dequant(w, out, k).astype(np.float64)
    bias = rng.uniform(-0.5, 0.5, out).astype(np.float32)
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    res = rng.uniform(-0.5, 0.5, (m, n)).astype(np.float32)
    y = O.gemm_q8_float(a, w, out, k, bias, first, n, res, True)
    pre = (a.astype(np.float64) @ dense.T + bias)[:, first:first + n] + res
    exact = 0.5 * pre * (1 + np.vectorize(math.erf)(pre / math.sqrt(2)))
    assert np.max(np.abs(y - exact)) < 1e-4


def test_dense_gemm_sums_depth_in_32_deep_chunks():
    # src/kernels.cpp:566-596: fp32 weights, depth in chunks of 32, each an FMA chain from zero, partials added left to
    # right. Row [2^24, 1 x63] against unit weights (exact 2^24 + 63): the first chunk's 1s round away next to 2^24,
    # the second chunk sums to 32 on its own, so 32-deep chunks give 2^24 + 32; one chain over the whole depth gives
    # 2^24 and 16-deep chunks give 2^24 + 48.
    a = np.ones((1, 64), np.float32)
    a[0, 0] = 2.0 ** 24
    w = np.ones((3, 64), np.float32)
    assert np.array_equal(O.gemm_dense(a, w), np.full((1, 3), 2.0 ** 24 + 32, np.float32))
    # bias after the depth sum; fp64 closeness with a ragged tail; exact erf-GELU after the bias
    rng = np.random.default_rng(11)
    for (m, n, k) in [(9, 14, 64), (5, 33, 100), (3, 1, 7)]:
        a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
        w = rng.uniform(-0.5, 0.5, (n, k)).astype(np.float32)
        bias = rng.uniform(-0.5, 0.5, n).astype(np.float32)
        pre = a.astype(np.float64) @ w.T.astype(np.float64) + bias
        assert np.max(np.abs(O.gemm_dense(a, w, bias) - pre)) < 1e-5
        exact = 0.5 * pre * (1 + np.vectorize(math.erf)(pre / math.sqrt(2)))
        assert np.max(np.abs(O.gemm_dense(a, w, bias, gelu=True) - exact)) < 1e-4


def test_dense_gemm_matches_reference_golden_bit_for_bit(golden):
    g = golden("gemm_dense")
    for i in range(int(g["cases"])):
        gelu = bool(g[f"c{i}_shape"][3])
        y = O.gemm_dense(g[f"c{i}_a"], g[f"c{i}_w"], g[f"c{i}_bias"], gelu=gelu)
        assert np.array_equal(bits(y), bits(g[f"c{i}_y"])), f"case {i}"


def test_int8_gemm_identities_and_closeness_to_float():
    rng = np.random.default_rng(7)
    m, n, k = 19, 37, 256
    w = O.q8_0_quantize(rng.uniform(-0.5, 0.5, (n, k)).astype(np.float32))
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    bias = rng.uniform(-0.5, 0.5, n).astype(np.float32)
    qa, sa, qs = O.quantize_act(a)
    dots = O.block_dots(qa, w, k, 0, n)
    q = w.reshape(n, k // 32, 34)[:, :, 2:].view(np.int8).astype(np.int64)
    brute = np.einsum("mbt,nbt->mnb", qa.reshape(m, k // 32, 32).astype(np.int64), q)
    assert np.array_equal(dots, brute)
    # sum qa * (q + 128) = dots + 128 * qsum, the unsigned form the reference's vpdpbusd accumulates
    unsigned = np.einsum("mbt,nbt->mnb", qa.reshape(m, k // 32, 32).astype(np.int64), q + 128)
    assert np.array_equal(unsigned, dots + 128 * qs[:, None, :])
    # tests/test_kernels.cpp:265-288: within 2% of the largest output of the float kernel
    y_int = O.gemm_q8_int8(a, w, n, k, bias)
    y_float = O.gemm_q8_float(a, w, n, k, bias)
    assert np.max(np.abs(y_int - y_float)) <= 0.02 * np.max(np.abs(y_float))


def test_quantize_act_matches_reference_golden_and_closed_form(golden):
    g = golden("quantize_act")
    qa, sa, qs = O.quantize_act(g["a"])
    assert np.array_equal(qa, g["qa"]) and np.array_equal(bits(sa), bits(g["sa"])) and np.array_equal(qs, g["qsum"])
    a = g["a"].reshape(g["a"].shape[0], -1, 32)
    amax = np.abs(a).max(-1)
    assert np.array_equal(sa, (amax / np.float32(127)).astype(np.float32))
    assert np.array_equal(qs, qa.reshape(a.shape).astype(np.int32).sum(-1))
    # ties round to even: row 6, block 0 holds +-127 and multiples of 127/31 * ... that scale onto .5 boundaries
    inv = np.where(amax > 0, np.float32(127) / np.where(amax > 0, amax, 1), 0).astype(np.float32)
    assert np.array_equal(qa.reshape(a.shape), np.rint(a * inv[..., None]).astype(np.int8))


# ------------------------------------------------------------------------------------------------ norms
def test_norms_match_reference_golden_bit_for_bit(golden):
    g = golden("norm")
    assert np.array_equal(bits(O.layer_norm(g["small"], g["g24"], g["b24"])), bits(g["layer_norm_small"]))
    assert np.array_equal(bits(O.layer_norm(g["x"], g["gamma"], g["beta"])), bits(g["layer_norm"]))
    assert np.array_equal(bits(O.norm_rows(g["x"], 1e-6)), bits(g["norm_plain"]))
    assert np.array_equal(bits(O.norm_rows(g["x"], 1e-6, gamma=g["gamma"], beta=g["beta"])), bits(g["norm_affine"]))
    assert np.array_equal(bits(O.norm_rows(g["x"], 1e-6, shift=g["shift"], scale=g["scale"])), bits(g["norm_ada"]))
    assert np.array_equal(bits(O.norm_rows(g["x"], 1e-5)), bits(g["norm_eps5"]))


def test_layer_norm_against_fp64_naive():
    # tests/test_kernels.cpp:157-182
    rng = np.random.default_rng(8)
    x = rng.uniform(-2, 2, (5, 24)).astype(np.float32)
    g, b = rng.uniform(-1, 1, 24).astype(np.float32), rng.uniform(-0.5, 0.5, 24).astype(np.float32)
    xd = x.astype(np.float64)
    mean = xd.mean(1, keepdims=True)
    var = ((xd - mean) ** 2).mean(1, keepdims=True)
    ref = (xd - mean) / np.sqrt(var + 1e-5) * g + b
    assert np.max(np.abs(O.layer_norm(x, g, b) - ref)) < 1e-4
    sh, sc = rng.normal(0, 0.1, (2, 24)).astype(np.float32), rng.normal(0, 0.1, (2, 24)).astype(np.float32)
    y = O.norm_rows(x, 1e-6, shift=sh, scale=sc, rows_per_batch=3)
    bidx = np.arange(5) // 3
    ref2 = (xd - mean) / np.sqrt(var + 1e-6) * (1 + sc[bidx]) + sh[bidx]
    assert np.max(np.abs(y - ref2)) < 1e-4


# ------------------------------------------------------------------------------------------------ attention
def _naive_attention(q, k, v, lq, lk, ldq, ldkv, heads, hd):
    q = q.astype(np.float64).reshape(lq, ldq)
    k = k.astype(np.float64).reshape(lk, ldkv)
    v = v.astype(np.float64).reshape(lk, ldkv)
    out = np.zeros((lq, heads * hd))
    for h in range(heads):
        s = q[:, h * hd:(h + 1) * hd] @ k[:, h * hd:(h + 1) * hd].T / math.sqrt(hd)
        p = np.exp(s - s.max(1, keepdims=True))
        out[:, h * hd:(h + 1) * hd] = (p / p.sum(1, keepdims=True)) @ v[:, h * hd:(h + 1) * hd]
    return out


def test_attention_matches_reference_golden_and_fp64(golden):
    g = golden("attention")
    for i in range(int(g["cases"])):
        lq, lk, heads, hd, ldq, ldkv = (int(v) for v in g[f"c{i}_shape"])
        q, k, v = g[f"c{i}_q"], g[f"c{i}_k"], g[f"c{i}_v"]
        y = O.attention(q, k, v, lq, lk, ldq, ldkv, heads, hd)
        assert np.array_equal(bits(y), bits(g[f"c{i}_out"])), f"case {i}"
        # tests/test_kernels.cpp:184-228: fp64 softmax attention, 1e-4
        assert np.max(np.abs(y - _naive_attention(q, k, v, lq, lk, ldq, ldkv, heads, hd))) < 1e-4


# ------------------------------------------------------------------------------------------------ elementwise
def test_exp_and_gelu_match_reference_golden_and_math(golden):
    g = golden("elementwise")
    assert np.array_equal(bits(O.exp256(g["x_exp"])), bits(g["exp256"]))
    assert np.array_equal(bits(O.gelu_erf(g["x_gelu"])), bits(g["gelu256"]))
    assert np.array_equal(bits(O.gelu_scalar(g["x_gelu"])), bits(g["gelu_scalar"]))
    assert np.array_equal(bits(O.gelu_tanh(g["x_tanh"])), bits(g["gelu_tanh"]))
    # tests/test_kernels.cpp:298-323
    x = g["x_exp"][:4000]
    assert np.max(np.abs(O.exp256(x) / np.exp(x.astype(np.float64)) - 1)) < 1e-6
    xg = g["x_gelu"][:1200].astype(np.float64)
    exact = 0.5 * xg * (1 + np.vectorize(math.erf)(xg / math.sqrt(2)))
    assert np.max(np.abs(O.gelu_erf(g["x_gelu"][:1200]) - exact)) < 2e-6
    assert np.max(np.abs(O.gelu_scalar(g["x_gelu"][:1200]) - exact)) < 2e-6
    xt = g["x_tanh"].astype(np.float64)
    tanh_gelu = 0.5 * xt * (1 + np.tanh(0.7978845608028654 * (xt + 0.044715 * xt ** 3)))
    assert np.max(np.abs(O.gelu_tanh(g["x_tanh"]) - tanh_gelu)) < 1e-5


def test_pos_embed_layout():
    freqs = (2.0 ** np.linspace(0, 10, 16)).astype(np.float32)
    coords = np.array([[0.25, -0.5, 1.0], [0.0, 0.1, -1.0]], np.float32)
    pe = O.pos_embed(freqs, coords)
    assert pe.shape == (2, 96)
    for r in range(2):
        for c in range(3):
            ang = (coords[r, c].astype(np.float64) * freqs.astype(np.float64)) * np.pi
            assert np.allclose(pe[r, c * 32:c * 32 + 16], np.sin(ang), atol=2e-4)
            assert np.allclose(pe[r, c * 32 + 16:c * 32 + 32], np.cos(ang), atol=2e-4)


# ------------------------------------------------------------------------------------------------ live reference
@needs_ref
def test_oracle_matches_live_reference_build_on_fresh_seeds():
    rng = np.random.default_rng(9)
    for (m, n, k) in [(13, 48, 192), (8, 30, 32), (41, 80, 512)]:
        w = O.q8_0_quantize(rng.normal(0, 0.1, (n, k)).astype(np.float32))
        blob = O.q8_0_to_panel(w, n, k)
        a = rng.normal(0, 1, (m, k)).astype(np.float32)
        bias = rng.normal(0, 0.1, n).astype(np.float32)
        for mode, fn in ((0, O.gemm_q8_float), (1, O.gemm_q8_int8)):
            for gelu in (False, True):
                ref = O.ref_gemm_panel(a, blob, bias, n, k, 0, n, None, gelu, mode=mode)
                assert np.array_equal(bits(fn(a, w, n, k, bias, 0, n, None, gelu)), bits(ref))
        wd = rng.normal(0, 0.1, (n, k)).astype(np.float32)
        for gelu in (False, True):
            assert np.array_equal(bits(O.gemm_dense(a, wd, bias, gelu)), bits(O.ref_gemm_dense(a, wd, bias, gelu=gelu)))
        qa, sa, qs = O.quantize_act(a)
        rqa, rsa, rqs = O.ref_quantize_activations(a)
        assert np.array_equal(qa, rqa) and np.array_equal(bits(sa), bits(rsa)) and np.array_equal(qs, rqs)
    x = rng.normal(0, 1, (7, 1280)).astype(np.float32)
    assert np.array_equal(bits(O.norm_rows(x, 1e-6)), bits(O.ref_norm_rows(x, 1e-6)))
    q = rng.normal(0, 1, 33 * 128).astype(np.float32)
    kv = rng.normal(0, 1, 45 * 128).astype(np.float32)
    assert np.array_equal(bits(O.attention(q, kv, kv, 33, 45, 128, 128, 2, 64)),
                          bits(O.ref_attention(q, kv, kv, 33, 45, 128, 128, 2, 64)))
