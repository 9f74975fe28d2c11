"""The real decoders on the GPU (src/decoders.cpp) against the reference's own outputs: the operators one by one
(bit-exact where the arithmetic is the same sequence of fp32 operations), the small fixture export with every weight
form, and a model-width export (dim 1024, 16 heads of 64) checked against the reference build when it is present.

Tolerance for decoder outputs: norm-relative 2e-5 against the reference's float kernel, the bar of its own decoder
check (tests/python/test_gguf_decoder.py:63-65, tools/idol_decode.cpp:55-68)."""
import importlib.util

import numpy as np
import pytest
import torch

import idol_kernels as K
import idolq_lib as L
import oracle as O
from conftest import GOLDEN, norm_rel
from decoders import Decoders

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _needs_ref():
    if not O.ref_available():
        pytest.skip("reference build absent (make -C oracle ref)")


# ------------------------------------------------------------------------------------------------ operators
@pytest.mark.parametrize("m,n,k", [(1, 64, 256), (37, 64, 3), (29, 128, 16), (70, 48, 100), (130, 200, 64), (5, 8, 1024),
                                   (77, 520, 32), (300, 1024, 16)])
def test_gemm_f32_is_bit_identical_to_the_reference_dense_gemm(m, n, k):
    _needs_ref()
    rng = np.random.default_rng(m * 7 + n)
    a = rng.standard_normal((m, k)).astype(np.float32)
    w = (rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    res = rng.standard_normal((m, n)).astype(np.float32)
    got = L.gemm_f32(_t(a), _t(w), bias=_t(b)).cpu().numpy()
    assert np.array_equal(got, O.ref_gemm_dense(a, w, b))
    # a residual aliasing the output (the Gaussian decoder's X = out(A) + X)
    y = _t(res)
    L.gemm_f32(_t(a), _t(w), bias=_t(b), residual=y, out=y)
    assert np.array_equal(y.cpu().numpy(), O.ref_gemm_dense(a, w, b, residual=res))
    # and the mathematics: fp64 brute force
    ref64 = a.astype(np.float64) @ w.astype(np.float64).T + b
    assert np.max(np.abs(got - ref64)) <= 1e-5 * max(1.0, np.max(np.abs(ref64)))


def test_gemm_f32_output_paths_give_the_same_bits():
    # 16-byte row stores (aligned output, the last columns of a row that does not fill 4 going out one by one) and
    # the element-wise stores (an output view 4 bytes off alignment), each with a residual aliasing the output
    _needs_ref()
    rng = np.random.default_rng(5)
    m, n, k = 50, 70, 16
    a = rng.standard_normal((m, k)).astype(np.float32)
    w = (rng.standard_normal((n, k)) / 4).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    res = rng.standard_normal((m, n)).astype(np.float32)
    want = O.ref_gemm_dense(a, w, b)
    want_res = O.ref_gemm_dense(a, w, b, residual=res)
    assert np.array_equal(L.gemm_f32(_t(a), _t(w), bias=_t(b)).cpu().numpy(), want)
    y = _t(res)
    L.gemm_f32(_t(a), _t(w), bias=_t(b), residual=y, out=y)
    assert np.array_equal(y.cpu().numpy(), want_res)
    big = torch.zeros((m, n + 5), device=DEV, dtype=torch.float32)
    view = big[:, 1:1 + n]  # data pointer 4 bytes past a 16-byte boundary, row stride n + 5
    L.gemm_f32(_t(a), _t(w), bias=_t(b), out=view)
    assert np.array_equal(view.cpu().numpy(), want)
    view.copy_(_t(res))
    L.gemm_f32(_t(a), _t(w), bias=_t(b), residual=view, out=view)
    assert np.array_equal(view.cpu().numpy(), want_res)
    assert not big[:, 0].any() and not big[:, 1 + n:].any()
    with pytest.raises(ValueError):
        L.gemm_f32(_t(a), _t(w), out=big[: m - 1, :n])  # an output with too few rows


@pytest.mark.parametrize("k", [1, 16, 32])
@pytest.mark.parametrize("act", [L.ACT_NONE, L.ACT_GELU_TANH])
def test_gemm_f32_vector_and_element_paths_agree_at_small_depth(k, act):
    # the 16-byte row stores (aligned output, n % 4 == 0) and the element-wise stores (an output view 4 bytes off
    # alignment) give the same bits at the latent projections' small depths, with an activation, with and without a
    # residual aliasing the output, over a partial last column tile and a partial last row tile
    rng = np.random.default_rng(k + 10 * act)
    m, n = 77, 520
    a = _t(rng.standard_normal((m, k)).astype(np.float32))
    w = _t((rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32))
    b = _t(rng.standard_normal(n).astype(np.float32))
    res = _t(rng.standard_normal((m, n)).astype(np.float32))
    fast = L.gemm_f32(a, w, bias=b, act=act)
    big = torch.zeros((m, n + 5), device=DEV, dtype=torch.float32)
    view = big[:, 1:1 + n]
    L.gemm_f32(a, w, bias=b, act=act, out=view)
    assert torch.equal(fast, view)
    y = res.clone()
    L.gemm_f32(a, w, bias=b, residual=y, act=act, out=y)
    view.copy_(res)
    L.gemm_f32(a, w, bias=b, residual=view, act=act, out=view)
    assert torch.equal(y, view)
    assert not big[:, 0].any() and not big[:, 1 + n:].any()


def test_gemm_f32_strided_rows_and_silu():
    rng = np.random.default_rng(1)
    a = rng.standard_normal((33, 80)).astype(np.float32)
    w = rng.standard_normal((40, 48)).astype(np.float32) * 0.2
    at = _t(a)[:, 16:64]
    got = L.gemm_f32(at, _t(w), act=L.ACT_SILU).cpu().numpy().astype(np.float64)
    v = a[:, 16:64].astype(np.float64) @ w.astype(np.float64).T
    assert np.max(np.abs(got - v / (1 + np.exp(-v)))) < 1e-5
    with pytest.raises(ValueError):
        L.gemm_f32(_t(a), _t(w))  # k mismatch


def test_rms_heads_and_add_gated_match_the_reference():
    _needs_ref()
    rng = np.random.default_rng(2)
    rows, heads, hd, ld = 45, 4, 64, 3 * 256
    x = rng.standard_normal((rows, ld)).astype(np.float32)
    x[3, 320:384] = 0.0  # a zero head: the 1e-12 floor
    g = rng.uniform(0.5, 1.5, heads * hd).astype(np.float32)
    xt = _t(x)
    L.rms_heads(xt[:, 256:], heads, hd, _t(g))
    want = x.copy()
    want[:, 256:] = O.ref_rms_heads(x[:, 256:].copy(), heads, hd, g)[:, :ld - 256]
    got = xt.cpu().numpy()
    assert np.array_equal(got[:, :256], x[:, :256]) and np.array_equal(got[:, 512:], x[:, 512:])
    assert np.max(np.abs(got - want)) <= 2e-7 * np.max(np.abs(want))
    # unit-norm heads times sqrt(hd) * gamma
    h = got[:, 256:512].reshape(rows, heads, hd) / g.reshape(heads, hd)
    norms = np.linalg.norm(h.astype(np.float64), axis=2)
    assert np.allclose(np.delete(norms, 3, axis=0), np.sqrt(hd), rtol=1e-5)
    assert np.all(got[3, 256 + 64:256 + 128] == 0)
    # a head size the 16-byte kernel does not take (general kernel), and bf16 rows
    x48 = rng.standard_normal((7, 3 * 48)).astype(np.float32)
    g48 = rng.uniform(0.5, 1.5, 3 * 48).astype(np.float32)
    xt = _t(x48)
    L.rms_heads(xt, 3, 48, _t(g48))
    assert np.max(np.abs(xt.cpu().numpy() - O.ref_rms_heads(x48, 3, 48, g48))) <= 2e-7 * 8
    xb = _t(x48).bfloat16()
    want_b = O.ref_rms_heads(xb.float().cpu().numpy(), 3, 48, g48)
    L.rms_heads(xb, 3, 48, _t(g48))
    assert np.max(np.abs(xb.float().cpu().numpy() - want_b)) <= 2e-2

    dim = 96
    xa = rng.standard_normal((rows, dim)).astype(np.float32)
    ha = rng.standard_normal((rows, dim)).astype(np.float32)
    gate = rng.standard_normal(dim).astype(np.float32)
    xt = _t(xa)
    L.add_gated(xt, _t(ha), _t(gate))
    assert np.array_equal(xt.cpu().numpy(), O.ref_add_gated(xa, ha, gate))


def test_level_embedding_and_silu():
    f = np.exp(-np.log(np.float32(1024)) * np.arange(128, dtype=np.float32) / 128, dtype=np.float32)
    for res in (2.0, 32.0, 1024.0):
        got = L.level_embed(res, _t(f)).cpu().numpy()
        ang = ((np.float32(res) * f) * np.float32(2.0)) * np.float32(np.pi)
        assert ang.dtype == np.float32
        want = np.concatenate([np.cos(ang.astype(np.float64)), np.sin(ang.astype(np.float64))])
        assert np.max(np.abs(got - want)) < 2e-6
    x = np.linspace(-30, 30, 4099).astype(np.float32)
    xt = _t(x)
    L.activation(xt, L.ACT_SILU)
    want = x.astype(np.float64) / (1 + np.exp(-x.astype(np.float64)))
    assert np.max(np.abs(xt.cpu().numpy() - want) / np.maximum(np.abs(want), 1e-30)) < 2e-6


# ------------------------------------------------------------------------------------------------ whole decoders
def _run(dec, anchors, cond, resolution):
    a, c = _t(anchors), _t(cond)
    oct_ = dec.octree_logits(a, a.shape[0], resolution, c, c.shape[0]).cpu().numpy()
    gs = dec.gaussian_features(a, a.shape[0], c, c.shape[0]).cpu().numpy()
    return oct_, gs


def test_small_export_matches_the_reference_decoders(golden):
    g = golden("decoders_small")
    dec = Decoders(GOLDEN / "decoders_small")
    try:
        K.set_quant_kernel(0)
        oct_, gs = _run(dec, g["anchors"], g["cond"], float(g["resolution"]))
        r_oct, r_gs = norm_rel(oct_, g["ref_oct"]), norm_rel(gs, g["ref_gs"])
        print(f"float kernel: octree {r_oct:.3e} gaussian {r_gs:.3e}")
        assert r_oct < 2e-5 and r_gs < 2e-5
    finally:
        K.set_quant_kernel(-1)
    # fewer rows than the buffers hold, and no rows
    o2 = dec.octree_logits(_t(g["anchors"]), 5, float(g["resolution"]), _t(g["cond"]), 29)
    assert o2.shape == (5, 8)
    assert dec.gaussian_features(_t(g["anchors"]), 0, _t(g["cond"]), 29).shape == (0, 60)


def _make_decoders_module():
    spec = importlib.util.spec_from_file_location("make_decoders", GOLDEN / "make_decoders.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_symmetric_export_matches_the_reference_integer_kernel(golden, tmp_path):
    # the fixture's weights with every panel symmetric, rebuilt from the generator's seed; the reference's outputs
    # on it with its float and its integer (AVX-VNNI) kernels are in the fixture
    g = golden("decoders_small")
    if "sym_gs_int8" not in g:
        pytest.skip("the fixture was written on a CPU without AVX-VNNI")
    md = _make_decoders_module()
    md.build_export(tmp_path / "sym", md.CFG, 11, md.SYM_FORMS)
    dec = Decoders(tmp_path / "sym")
    try:
        K.set_quant_kernel(0)
        oct_, gs = _run(dec, g["anchors"], g["cond"], float(g["resolution"]))
        f_oct, f_gs = norm_rel(oct_, g["sym_oct"]), norm_rel(gs, g["sym_gs"])
        K.set_quant_kernel(1)
        oct8, gs8 = _run(dec, g["anchors"], g["cond"], float(g["resolution"]))
        i_oct, i_gs = norm_rel(oct8, g["sym_oct_int8"]), norm_rel(gs8, g["sym_gs_int8"])
    finally:
        K.set_quant_kernel(-1)
    print(f"float kernel: octree {f_oct:.3e} gaussian {f_gs:.3e}; integer kernel: octree {i_oct:.3e} "
          f"gaussian {i_gs:.3e}; integer vs float {norm_rel(gs8, g['sym_gs']):.3e}")
    assert f_oct < 2e-5 and f_gs < 2e-5
    # the integer kernels agree far more closely than either agrees with the float kernel (about 1e-2 here)
    assert i_oct < 1e-4 and i_gs < 1e-4


def test_model_width_export_matches_the_reference_decoders(tmp_path):
    # dim 1024, 16 heads of 64, per_anchor 32: the real model's widths, one block of each decoder
    _needs_ref()
    md = _make_decoders_module()
    import idol_export as E
    cfg = E.DecoderConfig(dim=1024, heads=16, oct_blocks=1, gs_blocks=1, cond=16, per_anchor=32)
    forms = {name: "q8" for name in (
        "oct.input_layer", "oct.l_embedder.mlp.0", "oct.l_embedder.mlp.2", "oct.adaLN_modulation.1", "oct.out_proj",
        "oct.blocks.0.cross_attn.to_q", "oct.blocks.0.cross_attn.to_out", "oct.blocks.0.mlp.mlp.0",
        "oct.blocks.0.mlp.mlp.2", "gs.input_layer", "gs.out_proj", "gs.blocks.0.self_attn.to_qkv",
        "gs.blocks.0.self_attn.to_out", "gs.blocks.0.cross_attn.to_q", "gs.blocks.0.cross_attn.to_out",
        "gs.blocks.0.mlp.mlp.0", "gs.blocks.0.mlp.mlp.2")}
    md.build_export(tmp_path / "wide", cfg, 21, forms)
    rng = np.random.default_rng(22)
    anchors = rng.uniform(0, 1, (96, 3)).astype(np.float32)
    cond = rng.standard_normal((300, 16)).astype(np.float32)
    ref = O.RefDecoders(tmp_path / "wide")
    O.ref_lib().ref_set_quant_kernel(0)
    try:
        want_oct = ref.octree_logits(anchors, 64.0, cond)
        want_gs = ref.gaussian_features(anchors, cond)
    finally:
        O.ref_lib().ref_set_quant_kernel(-1)
        ref.close()
    dec = Decoders(tmp_path / "wide")
    K.set_quant_kernel(0)
    try:
        oct_, gs = _run(dec, anchors, cond, 64.0)
    finally:
        K.set_quant_kernel(-1)
    r_oct, r_gs = norm_rel(oct_, want_oct), norm_rel(gs, want_gs)
    print(f"dim 1024: octree {r_oct:.3e} gaussian {r_gs:.3e}")
    assert r_oct < 2e-5 and r_gs < 2e-5


@pytest.mark.parametrize("quant", ["Q8_0", "Q4_0"])
def test_decoders_from_gguf_match_the_reference(tmp_path, quant):
    # an Idol GGUF (Q8_0 or Q4_0 matrices, F32 / F16 vectors) run three ways: the reference's decoders on the
    # materialized native export, these decoders on the same export, and these decoders straight from the GGUF
    import idol_gguf as G
    from ggml_types import GGMLQuantizationType as Q
    from gguf_fixture import write_idol_gguf
    write_idol_gguf(tmp_path / "d.gguf", quant=getattr(Q, quant))
    m = G.IdolGGUF(tmp_path / "d.gguf")
    G.materialize(m, tmp_path / "native")
    rng = np.random.default_rng(31)
    anchors = rng.uniform(0, 1, (45, 3)).astype(np.float32)
    cond = rng.standard_normal((23, 16)).astype(np.float32)
    K.set_quant_kernel(0)
    try:
        a = _run(Decoders(tmp_path / "native"), anchors, cond, 16.0)
        b = _run(Decoders(G.decoder_export(m)), anchors, cond, 16.0)
    finally:
        K.set_quant_kernel(-1)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
    if O.ref_available():
        ref = O.RefDecoders(tmp_path / "native")
        O.ref_lib().ref_set_quant_kernel(0)
        try:
            r_oct, r_gs = ref.octree_logits(anchors, 16.0, cond), ref.gaussian_features(anchors, cond)
        finally:
            O.ref_lib().ref_set_quant_kernel(-1)
            ref.close()
        print(f"{quant}: octree {norm_rel(a[0], r_oct):.3e} gaussian {norm_rel(a[1], r_gs):.3e}")
        assert norm_rel(a[0], r_oct) < 2e-5 and norm_rel(a[1], r_gs) < 2e-5


def test_to_gaussians_sample_anchors_and_decode_match_the_reference():
    # src/decoders.cpp:335-442 around the decoders: to_gaussians on the same features (libm-level differences only),
    # the octree descent with the GPU decoders' logits, and decode end to end
    _needs_ref()
    from decoders import GaussianCloud, write_gaussian_ply  # noqa: F401
    dec = Decoders(GOLDEN / "decoders_small")
    ref = O.RefDecoders(GOLDEN / "decoders_small")
    rng = np.random.default_rng(41)
    cond = rng.standard_normal((29, 16)).astype(np.float32)
    anchors = rng.uniform(0, 1, (50, 3)).astype(np.float32)
    feats = (2 * rng.standard_normal((50, 60))).astype(np.float32)
    feats[0, :] = 30.0  # the softplus pass-through branch
    K.set_quant_kernel(0)
    O.ref_lib().ref_set_quant_kernel(0)
    try:
        cloud = dec.to_gaussians(_t(anchors), 50, _t(feats))
        want = ref.to_gaussians(anchors, feats)
        for key in ("xyz", "f_dc", "scale", "rotation", "opacity"):
            got = getattr(cloud, key).cpu().numpy()
            assert np.allclose(got, want[key], rtol=2e-6, atol=1e-7), key
        for num_points, level, seed in ((64, 2, 3), (500, 4, 9)):
            got = dec.sample_anchors(cond, 29, num_points, level, seed)
            exp = ref.sample_anchors(cond, num_points, level, seed)
            same = np.mean(np.all(got == exp, axis=1))
            print(f"sample_anchors {num_points} points, level {level}: {same:.4f} identical")
            assert got.shape == exp.shape and same == 1.0
        c = dec.decode(cond, 29, 400, 3, 5)
        assert c.size() == 400 and all(torch.isfinite(getattr(c, k)).all() for k in ("xyz", "scale", "opacity"))
        pts = ref.sample_anchors(cond, 100, 3, 5)
        rc = ref.to_gaussians(pts, ref.gaussian_features(pts, cond))
        for key in ("xyz", "f_dc", "scale", "rotation", "opacity"):
            assert norm_rel(getattr(c, key).cpu().numpy(), rc[key]) < 1e-4, key
    finally:
        K.set_quant_kernel(-1)
        O.ref_lib().ref_set_quant_kernel(-1)
        ref.close()
