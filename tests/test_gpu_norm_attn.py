"""GPU parity of the kernels between the GEMMs: layer norm (plain, affine, adaLN, in place), attention (MFMA and
fp32 kernels), activations and the position embedding, against the oracle and the reference's golden vectors."""
import numpy as np
import pytest
import torch

import idolq_lib as L
import oracle as O
from conftest import norm_rel

pytestmark = pytest.mark.gpu
DEV = "cuda"


def to_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def test_layer_norm_matches_reference_golden(golden):
    # fp64 accumulation as the reference's norm_rows: bit-identical except, rarely, one ulp (1e-6 abs bar)
    g = golden("norm")
    x = to_dev(g["x"])
    cases = [
        (L.layernorm(to_dev(g["small"]), 1e-5, gamma=to_dev(g["g24"]), beta=to_dev(g["b24"])), g["layer_norm_small"]),
        (L.layernorm(x, 1e-5, gamma=to_dev(g["gamma"]), beta=to_dev(g["beta"])), g["layer_norm"]),
        (L.layernorm(x, 1e-6), g["norm_plain"]),
        (L.layernorm(x, 1e-6, gamma=to_dev(g["gamma"]), beta=to_dev(g["beta"])), g["norm_affine"]),
        (L.layernorm(x, 1e-6, shift=to_dev(g["shift"]), scale=to_dev(g["scale"])), g["norm_ada"]),
        (L.layernorm(x, 1e-5), g["norm_eps5"]),
    ]
    for got, ref in cases:
        assert np.max(np.abs(got.cpu().numpy() - ref)) < 1e-5


def test_adaln_batches_in_place_and_bf16():
    rng = np.random.default_rng(20)
    rows, dim = 2 * 300, 1536
    x = rng.normal(0.2, 1.5, (rows, dim)).astype(np.float32)
    sh = rng.normal(0, 0.1, (2, dim)).astype(np.float32)
    sc = rng.normal(0, 0.1, (2, dim)).astype(np.float32)
    ref = O.norm_rows(x, 1e-6, shift=sh, scale=sc, rows_per_batch=300)
    xt = to_dev(x)
    L.layernorm(xt, 1e-6, shift=to_dev(sh), scale=to_dev(sc), rows_per_batch=300, out=xt)  # in place
    assert np.max(np.abs(xt.cpu().numpy() - ref)) < 1e-5
    xb = to_dev(x).bfloat16()
    yb = L.layernorm(xb, 1e-6, shift=to_dev(sh), scale=to_dev(sc), rows_per_batch=300)
    refb = O.norm_rows(xb.float().cpu().numpy(), 1e-6, shift=sh, scale=sc, rows_per_batch=300)
    assert norm_rel(yb.float().cpu().numpy(), torch.from_numpy(refb).bfloat16().float().numpy()) < 1e-3
    # dims above the register-resident limit take the re-reading path
    x2 = rng.normal(0, 1, (5, 6144)).astype(np.float32)
    assert np.max(np.abs(L.layernorm(to_dev(x2), 1e-6).cpu().numpy() - O.norm_rows(x2, 1e-6))) < 1e-5


@pytest.mark.parametrize("dtype,dim", [(torch.bfloat16, 1536), (torch.float16, 1024), (torch.float32, 1536),
                                       (torch.bfloat16, 512), (torch.bfloat16, 4096)])
def test_vector_rows_match_the_general_kernel(dtype, dim):
    # aligned rows take the one-wave-per-row kernel, a view with an odd row stride the general one: same arithmetic
    # (fp32 values, fp64 sums), so the results agree bit for bit, also in place and with adaLN per batch
    rng = np.random.default_rng(dim)
    rows = 2 * 515
    x = torch.from_numpy(rng.normal(0.1, 1.3, (rows, dim)).astype(np.float32)).to(DEV).to(dtype)
    wide = torch.zeros((rows, dim + 1), device=DEV, dtype=dtype)
    wide[:, :dim] = x
    odd = wide[:, :dim]
    sh = to_dev(rng.normal(0, 0.1, (2, dim)).astype(np.float32))
    sc = to_dev(rng.normal(0, 0.1, (2, dim)).astype(np.float32))
    g = to_dev(rng.normal(1, 0.1, dim).astype(np.float32))
    b = to_dev(rng.normal(0, 0.1, dim).astype(np.float32))
    for kw in (dict(), dict(gamma=g, beta=b), dict(shift=sh, scale=sc, rows_per_batch=515)):
        vec = L.layernorm(x, 1e-6, **kw)
        gen = L.layernorm(odd, 1e-6, **kw)
        assert torch.equal(vec, gen), kw
    xi = x.clone()
    L.layernorm(xi, 1e-6, shift=sh, scale=sc, rows_per_batch=515, out=xi)
    assert torch.equal(xi, L.layernorm(odd, 1e-6, shift=sh, scale=sc, rows_per_batch=515))


@pytest.mark.parametrize("dtype,dim", [(torch.bfloat16, 1536), (torch.float16, 1024), (torch.float32, 1024),
                                       (torch.bfloat16, 512), (torch.bfloat16, 2048)])
def test_streaming_rows_match_the_one_row_per_wave_kernel(dtype, dim):
    # 4096 rows and more, with adaLN batches of whole 4-row groups, take the streaming form (4 rows per wave, all
    # requested up front); below 4096 rows one row per wave. Both sum each row in the same order, so the streaming
    # form's results equal, bit for bit, the one-row-per-wave kernel run on each half (one adaLN batch each): a
    # ragged row count (not a multiple of the 16 rows of a workgroup), every parameter combination, in place. fp32
    # results are within 1e-5 of the oracle.
    rng = np.random.default_rng(dim + 7)
    half = 2060
    rows = 2 * half  # 4120 = 16 * 257 + 8
    x = torch.from_numpy(rng.normal(-0.3, 2.0, (rows, dim)).astype(np.float32)).to(DEV).to(dtype)
    sh = to_dev(rng.normal(0, 0.1, (2, dim)).astype(np.float32))
    sc = to_dev(rng.normal(0, 0.1, (2, dim)).astype(np.float32))
    g = to_dev(rng.normal(1, 0.1, dim).astype(np.float32))
    b = to_dev(rng.normal(0, 0.1, dim).astype(np.float32))
    for kw in (dict(), dict(gamma=g, beta=b), dict(gamma=g), dict(shift=sh, scale=sc),
               dict(gamma=g, beta=b, shift=sh, scale=sc)):
        ada = "shift" in kw
        got = L.layernorm(x, 1e-6, rows_per_batch=half if ada else 0, **kw)
        for h in (0, 1):
            part = {k: (v[h].contiguous() if k in ("shift", "scale") else v) for k, v in kw.items()}
            one = L.layernorm(x[h * half:(h + 1) * half], 1e-6, **part)
            assert torch.equal(got[h * half:(h + 1) * half], one), (kw.keys(), h)
        if dtype == torch.float32 and ("gamma" not in kw or "beta" in kw):  # the oracle takes gamma with beta
            ref = O.norm_rows(x.cpu().numpy(), 1e-6, rows_per_batch=half if ada else 0,
                              **{k: v.cpu().numpy() for k, v in kw.items()})
            assert np.max(np.abs(got.cpu().numpy() - ref)) < 1e-5, kw.keys()
    want = L.layernorm(x, 1e-6, shift=sh, scale=sc, rows_per_batch=half)
    xi = x.clone()
    L.layernorm(xi, 1e-6, shift=sh, scale=sc, rows_per_batch=half, out=xi)
    assert torch.equal(xi, want)


def test_attention_fp32_matches_reference_golden(golden):
    # the reference test shapes, strided rows (tests/test_kernels.cpp:184-228); fp32 kernel, 1e-5 norm-relative
    g = golden("attention")
    for i in range(int(g["cases"])):
        lq, lk, heads, hd, ldq, ldkv = (int(v) for v in g[f"c{i}_shape"])
        dim = heads * hd
        out = torch.empty((lq, dim), device=DEV)
        L.attention(to_dev(g[f"c{i}_q"]), to_dev(g[f"c{i}_k"]), to_dev(g[f"c{i}_v"]), 1, lq, lk, heads, hd, ldq,
                    ldkv, 0, 0, out, dim, 0)
        assert norm_rel(out.cpu().numpy(), g[f"c{i}_out"]) < 1e-5, i


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("lq,lk,heads", [(130, 77, 2), (256, 256, 3), (1, 1, 1), (128, 1024, 2), (300, 64, 1)])
def test_attention_mfma_tracks_fp32_attention(dtype, lq, lk, heads):
    # 16-bit inputs, head_dim 64: against the oracle on the upcast inputs, output rounded to the input dtype, 1e-3
    rng = np.random.default_rng(21)
    hd, dim = 64, heads * 64
    q = to_dev(rng.normal(0, 1, (lq, dim)).astype(np.float32)).to(dtype)
    k = to_dev(rng.normal(0, 1, (lk, dim)).astype(np.float32)).to(dtype)
    v = to_dev(rng.normal(0, 1, (lk, dim)).astype(np.float32)).to(dtype)
    out = torch.empty((lq, dim), device=DEV, dtype=dtype)
    L.attention(q, k, v, 1, lq, lk, heads, hd, dim, dim, 0, 0, out, dim, 0)
    ref = O.attention(q.float().cpu().numpy(), k.float().cpu().numpy(), v.float().cpu().numpy(), lq, lk, dim, dim,
                      heads, hd)
    assert norm_rel(out.float().cpu().numpy(), torch.from_numpy(ref).to(dtype).float().numpy()) < 1e-3


def test_attention_batched_strided_views_of_a_qkv_buffer():
    # batch 2 (guidance pairs), q/k/v as column slices of one [B*S, 3*D] projection buffer, out written strided
    rng = np.random.default_rng(22)
    B, S, heads, hd = 2, 200, 3, 64
    D = heads * hd
    qkv = to_dev(rng.normal(0, 1, (B * S, 3 * D)).astype(np.float32)).bfloat16()
    out = torch.zeros((B * S, D + 8), device=DEV, dtype=torch.bfloat16)
    L.attention(qkv[:, :D], qkv[:, D:2 * D], qkv[:, 2 * D:], B, S, S, heads, hd, 3 * D, 3 * D, S * 3 * D, S * 3 * D,
                out, D + 8, S * (D + 8))
    host = qkv.float().cpu().numpy()
    for b in range(B):
        blk = host[b * S:(b + 1) * S]
        ref = O.attention(blk[:, :D], blk[:, D:2 * D], blk[:, 2 * D:], S, S, D, D, heads, hd)
        got = out[b * S:(b + 1) * S, :D].float().cpu().numpy()
        assert norm_rel(got, torch.from_numpy(ref).bfloat16().float().numpy()) < 1e-3
    assert not out[:, D:].any()


def test_cross_attention_shape_sample():
    # cross-attention: 4096 queries against 1024 context tokens, 24 heads of 64, on a 256-query sample for the oracle
    rng = np.random.default_rng(23)
    lq, lk, heads, hd = 4096, 1024, 24, 64
    D = heads * hd
    q = to_dev(rng.normal(0, 1, (lq, D)).astype(np.float32)).bfloat16()
    kv = to_dev(rng.normal(0, 1, (lk, 2 * D)).astype(np.float32)).bfloat16()
    out = torch.empty((lq, D), device=DEV, dtype=torch.bfloat16)
    L.attention(q, kv[:, :D], kv[:, D:], 1, lq, lk, heads, hd, D, 2 * D, 0, 0, out, D, 0)
    rows = np.arange(0, lq, 16)
    kvh = kv.float().cpu().numpy()
    ref = O.attention(q.float().cpu().numpy()[rows], kvh[:, :D], kvh[:, D:], len(rows), lk, D, D, heads, hd)
    assert norm_rel(out[rows].float().cpu().numpy(), torch.from_numpy(ref).bfloat16().float().numpy()) < 1e-3


def test_activations_and_position_embedding(golden):
    g = golden("elementwise")
    xt = to_dev(g["x_tanh"].copy())
    L.activation(xt, L.ACT_GELU_TANH)
    assert np.max(np.abs(xt.cpu().numpy() - g["gelu_tanh"])) < 1e-5
    xg = to_dev(g["x_gelu"].copy())
    L.activation(xg, L.ACT_GELU_ERF)
    assert np.max(np.abs(xg.cpu().numpy() - g["gelu256"])) < 2e-6
    freqs = (2.0 ** np.linspace(0, 10, 16)).astype(np.float32)
    coords = np.random.default_rng(24).uniform(-1, 1, (1000, 3)).astype(np.float32)
    out = torch.zeros((1000, 352), device=DEV)
    L.pos_embed(to_dev(coords), to_dev(freqs), out[:, 256:])
    ref = O.pos_embed(freqs, coords)
    got = out.cpu().numpy()
    assert np.max(np.abs(got[:, 256:] - ref)) < 1e-4 and not got[:, :256].any()


@pytest.mark.parametrize("hd", [32, 64])
@pytest.mark.parametrize("lq,lk,heads,batch", [(1, 1, 1, 1), (37, 29, 2, 1), (130, 77, 2, 2), (64, 1000, 3, 1),
                                               (300, 64, 1, 1), (33, 4133, 2, 1)])
def test_attention_fp32_matrix_cores_match_the_reference(hd, lq, lk, heads, batch):
    # fp32 inputs with 16-byte aligned rows and head_dim 32 / 64 take the fp32 matrix-core kernel: fp32 products and
    # sums, so it tracks the reference's fp32 attention as closely as its fp32 kernel does (1e-5 bar, usually ~1e-7);
    # q, k and v are views into one projection buffer, with a batch stride
    rng = np.random.default_rng(lq * 31 + lk + hd)
    dim = heads * hd
    qkv = rng.normal(0, 1, (batch, max(lq, lk), 3 * dim)).astype(np.float32)
    buf = to_dev(qkv)
    bs = max(lq, lk) * 3 * dim
    out = torch.full((batch, lq, dim + 4), float("nan"), device=DEV)
    L.attention(buf[:, :, :dim], buf[:, :, dim:2 * dim], buf[:, :, 2 * dim:], batch, lq, lk, heads, hd, 3 * dim,
                3 * dim, bs, bs, out, dim + 4, lq * (dim + 4))
    got = out.cpu().numpy()
    assert np.all(np.isnan(got[:, :, dim:]))  # nothing written past the row
    for bi in range(batch):
        blk = qkv[bi]
        q, k, v = blk[:lq, :dim], blk[:lk, dim:2 * dim], blk[:lk, 2 * dim:]
        want = O.attention(q, k, v, lq, lk, dim, dim, heads, hd)
        assert norm_rel(got[bi, :, :dim], want) < 1e-5
        if O.ref_available():
            assert norm_rel(got[bi, :, :dim], O.ref_attention(q, k, v, lq, lk, dim, dim, heads, hd)) < 1e-5
        # fp64 softmax attention, one head
        s = q[:, :hd].astype(np.float64) @ k[:, :hd].astype(np.float64).T / np.sqrt(hd)
        pr = np.exp(s - s.max(axis=1, keepdims=True))
        o64 = (pr / pr.sum(axis=1, keepdims=True)) @ v[:, :hd].astype(np.float64)
        assert np.max(np.abs(got[bi, :, :hd] - o64)) < 2e-5


def test_self_attention_seq4096_sample():
    # config-2 self-attention at its real shape: batch 2 x 4096 tokens, 24 heads of 64, q/k/v column slices of one
    # [8192, 4608] bf16 projection buffer; 128 sampled queries of each batch against the oracle over all 4096 keys
    rng = np.random.default_rng(25)
    B, S, heads, hd = 2, 4096, 24, 64
    D = heads * hd
    qkv = to_dev(rng.normal(0, 1, (B * S, 3 * D)).astype(np.float32)).bfloat16()
    out = torch.empty((B * S, D), device=DEV, dtype=torch.bfloat16)
    L.attention(qkv[:, :D], qkv[:, D:2 * D], qkv[:, 2 * D:], B, S, S, heads, hd, 3 * D, 3 * D, S * 3 * D, S * 3 * D,
                out, D, S * D)
    host = qkv.float().cpu().numpy()
    got = out.float().cpu().numpy()
    rows = np.arange(5, S, 32)
    for b in range(B):
        blk = host[b * S:(b + 1) * S]
        ref = O.attention(np.ascontiguousarray(blk[rows, :D]), blk[:, D:2 * D], blk[:, 2 * D:], len(rows), S, D, D,
                          heads, hd)
        assert norm_rel(got[b * S + rows], torch.from_numpy(ref).bfloat16().float().numpy()) < 1e-3, b
    assert np.isfinite(got).all()


@pytest.mark.parametrize("lk", [4096, 1024])
def test_attention_full_size_scales_exactly_with_v(lk):
    # Every output of the denoiser's attention shapes: self-attention over 4096 keys (V staged once as fp16 V^T
    # tiles) and cross-attention over 1024 context keys (V converted in the workgroups), batch 2, 24 heads of 64.
    # Scaling V up by a power of two scales each staged fp16 value, each P.V product and sum and the normalised output
    # exactly, so the outputs must scale bit for bit; a misplaced key tile, head or query row anywhere breaks this.
    # (Scaling down is not exact: V's smallest values become fp16 subnormals and lose bits.)
    rng = np.random.default_rng(26 + lk)
    B, S, heads, hd = 2, 4096, 24, 64
    D = heads * hd
    q = to_dev(rng.normal(0, 1, (B * S, D)).astype(np.float32)).bfloat16()
    kv = to_dev(rng.normal(0, 1, (B * lk, 2 * D)).astype(np.float32)).bfloat16()
    outs = []
    for f in (1.0, 2.0, 4.0):
        kvf = kv.clone()
        kvf[:, D:] *= f
        out = torch.empty((B * S, D), device=DEV, dtype=torch.bfloat16)
        L.attention(q, kvf[:, :D], kvf[:, D:], B, S, lk, heads, hd, D, 2 * D, S * D, lk * 2 * D, out, D, S * D)
        outs.append(out)
    assert torch.isfinite(outs[0]).all()
    assert torch.equal(outs[1], outs[0] * 2.0) and torch.equal(outs[2], outs[0] * 4.0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_attention_raises_the_running_maximum(dtype):
    # scores that grow along the keys (key rows scaled from 0.5 to 4, positive means) and, in head 0, one key whose
    # scores exceed every earlier one by far: the first tile's maximum must be raised again and again (without that,
    # later probabilities would leave fp16), against the oracle on the upcast inputs at 1e-3
    rng = np.random.default_rng(27)
    lq, lk, heads, hd = 160, 700, 2, 64
    dim = heads * hd
    q = rng.normal(0.5, 1, (lq, dim)).astype(np.float32)
    k = (rng.normal(0.5, 1, (lk, dim)) * np.linspace(0.5, 4, lk)[:, None]).astype(np.float32)
    k[450, :hd] = 6.0
    v = rng.normal(0, 1, (lk, dim)).astype(np.float32)
    qd, kd, vd = (to_dev(a).to(dtype) for a in (q, k, v))
    out = torch.empty((lq, dim), device=DEV, dtype=dtype)
    L.attention(qd, kd, vd, 1, lq, lk, heads, hd, dim, dim, 0, 0, out, dim, 0)
    ref = O.attention(qd.float().cpu().numpy(), kd.float().cpu().numpy(), vd.float().cpu().numpy(), lq, lk, dim, dim,
                      heads, hd)
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    for h in range(heads):
        cols = slice(h * hd, (h + 1) * hd)
        assert norm_rel(got[:, cols], torch.from_numpy(ref[:, cols]).to(dtype).float().numpy()) < 1e-3, h


@pytest.mark.parametrize("hd", [32, 64])
def test_attention_fp32_running_maximum_rises_tile_after_tile(hd):
    # fp32 matrix-core kernel: scores that grow along the keys, so every tile raises the running maximum and rescales
    # the output before its product, and one key far above all others; the waves walk 6, 6, 6 and 4 tiles of their
    # quarters, so the pipelined loop's branches run with rescale factors below 1. Against the oracle and fp64.
    rng = np.random.default_rng(28)
    lq, lk, heads = 96, 700, 2
    dim = heads * hd
    q = rng.normal(0.5, 1, (lq, dim)).astype(np.float32)
    k = (rng.normal(0.5, 1, (lk, dim)) * np.linspace(0.5, 4, lk)[:, None]).astype(np.float32)
    k[450, :hd] = 6.0
    v = rng.normal(0, 1, (lk, dim)).astype(np.float32)
    out = torch.empty((lq, dim), device=DEV)
    L.attention(to_dev(q), to_dev(k), to_dev(v), 1, lq, lk, heads, hd, dim, dim, 0, 0, out, dim, 0)
    got = out.cpu().numpy()
    assert norm_rel(got, O.attention(q, k, v, lq, lk, dim, dim, heads, hd)) < 1e-5
    for h in range(heads):
        cols = slice(h * hd, (h + 1) * hd)
        s = q[:, cols].astype(np.float64) @ k[:, cols].astype(np.float64).T / np.sqrt(hd)
        pr = np.exp(s - s.max(axis=1, keepdims=True))
        o64 = (pr / pr.sum(axis=1, keepdims=True)) @ v[:, cols].astype(np.float64)
        assert np.max(np.abs(got[:, cols] - o64)) < 2e-5, h


def test_attention_bf16_values_beyond_fp16_range():
    # bf16 V holds values far beyond fp16's 65504 (the reference's fp32 attention takes them): the tiles that hold
    # them are staged with an exact power-of-two scale, so the output stays finite and within the 16-bit bar, with
    # large scores (peaky softmax) as well. Head 1 holds ordinary values: its workgroups take the plain path and
    # give the same bits as a call where no head holds large values.
    rng = np.random.default_rng(26)
    lq, lk, heads, hd = 200, 300, 2, 64
    dim = heads * hd
    q = rng.normal(0, 2.5, (lq, dim)).astype(np.float32)
    k = rng.normal(0, 2.5, (lk, dim)).astype(np.float32)
    v = rng.normal(0, 1, (lk, dim)).astype(np.float32)
    big = v.copy()
    big[64:128, :hd] *= 1e5           # tile 1: |v| up to ~4e5
    big[130, 7] = 3.0e30              # tile 2: one huge value
    big[256:300, :hd] *= -7e4         # the partial last tile
    qd, kd = to_dev(q).bfloat16(), to_dev(k).bfloat16()
    outs = []
    for vals in (v, big):
        vd = to_dev(vals).bfloat16()
        out = torch.empty((lq, dim), device=DEV, dtype=torch.float32)
        L.attention(qd, kd, vd, 1, lq, lk, heads, hd, dim, dim, 0, 0, out, dim, 0)
        outs.append(out)
        ref = O.attention(qd.float().cpu().numpy(), kd.float().cpu().numpy(), vd.float().cpu().numpy(), lq, lk, dim,
                          dim, heads, hd)
        got = out.cpu().numpy()
        assert np.isfinite(got).all()
        for h in range(heads):
            cols = slice(h * hd, (h + 1) * hd)
            assert norm_rel(got[:, cols], ref[:, cols]) < 1e-3, h
    assert torch.equal(outs[0][:, hd:], outs[1][:, hd:])
    assert float(outs[1][:, :hd].abs().max()) > 1e5


@pytest.mark.parametrize("batch,lq,lk,heads", [(1, 200, 300, 2), (2, 1000, 777, 3), (2, 640, 4096, 4), (1, 64, 64, 1)])
def test_attention_staged_v_tiles_give_the_same_bits(batch, lq, lk, heads):
    # bf16 inputs with head_dim 64: V converted once per call into fp16 V^T tiles (attn_v_tiles, the workspace entry
    # point) against V converted in every query workgroup (no workspace): the same operands and arithmetic, so the
    # same bits; with tiles beyond fp16's range (scaled per tile by the same rule), an infinity-free huge value, and
    # ragged key and query counts (the last tile's keys past lk are zero in the staged tiles)
    print(f"staged V batch={batch} lq={lq} lk={lk} heads={heads}", flush=True)
    rng = np.random.default_rng(batch * 1000 + lk)
    hd = 64
    dim = heads * hd
    q = rng.normal(0, 2.0, (batch * lq, dim)).astype(np.float32)
    k = rng.normal(0, 2.0, (batch * lk, dim)).astype(np.float32)
    v = rng.normal(0, 1, (batch * lk, dim)).astype(np.float32)
    if lk > 130:
        v[64:128, :hd] *= 1e5
        v[130, 7] = 3.0e30
    qd, kd, vd = (to_dev(a).bfloat16() for a in (q, k, v))
    outs = []
    for staged in (True, False):
        out = torch.empty((batch * lq, dim), device=DEV, dtype=torch.bfloat16)
        L.attention(qd, kd, vd, batch, lq, lk, heads, hd, dim, dim, lq * dim, lk * dim, out, dim, lq * dim,
                    staged_v=staged)
        outs.append(out)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    assert torch.isfinite(outs[0].float()).all()
    lib = L.load()
    assert lib.idolq_attention_workspace(L.BF16, batch, lk, heads, hd) >= batch * heads * ((lk + 63) // 64) * 8192
    assert lib.idolq_attention_workspace(L.F16, batch, lk, heads, hd) == 0


def test_attention_workspace_entry_point_through_the_c_abi():
    # idolq_attention_ws called directly: with its workspace (V staged), with one byte short of it (the call falls
    # back to converting V in the workgroups) and through idolq_attention: the same bits each time
    import ctypes
    lib = L.load()
    rng = np.random.default_rng(61)
    batch, lq, lk, heads, hd = 2, 256, 640, 3, 64
    dim = heads * hd
    q, k, v = (to_dev(rng.normal(0, 1, (batch * n, dim)).astype(np.float32)).bfloat16() for n in (lq, lk, lk))
    need = int(lib.idolq_attention_workspace(L.BF16, batch, lk, heads, hd))
    assert need >= batch * heads * ((lk + 63) // 64) * 8192
    ws = torch.empty(need, device=DEV, dtype=torch.uint8)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    outs = []
    for nbytes in (need, need - 1, None):
        out = torch.empty((batch * lq, dim), device=DEV, dtype=torch.bfloat16)
        args = [ctypes.c_void_p(t.data_ptr()) for t in (q, k, v)] + [L.BF16, batch, lq, lk, heads, hd, dim, dim,
                                                                    lq * dim, lk * dim, ctypes.c_void_p(out.data_ptr()),
                                                                    L.BF16, dim, lq * dim]
        if nbytes is None:
            rc = lib.idolq_attention(*args, stream)
        else:
            rc = lib.idolq_attention_ws(*args, ctypes.c_void_p(ws.data_ptr()), nbytes, stream)
        assert rc == 0, lib.idolq_last_error()
        outs.append(out)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
