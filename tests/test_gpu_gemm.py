"""GPU parity of the Q8_0 path: libidolq's kernels against the oracle on the same seeded inputs.

Bars (written per test): integer work (Q8_0 quantization, activation quantization, int8 block dot products,
Q8_0 expansion) is bit-exact; float outputs are within 1e-3 norm-relative error of the reference's float / integer
kernels (EXACT / INT8 modes) and 2e-2 for the bf16-dequant path (DEQUANT), measured against the CPU result rounded
to the output dtype.
"""
import ctypes

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


def q8(rng, n, k, std=0.02):
    return O.q8_0_quantize(rng.normal(0, std, (n, k)).astype(np.float32))


def rounded(a, dtype):
    return torch.from_numpy(np.asarray(a, np.float32)).to(dtype).float().numpy()


def test_q8_0_quantize_is_bit_exact():
    rng = np.random.default_rng(10)
    for n, k in ((1, 32), (37, 64), (256, 1536), (64, 352)):
        w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
        w[0, :32] = 0.0  # an all-zero block
        assert np.array_equal(L.quantize_q8_0(to_dev(w)).cpu().numpy(), O.q8_0_quantize(w))


def test_q8_0_dequant_matches_closed_form():
    rng = np.random.default_rng(11)
    for n, k in ((48, 96), (513, 1024)):
        w = q8(rng, n, k, 0.5)
        ref = O.q8_0_dequant(w, n, k)
        for dt in (torch.float32, torch.bfloat16, torch.float16):
            got = L.dequant(to_dev(w), n, k, dt).cpu()
            assert torch.equal(got, torch.from_numpy(ref).to(dt)), dt


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_activation_quantization_is_bit_exact(golden, dtype):
    g = golden("quantize_act")
    if dtype == torch.float32:
        qa, sa, qs = L.quantize_act(to_dev(g["a"]))
        assert np.array_equal(qa.cpu().numpy(), g["qa"])
        assert np.array_equal(sa.cpu().numpy().view(np.uint32), g["sa"].view(np.uint32))
        assert np.array_equal(qs.cpu().numpy(), g["qsum"])
    rng = np.random.default_rng(12)
    a = rng.normal(0, 1, (300, 1536)).astype(np.float32)
    x = to_dev(a).to(dtype)
    qa, sa, qs = L.quantize_act(x)
    rqa, rsa, rqs = O.quantize_act(x.float().cpu().numpy())
    assert np.array_equal(qa.cpu().numpy(), rqa)
    assert np.array_equal(sa.cpu().numpy().view(np.uint32), rsa.view(np.uint32))
    assert np.array_equal(qs.cpu().numpy(), rqs)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_activation_quantization_without_sums_is_bit_exact(dtype):
    # without code sums, 16-bit rows take the four-threads-per-block quantizer (the INT8 GEMM's): the same codes and
    # scales as the oracle, with an odd row count (a partial last workgroup), an all-zero block and ties to even
    rng = np.random.default_rng(13)
    a = rng.normal(0, 3, (301, 1536)).astype(np.float32)
    a[7, 64:96] = 0.0
    a[8, :32] = np.concatenate([[127.0], np.arange(31) * 0.5 - 7.5]).astype(np.float32)  # amax 127: x.5 ties
    x = to_dev(a).to(dtype)
    qa, sa, qs = L.quantize_act(x, with_qsum=False)
    rqa, rsa, _ = O.quantize_act(x.float().cpu().numpy())
    assert qs is None
    assert np.array_equal(qa.cpu().numpy(), rqa)
    assert np.array_equal(sa.cpu().numpy().view(np.uint32), rsa.view(np.uint32))
    assert not qa[7, 64:96].any() and float(sa[7, 2]) == 0.0


@pytest.mark.parametrize("m,n,k,off,cnt", [(70, 100, 352, 0, 100), (130, 200, 256, 16, 150), (5, 21, 32, 0, 21),
                                           (256, 384, 1536, 128, 256), (1, 7, 64, 0, 7)])
def test_int8_mfma_block_dots_are_bit_exact(m, n, k, off, cnt):
    rng = np.random.default_rng(13)
    a = rng.normal(0, 1, (m, k)).astype(np.float32)
    w = q8(rng, n, k, 0.05)
    qa, _, _ = O.quantize_act(a)
    got = L.block_dots(to_dev(qa), to_dev(w), n, off, cnt).cpu().numpy()
    assert np.array_equal(got, O.block_dots(qa, w, k, off, cnt))


def test_gemm_against_reference_golden_vectors(golden):
    # The reference's own outputs for its test shapes (tests/golden/gemm_q8.npz): EXACT vs the float kernel and INT8
    # vs the integer kernel, fp32 in and out, each within 1e-5 norm-relative, on row-major Q8_0 blocks and (five of
    # the ten cases) on the tiled layout.
    g = golden("gemm_q8")
    for i in range(int(g["cases"])):
        m, n, k, off, cnt, res, gelu = (int(v) for v in g[f"c{i}_shape"])
        a, w, bias = g[f"c{i}_a"], g[f"c{i}_w"], g[f"c{i}_bias"]
        r = to_dev(g[f"c{i}_residual"]) if res else None
        act = L.ACT_GELU_ERF if gelu else L.ACT_NONE
        # the same weights in the tiled layout where it applies (k % 64 == 0, window starting at a multiple of 32)
        layouts = [(to_dev(w), False)]
        if k % 64 == 0 and off % 32 == 0:
            layouts.append((L.tile_q8_0(to_dev(w), n, k), True))
        for wd, tiled in layouts:
            for mode, key, bar in ((L.MODE_EXACT, "y_float", 1e-5), (L.MODE_INT8, "y_int8", 1e-5)):
                y = L.gemm(to_dev(a), wd, n, off, cnt, bias=to_dev(bias), residual=r, act=act, mode=mode,
                           tiled=tiled)
                err = norm_rel(y.cpu().numpy(), g[f"c{i}_{key}"])
                assert err < bar, (i, key, tiled, err)


@pytest.mark.parametrize("m,n,k", [(256, 1024, 1024), (70, 100, 352), (33, 37, 64), (5, 21, 32), (300, 96, 1280)])
def test_exact_and_int8_modes_track_the_reference_kernels(m, n, k):
    # Config-0 shape (256 x 1024 x 1024) and ragged tails in every direction.
    rng = np.random.default_rng(14)
    a = rng.normal(0, 1, (m, k)).astype(np.float32)
    w = q8(rng, n, k)
    b = rng.normal(0, 0.01, n).astype(np.float32)
    at, wt, bt = to_dev(a), to_dev(w), to_dev(b)
    assert norm_rel(L.gemm(at, wt, n, bias=bt, mode=L.MODE_EXACT).cpu().numpy(), O.gemm_q8_float(a, w, n, k, b)) < 1e-5
    assert norm_rel(L.gemm(at, wt, n, bias=bt, mode=L.MODE_INT8).cpu().numpy(), O.gemm_q8_int8(a, w, n, k, b)) < 1e-5
    # 16-bit activations: EXACT stays within 1e-3 of the float kernel on the same (upcast) inputs, DEQUANT within 2e-2
    for dt in (torch.bfloat16, torch.float16):
        xr = rounded(a, dt)
        ref = O.gemm_q8_float(xr, w, n, k, b)
        ye = L.gemm(at.to(dt), wt, n, bias=bt, mode=L.MODE_EXACT, out_dtype=torch.float32).cpu().numpy()
        yd = L.gemm(at.to(dt), wt, n, bias=bt, mode=L.MODE_DEQUANT, out_dtype=torch.float32).cpu().numpy()
        assert norm_rel(ye, ref) < 1e-5
        assert norm_rel(yd, ref) < 2e-2
        # output rounded to the activation dtype, compared with the CPU result rounded the same way
        yo = L.gemm(at.to(dt), wt, n, bias=bt, mode=L.MODE_EXACT).float().cpu().numpy()
        assert norm_rel(yo, rounded(ref, dt)) < 1e-3


@pytest.mark.parametrize("m,n_total,k,off,cnt,xdt", [
    (256, 1024, 1024, 0, 1024, torch.float32),   # config 0's shape, fp32 activations (the reference's input)
    (300, 520, 512, 32, 448, torch.bfloat16),    # ragged rows and a column window
    (1, 96, 128, 0, 96, torch.float16),          # one row (the scale pairs past m), two stages
    (512, 512, 4096, 0, 512, torch.bfloat16),    # stream-K (every tile split)
    (4096, 1536, 6144, 0, 1536, torch.bfloat16), # the MLP block's down projection (stream-K)
])
def test_int8_on_tiled_weights_matches_the_row_major_int8_kernel(m, n_total, k, off, cnt, xdt):
    # INT8 mode on tiled weights (int8 MFMA on the tiled fragments, the block scale fold in the wide kernel) against
    # the row-major INT8 kernel on the same blocks: whole tiles give the same bits (the same int32 block dots, folded
    # in the same order with the same roundings); with the tiles' k range split over the CUs the parts' sums differ
    # only by fp32 reassociation, repeated calls are bit-identical, and every tile counter ends at zero. The small
    # shapes also against the oracle's integer kernel (1e-5).
    print(f"int8 tiled m={m} n={n_total} k={k} window {off}+{cnt} {xdt}", flush=True)
    rng = np.random.default_rng(m + k)
    a = rng.normal(0, 1, (m, k)).astype(np.float32)
    wq = q8(rng, n_total, k)
    b = rng.normal(0, 0.01, n_total).astype(np.float32)
    x, wd, bt = to_dev(a).to(xdt), to_dev(wq), to_dev(b)
    wt = L.tile_q8_0(wd, n_total, k)
    kw = dict(bias=bt, mode=L.MODE_INT8, out_dtype=torch.float32)
    raw = L.gemm(x, wd, n_total, off, cnt, **kw)
    til = L.gemm(x, wt, n_total, off, cnt, tiled=True, **kw)
    # an explicit workspace whose tile counters (after the codes and scales) start as garbage: the quantizer clears
    # them, and the split GEMM leaves them at zero
    lib = L.load()
    full = int(lib.idolq_q8_0_gemm_workspace(m, k, L.MODE_INT8))
    prefix = full - int(lib.idolq_q8_0_gemm_workspace(m, k, L.MODE_DEQUANT))
    ws = torch.zeros(full, device=DEV, dtype=torch.uint8)
    ws[prefix:prefix + 4096] = 7
    spl = [L.gemm(x, wt, n_total, off, cnt, tiled=True, split=True, workspace=ws, **kw) for _ in range(2)]
    torch.cuda.synchronize()
    assert torch.equal(raw, til)
    assert torch.equal(spl[0], spl[1])
    assert norm_rel(spl[0].cpu().numpy(), til.cpu().numpy()) < 1e-6
    assert int(ws[prefix:prefix + 4096].view(torch.int32).abs().sum().item()) == 0
    if m * k <= 2 ** 20:
        wrows = wq.reshape(n_total, -1)[off:off + cnt].reshape(-1)
        ref = O.gemm_q8_int8(x.float().cpu().numpy(), wrows, cnt, k, b[off:off + cnt])
        assert norm_rel(til.cpu().numpy(), ref) < 1e-5


@pytest.mark.parametrize("m,n_total,k,off,cnt,xdt", [
    (256, 1024, 1024, 0, 1024, torch.float32),   # config 0's shape, fp32 activations (the reference's input)
    (300, 520, 512, 32, 448, torch.float32),     # ragged rows and a column window
    (1, 96, 128, 0, 96, torch.float16),          # one row, two stages
    (70, 200, 320, 64, 136, torch.bfloat16),     # ragged everything, five stages
    (512, 512, 4096, 0, 512, torch.float32),     # stream-K (every tile split)
    (2048, 1536, 1536, 0, 1536, torch.float32),  # a full wave of tiles and a partial one
])
def test_exact_on_tiled_weights_matches_the_row_major_exact_kernel(m, n_total, k, off, cnt, xdt):
    # EXACT mode on tiled weights (activations split into bf16 high and low parts, two bf16 MFMA products per block,
    # the block scale folded in fp32) against the row-major EXACT kernel and the oracle's float kernel: both within
    # 1e-5 of the oracle, within 1e-6 of each other (fp32 reassociation only); with the k range split over the CUs
    # repeated calls are bit-identical and every tile counter ends at zero (an explicit workspace whose counters
    # start as garbage: the split prepass clears them)
    print(f"exact tiled m={m} n={n_total} k={k} window {off}+{cnt} {xdt}", flush=True)
    rng = np.random.default_rng(m + k + 1)
    a = rng.normal(0, 1, (m, k)).astype(np.float32)
    wq = q8(rng, n_total, k)
    b = rng.normal(0, 0.01, n_total).astype(np.float32)
    x, wd, bt = to_dev(a).to(xdt), to_dev(wq), to_dev(b)
    wt = L.tile_q8_0(wd, n_total, k)
    kw = dict(bias=bt, mode=L.MODE_EXACT, out_dtype=torch.float32)
    raw = L.gemm(x, wd, n_total, off, cnt, **kw)
    til = L.gemm(x, wt, n_total, off, cnt, tiled=True, **kw)
    lib = L.load()
    full = int(lib.idolq_q8_0_gemm_workspace(m, k, L.MODE_EXACT))
    prefix = full - int(lib.idolq_q8_0_gemm_workspace(m, k, L.MODE_DEQUANT))
    assert prefix >= 4 * m * k
    ws = torch.zeros(full, device=DEV, dtype=torch.uint8)
    ws[prefix:prefix + 4096] = 7
    spl = [L.gemm(x, wt, n_total, off, cnt, tiled=True, split=True, workspace=ws, **kw) for _ in range(2)]
    torch.cuda.synchronize()
    assert norm_rel(til.cpu().numpy(), raw.cpu().numpy()) < 1e-6
    assert torch.equal(spl[0], spl[1])
    assert norm_rel(spl[0].cpu().numpy(), til.cpu().numpy()) < 1e-6
    assert int(ws[prefix:prefix + 4096].view(torch.int32).abs().sum().item()) == 0
    if m * k <= 2 ** 20:
        wrows = wq.reshape(n_total, -1)[off:off + cnt].reshape(-1)
        ref = O.gemm_q8_float(x.float().cpu().numpy(), wrows, cnt, k, b[off:off + cnt])
        assert norm_rel(til.cpu().numpy(), ref) < 1e-5


def test_exact_on_tiled_weights_epilogue_and_workspace_check():
    # fp32 output with bias, residual aliasing y and erf-GELU (the reference's float-kernel epilogue) through the
    # tiled EXACT path, against the row-major EXACT kernel; a workspace below the high and low parts is refused
    rng = np.random.default_rng(33)
    m, n, k = 333, 416, 768
    x = to_dev(rng.normal(0, 1, (m, k)).astype(np.float32))
    wq = to_dev(q8(rng, n, k))
    wt = L.tile_q8_0(wq, n, k)
    bt = to_dev(rng.normal(0, 0.1, n).astype(np.float32))
    res = to_dev(rng.normal(0, 1, (m, n)).astype(np.float32))
    outs = []
    for w, tiled in ((wq, False), (wt, True)):
        y = res.clone()
        L.gemm(x, w, n, bias=bt, residual=y, act=L.ACT_GELU_ERF, mode=L.MODE_EXACT, out=y, tiled=tiled)
        outs.append(y)
    torch.cuda.synchronize()
    assert norm_rel(outs[1].cpu().numpy(), outs[0].cpu().numpy()) < 1e-6
    lib = L.load()
    small = torch.zeros(4 * m * k - 256, device=DEV, dtype=torch.uint8)
    y = torch.empty((m, n), device=DEV)
    rc = lib.idolq_q8_0_gemm(ctypes.c_void_p(x.data_ptr()), L.F32, m, k, k, ctypes.c_void_p(wt.data_ptr()), n, 0, n,
                             None, 0, None, 0, 0, L.ACT_NONE, L.MODE_EXACT, L.FLAG_TILED_WEIGHTS,
                             ctypes.c_void_p(y.data_ptr()), L.F32, n, ctypes.c_void_p(small.data_ptr()), small.numel(),
                             ctypes.c_void_p(torch.cuda.current_stream(DEV).cuda_stream))
    assert rc == L.EINVAL and b"workspace" in lib.idolq_last_error()


def test_int8_on_tiled_weights_register_epilogue():
    # bf16 output through the register epilogue (bias, residual aliasing y, tanh-GELU), whole tiles and split: the
    # same bits as the row-major INT8 kernel's epilogue for whole tiles, within the output rounding when split
    rng = np.random.default_rng(31)
    m, n, k = 1000, 768, 2048
    x = to_dev(rng.normal(0, 1, (m, k)).astype(np.float32)).bfloat16()
    wq = to_dev(q8(rng, n, k))
    wt = L.tile_q8_0(wq, n, k)
    bt = to_dev(rng.normal(0, 0.1, n).astype(np.float32))
    res = to_dev(rng.normal(0, 1, (m, n)).astype(np.float32)).bfloat16()
    outs = []
    for w, tiled, split in ((wq, False, False), (wt, True, False), (wt, True, True)):
        y = res.clone()
        L.gemm(x, w, n, bias=bt, residual=y, act=L.ACT_GELU_TANH, mode=L.MODE_INT8, out=y, tiled=tiled, split=split)
        outs.append(y)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    assert norm_rel(outs[2].float().cpu().numpy(), outs[0].float().cpu().numpy()) < 1e-2


def test_epilogue_window_residual_alias_and_activations():
    rng = np.random.default_rng(15)
    m, n, k = 67, 160, 256
    a = rng.normal(0, 1, (m, k)).astype(np.float32)
    w = q8(rng, n, k, 0.05)
    b = rng.normal(0, 0.1, n).astype(np.float32)
    off, cnt = 32, 96
    res = rng.normal(0, 1, (m, cnt)).astype(np.float32)
    # residual aliasing the output (src/decoders.cpp:303 passes X as both)
    y = to_dev(res.copy())
    L.gemm(to_dev(a), to_dev(w), n, off, cnt, bias=to_dev(b), residual=y, act=L.ACT_GELU_ERF, mode=L.MODE_EXACT,
           out=y)
    ref = O.gemm_q8_float(a, w, n, k, b, off, cnt, res, True)
    assert norm_rel(y.cpu().numpy(), ref) < 1e-5
    pre = O.gemm_q8_float(a, w, n, k, b, off, cnt)
    for act, fn in ((L.ACT_GELU_TANH, lambda v: O.gelu_tanh(v)), (L.ACT_RELU, lambda v: np.maximum(v, 0))):
        got = L.gemm(to_dev(a), to_dev(w), n, off, cnt, bias=to_dev(b), act=act, mode=L.MODE_EXACT).cpu().numpy()
        assert norm_rel(got, fn(pre)) < 1e-5
    # strided activation rows (ldx > k) and an output written into a wider buffer
    wide = np.zeros((m, k + 40), np.float32)
    wide[:, 8:8 + k] = a
    xt = to_dev(wide)[:, 8:8 + k]
    out = torch.zeros((m, cnt + 10), device=DEV)
    L.gemm(xt, to_dev(w), n, off, cnt, bias=to_dev(b), mode=L.MODE_EXACT, out=out[:, 5:5 + cnt])
    got = out.cpu().numpy()
    assert norm_rel(got[:, 5:5 + cnt], pre) < 1e-5 and not got[:, :5].any() and not got[:, 5 + cnt:].any()


def test_triton_compatible_rounding_before_bias():
    # tools/idol_triton.py:84-89: acc rounded to the output dtype, then bias added, then rounded again.
    rng = np.random.default_rng(16)
    m, n, k = 64, 96, 512
    x = to_dev(rng.normal(0, 1, (m, k)).astype(np.float32)).bfloat16()
    w = q8(rng, n, k, 0.25)
    bias = to_dev(rng.normal(0, 1, n).astype(np.float32)).bfloat16()
    y = L.gemm(x, to_dev(w), n, bias=bias, mode=L.MODE_DEQUANT, flags=L.FLAG_ROUND_BEFORE_BIAS)
    dense = L.dequant(to_dev(w), n, k, torch.bfloat16)
    ref = (x.float() @ dense.float().T).bfloat16() + bias
    assert torch.equal(y, ref) or norm_rel(y.float().cpu().numpy(), ref.float().cpu().numpy()) < 1e-3


def test_mlp_block_config_shape_parity_on_a_row_sample():
    # x bf16 [4096, 1536]; up Q8_0 [6144 x 1536] + bias + tanh-GELU; down Q8_0 [1536 x 6144] + bias + residual.
    # Full-size GPU run, parity on 64 sampled rows against the oracle (float kernel on the upcast inputs, the GELU
    # applied after the GEMM as the reference's decoders do, intermediates rounded to bf16 as the GPU stores them).
    rng = np.random.default_rng(17)
    M, D, H = 4096, 1536, 6144
    x = to_dev(rng.normal(0, 1, (M, D)).astype(np.float32)).bfloat16()
    wu, wd = q8(rng, H, D), q8(rng, D, H)
    bu, bd = rng.normal(0, 0.01, H).astype(np.float32), rng.normal(0, 0.01, D).astype(np.float32)
    for mode, bar in ((L.MODE_DEQUANT, 2e-2), (L.MODE_EXACT, 1e-3)):
        h = L.gemm(x, to_dev(wu), H, bias=to_dev(bu), act=L.ACT_GELU_TANH, mode=mode)
        y = L.gemm(h, to_dev(wd), D, bias=to_dev(bd), residual=x, mode=mode)
        rows = rng.choice(M, 64, replace=False)
        xs = x[rows].float().cpu().numpy()
        h_ref = rounded(O.gelu_tanh(O.gemm_q8_float(xs, wu, H, D, bu)), torch.bfloat16)
        assert norm_rel(h[rows].float().cpu().numpy(), h_ref) < bar
        y_ref = O.gemm_q8_float(h[rows].float().cpu().numpy(), wd, D, H, bd, residual=xs)
        assert norm_rel(y[rows].float().cpu().numpy(), rounded(y_ref, torch.bfloat16)) < bar
        assert torch.isfinite(y).all()


def test_mlp_block_benchmarked_path_against_the_oracle():
    # The MLP block exactly as bench.py times it: tiled weights with the split workspace (the up projection's launch
    # plan at 4096 x 1536 -> 6144 is the split-column pair kernel, the down projection's 4096 x 6144 -> 1536 is
    # stream-K), tanh-GELU and bias on the way up, bias and residual on the way down; then the down projection once
    # more with the residual aliasing its output (y += h W^T + b, as the denoiser layers add into the stream).
    # 64 sampled rows against the oracle's float kernel on the upcast inputs (2e-2, the DEQUANT bar), and against the
    # oracle's dense fp32 kernel on the weights the DEQUANT arithmetic multiplies (each Q8_0 value rounded to bf16)
    # within 1e-3 (the bar of the reference's fused test, tests/python/test_fused_packed.py:53-57), both rounded to
    # bf16 as the GPU stores them; the down projection's 1e-3 check runs on the GPU's own h.
    rng = np.random.default_rng(23)
    M, D, H = 4096, 1536, 6144
    x = to_dev(rng.normal(0, 1, (M, D)).astype(np.float32)).bfloat16()
    wu, wd = q8(rng, H, D), q8(rng, D, H)
    bu, bd = rng.normal(0, 0.01, H).astype(np.float32), rng.normal(0, 0.01, D).astype(np.float32)
    tu, td = L.tile_q8_0(to_dev(wu), H, D), L.tile_q8_0(to_dev(wd), D, H)
    h = torch.empty((M, H), device=DEV, dtype=torch.bfloat16)
    y = torch.empty((M, D), device=DEV, dtype=torch.bfloat16)
    L.gemm(x, tu, H, bias=to_dev(bu), act=L.ACT_GELU_TANH, mode=L.MODE_DEQUANT, out=h, tiled=True, split=True)
    L.gemm(h, td, D, bias=to_dev(bd), residual=x, mode=L.MODE_DEQUANT, out=y, tiled=True, split=True)
    acc = x.clone()
    L.gemm(h, td, D, bias=to_dev(bd), residual=acc, mode=L.MODE_DEQUANT, out=acc, tiled=True, split=True)
    torch.cuda.synchronize()
    assert torch.equal(acc, y)  # aliasing the residual changes nothing
    rows = rng.choice(M, 64, replace=False)
    xs = x[rows].float().cpu().numpy()
    wu_t, wd_t = rounded(O.q8_0_dequant(wu, H, D), torch.bfloat16), rounded(O.q8_0_dequant(wd, D, H), torch.bfloat16)
    h_ref = rounded(O.gelu_tanh(O.gemm_q8_float(xs, wu, H, D, bu)), torch.bfloat16)
    h_deq = rounded(O.gelu_tanh(O.gemm_dense(xs, wu_t, bu)), torch.bfloat16)
    hs = h[rows].float().cpu().numpy()
    assert norm_rel(hs, h_ref) < 2e-2 and norm_rel(hs, h_deq) < 1e-3
    y_chain = rounded(O.gemm_q8_float(h_ref, wd, D, H, bd, residual=xs), torch.bfloat16)
    y_deq = rounded(O.gemm_dense(hs, wd_t, bd) + xs, torch.bfloat16)
    ys = y[rows].float().cpu().numpy()
    assert norm_rel(ys, y_chain) < 2e-2 and norm_rel(ys, y_deq) < 1e-3
    assert torch.isfinite(h).all() and torch.isfinite(y).all()
    ws = L.split_workspace_of(x.device)
    assert int(ws[:4096].view(torch.int32).abs().sum().item()) == 0  # every split tile was finished


@pytest.mark.parametrize("mode", [L.MODE_DEQUANT, L.MODE_INT8])
@pytest.mark.parametrize("m,n,k", [(4096, 6144, 1536), (4096, 1536, 6144), (8192, 1536, 1536)])
def test_launch_plans_scale_exactly_at_full_size(m, n, k, mode):
    # Every output of the full-size plans: the split-column pair kernel (DEQUANT, 4096 x 1536 -> 6144), stream-K
    # (4096 x 6144 -> 1536), whole 128 x 384 tiles (8192 x 1536 -> 1536), and the INT8 fold with its two workgroups per
    # CU. Scaling x by a power of two scales every product and every fp32 partial sum exactly, whatever tile, stage or
    # stream-K part computed it; in INT8 mode it leaves the codes alone and scales the activation scales exactly. So
    # the outputs must scale bit for bit, and a misplaced row, column or partial tile anywhere breaks this.
    rng = np.random.default_rng(m + n + k)
    x = to_dev(rng.normal(0, 1, (m, k)).astype(np.float32)).bfloat16()
    w = L.tile_q8_0(to_dev(q8(rng, n, k)), n, k)
    y = L.gemm(x, w, n, mode=mode, tiled=True, split=True)
    for f in (2.0, 0.25):
        yf = L.gemm(x * f, w, n, mode=mode, tiled=True, split=True)
        assert torch.equal(yf, y * f), f
    assert torch.isfinite(y).all() and y.float().abs().max().item() > 0


def test_wrappers_reject_wrong_dtypes_and_short_views_on_the_device():
    # Outputs and residuals must cover [m, n] (a short-row view or a narrower column slice of a wider buffer is
    # rejected before any launch) and have a dtype the library writes; a column slice of the right width inside a
    # wider buffer is accepted and leaves the columns around it untouched.
    rng = np.random.default_rng(24)
    m, n, k = 64, 96, 128
    x = to_dev(rng.normal(0, 1, (m, k)).astype(np.float32)).bfloat16()
    w = to_dev(q8(rng, n, k))
    wide = torch.zeros((m, n + 16), device=DEV, dtype=torch.bfloat16)
    for bad in (wide[:m - 1, :n], wide[:, :n - 1], torch.zeros((m, n), device=DEV, dtype=torch.float64),
                torch.zeros((m, n), device=DEV, dtype=torch.int32)):
        with pytest.raises(ValueError):
            L.gemm(x, w, n, out=bad, mode=L.MODE_DEQUANT)
    with pytest.raises(ValueError):
        L.gemm(x, w, n, residual=torch.zeros((m, n), device=DEV, dtype=torch.int16), mode=L.MODE_DEQUANT)
    with pytest.raises(ValueError):
        L.layernorm(x, 1e-6, out=torch.zeros((m, k), device=DEV, dtype=torch.int8))
    with pytest.raises(ValueError):
        L.layernorm(x, 1e-6, out=wide[:m // 2, :k])
    L.gemm(x, w, n, out=wide[:, 8:8 + n], mode=L.MODE_DEQUANT)
    ref = L.gemm(x, w, n, mode=L.MODE_DEQUANT)
    assert torch.equal(wide[:, 8:8 + n], ref) and not wide[:, :8].any() and not wide[:, 8 + n:].any()


def test_empty_and_tiny_inputs():
    rng = np.random.default_rng(18)
    w = q8(rng, 7, 64)
    x = torch.empty((0, 64), device=DEV)
    assert L.gemm(x, to_dev(w), 7, mode=L.MODE_EXACT).shape == (0, 7)
    a = rng.normal(0, 1, (1, 64)).astype(np.float32)
    y = L.gemm(to_dev(a), to_dev(w), 7, 3, 1, mode=L.MODE_EXACT).cpu().numpy()
    ref = O.gemm_q8_float(a, w, 7, 64, None, 3, 1)
    # a single output that is a cancelling sum: the 1e-3 bar, and an absolute bound of the bf16 high/low split of
    # fp32 activations (2^-16 of each term) against the sum of the terms' magnitudes
    terms = np.abs(a[0] * O.q8_0_dequant(w, 7, 64)[3]).sum()
    assert norm_rel(y, ref) < 1e-3 and abs(float(y[0, 0] - ref[0, 0])) <= terms * 2.0 ** -16


@pytest.mark.parametrize("m,n,k", [(1024, 1536, 2048), (512, 384, 1280), (4096, 1536, 6144), (300, 520, 3072),
                                   (4096, 6144, 1536), (1000, 1536, 1536)])
def test_split_k_matches_whole_tiles(m, n, k):
    # DEQUANT on tiled weights with the k stages of the leftover tiles split over the CUs (stream-K: partial tiles
    # added through the workspace) against whole tiles per workgroup: the same products summed in another grouping
    # (fp32), so within 1e-5 norm-relative before the output rounding (fp32 output here); both within 1e-3 of an fp32
    # product of the dequantized weights. Repeated calls are bit-identical (the parts of a split tile are added in a
    # fixed order, whichever part finishes it), and every tile counter in the workspace is back to zero afterwards.
    rng = np.random.default_rng(m + n + k)
    wq = to_dev(q8(rng, n, k))
    w = L.tile_q8_0(wq, n, k)
    x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(DEV).bfloat16()
    b = torch.from_numpy(rng.normal(0, 0.01, n).astype(np.float32)).to(DEV)
    whole = L.gemm(x, w, n, bias=b, mode=L.MODE_DEQUANT, out_dtype=torch.float32, split=False, tiled=True)
    runs = [L.gemm(x, w, n, bias=b, mode=L.MODE_DEQUANT, out_dtype=torch.float32, split=True, tiled=True)
            for _ in range(3)]
    bf = [L.gemm(x, w, n, bias=b, residual=x[:, :n] if n <= k else None, mode=L.MODE_DEQUANT, split=s, tiled=True)
          for s in (False, True)]
    torch.cuda.synchronize()
    # the finishing part sums the parts in range order whichever part arrives last: repeats are bit-identical
    assert torch.equal(runs[1], runs[0]) and torch.equal(runs[2], runs[0])
    assert torch.equal(L.gemm(x, w, n, bias=b, mode=L.MODE_DEQUANT, split=True, tiled=True),
                       L.gemm(x, w, n, bias=b, mode=L.MODE_DEQUANT, split=True, tiled=True))
    assert norm_rel(runs[0].cpu().numpy(), whole.cpu().numpy()) < 1e-5
    # bf16 output through the register epilogue: split and whole differ at most by the output rounding
    assert norm_rel(bf[1].float().cpu().numpy(), bf[0].float().cpu().numpy()) < 1e-3
    ref = x.float() @ L.dequant(wq, n, k, torch.bfloat16).float().T + b
    assert norm_rel(runs[0].cpu().numpy(), ref.cpu().numpy()) < 1e-3
    ws = L.split_workspace_of(x.device)
    assert int(ws[:4096].view(torch.int32).abs().sum().item()) == 0  # every split tile was finished


def tiled_layout(blocks, n, k):
    """The tiled (grouped) Q8_0 layout restated in numpy: rows in groups of 32 (zero rows past n), k in stages of 64;
    chunk (g, s) = block 2s codes, block 2s+1 codes (each 64 lanes x 16 bytes: lane l holds codes 8h..8h+7 and
    16+8h..16+8h+7 of row l % 32, h = l // 32), then the two fp16 scales of each of the 32 rows; chunks group-major."""
    S = k // 64
    G = (n + 31) // 32
    pad = np.zeros((G * 32, S * 68), np.uint8)
    pad[:n] = blocks.reshape(n, S * 68)
    raw = pad.reshape(G, 32, S, 68)
    parts = []
    for q in (raw[..., 2:34], raw[..., 36:68]):
        lanes = np.stack([np.concatenate([q[..., 8 * h:8 * h + 8], q[..., 16 + 8 * h:24 + 8 * h]], axis=-1)
                          for h in (0, 1)], axis=1)  # (G, h, r, S, 16)
        parts.append(lanes.transpose(0, 3, 1, 2, 4).reshape(G, S, 1024))
    scales = np.concatenate([raw[..., 0:2], raw[..., 34:36]], axis=-1).transpose(0, 2, 1, 3).reshape(G, S, 128)
    return np.concatenate(parts + [scales], axis=-1).reshape(-1)


@pytest.mark.parametrize("m,n,k,off,cnt", [(256, 128, 64, 0, 128), (300, 200, 192, 128, 72), (1000, 1536, 1536, 0, 1536),
                                         (513, 4608, 1280, 1536, 1536), (512, 512, 256, 96, 256), (256, 512, 128, 0, 512),
                                         (700, 2048, 384, 0, 2048), (256, 64, 128, 0, 64)])
def test_tiled_weights_match_row_major(m, n, k, off, cnt):
    # the tiled layout is a pure reordering of the blocks (bit-exact against the numpy restatement), and the GEMM on it
    # gives bit-identical results to the GEMM on the row-major blocks (same kernel arithmetic)
    rng = np.random.default_rng(m * 7 + n)
    wq = q8(rng, n, k)
    w = to_dev(wq)
    wt = L.tile_q8_0(w, n, k)
    assert np.array_equal(wt.cpu().numpy(), tiled_layout(wq, n, k))
    x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(DEV).bfloat16()
    b = torch.from_numpy(rng.normal(0, 0.01, n).astype(np.float32)).to(DEV)
    res = torch.from_numpy(rng.standard_normal((m, cnt)).astype(np.float32)).to(DEV).bfloat16()
    for act in (L.ACT_NONE, L.ACT_GELU_TANH):
        raw = L.gemm(x, w, n, off, cnt, bias=b, residual=res, act=act, mode=L.MODE_DEQUANT)
        til = L.gemm(x, wt, n, off, cnt, bias=b, residual=res, act=act, mode=L.MODE_DEQUANT, tiled=True)
        assert torch.equal(raw, til)
    with pytest.raises(ValueError):
        L.gemm(x, wt, n, 16, 16, mode=L.MODE_DEQUANT, tiled=True)  # window not on a 32-row group


def test_exact_on_tiled_weights_with_strided_activation_rows():
    # x a column slice of a wider fp32 buffer (row stride 1280 > k = 1024): the split prepass reads the rows at their
    # stride; the result matches the row-major EXACT kernel on the same view within 1e-6 and the oracle within 1e-5
    rng = np.random.default_rng(71)
    m, k, n = 150, 1024, 320
    big = rng.normal(0, 1, (m, 1280)).astype(np.float32)
    xb = to_dev(big)
    x = xb[:, 64:64 + k]
    wq = q8(rng, n, k)
    wd = to_dev(wq)
    wt = L.tile_q8_0(wd, n, k)
    b = rng.normal(0, 0.01, n).astype(np.float32)
    bt = to_dev(b)
    raw = L.gemm(x, wd, n, bias=bt, mode=L.MODE_EXACT, out_dtype=torch.float32)
    til = L.gemm(x, wt, n, bias=bt, mode=L.MODE_EXACT, out_dtype=torch.float32, tiled=True)
    torch.cuda.synchronize()
    assert norm_rel(til.cpu().numpy(), raw.cpu().numpy()) < 1e-6
    ref = O.gemm_q8_float(np.ascontiguousarray(big[:, 64:64 + k]), wq, n, k, b)
    assert norm_rel(til.cpu().numpy(), ref) < 1e-5


def test_int8_on_tiled_weights_with_strided_activation_rows():
    # bf16 x a column slice of a wider buffer (row stride 1600 > k = 1024): the tiled-layout quantizer reads the rows
    # at their stride; whole tiles give the same bits as the row-major INT8 kernel on the same view
    rng = np.random.default_rng(72)
    m, k, n = 200, 1024, 256
    xb = to_dev(rng.normal(0, 1, (m, 1600)).astype(np.float32)).bfloat16()
    x = xb[:, 128:128 + k]
    wd = to_dev(q8(rng, n, k))
    wt = L.tile_q8_0(wd, n, k)
    bt = to_dev(rng.normal(0, 0.01, n).astype(np.float32))
    raw = L.gemm(x, wd, n, bias=bt, mode=L.MODE_INT8, out_dtype=torch.float32)
    til = L.gemm(x, wt, n, bias=bt, mode=L.MODE_INT8, out_dtype=torch.float32, tiled=True)
    torch.cuda.synchronize()
    assert torch.equal(raw, til)
