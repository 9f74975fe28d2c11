"""The small-m form of the Q8_0 GEMM (q8_gemv_kernel: m <= 16 on GGUF row-major weights), through idolq_q8_0_gemm:
EXACT against the reference's float kernel (the oracle, 1e-5), DEQUANT against an fp32 product of the weights it
multiplies, T(fp32(d) * q) (1e-5, the accumulation order aside) and against the float kernel within the bf16-dequant
bar; the epilogue (bias, residual aliasing y, activation, rounding before the bias), ragged and strided shapes, the
m = 17 boundary to the tiled kernels, and deterministic repeats."""
import numpy as np
import pytest
import torch

import idolq_lib as L
import oracle as O
from conftest import norm_rel

pytestmark = pytest.mark.gpu
DEV = "cuda"


def q8(rng, n, k, std=0.02):
    return O.q8_0_quantize(rng.normal(0, std, (n, k)).astype(np.float32))


SHAPES = [(6144, 1024), (1024, 256), (333, 1536), (4096, 4096), (20, 192)]


@pytest.mark.parametrize("m", [1, 2, 7, 16])
@pytest.mark.parametrize("n,k", SHAPES)
def test_gemv_exact_tracks_the_reference_float_kernel(m, n, k):
    print(f"gemv exact m={m} n={n} k={k}", flush=True)
    rng = np.random.default_rng(m * 100 + n + k)
    a = rng.standard_normal((m, k)).astype(np.float32)
    w = q8(rng, n, k)
    b = rng.normal(0, 0.01, n).astype(np.float32)
    y = L.gemm(torch.from_numpy(a).to(DEV), torch.from_numpy(w).to(DEV), n, bias=torch.from_numpy(b).to(DEV),
               mode=L.MODE_EXACT).cpu().numpy()
    assert norm_rel(y, O.gemm_q8_float(a, w, n, k, b)) < 1e-5


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m", [1, 2, 7, 16])
@pytest.mark.parametrize("n,k", SHAPES)
def test_gemv_dequant_multiplies_the_dequantized_weights(dtype, m, n, k):
    print(f"gemv dequant {dtype} m={m} n={n} k={k}", flush=True)
    rng = np.random.default_rng(m * 31 + n + k)
    x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(DEV).to(dtype)
    w = q8(rng, n, k)
    wd = torch.from_numpy(w).to(DEV)
    b = torch.from_numpy(rng.normal(0, 0.01, n).astype(np.float32)).to(DEV)
    y = L.gemm(x, wd, n, bias=b, mode=L.MODE_DEQUANT, out_dtype=torch.float32)
    ref = x.float() @ L.dequant(wd, n, k, dtype).float().T + b  # the products DEQUANT multiplies, in fp32
    assert norm_rel(y.cpu().numpy(), ref.cpu().numpy()) < 1e-5
    cpu = O.gemm_q8_float(x.float().cpu().numpy(), w, n, k, b.cpu().numpy())
    assert norm_rel(y.cpu().numpy(), cpu) < 2e-2


@pytest.mark.parametrize("m", [1, 5, 16])
def test_gemv_epilogue_window_residual_and_strides(m):
    # column window, bias, residual aliasing y (strided rows), erf-GELU; x rows strided; against the oracle
    rng = np.random.default_rng(60 + m)
    n_total, k, off, n = 700, 512, 96, 257
    a = rng.standard_normal((m, k + 8)).astype(np.float32)
    w = q8(rng, n_total, k)
    b = rng.normal(0, 0.01, n_total).astype(np.float32)
    res = rng.standard_normal((m, n + 3)).astype(np.float32)
    x = torch.from_numpy(a).to(DEV)[:, :k]
    y = torch.from_numpy(res.copy()).to(DEV)
    L.gemm(x, torch.from_numpy(w).to(DEV), n_total, off, n, bias=torch.from_numpy(b).to(DEV), residual=y[:, :n],
           act=L.ACT_GELU_ERF, mode=L.MODE_EXACT, out=y[:, :n])
    want = O.gemm_q8_float(np.ascontiguousarray(a[:, :k]), w, n_total, k, b, off, n,
                           residual=np.ascontiguousarray(res[:, :n]), gelu=True)
    got = y.cpu().numpy()
    assert norm_rel(got[:, :n], want) < 1e-5
    assert np.array_equal(got[:, n:], res[:, n:])  # nothing written past the window


def test_gemv_rounds_before_bias_like_the_fused_path():
    # fused_linear's order (tools/idol_triton.py:84-89): the product rounded to the output dtype, then the bias
    rng = np.random.default_rng(70)
    m, n, k = 3, 96, 256
    x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(DEV).bfloat16()
    w = torch.from_numpy(q8(rng, n, k)).to(DEV)
    b = torch.from_numpy(rng.normal(0, 1.0, n).astype(np.float32)).to(DEV)
    y = L.gemm(x, w, n, bias=b, mode=L.MODE_DEQUANT, flags=L.FLAG_ROUND_BEFORE_BIAS)
    plain = L.gemm(x, w, n, mode=L.MODE_DEQUANT)
    assert torch.equal(y, (plain.float() + b).bfloat16())


def test_gemv_meets_the_tiled_kernels_at_m_16_17_and_repeats():
    # m = 16 takes the small-m kernel, m = 17 the tiled kernels: the same products, fp32 sums in another order
    rng = np.random.default_rng(80)
    n, k = 1536, 6144
    x = torch.from_numpy(rng.standard_normal((17, k)).astype(np.float32)).to(DEV).bfloat16()
    w = torch.from_numpy(q8(rng, n, k)).to(DEV)
    y16 = L.gemm(x[:16], w, n, mode=L.MODE_DEQUANT, out_dtype=torch.float32)
    y17 = L.gemm(x, w, n, mode=L.MODE_DEQUANT, out_dtype=torch.float32)
    assert norm_rel(y16.cpu().numpy(), y17[:16].cpu().numpy()) < 1e-5
    again = L.gemm(x[:16], w, n, mode=L.MODE_DEQUANT, out_dtype=torch.float32)
    assert torch.equal(y16, again)
