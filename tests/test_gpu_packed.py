"""GPU tests of the drop-in Python surfaces, restating the reference's tests/python/test_fused_packed.py (shapes,
dtypes, strided input, bias on/off, layer(x) == fused_linear(x) exactly, norm-relative error < 1e-3 against
(x.float() @ dequantize(dtype).float().T).to(dtype) + bias), plus the kernels.hpp mirror used by the decoders."""
from types import SimpleNamespace

import numpy as np
import pytest
import torch

import idol_kernels as K
import oracle as O
from conftest import norm_rel
from ggml_types import GGMLQuantizationType as T
from idol_hip import fused_linear
from idol_packed import PackedLinear, enable_fused_packed

pytestmark = pytest.mark.gpu
DEV = "cuda"
SHAPES = [(1, 7, 256), (41, 71, 256), (5, 33, 512), (4097, 71, 256), (4097, 3072, 32), (4097, 1024, 1024)]


@pytest.mark.parametrize("rows,columns,width", SHAPES)
def test_fused_packed_matches_reference_test(rows, columns, width):
    rng = np.random.default_rng(144)
    weights = rng.normal(0, 0.25, (columns, width)).astype(np.float32)
    tensor = SimpleNamespace(shape=np.array([width, columns]), tensor_type=T.Q8_0, data=O.q8_0_quantize(weights))
    layer = PackedLinear(tensor, None).to(DEV)
    gen = torch.Generator(device=DEV).manual_seed(rows * 7 + columns)
    for dtype in (torch.float16, torch.bfloat16):
        base = torch.randn(rows, width * 2, device=DEV, dtype=dtype, generator=gen)
        value = base[:, ::2]
        for bias in (None, torch.randn(columns, device=DEV, dtype=dtype, generator=gen)):
            with torch.no_grad():
                output = fused_linear(value, layer.packed, layer.shape, 8, bias)
                layer.bias = torch.nn.Parameter(bias, requires_grad=False) if bias is not None else None
                assert enable_fused_packed(layer) == 1
                torch.testing.assert_close(layer(value), output, rtol=0, atol=0)
                dense = layer.dequantize(dtype)
                reference = (value.float() @ dense.float().T).to(dtype)
                if bias is not None:
                    reference = reference + bias
            relative = norm_rel(output.float().cpu().numpy(), reference.float().cpu().numpy())
            assert torch.isfinite(output).all() and relative < 1e-3, (dtype, relative)


def test_fused_linear_keeps_leading_dims_empty_input_and_errors():
    rng = np.random.default_rng(1)
    w = O.q8_0_quantize(rng.normal(0, 0.1, (48, 64)).astype(np.float32))
    packed = torch.from_numpy(w).to(DEV)
    x = torch.randn(2, 3, 64, device=DEV, dtype=torch.bfloat16)
    with torch.no_grad():
        assert fused_linear(x, packed, (48, 64), 8).shape == (2, 3, 48)
        assert fused_linear(x[:, :0], packed, (48, 64), 8).shape == (2, 0, 48)
    with pytest.raises(ValueError, match="inference only"):
        fused_linear(x.clone().requires_grad_(True), packed, (48, 64), 8)
    with pytest.raises(ValueError, match="invalid packed linear dimensions"):
        fused_linear(x, packed[:-1], (48, 64), 8)
    with pytest.raises(ValueError, match="invalid fused linear bias"):
        fused_linear(x, packed, (48, 64), 8, torch.zeros(48, device=DEV))
    with pytest.raises(ValueError, match="unsupported fused linear input"):
        fused_linear(x.float(), packed, (48, 64), 8)


def test_packed_linear_gpu_dequantize_equals_expansion_kernel():
    rng = np.random.default_rng(2)
    w = O.q8_0_quantize(rng.normal(0, 0.1, (96, 256)).astype(np.float32))
    layer = PackedLinear(SimpleNamespace(shape=np.array([256, 96]), tensor_type=T.Q8_0, data=w), None).to(DEV)
    ref = O.q8_0_dequant(w, 96, 256)
    for dt in (torch.float32, torch.bfloat16, torch.float16):
        assert torch.equal(layer.dequantize(dt).cpu(), torch.from_numpy(ref).to(dt))


def test_kernels_mirror_gemm_packed_with_panel_blobs():
    # src/kernels.hpp gemm_packed / quantized_linear on a panel blob from the Q8_0 bridge: the float kernel (EXACT)
    # and the integer kernel (INT8) against the oracle, a column window and a residual aliasing the output with GELU
    rng = np.random.default_rng(3)
    m, out, inp = 19, 37, 128
    blocks = O.q8_0_quantize(rng.uniform(-0.5, 0.5, (out, inp)).astype(np.float32))
    bias = rng.uniform(-0.5, 0.5, out).astype(np.float32)
    a = rng.uniform(-1, 1, (m, inp)).astype(np.float32)
    w = K.quantized_linear(O.q8_0_to_panel(blocks, out, inp), bias, out, inp, 8, 32)
    assert np.array_equal(K.dequantize_linear(w).cpu().numpy(), O.q8_0_dequant(blocks, out, inp))
    at = torch.from_numpy(a).to(DEV)
    for mode, ref_fn in ((0, O.gemm_q8_float), (1, O.gemm_q8_int8)):
        K.set_quant_kernel(mode)
        c = torch.empty((m, out), device=DEV)
        K.gemm_packed(at, m, w, 0, out, None, False, c)
        assert norm_rel(c.cpu().numpy(), ref_fn(a, blocks, out, inp, bias)) < 1e-5
        res = rng.uniform(-0.5, 0.5, (m, 16)).astype(np.float32)
        c2 = torch.from_numpy(res.copy()).to(DEV)
        K.gemm_packed(at, m, w, 16, 16, c2, True, c2)
        assert norm_rel(c2.cpu().numpy(), ref_fn(a, blocks, out, inp, bias, 16, 16, res, True)) < 1e-5
    K.set_quant_kernel(-1)


def test_kernels_mirror_layer_norm_and_attention():
    rng = np.random.default_rng(4)
    x = rng.uniform(-2, 2, (5, 24)).astype(np.float32)
    g, b = rng.uniform(-1, 1, 24).astype(np.float32), rng.uniform(-0.5, 0.5, 24).astype(np.float32)
    xt = torch.from_numpy(x).to(DEV)
    K.layer_norm(xt, 5, 24, torch.from_numpy(g).to(DEV), torch.from_numpy(b).to(DEV), xt)  # in place
    assert np.max(np.abs(xt.cpu().numpy() - O.layer_norm(x, g, b))) < 1e-5
    lq, lk, heads, hd = 70, 130, 2, 64
    dim = heads * hd
    q = rng.uniform(-1, 1, lq * (dim + 3)).astype(np.float32)
    kv = rng.uniform(-1, 1, lk * (dim + 1)).astype(np.float32)
    out = torch.empty((lq, dim), device=DEV)
    K.attention(torch.from_numpy(q).to(DEV), lq, dim + 3, torch.from_numpy(kv).to(DEV), torch.from_numpy(kv).to(DEV),
                lk, dim + 1, heads, hd, out, dim)
    assert norm_rel(out.cpu().numpy(), O.attention(q, kv, kv, lq, lk, dim + 3, dim + 1, heads, hd)) < 1e-5


@pytest.mark.parametrize("kind", [T.Q8_0, T.Q4_0])
def test_packed_linear_runs_its_tiled_copy_with_the_same_bits(kind):
    # PackedLinear keeps the layer's Q8_0 blocks (Q4_0: their exact re-encoding) in the tiled GEMM layout, made once per
    # device, and serves calls of more than 16 rows from it: layer(x) equals fused_linear on the GGUF bytes bit for
    # bit (the tiled and row-major kernels compute the same products), shorter calls keep the row-major small-m
    # kernel, and writing the packed bytes (load_state_dict) remakes the copy.
    import idolq_lib as L
    rng = np.random.default_rng(31)
    n, k = 520, 1536
    weights = rng.normal(0, 0.05, (n, k)).astype(np.float32)
    data = O.q8_0_quantize(weights) if kind == T.Q8_0 else O.q4_0_quantize(weights)
    layer = PackedLinear(SimpleNamespace(shape=np.array([k, n]), tensor_type=kind, data=data), None).to(DEV)
    enable_fused_packed(layer)
    code = 8 if kind == T.Q8_0 else 4
    gen = torch.Generator(device=DEV).manual_seed(5)
    for dtype in (torch.bfloat16, torch.float16):
        bias = torch.randn(n, device=DEV, dtype=dtype, generator=gen)
        layer.bias = torch.nn.Parameter(bias, requires_grad=False)
        for rows in (300, 7):
            x = torch.randn(rows, k, device=DEV, dtype=dtype, generator=gen)
            with torch.no_grad():
                got = layer(x)
                want = fused_linear(x, layer.packed, layer.shape, code, bias)
            assert torch.equal(got, want), (dtype, rows)
    assert layer._q8_tiled is not None and layer._q8_tiled.numel() == L.tiled_q8_0_bytes(n, k)
    first = layer._q8_tiled
    other = O.q8_0_quantize(weights[::-1].copy()) if kind == T.Q8_0 else O.q4_0_quantize(weights[::-1].copy())
    layer.load_state_dict({"packed": torch.from_numpy(other), "bias": layer.bias.detach()})
    x = torch.randn(64, k, device=DEV, dtype=torch.bfloat16, generator=gen)
    layer.bias = None
    with torch.no_grad():
        assert torch.equal(layer(x), fused_linear(x, layer.packed, layer.shape, code))
    assert layer._q8_tiled is not first


def test_fp16_large_m_q8_0_adds_the_bias_before_its_rounding():
    # tools/idol_triton.py:112-117: fp16 activations, m >= 4096, n >= 1024, k >= 1024 go through F.linear, whose fused
    # bias enters the fp32 accumulator before the single rounding to fp16; below that size (and in bf16) the product
    # is rounded first (tools/idol_triton.py:84-89). The output is compared element by element with both orders
    # applied to an fp32 product of the dequantized weights: almost every element matches the branch's own order.
    rng = np.random.default_rng(32)
    n, k = 1024, 1024
    w = O.q8_0_quantize(rng.normal(0, 0.25, (n, k)).astype(np.float32))
    packed = torch.from_numpy(w).to(DEV)
    dense = torch.from_numpy(O.q8_0_dequant(w, n, k)).to(DEV).half().float()
    gen = torch.Generator(device=DEV).manual_seed(9)
    bias = torch.randn(n, device=DEV, dtype=torch.float16, generator=gen)
    for m, bias_first in ((4096, True), (4095, False)):
        x = torch.randn(m, k, device=DEV, dtype=torch.float16, generator=gen)
        with torch.no_grad():
            y = fused_linear(x, packed, (n, k), 8, bias)
        acc = x.float() @ dense.T
        one = (acc + bias.float()).half()
        two = (acc.half().float() + bias.float()).half()
        match_one, match_two = (y == one).float().mean().item(), (y == two).float().mean().item()
        if bias_first:
            assert match_one > 0.99 and match_two < match_one - 0.05, (match_one, match_two)
        else:
            assert match_two > 0.99 and match_one < match_two - 0.05, (match_one, match_two)
