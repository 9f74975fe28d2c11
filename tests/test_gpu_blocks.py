"""The other GGUF block formats on the GPU: libidolq's expansion of Q4_0 / Q8_0 / Q2_K / Q4_K / Q6_K against the
oracle (bit-exact in fp32 and after rounding to bf16 / fp16), the exact Q4_0 -> Q8_0 re-encoding, and the fused
Q4_0 and Q4_K linears on the reference's own test shapes and bar (tests/python/test_fused_packed.py)."""
from types import SimpleNamespace

import numpy as np
import pytest
import torch

import idolq_lib as L
import oracle as O
from conftest import norm_rel
from ggml_types import GGMLQuantizationType as T
from idol_hip import fused_linear
from idol_packed import PackedLinear, enable_fused_packed

pytestmark = pytest.mark.gpu
DEV = "cuda"
SCALES = {O.KIND_Q4_0: (0,), O.KIND_Q8_0: (0,), O.KIND_Q2_K: (80, 82), O.KIND_Q4_K: (0, 2), O.KIND_Q6_K: (208,)}


def random_blocks(kind, n, k, seed):
    rng = np.random.default_rng(seed)
    values, size = O.BLOCK_SHAPE[kind]
    raw = rng.integers(0, 256, n * (k // values) * size, dtype=np.uint8)
    blocks = raw.reshape(-1, size)
    for off in SCALES[kind]:
        blocks[:, off:off + 2] = np.float16(rng.uniform(-1, 1, blocks.shape[0])).view(np.uint8).reshape(-1, 2)
    return raw


@pytest.mark.parametrize("kind", [O.KIND_Q4_0, O.KIND_Q8_0, O.KIND_Q2_K, O.KIND_Q4_K, O.KIND_Q6_K])
@pytest.mark.parametrize("n,k", [(1, 256), (37, 512), (300, 1024)])
def test_block_expansion_matches_the_oracle(kind, n, k):
    raw = random_blocks(kind, n, k, kind * 100 + n)
    want = torch.from_numpy(O.blocks_values(raw, kind, n, k))
    w = torch.from_numpy(raw).to(DEV)
    for dtype in (torch.float32, torch.bfloat16, torch.float16):
        got = L.blocks_dequant(w, kind, n, k, dtype).cpu()
        assert torch.equal(got, want.to(dtype)), dtype
    layer = PackedLinear(SimpleNamespace(shape=np.array([k, n]), tensor_type=T(kind), data=raw), None)
    host = layer.dequantize(torch.bfloat16)
    assert torch.equal(layer.to(DEV).dequantize(torch.bfloat16).cpu(), host)


def test_q4_0_reencoding_and_errors():
    raw = random_blocks(O.KIND_Q4_0, 70, 320, 5)
    q8 = L.q4_0_to_q8_0(torch.from_numpy(raw).to(DEV), 70, 320).cpu().numpy()
    assert np.array_equal(q8, O.q4_0_to_q8_0(raw, 70, 320))
    assert np.array_equal(O.q8_0_dequant(q8, 70, 320), O.blocks_values(raw, O.KIND_Q4_0, 70, 320))
    with pytest.raises(ValueError, match="does not match"):
        L.blocks_dequant(torch.from_numpy(raw).to(DEV)[:-1], O.KIND_Q4_0, 70, 320, torch.float32)
    with pytest.raises(ValueError, match="does not match"):
        L.blocks_dequant(torch.from_numpy(raw).to(DEV), O.KIND_Q4_K, 70, 320, torch.float32)


@pytest.mark.parametrize("kind,code", [(T.Q4_0, 4), (T.Q4_K, 44)])
@pytest.mark.parametrize("rows,columns,width", [(1, 7, 256), (41, 71, 256), (5, 33, 512), (2048, 1536, 1536)])
def test_fused_q4_matches_reference_test(kind, code, rows, columns, width):
    # tests/python/test_fused_packed.py: Q4_0 from N(0, 0.25) weights, Q4_K from random bytes with d = 1, dmin = 0.5;
    # strided fp16 / bf16 input, bias on and off; the module equals fused_linear exactly and both are within 1e-3 of
    # the fp32 product of the expanded weights
    rng = np.random.default_rng(144)
    if kind == T.Q4_K:
        data = rng.integers(0, 256, size=(columns, width // 256 * 144), dtype=np.uint8)
        data.reshape(-1, 144)[:, :4] = np.array([0, 60, 0, 56], dtype=np.uint8)
    else:
        data = O.q4_0_quantize(rng.normal(0, 0.25, (columns, width)).astype(np.float32))
    layer = PackedLinear(SimpleNamespace(shape=np.array([width, columns]), tensor_type=kind, data=data), None).to(DEV)
    gen = torch.Generator(device=DEV).manual_seed(rows + columns)
    for dtype in (torch.float16, torch.bfloat16):
        base = torch.randn(rows, width * 2, device=DEV, dtype=dtype, generator=gen)
        value = base[:, ::2]
        for bias in (None, torch.randn(columns, device=DEV, dtype=dtype, generator=gen)):
            with torch.no_grad():
                output = fused_linear(value, layer.packed, layer.shape, code, bias)
                layer.bias = torch.nn.Parameter(bias, requires_grad=False) if bias is not None else None
                assert enable_fused_packed(layer) == 1
                torch.testing.assert_close(layer(value), output, rtol=0, atol=0)
                dense = layer.dequantize(dtype)
                reference = (value.float() @ dense.float().T).to(dtype)
                if bias is not None:
                    reference = reference + bias
            relative = norm_rel(output.float().cpu().numpy(), reference.float().cpu().numpy())
            assert torch.isfinite(output).all() and relative < 1e-3, (dtype, relative)
    # the expanded weights are the oracle's values
    want = O.blocks_values(data.reshape(-1), int(kind), columns, width)
    assert torch.equal(layer.dequantize(torch.float32).cpu(), torch.from_numpy(want))


def q4k_blocks(n, k, seed, d=0.01, dmin=0.02):
    """Random Q4_K super-blocks with finite scales (random 6-bit scales and minimums, random codes)."""
    rng = np.random.default_rng(seed)
    raw = rng.integers(0, 256, (n * (k // 256), 144), dtype=np.uint8)
    raw[:, 0:2] = np.float16(rng.uniform(0.2, 1.0, raw.shape[0]) * d).view(np.uint8).reshape(-1, 2)
    raw[:, 2:4] = np.float16(rng.uniform(0.2, 1.0, raw.shape[0]) * dmin).view(np.uint8).reshape(-1, 2)
    return raw.reshape(-1)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_q4_k_gemm_decodes_every_weight_exactly(dtype):
    # one-hot activation rows: y[i, j] = T(w[j, i]) exactly (a product by 1, sums of zeros), so the decode inside the
    # GEMM's weight loader equals the expansion (and so the oracle) bit for bit at every position, for all 8 groups
    n, k = 96, 512
    raw = q4k_blocks(n, k, 31)
    w = torch.from_numpy(raw).to(DEV)
    x = torch.eye(k, device=DEV, dtype=dtype)
    y = L.q4_k_gemm(x, w, n, out_dtype=torch.float32)
    want = L.blocks_dequant(w, L.KIND_Q4_K, n, k, dtype).float().T
    assert torch.equal(y, want)
    assert torch.equal(want.T.cpu(), torch.from_numpy(O.blocks_values(raw, O.KIND_Q4_K, n, k)).to(dtype).float())


@pytest.mark.parametrize("m,n_total,k,off,cnt,split", [(1, 7, 256, 0, 7, False), (300, 520, 1024, 0, 520, False),
                                                         (513, 384, 2048, 96, 200, False), (4096, 1536, 1536, 0, 1536, True),
                                                         (1024, 768, 6144, 0, 768, True), (128, 64, 256, 0, 64, False)])
def test_q4_k_gemm_multiplies_the_decoded_weights(m, n_total, k, off, cnt, split):
    # against an fp32 product of the expanded weights (the same products; fp32 sums in another order): 1e-5
    print(f"q4_k gemm m={m} n={n_total} k={k} window {off}+{cnt} split={split}", flush=True)
    raw = q4k_blocks(n_total, k, m + k)
    w = torch.from_numpy(raw).to(DEV)
    rng = np.random.default_rng(m)
    x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(DEV).bfloat16()
    b = torch.from_numpy(rng.normal(0, 0.1, n_total).astype(np.float32)).to(DEV)
    y = L.q4_k_gemm(x, w, n_total, off, cnt, bias=b, out_dtype=torch.float32, split=split)
    dense = L.blocks_dequant(w, L.KIND_Q4_K, n_total, k, torch.bfloat16).float()[off:off + cnt]
    ref = x.float() @ dense.T + b[off:off + cnt]
    assert norm_rel(y.cpu().numpy(), ref.cpu().numpy()) < 1e-5
    again = L.q4_k_gemm(x, w, n_total, off, cnt, bias=b, out_dtype=torch.float32, split=split)
    assert torch.equal(y, again)


def test_q4_k_gemm_epilogue_and_fused_rounding():
    # bias, residual aliasing y, tanh-GELU in the register epilogue (bf16 out) against the same steps in fp32 on the
    # expanded weights; and the fused path's order: product rounded to bf16, then the bias
    m, n, k = 512, 768, 1024
    raw = q4k_blocks(n, k, 77)
    w = torch.from_numpy(raw).to(DEV)
    rng = np.random.default_rng(78)
    x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(DEV).bfloat16()
    b = torch.from_numpy(rng.normal(0, 0.1, n).astype(np.float32)).to(DEV)
    res = torch.from_numpy(rng.standard_normal((m, n)).astype(np.float32)).to(DEV).bfloat16()
    y = res.clone()
    L.q4_k_gemm(x, w, n, bias=b, residual=y, act=L.ACT_GELU_TANH, out=y)
    dense = L.blocks_dequant(w, L.KIND_Q4_K, n, k, torch.bfloat16).float()
    v = x.float() @ dense.T + b + res.float()
    ref = 0.5 * v * (1 + torch.tanh(0.7978845608028654 * (v + 0.044715 * v ** 3)))
    assert norm_rel(y.float().cpu().numpy(), ref.bfloat16().float().cpu().numpy()) < 1e-3
    plain = L.q4_k_gemm(x, w, n)
    rounded = L.q4_k_gemm(x, w, n, bias=b, flags=L.FLAG_ROUND_BEFORE_BIAS)
    assert torch.equal(rounded, (plain.float() + b).bfloat16())
    with pytest.raises(ValueError):  # k = 320 is not a whole number of super-blocks
        L.q4_k_gemm(x[:, :320], torch.zeros(n * 144, device=DEV, dtype=torch.uint8), n)


def test_packed_q4_0_reencodes_once():
    raw = random_blocks(O.KIND_Q4_0, 64, 256, 9)
    layer = PackedLinear(SimpleNamespace(shape=np.array([256, 64]), tensor_type=T.Q4_0, data=raw), None).to(DEV)
    enable_fused_packed(layer)
    x = torch.randn(3, 256, device=DEV, dtype=torch.bfloat16)
    with torch.no_grad():
        a = layer(x)
        cache = layer._q8_blocks
        b = layer(x)
    assert cache is not None and layer._q8_blocks is cache and torch.equal(a, b)
    assert torch.equal(a, fused_linear(x, layer.packed, (64, 256), 4))
