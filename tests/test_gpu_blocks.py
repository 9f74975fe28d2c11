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
