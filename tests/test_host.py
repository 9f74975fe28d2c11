"""CPU tests of the boundary and the host logic: the C ABI library loads and exports what include/idolq.h declares,
host-side argument checks reject bad calls before anything is launched, and the drop-in Python surfaces
(PackedLinear, fused_linear, the kernels.hpp mirror) keep the reference's behaviour on the CPU side."""
import ctypes
import re
from pathlib import Path
from types import SimpleNamespace

import numpy as np
import pytest
import torch

import idolq_lib as L
import idol_kernels as K
import oracle as O
from ggml_types import GGMLQuantizationType as T
from idol_hip import fused_linear
from idol_packed import PackedLinear, enable_fused_packed, replace_quantized_linear_layers

HEADER = Path(__file__).resolve().parents[1] / "include" / "idolq.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(idolq_\w+)\s*\(", text)))


def source(weights, kind=T.Q8_0):
    n, k = weights.shape
    return SimpleNamespace(shape=np.array([k, n]), tensor_type=kind, data=O.q8_0_quantize(weights))


# ------------------------------------------------------------------------------------------------ C ABI
def test_library_exports_every_declared_entry_point():
    lib = L.load()
    declared = declared_functions()
    assert len(declared) >= 14
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(L.exported_symbols())
    assert b"gfx950" in lib.idolq_version()


def test_c_abi_rejects_bad_arguments_on_the_host():
    lib = L.load()
    assert lib.idolq_q8_0_bytes(6144, 1536) == 6144 * 48 * 34
    assert lib.idolq_q8_0_bytes(10, 33) == 0
    # EXACT: the bf16 high and low parts of the tiled path, then the same split room as DEQUANT
    assert lib.idolq_q8_0_gemm_workspace(4096, 1536, L.MODE_EXACT) == (
        4096 * 1536 * 4 + lib.idolq_q8_0_gemm_workspace(4096, 1536, L.MODE_DEQUANT))
    # DEQUANT: one 256 x 128 fp32 partial tile and a flag per CU (256 where no device is visible), and an error word
    assert lib.idolq_q8_0_gemm_workspace(4096, 1536, L.MODE_DEQUANT) >= 256 * (256 * 128 * 4 + 4)
    assert lib.idolq_q8_0_gemm_workspace(4096, 1536, L.MODE_INT8) >= 4096 * 1536 + 4096 * 48 * 4
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: every call below fails its checks first
    rc = lib.idolq_q8_0_gemm(None, L.BF16, 4, 64, 64, fake, 8, 0, 8, None, 0, None, 0, 0, 0, 0, 0, fake, L.BF16, 8,
                             None, 0, None)
    assert rc == L.EINVAL and b"non-null" in lib.idolq_last_error()
    rc = lib.idolq_q8_0_gemm(fake, L.BF16, 4, 48, 48, fake, 8, 0, 8, None, 0, None, 0, 0, 0, 0, 0, fake, L.BF16, 8,
                             None, 0, None)
    assert rc == L.EINVAL and b"multiple of 32" in lib.idolq_last_error()
    rc = lib.idolq_q8_0_gemm(fake, L.BF16, 4, 64, 64, fake, 8, 4, 8, None, 0, None, 0, 0, 0, 0, 0, fake, L.BF16, 8,
                             None, 0, None)
    assert rc == L.EINVAL and b"window" in lib.idolq_last_error()
    rc = lib.idolq_q8_0_gemm(fake, L.F32, 4, 64, 64, fake, 8, 0, 8, None, 0, None, 0, 0, 0, L.MODE_DEQUANT, 0, fake,
                             L.F32, 8, None, 0, None)
    assert rc == L.EINVAL and b"DEQUANT" in lib.idolq_last_error()
    rc = lib.idolq_q8_0_gemm(fake, L.BF16, 4, 64, 64, fake, 8, 0, 8, None, 0, None, 0, 0, 0, L.MODE_INT8, 0, fake,
                             L.BF16, 8, None, 0, None)
    assert rc == L.EINVAL and b"workspace" in lib.idolq_last_error()
    rc = lib.idolq_q8_0_gemm(fake, L.F32, 4, 64, 64, fake, 8, 0, 8, None, 0, None, 0, 0, 0, L.MODE_EXACT,
                             L.FLAG_TILED_WEIGHTS, fake, L.F32, 8, None, 0, None)
    assert rc == L.EINVAL and b"workspace" in lib.idolq_last_error()
    rc = lib.idolq_q8_0_gemm(fake, 7, 4, 64, 64, fake, 8, 0, 8, None, 0, None, 0, 0, 0, 0, 0, fake, L.BF16, 8, None,
                             0, None)
    assert rc == L.EINVAL and b"dtype" in lib.idolq_last_error()
    assert lib.idolq_layernorm(fake, L.F32, 4, 16, 8, 1e-6, None, None, None, None, 0, fake, L.F32, 16, None) == L.EINVAL
    assert lib.idolq_layernorm(fake, L.F32, 4, 16, 16, 1e-6, None, None, fake, None, 0, fake, L.F32, 16, None) == L.EINVAL
    assert lib.idolq_attention(fake, fake, fake, L.BF16, 1, 4, 0, 2, 64, 128, 128, 0, 0, fake, L.BF16, 128, 0,
                               None) == L.EINVAL
    assert lib.idolq_attention(fake, fake, fake, L.BF16, 1, 4, 4, 2, 64, 100, 128, 0, 0, fake, L.BF16, 128, 0,
                               None) == L.EINVAL
    assert lib.idolq_q8_0_dequant(fake, 4, 40, fake, L.F32, None) == L.EINVAL
    assert lib.idolq_quantize_act_q8(fake, L.F32, 4, 64, 32, fake, fake, None, None) == L.EINVAL
    assert lib.idolq_q8_0_block_dots(fake, 4, 64, fake, 8, 0, 16, fake, None) == L.EINVAL
    assert lib.idolq_activation(fake, L.F32, 10, 9, None) == L.EINVAL
    assert lib.idolq_pos_embed(fake, 4, fake, 16, fake, L.F32, 90, None) == L.EINVAL
    assert lib.idolq_copy2d(fake, L.F32, 4, fake, L.F32, 8, 2, 8, None) == L.EINVAL
    # EXACT on tiled weights addresses its bf16 high / low parts and the weight groups with 32-bit byte offsets
    big_ws = ctypes.c_size_t(1 << 36)
    rc = lib.idolq_q8_0_gemm(fake, L.F32, 1 << 20, 2048, 2048, fake, 64, 0, 64, None, 0, None, 0, 0, 0, L.MODE_EXACT,
                             L.FLAG_TILED_WEIGHTS, fake, L.F32, 64, fake, big_ws, None)
    assert rc == L.EINVAL and b"2^32" in lib.idolq_last_error()
    rc = lib.idolq_q8_0_gemm(fake, L.F32, 64, 64, 64, fake, 1 << 27, 0, 32, None, 0, None, 0, 0, 0, L.MODE_EXACT,
                             L.FLAG_TILED_WEIGHTS, fake, L.F32, 32, fake, big_ws, None)
    assert rc == L.EINVAL and b"2^32" in lib.idolq_last_error()
    # m == 0 or n == 0 is a no-op, as fused_linear's empty input is
    assert lib.idolq_q8_0_gemm(fake, L.BF16, 0, 64, 64, fake, 8, 0, 8, None, 0, None, 0, 0, 0, 0, 0, fake, L.BF16, 8,
                               None, 0, None) == 0


def test_wrappers_reject_outputs_and_residuals_that_do_not_cover_the_result():
    # The C ABI sees a pointer and a row stride only; the Python wrappers require every output and residual to be
    # the [m, n] extent the kernel writes or reads, so a shorter or narrower view cannot send it past its memory.
    # These checks come before any device work (CPU tensors reach them).
    x = torch.zeros((64, 128), dtype=torch.bfloat16)
    w = torch.zeros(L.q8_0_bytes(96, 128), dtype=torch.uint8)
    big = torch.zeros((64, 200), dtype=torch.bfloat16)
    for bad, what in ((torch.zeros((63, 96), dtype=torch.bfloat16), "out"),     # a row short
                      (big[:32], "out"),                                         # a short-row view
                      (big[:, :95], "out"),                                      # a column slice narrower than n
                      (big[:, ::2][:, :96], "out"),                              # strided columns
                      (torch.zeros(64 * 96, dtype=torch.bfloat16), "out")):      # not 2-D
        with pytest.raises(ValueError, match=what):
            L.gemm(x, w, 96, out=bad)
    with pytest.raises(ValueError, match="residual"):
        L.gemm(x, w, 96, residual=big[:60, :96])
    with pytest.raises(ValueError, match="residual"):
        L.gemm(x, w, 96, residual=big[:, :64])
    with pytest.raises(ValueError, match="x must be"):
        L.gemm(x.reshape(-1), w, 96)
    # a window: out and the residual are [m, n] of the window, not of the whole layer
    with pytest.raises(ValueError, match="out"):
        L.gemm(x, w, 96, 32, 32, out=big[:, :96])
    with pytest.raises(ValueError, match="out"):
        L.q4_k_gemm(x, torch.zeros(1, dtype=torch.uint8), 96, out=big[:, :90])
    with pytest.raises(ValueError, match="out"):
        L.layernorm(x, 1e-6, out=big[:48, :128])
    with pytest.raises(ValueError, match="out"):
        L.layernorm(x, 1e-6, out=big[:, :100])
    with pytest.raises(ValueError, match="rows overlap"):
        L.layernorm(x, 1e-6, out=big.as_strided((64, 128), (100, 1)))
    with pytest.raises(ValueError, match="x must be"):
        L.layernorm(x[0], 1e-6)


# ------------------------------------------------------------------------------------------------ fused_linear
def test_fused_linear_validates_like_the_reference():
    rng = np.random.default_rng(0)
    src = source(rng.normal(0, 0.25, (8, 64)).astype(np.float32))
    packed = torch.from_numpy(src.data)
    x = torch.randn(3, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="unsupported fused linear input"):
        fused_linear(x, packed, (8, 64), 8)  # CPU tensors
    with pytest.raises(ValueError, match="unsupported fused linear input"):
        fused_linear(x, packed, (8, 32), 8)  # k mismatch
    with pytest.raises(ValueError, match="unsupported fused linear input"):
        fused_linear(x, packed, (8, 64), 5)  # unknown kind


# ------------------------------------------------------------------------------------------------ PackedLinear
def test_packed_linear_holds_blocks_and_expands_them_on_the_cpu():
    rng = np.random.default_rng(1)
    w = rng.normal(0, 0.25, (71, 256)).astype(np.float32)
    src = source(w)
    bias = torch.randn(71)
    layer = PackedLinear(src, bias)
    assert layer.shape == (71, 256) and layer.kind == T.Q8_0 and not layer.fused
    assert layer.packed.dtype == torch.uint8 and layer.packed.numel() == 71 * 8 * 34
    assert "packed" in dict(layer.named_buffers()) and not layer.bias.requires_grad
    dense = layer.dequantize(torch.float32).numpy()
    assert np.array_equal(dense, O.q8_0_dequant(src.data, 71, 256))
    x = torch.randn(5, 256)
    assert torch.equal(layer(x), torch.nn.functional.linear(x, torch.from_numpy(dense), bias))
    layer.fused = True  # a CPU input never takes the fused path (tools/idol_packed.py:79-80)
    assert torch.equal(layer(x), torch.nn.functional.linear(x, torch.from_numpy(dense), bias))
    with pytest.raises(ValueError, match="unsupported packed matrix"):
        PackedLinear(SimpleNamespace(shape=np.array([64, 8]), tensor_type=T.Q5_0, data=np.zeros(10, np.uint8)), None)


def test_q4_0_and_f16_expansion_closed_form():
    d = np.float16(0.5)
    nibbles = np.arange(16, dtype=np.uint8)
    block = np.concatenate([np.array([d]).view(np.uint8), (nibbles | (15 - nibbles) << 4).astype(np.uint8)])
    layer = PackedLinear(SimpleNamespace(shape=np.array([32, 1]), tensor_type=T.Q4_0, data=block), None)
    expect = np.concatenate([nibbles.astype(np.float32) - 8, (15 - nibbles).astype(np.float32) - 8]) * 0.5
    assert np.array_equal(layer.dequantize(torch.float32).numpy()[0], expect)
    half = np.arange(6, dtype=np.float16).reshape(2, 3)
    layer = PackedLinear(SimpleNamespace(shape=np.array([3, 2]), tensor_type=T.F16, data=half.view(np.uint8)), None)
    assert np.array_equal(layer.dequantize(torch.float32).numpy(), half.astype(np.float32))


def test_enable_and_replace_follow_the_reference_mapping():
    rng = np.random.default_rng(2)

    class Net(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.a = torch.nn.Linear(64, 32)
            self.b = torch.nn.Sequential(torch.nn.Linear(32, 16))
            self.norm = torch.nn.LayerNorm(16)

    net = Net()
    tensors = {"a.weight": source(rng.normal(0, 0.1, (32, 64)).astype(np.float32)),
               "b.0.weight": source(rng.normal(0, 0.1, (16, 32)).astype(np.float32))}
    names = replace_quantized_linear_layers(net, tensors)
    assert names == ["a.weight", "b.0.weight"]
    assert isinstance(net.a, PackedLinear) and isinstance(net.b[0], PackedLinear)
    assert enable_fused_packed(net) == 2 and net.a.fused and net.b[0].fused
    with pytest.raises(ValueError, match="not a linear weight"):
        replace_quantized_linear_layers(Net(), {"a.bias": tensors["a.weight"]})
    with pytest.raises(ValueError, match="missing"):
        replace_quantized_linear_layers(Net(), {"c.weight": tensors["a.weight"]})
    with pytest.raises(ValueError, match="does not match"):
        replace_quantized_linear_layers(Net(), {"b.0.weight": tensors["a.weight"]})


# ------------------------------------------------------------------------------------------------ kernels.hpp mirror
def test_quantized_linear_rejects_shapes_the_format_cannot_hold():
    # tests/test_kernels.cpp:290-296
    bias = np.zeros(16, np.float32)
    with pytest.raises(ValueError, match="wrong size"):
        K.quantized_linear(bytes(10), bias, 16, 64, 4, 32)
    with pytest.raises(ValueError, match="2, 3, 4, 5, 6 or 8 bits"):
        K.quantized_linear(bytes(10), bias, 16, 64, 7, 32)
    with pytest.raises(ValueError, match="multiple of 32"):
        K.quantized_linear(bytes(10), bias, 16, 64, 4, 48)
    with pytest.raises(ValueError, match="multiple of 32"):
        K.quantized_linear(bytes(10), bias, 16, 96, 4, 64)
    assert K.quant_panel_bytes(1024, 8, 32) == 32 * 576 == O.panel_bytes(16, 1024)


def test_panel_to_q8_0_inverts_the_gguf_bridge():
    rng = np.random.default_rng(3)
    for n, k in ((37, 64), (16, 352), (70, 1024)):
        blocks = O.q8_0_quantize(rng.normal(0, 0.05, (n, k)).astype(np.float32))
        blob = O.q8_0_to_panel(blocks, n, k)
        assert np.array_equal(K.panel_to_q8_0(blob, n, k), blocks)
    bad = O.q8_0_to_panel(blocks, 70, 1024).copy()
    bad[32:34] = np.array([np.float16(0.25)]).view(np.uint8)  # a minimum that is not -128 * scale
    with pytest.raises(ValueError, match="-128"):
        K.panel_to_q8_0(bad, 70, 1024)
