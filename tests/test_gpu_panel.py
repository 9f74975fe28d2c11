"""The native panel entry points on the device (idolq_panel_expand_f32, idolq_panel_to_q8_0, idolq_panel_bytes)
through the C ABI: bit-exact against the reference build's own dequantizer (src/kernels.cpp:535-550
dequantize_linear) for every width and group, the inverse of the GGUF bridge, the inexact-minimum count, and the
argument checks and messages of src/kernels.cpp:516-533 quantized_linear."""
import numpy as np
import pytest
import torch

import idol_kernels as K
import idolq_lib as L
import oracle as O

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def panel(rng, out, inp, bits, group, symmetric):
    codes = rng.integers(0, 1 << bits, (out, inp)).astype(np.uint8)
    s = rng.uniform(0.001, 0.2, (out, inp // group)).astype(np.float16).astype(np.float32)
    m = -float(1 << (bits - 1)) * s if symmetric else \
        rng.uniform(-1, 1, (out, inp // group)).astype(np.float16).astype(np.float32)
    return K.pack_panel(codes, s, m, bits, group), codes, s, m


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("group", [32, 64, 128])
def test_panel_expand_matches_the_reference_dequantizer(bits, group):
    rng = np.random.default_rng(bits * 1000 + group)
    out, inp = 37, 384
    blob, codes, s, m = panel(rng, out, inp, bits, group, symmetric=False)
    assert L.panel_bytes(out, inp, bits, group) == blob.size
    dev_blob = torch.from_numpy(blob).to(DEV)
    wide = torch.full((out, inp + 5), float("nan"), device=DEV)
    L.panel_expand_f32(dev_blob, out, inp, bits, group, w=wide[:, :inp])
    got = wide.cpu().numpy()
    want = (codes.astype(np.float32) * np.repeat(s, group, 1) + np.repeat(m, group, 1)).astype(np.float32)
    assert np.array_equal(got[:, :inp], want)
    assert np.isnan(got[:, inp:]).all()  # nothing written past the row
    if O.ref_available():
        assert np.array_equal(got[:, :inp], O.ref_dequantize_panel(blob, out, inp, bits, group))
    # the exact minimum is not met, so every (row, group) is counted and the layer stays fp32
    _, inexact = L.panel_to_q8_0(dev_blob, out, inp, bits, group)
    exact = m == -float(1 << (bits - 1)) * s
    assert int(inexact.item()) == int((~exact).sum()) > 0


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("group", [32, 64, 128])
def test_symmetric_panel_to_q8_0_holds_the_panel_values(bits, group):
    rng = np.random.default_rng(bits * 7 + group)
    out, inp = 50, 256
    blob, codes, s, _ = panel(rng, out, inp, bits, group, symmetric=True)
    q8, inexact = L.panel_to_q8_0(torch.from_numpy(blob).to(DEV), out, inp, bits, group)
    assert int(inexact.item()) == 0
    blocks = q8.cpu().numpy()
    assert np.array_equal(blocks, K.panel_to_q8_0(blob, out, inp, bits, group))
    values = O.q8_0_dequant(blocks, out, inp)
    half = float(1 << (bits - 1))
    assert np.array_equal(values, (np.repeat(s, group, 1) * (codes.astype(np.float32) - half)).astype(np.float32))
    if O.ref_available():
        assert np.array_equal(values, O.ref_dequantize_panel(blob, out, inp, bits, group))


def test_panel_to_q8_0_inverts_the_gguf_bridge_on_the_device():
    rng = np.random.default_rng(4)
    for n, k in ((37, 64), (16, 352), (70, 1024)):
        blocks = O.q8_0_quantize(rng.normal(0, 0.05, (n, k)).astype(np.float32))
        blob = O.q8_0_to_panel(blocks, n, k)
        q8, inexact = L.panel_to_q8_0(torch.from_numpy(blob).to(DEV), n, k, 8, 32)
        assert int(inexact.item()) == 0 and np.array_equal(q8.cpu().numpy(), blocks)
    bad = blob.copy()
    bad[32:34] = np.array([np.float16(0.25)]).view(np.uint8)  # one minimum that is not -128 * scale
    _, inexact = L.panel_to_q8_0(torch.from_numpy(bad).to(DEV), 70, 1024, 8, 32)
    assert int(inexact.item()) == 1


def test_quantized_linear_on_the_device_takes_the_exact_form():
    # quantized_linear routes a symmetric panel to Q8_0 blocks and an asymmetric one to fp32 values, on the device
    rng = np.random.default_rng(5)
    out, inp = 40, 128
    sym, codes, s, _ = panel(rng, out, inp, 4, 64, symmetric=True)
    asym, codes2, s2, m2 = panel(rng, out, inp, 6, 32, symmetric=False)
    bias = rng.normal(0, 0.1, out).astype(np.float32)
    a = K.quantized_linear(sym, bias, out, inp, 4, 64)
    b = K.quantized_linear(asym, bias, out, inp, 6, 32)
    assert a.q8 is not None and a.weight is None and (a.qbits, a.qgroup) == (4, 64)
    assert b.q8 is None and b.weight is not None and (b.qbits, b.qgroup) == (6, 32)
    assert np.array_equal(K.dequantize_linear(b).cpu().numpy(), K.panel_values(asym, out, inp, 6, 32))
    assert np.array_equal(K.dequantize_linear(a).cpu().numpy(), K.panel_values(sym, out, inp, 4, 64))


def test_panel_argument_checks():
    blob = torch.zeros(L.panel_bytes(16, 64, 4, 32), device=DEV, dtype=torch.uint8)
    assert L.panel_bytes(16, 64, 7, 32) == 0 and L.panel_bytes(16, 96, 4, 64) == 0
    with pytest.raises(ValueError, match="2, 3, 4, 5, 6 or 8 bits"):
        L.panel_expand_f32(blob, 16, 64, 7, 32)
    with pytest.raises(ValueError, match="multiple of 32 that divides"):
        L.panel_expand_f32(blob, 16, 64, 4, 48)
    with pytest.raises(ValueError, match="wrong size"):
        L.panel_expand_f32(blob[:-1], 16, 64, 4, 32)
    with pytest.raises(ValueError, match="wrong size"):
        L.panel_to_q8_0(blob, 17, 64, 4, 32)
