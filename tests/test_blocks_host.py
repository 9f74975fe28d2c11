"""GGUF block formats on the CPU: the oracle's element-by-element restatement pinned by hand-computed known answers
(one element per code position, scale group and bit field that a layout mistake would move), the host expansion of
PackedLinear against the oracle, and the Q4_0 -> Q8_0 re-encoding invariant."""
import numpy as np
import pytest
import torch

import oracle as O
import idol_packed as P
from ggml_types import GGMLQuantizationType as T


def _f16(v):
    return np.array([np.float16(v)]).view(np.uint8)


def _single(kind, fill):
    values, size = O.BLOCK_SHAPE[kind]
    b = np.zeros(size, np.uint8)
    fill(b)
    return b, O.blocks_values(b, kind, 1, values)[0]


def test_q4_0_known_answers():
    def fill(b):
        b[0:2] = _f16(0.5)
        b[2 + 4] = 0xF0  # element 4: low nibble 0, element 20: high nibble 15
    _, v = _single(O.KIND_Q4_0, fill)
    assert v[4] == (0 - 8) * 0.5 and v[20] == (15 - 8) * 0.5 and v[0] == -4.0


def test_q2_k_known_answers():
    def fill(b):
        b[80:82], b[82:84] = _f16(0.5), _f16(0.25)
        b[16 + 32 + 7] = 0b10_000000  # element 128 + 96 + 7 = 231: bits 6..7 of byte 32 + 7 of the codes
        b[14] = 0x36                  # group 231 // 16 = 14: scale 6, min 3
        b[16 + 0 + 3] = 0b00_00_01_11  # element 3: 3 (bits 0..1); element 32 + 3: 1 (bits 2..3)
        b[0] = 0x21                   # group 0: scale 1, min 2
        b[2] = 0x05                   # group 2 (elements 32..47): scale 5, min 0
    _, v = _single(O.KIND_Q2_K, fill)
    assert v[231] == (0.5 * 6) * 2 - 0.25 * 3
    assert v[3] == (0.5 * 1) * 3 - 0.25 * 2
    assert v[35] == (0.5 * 5) * 1
    assert v[230] == -0.25 * 3  # same group, code 0


def test_q4_k_known_answers():
    def fill(b):
        b[0:2], b[2:4] = _f16(2.0), _f16(1.0)
        s = b[4:16]
        s[1] = 0b11_000101   # sc_1 = 5; its top bits are bits 4..5 of sc_5
        s[5] = 0b10_000011   # m_1 = 3; its top bits are bits 4..5 of m_5
        s[9] = 0x7A          # low nibble: sc_5 bits 0..3, high nibble: m_5 bits 0..3
        b[16 + 32 * 2 + 3] = 0xB0  # element 5 * 32 + 3: high nibble of byte 64 + 3 of the codes
        b[16 + 0 + 7] = 0x90       # element 32 + 7: high nibble of byte 7
        b[16 + 32 * 1 + 9] = 0x0C  # element 2 * 32 + 9: low nibble of byte 32 + 9
    _, v = _single(O.KIND_Q4_K, fill)
    sc5, m5 = 0xA | (3 << 4), 0x7 | (2 << 4)
    assert v[5 * 32 + 3] == (2.0 * sc5) * 11 - 1.0 * m5
    assert v[32 + 7] == (2.0 * 5) * 9 - 1.0 * 3
    assert v[2 * 32 + 9] == (2.0 * 0) * 12 - 0.0  # sc_2 = m_2 = 0
    assert v[5 * 32] == -1.0 * m5


def test_q6_k_known_answers():
    def fill(b):
        b[208:210] = _f16(0.5)
        b[64 + 0 + 5] = 0xD0          # element 128 + 64 + 5 = 197: high nibble of low byte 64 * 1 + 5
        b[128 + 32 + 5] = 0b00_10_00_00  # its top bits: bits 4..5 of high byte 32 * 1 + 5
        b[192 + 12] = np.uint8(np.int8(-3).view(np.uint8))  # group 197 // 16 = 12
        b[32 + 1] = 0x07              # element 32 + 1: low nibble of byte 32 + 1, top bits 0
        b[192 + 2] = 4                # group 33 // 16 = 2
    _, v = _single(O.KIND_Q6_K, fill)
    assert v[197] == (0.5 * -3) * ((13 | (2 << 4)) - 32)
    assert v[33] == (0.5 * 4) * (7 - 32)


@pytest.mark.parametrize("kind", [O.KIND_Q4_0, O.KIND_Q8_0, O.KIND_Q2_K, O.KIND_Q4_K, O.KIND_Q6_K])
def test_host_expansion_matches_the_oracle(kind):
    rng = np.random.default_rng(kind)
    values, size = O.BLOCK_SHAPE[kind]
    n, k = 7, 512
    raw = rng.integers(0, 256, n * (k // values) * size, dtype=np.uint8)
    blocks = raw.reshape(-1, size)
    scale_at = {O.KIND_Q4_0: (0,), O.KIND_Q8_0: (0,), O.KIND_Q2_K: (80, 82), O.KIND_Q4_K: (0, 2), O.KIND_Q6_K: (208,)}
    for off in scale_at[kind]:  # finite fp16 scales
        blocks[:, off:off + 2] = np.float16(rng.uniform(-2, 2, blocks.shape[0])).view(np.uint8).reshape(-1, 2)
    want = O.blocks_values(raw, kind, n, k)
    layer = P.PackedLinear(type("S", (), {"shape": np.array([k, n]), "tensor_type": T(kind), "data": raw})(), None)
    for dtype in (torch.float32, torch.bfloat16, torch.float16):
        got = layer.dequantize(dtype)
        assert torch.equal(got, torch.from_numpy(want).to(dtype))


def test_q4_0_reencoding_is_exact():
    rng = np.random.default_rng(3)
    w = rng.normal(0, 0.25, (9, 256)).astype(np.float32)
    q4 = O.q4_0_quantize(w)
    vals = O.blocks_values(q4, O.KIND_Q4_0, 9, 256)
    assert np.array_equal(O.q8_0_dequant(O.q4_0_to_q8_0(q4, 9, 256), 9, 256), vals)
    # the quantizer's rounding: within half a step, except the top code, clipped at 15 (up to one step); the value of
    # largest magnitude maps to code 0 exactly (d = m / -8)
    d = np.abs(np.ascontiguousarray(q4.reshape(-1, 18)[:, :2]).view("<f2").astype(np.float32))
    err = np.abs(vals - w).reshape(-1, 32)
    assert np.all(err <= d * 1.0 + 1e-3 * d + 1e-7)
    top = np.abs(w).reshape(-1, 32).argmax(1)
    assert np.all(err[np.arange(err.shape[0]), top] <= 1e-3 * d[:, 0] * 8 + 1e-7)
