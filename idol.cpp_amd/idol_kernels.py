"""The matmul, norm and attention entry points of the reference's src/kernels.hpp (namespace idol::detail), as used
by its octree and Gaussian decoders (src/decoders.cpp), on MI355X.

Names, argument order and meaning, and error behaviour follow src/kernels.hpp:53-90; C++ exceptions become
ValueError (std::invalid_argument) and raw pointers become GPU tensors (views into a wider buffer stand for a
pointer offset, with the row strides passed explicitly as in the reference). Quantized layers arrive as the native
panel blob (src/kernels.hpp:33-51) and are turned into GGUF Q8_0 blocks once, at load time: the exact inverse of
tools/gguf_to_decoder.py:16-40, so only 8-bit, group-32 panels whose minimum is -128 * scale qualify (the panels
the Q8_0 bridge writes); other widths are outside this path.
"""
import os

import numpy as np
import torch

import idolq_lib as L

K_COLS = 16          # output columns per panel (src/kernels.hpp:25)
K_QUANT_HEADER = 64  # 16 half scales and 16 half minimums per group (src/kernels.cpp:144)
_QUANT_BITS = (2, 3, 4, 5, 6, 8)

_quant_kernel = -1   # -1: IDOL_QUANT_KERNEL decides; 0: float kernel; 1: integer kernel


class QuantizedLinear:
    """idol::detail::PackedLinear for a quantized layer: `out`, `in_`, `qbits`, `qgroup`, the weights as Q8_0 blocks
    on the device (`q8`) and the bias padded to a multiple of 16 (src/kernels.hpp:33-51)."""

    def __init__(self, out, in_, q8, bias, qbits=8, qgroup=32):
        self.out, self.in_, self.qbits, self.qgroup = out, in_, qbits, qgroup
        self.q8 = q8
        self.bias = bias

    def bytes(self):
        return self.q8.numel() + self.bias.numel() * 4


def quant_panel_bytes(in_, bits, group):
    """Bytes of one quantized 16-column panel (src/kernels.cpp:512-514)."""
    return (in_ // group) * (K_QUANT_HEADER + 2 * group * bits)


def set_quant_kernel(mode):
    """src/kernels.hpp:64-68. -1: IDOL_QUANT_KERNEL decides ("float" forces the float kernel), 0: float, 1: int8."""
    global _quant_kernel
    _quant_kernel = int(mode)


def quant_int8_supported():
    """The integer kernel (int8 MFMA) is available on every gfx950 device."""
    return True


def _use_int8():
    mode = _quant_kernel
    if mode < 0:
        mode = 0 if os.environ.get("IDOL_QUANT_KERNEL") == "float" else 1
    return mode == 1


def panel_to_q8_0(blob, out, in_):
    """GGUF Q8_0 blocks (uint8 [out * in_/32 * 34]) of an 8-bit, group-32 panel blob; the inverse of
    tools/gguf_to_decoder.py:16-40. Raises ValueError if a minimum is not exactly -128 * scale."""
    blob = np.asarray(blob, dtype=np.uint8).reshape(-1)
    npanels, ng = (out + K_COLS - 1) // K_COLS, in_ // 32
    groups = blob.reshape(npanels, ng, K_QUANT_HEADER + 2 * 32 * 8)
    scales = np.ascontiguousarray(groups[:, :, :32]).view("<f2").reshape(npanels, ng, K_COLS)
    mins = np.ascontiguousarray(groups[:, :, 32:64]).view("<f2").reshape(npanels, ng, K_COLS)
    codes = groups[:, :, 64:].reshape(npanels, ng, 32, K_COLS)
    s32, m32 = scales.astype(np.float32), mins.astype(np.float32)
    valid = np.arange(npanels * K_COLS).reshape(npanels, 1, K_COLS) < out
    if not np.all(np.where(valid, m32 == -128.0 * s32, True)):
        raise ValueError("an 8-bit panel whose minimum is not -128 * scale does not hold GGUF Q8_0 blocks")
    # [panel, group, k, column] -> [row = panel * 16 + column, group, k]
    q = (codes.astype(np.int16) - 128).astype(np.int8).transpose(0, 3, 1, 2).reshape(npanels * K_COLS, ng, 32)
    d = scales.transpose(0, 2, 1).reshape(npanels * K_COLS, ng)
    blocks = np.empty((npanels * K_COLS, ng, 34), np.uint8)
    blocks[:, :, :2] = np.ascontiguousarray(d).view(np.uint8).reshape(npanels * K_COLS, ng, 2)
    blocks[:, :, 2:] = q.view(np.uint8)
    return blocks[:out].reshape(-1)


def quantized_linear(blob, bias, out, in_, bits, group, device="cuda"):
    """Wraps an already-quantized panel blob (src/kernels.cpp:516-533), with the same rejections."""
    if bits not in _QUANT_BITS:
        raise ValueError("quantized layers use 2, 3, 4, 5, 6 or 8 bits")
    if group <= 0 or group % 32 != 0 or in_ % group != 0:
        raise ValueError("the quantization group must be a multiple of 32 that divides the input size")
    blob = np.frombuffer(bytes(blob), dtype=np.uint8) if not isinstance(blob, np.ndarray) else blob
    npanels = (out + K_COLS - 1) // K_COLS
    if blob.size != npanels * quant_panel_bytes(in_, bits, group):
        raise ValueError("a quantized blob has the wrong size for its shape")
    if bits != 8 or group != 32:
        raise NotImplementedError("only 8-bit, group-32 panels (GGUF Q8_0 blocks) run on the GPU")
    q8 = torch.from_numpy(panel_to_q8_0(blob, out, in_)).to(device)
    return q8_0_linear(q8, bias, out, in_, device=device)


def q8_0_linear(q8, bias, out, in_, device="cuda"):
    """A quantized layer straight from GGUF Q8_0 blocks (the form tools/gguf_to_decoder.py:16-40 starts from)."""
    if in_ % 32:
        raise ValueError("the quantization group must be a multiple of 32 that divides the input size")
    q8 = torch.as_tensor(q8, dtype=torch.uint8).reshape(-1).to(device)
    if q8.numel() != out * (in_ // 32) * 34:
        raise ValueError("a quantized blob has the wrong size for its shape")
    npad = (out + K_COLS - 1) // K_COLS * K_COLS
    b = torch.zeros(npad, dtype=torch.float32, device=device)
    if bias is not None:
        b[:out] = torch.as_tensor(bias, dtype=torch.float32).reshape(-1)[:out].to(device)
    return QuantizedLinear(out, in_, q8, b)


def dequantize_linear(w):
    """The out x in row-major weights the GEMM sees (src/kernels.cpp:535-550), fp32 on the device."""
    return L.dequant(w.q8, w.out, w.in_, torch.float32)


def gemm_packed(a, m, w, n_offset, n, residual, gelu, c):
    """c[m x n] = a[m x in] * W^T + bias for output columns [n_offset, n_offset + n) (src/kernels.hpp:73-76).

    a is [m, in] fp32 (rows unit-stride); c and residual are [m, n] (residual may alias c); the residual is added
    before the optional erf-GELU."""
    if n_offset < 0 or n < 0 or n_offset + n > w.out:
        raise ValueError("column window outside the layer")
    if m == 0 or n == 0:
        return c
    mode = L.MODE_INT8 if _use_int8() else L.MODE_EXACT
    L.gemm(a[:m], w.q8, w.out, n_offset, n, bias=w.bias[:w.out], residual=residual,
           act=L.ACT_GELU_ERF if gelu else L.ACT_NONE, mode=mode, out=c)
    return c


def layer_norm(x, rows, dim, gamma, beta, y):
    """Layer norm over rows vectors of length dim, eps 1e-5 (src/kernels.cpp:599-618); y may alias x."""
    return L.layernorm(x[:rows, :dim], 1e-5, gamma=gamma, beta=beta, out=y)


def norm_rows(x, y, rows, dim, eps, gamma=None, beta=None, shift=None, scale=None, rows_per_batch=0):
    """src/decoders.cpp:23-42: layer norm, optional gamma/beta, optional adaLN (1 + scale) and shift."""
    return L.layernorm(x[:rows, :dim], eps, gamma=gamma, beta=beta, shift=shift, scale=scale,
                       rows_per_batch=rows_per_batch, out=y)


def attention(q, lq, ldq, k, v, lk, ldkv, heads, head_dim, out, dim):
    """Scaled dot-product attention over projected rows (src/kernels.hpp:81-84). q, k, v and out are flat GPU
    tensors (pointer offsets as views); q has lq rows of stride ldq, k and v lk rows of stride ldkv, out lq rows of
    stride dim."""
    return L.attention(q, k, v, 1, lq, lk, heads, head_dim, ldq, ldkv, 0, 0, out, dim, 0)


def gelu_tanh(x):
    """In-place tanh-GELU (src/decoders.cpp:55-71)."""
    return L.activation(x, L.ACT_GELU_TANH)
