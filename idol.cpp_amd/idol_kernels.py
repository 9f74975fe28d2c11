"""The matmul, norm and attention entry points of the reference's src/kernels.hpp (namespace idol::detail), as used
by its octree and Gaussian decoders (src/decoders.cpp), on MI355X.

Names, argument order and meaning, and error behaviour follow src/kernels.hpp:53-90; C++ exceptions become
ValueError (std::invalid_argument) and raw pointers become GPU tensors (views into a wider buffer stand for a
pointer offset, with the row strides passed explicitly as in the reference).

Weights. A quantized layer arrives as the native panel blob (src/kernels.hpp:33-51). When every group's minimum is
-2^(bits-1) * scale (the form the GGUF Q8_0 and Q4_0 bridges write, tools/gguf_to_decoder.py:16-40), its values are
exactly fp32(scale) * (code - 2^(bits-1)) and it is turned, losslessly and once at load time, into GGUF Q8_0 blocks
for the Q8_0 GEMM. Any other panel (asymmetric minimums from a search quantizer) is expanded once to the fp32 values
the reference's dequantizer produces, fma(code, scale, min), and runs on the dense fp32 GEMM, which sums in the
reference's order: the reference's float kernel treats a quantized layer and a dense layer holding its dequantized
values identically (src/kernels.cpp:272-273). Unquantized layers (pack_linear) hold their fp32 weights.
"""
import os

import numpy as np
import torch

import idolq_lib as L

K_COLS = 16          # output columns per panel (src/kernels.hpp:25)
K_QUANT_HEADER = 64  # 16 half scales and 16 half minimums per group (src/kernels.cpp:144)
_QUANT_BITS = (2, 3, 4, 5, 6, 8)
_PLANES = {2: (2,), 3: (2, 1), 4: (4,), 5: (4, 1), 6: (4, 2), 8: (8,)}  # bit-plane widths, low bits first

_quant_kernel = -1   # -1: IDOL_QUANT_KERNEL decides; 0: float kernel; 1: integer kernel


class PackedLinear:
    """idol::detail::PackedLinear on the device: `out`, `in_`, `qbits` (0: unquantized), `qgroup`, the weights either
    as Q8_0 blocks (`q8`) or as fp32 [out, in] (`weight`), and the bias padded to a multiple of 16
    (src/kernels.hpp:33-51)."""

    def __init__(self, out, in_, q8, bias, qbits=8, qgroup=32, weight=None):
        self.out, self.in_, self.qbits, self.qgroup = out, in_, qbits, qgroup
        self.q8 = q8
        self.weight = weight
        self.bias = bias

    def bytes(self):
        """Bytes held on the device: the weights as stored here plus the padded bias."""
        held = self.q8.numel() if self.q8 is not None else self.weight.numel() * 4
        return held + self.bias.numel() * 4


QuantizedLinear = PackedLinear


def _padded_bias(bias, out, device):
    npad = (out + K_COLS - 1) // K_COLS * K_COLS
    b = torch.zeros(npad, dtype=torch.float32, device=device)
    if bias is not None:
        b[:out] = torch.as_tensor(np.asarray(bias, np.float32).reshape(-1)[:out]).to(device)
    return b


def pack_linear(weight, bias, out, in_, device="cuda"):
    """An unquantized layer from fp32 weights [out x in] and bias [out] (src/kernels.cpp:144-160)."""
    w = torch.as_tensor(np.ascontiguousarray(np.asarray(weight, np.float32).reshape(out, in_))).to(device)
    return PackedLinear(out, in_, None, _padded_bias(bias, out, device), qbits=0, qgroup=0, weight=w)


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


def unpack_panel(blob, out, in_, bits, group):
    """(codes uint8 [out, in], scales fp32 [out, in/group], minimums fp32 [out, in/group]) of a panel blob: per
    16-column panel and group, 16 fp16 scales, 16 fp16 minimums, then per 8 rows of k the bit planes, low bits first,
    a plane of width w packing rows w_i * (8 / w) + j at bit j * w of byte row w_i (the reader's order,
    src/kernels.cpp:167-209)."""
    blob = np.asarray(blob, dtype=np.uint8).reshape(-1)
    npanels, ng = (out + K_COLS - 1) // K_COLS, in_ // group
    groups = blob.reshape(npanels, ng, K_QUANT_HEADER + 2 * group * bits)
    scales = np.ascontiguousarray(groups[:, :, :32]).view("<f2").reshape(npanels, ng, K_COLS).astype(np.float32)
    mins = np.ascontiguousarray(groups[:, :, 32:64]).view("<f2").reshape(npanels, ng, K_COLS).astype(np.float32)
    body = groups[:, :, 64:].reshape(npanels, ng, group // 8, bits, K_COLS)
    codes = np.zeros((npanels, ng, group // 8, 8, K_COLS), np.uint8)
    plane0, shift = 0, 0
    for width in _PLANES[bits]:
        per = 8 // width
        for wi in range(width):
            byte = body[:, :, :, plane0 + wi, :]
            for sub in range(per):
                codes[:, :, :, wi * per + sub, :] |= ((byte >> (sub * width)) & ((1 << width) - 1)) << shift
        plane0 += width
        shift += width
    # [panel, group, k, column] -> [row, k]
    codes = codes.reshape(npanels, in_, K_COLS).transpose(0, 2, 1).reshape(npanels * K_COLS, in_)[:out]
    scales = scales.transpose(0, 2, 1).reshape(npanels * K_COLS, ng)[:out]
    mins = mins.transpose(0, 2, 1).reshape(npanels * K_COLS, ng)[:out]
    return np.ascontiguousarray(codes), np.ascontiguousarray(scales), np.ascontiguousarray(mins)


def pack_panel(codes, scales, mins, bits, group):
    """The panel blob (uint8) of codes [out, in] (values < 2^bits), scales and minimums [out, in/group] (stored as
    fp16): the layout unpack_panel reads, as the reference's writer lays it out (tools/idolq.py:137-170)."""
    codes = np.asarray(codes, np.uint8)
    out, in_ = codes.shape
    npanels, ng = (out + K_COLS - 1) // K_COLS, in_ // group
    pad = npanels * K_COLS - out
    c = np.pad(codes, ((0, pad), (0, 0)))
    s = np.pad(np.asarray(scales, np.float32), ((0, pad), (0, 0))).astype(np.float16)
    m = np.pad(np.asarray(mins, np.float32), ((0, pad), (0, 0))).astype(np.float16)
    # [row, k] -> [panel, group, chunk of 8 k, k in chunk, column]
    ck = c.reshape(npanels, K_COLS, ng, group // 8, 8).transpose(0, 2, 3, 4, 1)
    body = np.zeros((npanels, ng, group // 8, bits, K_COLS), np.uint8)
    plane0, shift = 0, 0
    for width in _PLANES[bits]:
        per = 8 // width
        for wi in range(width):
            for sub in range(per):
                body[:, :, :, plane0 + wi, :] |= ((ck[:, :, :, wi * per + sub, :] >> shift) & ((1 << width) - 1)) \
                    << (sub * width)
        plane0 += width
        shift += width
    head_s = np.ascontiguousarray(s.reshape(npanels, K_COLS, ng).transpose(0, 2, 1)).view(np.uint8)
    head_m = np.ascontiguousarray(m.reshape(npanels, K_COLS, ng).transpose(0, 2, 1)).view(np.uint8)
    blob = np.concatenate([head_s.reshape(npanels, ng, 32), head_m.reshape(npanels, ng, 32),
                           body.reshape(npanels, ng, -1)], axis=2)
    return np.ascontiguousarray(blob).reshape(-1)


# ---- host restatement of the panel layout: the writers (tools/idolq.py:137-170 order) and loaders that hold their
# weights on the host (device="cpu"); on the GPU the blob is converted by idolq_panel_to_q8_0 / idolq_panel_expand_f32.
def panel_is_symmetric(scales, mins, bits):
    """True when every minimum is -2^(bits-1) * scale: the panel holds fp32(scale) * (code - 2^(bits-1))."""
    return bool(np.all(mins == -float(1 << (bits - 1)) * scales))


def panel_to_q8_0(blob, out, in_, bits=8, group=32):
    """GGUF Q8_0 blocks (uint8 [out * in_/32 * 34]) holding exactly the values of a symmetric panel blob: the inverse
    of tools/gguf_to_decoder.py:16-40 for 8-bit (Q8_0) and 4-bit (Q4_0) panels. Raises ValueError if a minimum is
    not -2^(bits-1) * scale."""
    codes, scales, mins = unpack_panel(blob, out, in_, bits, group)
    if not panel_is_symmetric(scales, mins, bits):
        raise ValueError(f"a {bits}-bit panel whose minimum is not -{1 << (bits - 1)} * scale does not hold GGUF "
                         "Q8_0 blocks")
    nb = in_ // 32
    q = (codes.astype(np.int16) - (1 << (bits - 1))).astype(np.int8).reshape(out, nb, 32)
    d = np.repeat(scales, group // 32, axis=1).astype(np.float16)
    blocks = np.empty((out, nb, 34), np.uint8)
    blocks[:, :, :2] = np.ascontiguousarray(d).view(np.uint8).reshape(out, nb, 2)
    blocks[:, :, 2:] = q.view(np.uint8)
    return blocks.reshape(-1)


def panel_values(blob, out, in_, bits, group):
    """The fp32 weights [out, in] the reference's dequantizer gives a panel: fma(code, scale, min) per value (the
    product of an 8-bit code and an fp16 scale is exact in fp32, so one rounding, as the fused multiply-add)."""
    codes, scales, mins = unpack_panel(blob, out, in_, bits, group)
    s = np.repeat(scales, group, axis=1)
    m = np.repeat(mins, group, axis=1)
    return (codes.astype(np.float32) * s + m).astype(np.float32)


def quantized_linear(blob, bias, out, in_, bits, group, device="cuda"):
    """Wraps an already-quantized panel blob (src/kernels.cpp:516-533), with the same rejections."""
    if bits not in _QUANT_BITS:
        raise ValueError("quantized layers use 2, 3, 4, 5, 6 or 8 bits")
    if group <= 0 or group % 32 != 0 or in_ % group != 0:
        raise ValueError("the quantization group must be a multiple of 32 that divides the input size")
    blob = np.frombuffer(bytes(blob), dtype=np.uint8) if not isinstance(blob, np.ndarray) else blob.reshape(-1)
    npanels = (out + K_COLS - 1) // K_COLS
    if blob.size != npanels * quant_panel_bytes(in_, bits, group):
        raise ValueError("a quantized blob has the wrong size for its shape")
    if torch.device(device).type == "cuda":
        # on the device: the blocks when every group's minimum is exact (checked by the kernel), else fp32 values
        dev_blob = torch.from_numpy(np.ascontiguousarray(blob)).to(device)
        q8, inexact = L.panel_to_q8_0(dev_blob, out, in_, bits, group)
        if int(inexact.item()) == 0:
            layer = q8_0_linear(q8, bias, out, in_, device=device)
        else:
            w = L.panel_expand_f32(dev_blob, out, in_, bits, group)
            layer = PackedLinear(out, in_, None, _padded_bias(bias, out, device), weight=w)
    else:
        codes, scales, mins = unpack_panel(blob, out, in_, bits, group)
        if panel_is_symmetric(scales, mins, bits):
            q8 = torch.from_numpy(panel_to_q8_0(blob, out, in_, bits, group)).to(device)
            layer = q8_0_linear(q8, bias, out, in_, device=device)
        else:
            w = torch.from_numpy(panel_values(blob, out, in_, bits, group)).to(device)
            layer = PackedLinear(out, in_, None, _padded_bias(bias, out, device), weight=w)
    layer.qbits, layer.qgroup = bits, group
    return layer


def q8_0_linear(q8, bias, out, in_, device="cuda"):
    """A quantized layer straight from GGUF Q8_0 blocks (the form tools/gguf_to_decoder.py:16-40 starts from)."""
    if in_ % 32:
        raise ValueError("the quantization group must be a multiple of 32 that divides the input size")
    q8 = torch.as_tensor(q8, dtype=torch.uint8).reshape(-1).to(device)
    if q8.numel() != out * (in_ // 32) * 34:
        raise ValueError("a quantized blob has the wrong size for its shape")
    return PackedLinear(out, in_, q8, _padded_bias(bias, out, device))


def dequantize_linear(w):
    """The out x in row-major weights the GEMM sees (src/kernels.cpp:535-550), fp32 on the device."""
    if w.q8 is None:
        return w.weight.clone()
    return L.dequant(w.q8, w.out, w.in_, torch.float32)


def gemm_packed(a, m, w, n_offset, n, residual, gelu, c):
    """c[m x n] = a[m x in] * W^T + bias for output columns [n_offset, n_offset + n) (src/kernels.hpp:73-76).

    a is [m, in] fp32 (rows unit-stride); c and residual are [m, n] (residual may alias c); the residual is added
    before the optional erf-GELU."""
    if n_offset < 0 or n < 0 or n_offset + n > w.out:
        raise ValueError("column window outside the layer")
    if m == 0 or n == 0:
        return c
    act = L.ACT_GELU_ERF if gelu else L.ACT_NONE
    if w.q8 is None:
        L.gemm_f32(a[:m], w.weight[n_offset:n_offset + n], bias=w.bias[n_offset:n_offset + n], residual=residual,
                   act=act, out=c)
        return c
    mode = L.MODE_INT8 if _use_int8() else L.MODE_EXACT
    L.gemm(a[:m], w.q8, w.out, n_offset, n, bias=w.bias[:w.out], residual=residual,
           act=act, mode=mode, out=c)
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
