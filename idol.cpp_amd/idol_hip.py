"""Fused packed linear on MI355X: the drop-in for the reference's tools/idol_triton.py:fused_linear.

fused_linear keeps the reference's signature, validation and error messages (tools/idol_triton.py:94-111) and its
numerics: weights dequantized to the activation dtype (the fp32 value, rounded), fp32 accumulation, the product
rounded to the output dtype before the bias is added (tools/idol_triton.py:84-89). Per kind:
  Q8_0 (8)   libidolq's Q8_0 GEMM (idolq_q8_0_gemm, DEQUANT mode) on the GGUF blocks as they are;
  Q4_K (44)  libidolq's Q4_K GEMM (idolq_q4_k_gemm) on the GGUF super-blocks as they are: each weight is decoded to
             T((d * sc) * q - dmin * m) inside the GEMM's weight loader, as the reference's kernel does
             (tools/idol_triton.py:61-82); nothing is expanded or allocated besides the output;
  Q4_0 (4)   the blocks as Q8_0 blocks with the same scale and codes q - 8 (exact), then the Q8_0 GEMM: the weights it
             multiplies are the reference's T(d * (q - 8)). PackedLinear makes that copy once per device and passes
             it as q8_blocks; a bare call re-encodes the blocks (idolq_q4_0_to_q8_0) first.
For Q8_0 and Q4_0, q8_tiled may carry the same Q8_0 blocks in the library's tiled layout (idolq_q8_0_tile, made once
by PackedLinear): calls of more than 16 rows then run the tiled-weight GEMM, whose products are bit-identical to the
row-major kernel's (whole tiles), and shorter ones keep the row-major small-m kernel.
Rounding: the product is rounded to the output dtype before the bias is added (tools/idol_triton.py:84-89), except
on the reference's fp16 large-M Q8_0 branch (fp16, m >= 4096, n >= 1024, k >= 1024: tools/idol_triton.py:112-117),
which calls F.linear, whose fused bias enters the fp32 accumulator before the one rounding; that branch keeps that
order here (same weights T(d * q), no dense copy).
"""
import torch

import idolq_lib as L

KIND_Q4_0, KIND_Q8_0, KIND_Q4_K = 4, 8, 44
SMALL_M = 16  # rows up to which the row-major small-m kernel serves a call (idolq_q8_0_gemm's m <= 16 form)


def fused_linear(value, packed, shape, kind, bias=None, *, q8_blocks=None, q8_tiled=None):
    """Multiply FP16/BF16 activations by Q4_0, Q8_0 or Q4_K weights on the GPU (tools/idol_triton.py:94-126).
    q8_blocks: for kind 4, the Q8_0 re-encoding of `packed` (L.q4_0_to_q8_0) made beforehand. q8_tiled: for kinds 8
    and 4, those Q8_0 blocks in the tiled layout (L.tile_q8_0), made beforehand."""
    if (not value.is_cuda or not packed.is_cuda or packed.dtype != torch.uint8
            or value.device != packed.device or value.dtype not in (torch.float16, torch.bfloat16)
            or len(shape) != 2 or value.shape[-1] != shape[1] or kind not in (KIND_Q4_0, KIND_Q8_0, KIND_Q4_K)):
        raise ValueError('unsupported fused linear input')
    if torch.is_grad_enabled() and (value.requires_grad or (bias is not None and bias.requires_grad)):
        raise ValueError('fused linear supports inference only')
    n, k = shape
    group, size = (256, 144) if kind == KIND_Q4_K else (32, 18 if kind == KIND_Q4_0 else 34)
    if n < 1 or k < 1 or k % group or packed.numel() != n * (k // group) * size:
        raise ValueError('invalid packed linear dimensions')
    if bias is not None and (bias.shape != (n,) or bias.device != value.device or bias.dtype != value.dtype):
        raise ValueError('invalid fused linear bias')
    x = value.reshape(-1, k)
    if x.shape[0] and x.stride(-1) != 1:
        x = x.contiguous()
    m = x.shape[0]
    if not m:
        return torch.empty((*value.shape[:-1], n), device=value.device, dtype=value.dtype)
    w = packed.reshape(-1)
    # the bias enters the epilogue as fp32, as the reference loads it (an exact widening)
    b32 = bias.float() if bias is not None else None
    if kind == KIND_Q4_K:
        if x.data_ptr() % 16:  # the Q4_K kernel reads 16-byte aligned rows (k % 256 == 0): only a view can miss it
            x = x.clone()
        out = L.q4_k_gemm(x, w, n, bias=b32, flags=L.FLAG_ROUND_BEFORE_BIAS)
        return out.reshape(*value.shape[:-1], n)
    # the reference's F.linear branch adds the bias before its one rounding; everywhere else the product is rounded
    # first
    dense_branch = kind == KIND_Q8_0 and value.dtype == torch.float16 and m >= 4096 and n >= 1024 and k >= 1024
    flags = 0 if dense_branch else L.FLAG_ROUND_BEFORE_BIAS
    # the tiled-weight GEMM reads 16-byte aligned activation rows; other views keep the row-major blocks
    aligned = x.data_ptr() % 16 == 0 and (m == 1 or (x.stride(0) * x.element_size()) % 16 == 0)
    if q8_tiled is not None and m > SMALL_M and aligned:
        if q8_tiled.numel() != L.tiled_q8_0_bytes(n, k) or q8_tiled.device != value.device:
            raise ValueError('invalid packed linear dimensions')
        out = L.gemm(x, q8_tiled.reshape(-1), n, bias=b32, mode=L.MODE_DEQUANT, flags=flags, tiled=True)
        return out.reshape(*value.shape[:-1], n)
    if kind == KIND_Q4_0:
        if q8_blocks is not None:
            if q8_blocks.numel() != n * (k // 32) * 34 or q8_blocks.device != value.device:
                raise ValueError('invalid packed linear dimensions')
            w = q8_blocks.reshape(-1)
        else:
            w = L.q4_0_to_q8_0(w, n, k)
    out = L.gemm(x, w, n, bias=b32, mode=L.MODE_DEQUANT, flags=flags)
    return out.reshape(*value.shape[:-1], n)
