"""Fused Q8_0 linear on MI355X: the drop-in for the reference's tools/idol_triton.py:fused_linear.

fused_linear keeps the reference's signature, validation and error messages (tools/idol_triton.py:94-111) and its
numerics: weights dequantized to the activation dtype (fp32(d) * q, rounded), fp32 accumulation, the product
rounded to the output dtype before the bias is added (tools/idol_triton.py:84-89). The arithmetic runs in
libidolq's gfx950 kernel (idolq_q8_0_gemm, DEQUANT mode); there is no other path.
"""
import torch

import idolq_lib as L

KIND_Q4_0, KIND_Q8_0, KIND_Q4_K = 4, 8, 44


def fused_linear(value, packed, shape, kind, bias=None):
    """Multiply FP16/BF16 activations by Q8_0 weights on the GPU (tools/idol_triton.py:94-126)."""
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
    if kind != KIND_Q8_0:
        raise NotImplementedError('only Q8_0 weights have a fused MI355X kernel')
    x = value.reshape(-1, k)
    if x.shape[0] and x.stride(-1) != 1:
        x = x.contiguous()
    m = x.shape[0]
    if not m:
        return torch.empty((*value.shape[:-1], n), device=value.device, dtype=value.dtype)
    out = L.gemm(x, packed.reshape(-1), n, bias=bias, mode=L.MODE_DEQUANT, flags=L.FLAG_ROUND_BEFORE_BIAS)
    return out.reshape(*value.shape[:-1], n)
