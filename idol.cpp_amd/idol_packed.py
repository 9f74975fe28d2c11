"""Quantized linear layers that keep their GGUF blocks packed: the drop-in for the reference's
tools/idol_packed.py (PackedLinear, enable_fused_packed, replace_quantized_linear_layers).

Signatures, attributes (`shape`, `kind`, `packed` buffer, `bias`, `fused`), validation and error messages follow the
reference. The fused GPU path is libidolq (idol_hip.fused_linear) for Q4_0, Q8_0 and Q4_K, the kinds the reference
fuses. dequantize() expands every kind: on the GPU with libidolq's kernels (idolq_q8_0_dequant,
idolq_blocks_dequant), for a module kept on the host with tensor arithmetic; both compute each value with the
reference expansion's fp32 operations (tools/idol_packed.py:25-71), then round once.
"""
import numpy as np
import torch
import torch.nn.functional as F

import idolq_lib as L
from ggml_types import GGMLQuantizationType
from idol_hip import fused_linear

_PACKED_KINDS = (GGMLQuantizationType.F16, GGMLQuantizationType.Q8_0, GGMLQuantizationType.Q4_0,
                 GGMLQuantizationType.Q2_K, GGMLQuantizationType.Q4_K, GGMLQuantizationType.Q6_K)
_FUSED_KINDS = {GGMLQuantizationType.Q4_0: 4, GGMLQuantizationType.Q8_0: 8, GGMLQuantizationType.Q4_K: 44}


class PackedLinear(torch.nn.Module):
    """A linear layer holding raw GGUF blocks (tools/idol_packed.py:12-23)."""

    def __init__(self, source, bias):
        super().__init__()
        self.shape = tuple(reversed(np.asarray(source.shape).tolist()))
        self.kind = source.tensor_type
        if len(self.shape) != 2 or self.kind not in _PACKED_KINDS:
            raise ValueError("unsupported packed matrix")
        self.register_buffer("packed", torch.from_numpy(np.array(source.data, copy=True)).reshape(-1))
        self.bias = torch.nn.Parameter(bias.detach(), requires_grad=False) if bias is not None else None
        self.fused = False

    def dequantize(self, dtype):
        """The dense (n, k) weight in `dtype` (tools/idol_packed.py:25-71)."""
        kind = self.kind
        n, k = self.shape
        if kind == GGMLQuantizationType.F16:
            return self.packed.view(torch.float16).reshape(self.shape).to(dtype)
        if self.packed.is_cuda:
            out_dtype = dtype if dtype in L.DTYPE_CODE else torch.float32
            if kind == GGMLQuantizationType.Q8_0:
                dense = L.dequant(self.packed, n, k, out_dtype)
            else:
                dense = L.blocks_dequant(self.packed, int(kind), n, k, out_dtype)
            return dense if out_dtype == dtype else dense.to(dtype)
        return _host_values(self.packed, kind, n, k).to(dtype)

    def forward(self, value):
        """Fused kernel for Q4_0, Q8_0 and Q4_K on the GPU with 16-bit activations and no autograd; otherwise a dense product
        (tools/idol_packed.py:73-82)."""
        needs_grad = torch.is_grad_enabled() and (value.requires_grad or
                                                  (self.bias is not None and self.bias.requires_grad))
        if (self.fused and value.is_cuda and value.dtype in (torch.float16, torch.bfloat16)
                and self.kind in _FUSED_KINDS and not needs_grad):
            return fused_linear(value, self.packed, self.shape, _FUSED_KINDS[self.kind], self.bias)
        return F.linear(value, self.dequantize(value.dtype), self.bias)


def _host_values(packed, kind, n, k):
    """fp32 values of a packed matrix held on the host: per block format, the products and differences of the
    reference's expansion, in fp32, without fused multiply-adds."""
    f16 = lambda b: b.contiguous().view(torch.float16).float()  # noqa: E731
    u = packed.reshape(-1)
    if kind == GGMLQuantizationType.Q8_0:
        blocks = u.reshape(-1, 34)
        return (blocks[:, 2:].contiguous().view(torch.int8).float() * f16(blocks[:, :2])).reshape(n, k)
    if kind == GGMLQuantizationType.Q4_0:
        blocks = u.reshape(-1, 18)
        nib = blocks[:, 2:]
        q = torch.cat((nib & 15, nib >> 4), dim=1).to(torch.int16).sub_(8).float()
        return (q * f16(blocks[:, :2])).reshape(n, k)
    if kind == GGMLQuantizationType.Q2_K:
        blocks = u.reshape(-1, 84)
        pairs = blocks[:, :16]
        sd = f16(blocks[:, 80:82]) * (pairs & 15).float()          # [blocks, 16]
        sm = f16(blocks[:, 82:84]) * (pairs >> 4).float()
        qs = blocks[:, 16:80].reshape(-1, 2, 1, 32)                  # [blocks, half, 1, l]
        shift = torch.arange(0, 8, 2, dtype=torch.uint8).reshape(1, 1, 4, 1)
        q = ((qs >> shift) & 3).reshape(-1, 16, 16).float()          # element 128 h + 32 s + l
        return (sd.unsqueeze(2) * q - sm.unsqueeze(2)).reshape(n, k)
    if kind == GGMLQuantizationType.Q4_K:
        blocks = u.reshape(-1, 144)
        s = blocks[:, 4:16].to(torch.int32)
        a, b, c = s[:, 0:4], s[:, 4:8], s[:, 8:12]
        sc = torch.cat((a & 63, (c & 15) | ((a >> 6) << 4)), dim=1).float()
        mn = torch.cat((b & 63, (c >> 4) | ((b >> 6) << 4)), dim=1).float()
        sd = f16(blocks[:, 0:2]) * sc
        sm = f16(blocks[:, 2:4]) * mn
        qs = blocks[:, 16:].reshape(-1, 4, 1, 32)
        q = ((qs >> torch.tensor([0, 4], dtype=torch.uint8).reshape(1, 1, 2, 1)) & 15).reshape(-1, 8, 32).float()
        return (sd.unsqueeze(2) * q - sm.unsqueeze(2)).reshape(n, k)
    if kind == GGMLQuantizationType.Q6_K:
        blocks = u.reshape(-1, 210)
        ql = blocks[:, :128].reshape(-1, 2, 1, 64)
        qh = blocks[:, 128:192].reshape(-1, 2, 1, 32)
        lo = ((ql >> torch.tensor([0, 4], dtype=torch.uint8).reshape(1, 1, 2, 1)) & 15).reshape(-1, 2, 4, 32)
        hi = ((qh >> torch.arange(0, 8, 2, dtype=torch.uint8).reshape(1, 1, 4, 1)) & 3).reshape(-1, 2, 4, 32)
        q = (lo.to(torch.int16) | (hi.to(torch.int16) << 4)).sub_(32).reshape(-1, 16, 16).float()
        sd = f16(blocks[:, 208:210]) * blocks[:, 192:208].contiguous().view(torch.int8).float()
        return (sd.unsqueeze(2) * q).reshape(n, k)
    raise NotImplementedError(f"dequantize is not implemented for {GGMLQuantizationType(kind).name}")


def enable_fused_packed(model):
    """Enable supported packed layers; return the number configured for the GPU (tools/idol_packed.py:85-94)."""
    count = 0
    for layer in model.modules():
        if isinstance(layer, PackedLinear) and layer.kind in _FUSED_KINDS:
            layer.fused = True
            count += 1
    return count


def replace_quantized_linear_layers(model, source, include_half=False):
    """Replace all quantized linear weights after checking the complete mapping (tools/idol_packed.py:97-129).

    `source` maps GGUF tensor names to source tensors. A quantized tensor that is not a linear weight is an error.
    """
    supported = {GGMLQuantizationType.Q8_0, GGMLQuantizationType.Q4_0, GGMLQuantizationType.Q2_K,
                 GGMLQuantizationType.Q4_K, GGMLQuantizationType.Q6_K}
    selected = {name: tensor for name, tensor in source.items()
                if tensor.tensor_type in supported or
                (include_half and tensor.tensor_type == GGMLQuantizationType.F16
                 and len(tensor.shape) == 2 and name.endswith('.weight'))}
    names = []
    for key, tensor in selected.items():
        if not key.endswith('.weight'):
            raise ValueError('quantized tensor is not a linear weight: ' + key)
        name = key[:-len('.weight')]
        try:
            module = model.get_submodule(name)
        except AttributeError as exc:
            raise ValueError('quantized linear layer is missing: ' + key) from exc
        if (not isinstance(module, torch.nn.Linear)
                or tuple(reversed(np.asarray(tensor.shape).tolist())) != tuple(module.weight.shape)):
            raise ValueError('quantized tensor does not match a linear layer: ' + key)
        names.append(name)
    for name in names:
        tensor = selected[name + '.weight']
        module = model.get_submodule(name)
        parent_name, _, leaf = name.rpartition(".")
        parent = model.get_submodule(parent_name) if parent_name else model
        setattr(parent, leaf, PackedLinear(tensor, module.bias).to(device=module.weight.device))
    return [name + '.weight' for name in names]
