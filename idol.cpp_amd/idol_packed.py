"""Quantized linear layers that keep their GGUF blocks packed: the drop-in for the reference's
tools/idol_packed.py (PackedLinear, enable_fused_packed, replace_quantized_linear_layers).

Signatures, attributes (`shape`, `kind`, `packed` buffer, `bias`, `fused`), validation and error messages follow the
reference. Differences:
  * the fused GPU path is libidolq's gfx950 kernel (idol_hip.fused_linear) and exists for Q8_0; enable_fused_packed
    therefore enables Q8_0 layers only;
  * dequantize() expands Q8_0 on the GPU with libidolq's kernel (tools/idol_triton.py:_unpack_q8 semantics) and
    F16 / Q4_0 with tensor arithmetic; the K-quant kinds are accepted as packed storage but cannot be expanded
    (NotImplementedError).
"""
import numpy as np
import torch
import torch.nn.functional as F

import idolq_lib as L
from ggml_types import GGMLQuantizationType
from idol_hip import fused_linear

_PACKED_KINDS = (GGMLQuantizationType.F16, GGMLQuantizationType.Q8_0, GGMLQuantizationType.Q4_0,
                 GGMLQuantizationType.Q2_K, GGMLQuantizationType.Q4_K, GGMLQuantizationType.Q6_K)
_FUSED_KINDS = {GGMLQuantizationType.Q8_0: 8}


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
        if kind == GGMLQuantizationType.F16:
            return self.packed.view(torch.float16).reshape(self.shape).to(dtype)
        if kind == GGMLQuantizationType.Q8_0:
            n, k = self.shape
            if self.packed.is_cuda:
                if dtype in L.DTYPE_CODE:
                    return L.dequant(self.packed, n, k, dtype)
                return L.dequant(self.packed, n, k, torch.float32).to(dtype)
            blocks = self.packed.reshape(-1, 34)
            scale = blocks[:, :2].contiguous().view(torch.float16).float()
            codes = blocks[:, 2:].contiguous().view(torch.int8).float()
            return (codes * scale).reshape(self.shape).to(dtype)
        if kind == GGMLQuantizationType.Q4_0:
            blocks = self.packed.reshape(-1, 18)
            scale = blocks[:, :2].contiguous().view(torch.float16).float()
            nib = blocks[:, 2:]
            codes = torch.cat((nib & 15, nib >> 4), dim=1).to(torch.int16).sub_(8).float()
            return (codes * scale).reshape(self.shape).to(dtype)
        raise NotImplementedError(f"dequantize is not implemented for {GGMLQuantizationType(kind).name}")

    def forward(self, value):
        """Fused kernel for Q8_0 on the GPU with 16-bit activations and no autograd; otherwise a dense product
        (tools/idol_packed.py:73-82)."""
        needs_grad = torch.is_grad_enabled() and (value.requires_grad or
                                                  (self.bias is not None and self.bias.requires_grad))
        if (self.fused and value.is_cuda and value.dtype in (torch.float16, torch.bfloat16)
                and self.kind in _FUSED_KINDS and not needs_grad):
            return fused_linear(value, self.packed, self.shape, _FUSED_KINDS[self.kind], self.bias)
        return F.linear(value, self.dequantize(value.dtype), self.bias)


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
