"""Quantized linear layers that keep their GGUF blocks packed: the drop-in for the reference's
tools/idol_packed.py (PackedLinear, enable_fused_packed, replace_quantized_linear_layers).

Signatures, attributes (`shape`, `kind`, `packed` buffer, `bias`, `fused`), the accepted inputs and the error
messages are the reference's interface; the code is this package's own. The fused GPU path is libidolq
(idol_hip.fused_linear) for Q4_0, Q8_0 and Q4_K, the kinds the reference fuses. dequantize() expands every kind: on the GPU with libidolq's kernels (idolq_q8_0_dequant,
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
_BLOCK_KINDS = frozenset(_PACKED_KINDS[1:])
_FUSED_KINDS = {GGMLQuantizationType.Q4_0: 4, GGMLQuantizationType.Q8_0: 8, GGMLQuantizationType.Q4_K: 44}
_FUSED_DTYPES = (torch.float16, torch.bfloat16)
_TILED_KINDS = (GGMLQuantizationType.Q8_0, GGMLQuantizationType.Q4_0)  # fused through the Q8_0 GEMM


class PackedLinear(torch.nn.Module):
    """A linear layer that keeps a GGUF matrix's raw bytes (the interface of tools/idol_packed.py:12-82).

    `shape` is (out, in) -- the GGUF dimensions reversed --, `kind` the GGUF type, `packed` a uint8 buffer (it moves
    with .to(device)), `bias` a frozen parameter or None, and `fused` whether forward may take the fused kernel."""

    def __init__(self, source, bias):
        super().__init__()
        shape = tuple(int(d) for d in reversed(np.asarray(source.shape).tolist()))
        if len(shape) != 2 or source.tensor_type not in _PACKED_KINDS:
            raise ValueError("unsupported packed matrix")
        self.shape, self.kind, self.fused = shape, source.tensor_type, False
        self.register_buffer("packed", torch.from_numpy(np.array(source.data, dtype=np.uint8, copy=True).reshape(-1)))
        self.bias = None if bias is None else torch.nn.Parameter(bias.detach(), requires_grad=False)
        # derived device copies, made once and remade when `packed` moves or is written (its storage or version
        # changes): Q4_0's exact Q8_0 re-encoding, and the Q8_0 blocks in the tiled GEMM layout
        self._q8_blocks = self._q8_tiled = None
        self._q8_blocks_key = self._q8_tiled_key = None

    def _packed_key(self):
        return (self.packed.device, self.packed.data_ptr(), self.packed._version)

    def _q4_0_as_q8_0(self):
        if self._q8_blocks is None or self._q8_blocks_key != self._packed_key():
            n, k = self.shape
            self._q8_blocks = L.q4_0_to_q8_0(self.packed, n, k)
            self._q8_blocks_key = self._packed_key()
        return self._q8_blocks

    def _q8_0_tiled(self):
        """The layer's Q8_0 blocks (Q4_0: their exact Q8_0 re-encoding) in the library's tiled layout on the packed
        buffer's device, made on the first fused call there (k % 64 == 0; None otherwise). It costs
        L.tiled_q8_0_bytes(n, k) bytes of device memory beside `packed` (about 1.06 bytes per weight) and serves the
        calls of more than 16 rows with the tiled-weight GEMM (bit-identical products)."""
        n, k = self.shape
        if k % 64:
            return None
        if self._q8_tiled is None or self._q8_tiled_key != self._packed_key():
            blocks = self._q4_0_as_q8_0() if self.kind == GGMLQuantizationType.Q4_0 else self.packed
            self._q8_tiled = L.tile_q8_0(blocks, n, k)
            self._q8_tiled_key = self._packed_key()
        return self._q8_tiled

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

    def _fusable(self, value):
        """The fused kernel serves enabled layers of the fused kinds on 16-bit GPU activations when no gradient is
        being recorded for the input or the bias."""
        if not (self.fused and self.kind in _FUSED_KINDS and value.is_cuda and value.dtype in _FUSED_DTYPES):
            return False
        if not torch.is_grad_enabled():
            return True
        return not value.requires_grad and not (self.bias is not None and self.bias.requires_grad)

    def forward(self, value):
        if self._fusable(value):
            q8 = self._q4_0_as_q8_0() if self.kind == GGMLQuantizationType.Q4_0 else None
            tiled = self._q8_0_tiled() if self.kind in _TILED_KINDS else None
            return fused_linear(value, self.packed, self.shape, _FUSED_KINDS[self.kind], self.bias, q8_blocks=q8,
                                q8_tiled=tiled)
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
    """Marks every PackedLinear of a fused kind for the fused path; returns how many (tools/idol_packed.py:85-94)."""
    layers = [m for m in model.modules() if isinstance(m, PackedLinear) and m.kind in _FUSED_KINDS]
    for layer in layers:
        layer.fused = True
    return len(layers)


def _replaceable(key, tensor, include_half):
    """Whether replace_quantized_linear_layers takes this source tensor: block formats always, F16 matrix weights
    with include_half."""
    if tensor.tensor_type in _BLOCK_KINDS:
        return True
    return (include_half and tensor.tensor_type == GGMLQuantizationType.F16 and len(np.asarray(tensor.shape)) == 2
            and key.endswith(".weight"))


def _target_layer(model, key, tensor):
    """The nn.Linear whose weight `key` names, with the same shape as the source tensor, or the error for it."""
    if not key.endswith(".weight"):
        raise ValueError("quantized tensor is not a linear weight: " + key)
    try:
        layer = model.get_submodule(key[:-len(".weight")])
    except AttributeError as exc:
        raise ValueError("quantized linear layer is missing: " + key) from exc
    shape = tuple(int(d) for d in reversed(np.asarray(tensor.shape).tolist()))
    if not isinstance(layer, torch.nn.Linear) or shape != tuple(layer.weight.shape):
        raise ValueError("quantized tensor does not match a linear layer: " + key)
    return layer


def replace_quantized_linear_layers(model, source, include_half=False):
    """Swaps the nn.Linear layers whose weights `source` (GGUF tensor name -> tensor) holds packed for PackedLinear
    layers on the same device, after every one of them has been checked; returns the weight names replaced (the
    interface of tools/idol_packed.py:97-129)."""
    plan = [(key, tensor, _target_layer(model, key, tensor)) for key, tensor in source.items()
            if _replaceable(key, tensor, include_half)]
    for key, tensor, layer in plan:
        parent, _, leaf = key[:-len(".weight")].rpartition(".")
        setattr(model.get_submodule(parent) if parent else model, leaf,
                PackedLinear(tensor, layer.bias).to(device=layer.weight.device))
    return [key for key, _, _ in plan]
