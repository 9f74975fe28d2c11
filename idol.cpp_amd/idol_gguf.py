"""The Idol GGUF container without gguf-py: a GGUF v2/v3 reader and writer, host dequantization, and the reference's
Idol loader on top (tools/idol_gguf.py: IdolGGUF, validate_tensor_values, validate_runtime_half_storage) plus the
decoder bridge (tools/gguf_to_decoder.py: native_blob, materialize).

The reference imports gguf-py (0.19.0 pinned in requirements-runtime.txt) for the container; gguf-py is not
available here, so the container is read with this module, which restates the published GGUF layout:
    magic "GGUF" | u32 version (2 or 3) | u64 tensor count | u64 key-value count
    key-values: string key (u64 length + UTF-8) | u32 value type | value (arrays: u32 element type, u64 count, items)
    tensor infos: string name | u32 n_dims | u64 dims[n_dims] (innermost first) | u32 ggml type | u64 data offset
    padding to `general.alignment` (default 32) | tensor data, each tensor at its offset from the data start
All integers little-endian. Tensor objects expose what the reference's code reads from gguf-py's ReaderTensor:
`name`, `shape` (dims innermost first, a numpy array), `tensor_type`, `n_elements`, `n_bytes` and `data` (a
read-only numpy view of the file: float32 / float16 / float64 / integer arrays shaped outermost first for the plain
types, uint8 [rows, bytes per row] for block formats and BF16), and fields `contents()` as gguf-py's do.
Host code only: tensors move to the GPU through PackedLinear / Decoders.
"""
import json
import os
import struct
from enum import IntEnum
from pathlib import Path

import numpy as np
import torch

import idol_export as E
import idol_kernels as K
from ggml_types import GGMLQuantizationType as Q, TYPE_SIZE

GGUF_MAGIC = b"GGUF"
DEFAULT_ALIGNMENT = 32


class GGUFValueType(IntEnum):
    UINT8 = 0
    INT8 = 1
    UINT16 = 2
    INT16 = 3
    UINT32 = 4
    INT32 = 5
    FLOAT32 = 6
    BOOL = 7
    STRING = 8
    ARRAY = 9
    UINT64 = 10
    INT64 = 11
    FLOAT64 = 12


_SCALAR = {GGUFValueType.UINT8: "<u1", GGUFValueType.INT8: "<i1", GGUFValueType.UINT16: "<u2",
           GGUFValueType.INT16: "<i2", GGUFValueType.UINT32: "<u4", GGUFValueType.INT32: "<i4",
           GGUFValueType.FLOAT32: "<f4", GGUFValueType.BOOL: "<u1", GGUFValueType.UINT64: "<u8",
           GGUFValueType.INT64: "<i8", GGUFValueType.FLOAT64: "<f8"}
_PLAIN = {Q.F32: np.float32, Q.F16: np.float16, Q.F64: np.float64, Q.I8: np.int8, Q.I16: np.int16, Q.I32: np.int32,
          Q.I64: np.int64}


class ReaderField:
    """A key-value pair: `name`, `types` (the value type, then element types for arrays) and the decoded value."""

    def __init__(self, name, types, value):
        self.name, self.types, self.value = name, types, value

    def contents(self):
        return self.value


class ReaderTensor:
    def __init__(self, name, shape, tensor_type, n_elements, n_bytes, data_offset, data):
        self.name, self.shape, self.tensor_type = name, shape, tensor_type
        self.n_elements, self.n_bytes, self.data_offset, self.data = n_elements, n_bytes, data_offset, data


class GGUFReader:
    """A GGUF file mapped read-only: `fields` (name -> ReaderField), `tensors` (list of ReaderTensor)."""

    def __init__(self, path):
        self.path = Path(path)
        self.mm = np.memmap(self.path, mode="r")
        self.pos = 0
        if self._bytes(4) != GGUF_MAGIC:
            raise ValueError("GGUF magic invalid")
        self.version = self._scalar("<u4")
        if self.version not in (2, 3):
            raise ValueError(f"unsupported GGUF version {self.version}")
        n_tensors, n_kv = self._scalar("<u8"), self._scalar("<u8")
        self.fields = {}
        for _ in range(n_kv):
            name = self._string()
            vtype = GGUFValueType(self._scalar("<u4"))
            types, value = self._value(vtype)
            if name in self.fields:
                raise KeyError(f"duplicate key {name}")
            self.fields[name] = ReaderField(name, types, value)
        align = self.fields.get("general.alignment")
        self.alignment = int(align.contents()) if align is not None else DEFAULT_ALIGNMENT
        if self.alignment <= 0 or self.alignment & (self.alignment - 1):
            raise ValueError("invalid GGUF alignment")
        infos = []
        for _ in range(n_tensors):
            name = self._string()
            n_dims = self._scalar("<u4")
            dims = np.array([self._scalar("<u8") for _ in range(n_dims)], np.uint64)
            ttype = Q(self._scalar("<u4"))
            offset = self._scalar("<u8")
            infos.append((name, dims, ttype, offset))
        self.data_start = -(-self.pos // self.alignment) * self.alignment
        self.tensors = []
        names = set()
        for name, dims, ttype, offset in infos:
            if name in names:
                raise ValueError(f"found duplicated tensor with name {name}")
            names.add(name)
            if ttype not in TYPE_SIZE:
                raise ValueError(f"unsupported GGML type {int(ttype)} for tensor {name}")
            values, size = TYPE_SIZE[ttype]
            n_el = int(np.prod(dims, dtype=np.uint64)) if len(dims) else 1
            inner = int(dims[0]) if len(dims) else 1
            if inner % values:
                raise ValueError(f"tensor {name}: innermost dimension is not a whole number of blocks")
            n_bytes = n_el // values * size
            start = self.data_start + int(offset)
            if start + n_bytes > self.mm.size:
                raise ValueError(f"tensor {name} lies outside the file")
            raw = self.mm[start:start + n_bytes]
            outer = [int(v) for v in reversed(dims.tolist())]
            if ttype in _PLAIN:
                data = raw.view(_PLAIN[ttype]).reshape(outer if outer else [1])
            else:
                rows = n_el // inner if inner else 0
                data = raw.reshape(rows, inner // values * size)
            self.tensors.append(ReaderTensor(name, dims, ttype, n_el, n_bytes, start, data))

    def get_field(self, name):
        return self.fields.get(name)

    # ---------------------------------------------------------------------------------------------------- parsing
    def _bytes(self, n):
        if self.pos + n > self.mm.size:
            raise ValueError("truncated GGUF file")
        b = self.mm[self.pos:self.pos + n].tobytes()
        self.pos += n
        return b

    def _scalar(self, fmt):
        dt = np.dtype(fmt)
        v = np.frombuffer(self._bytes(dt.itemsize), dt)[0]
        return v.item()

    def _string(self):
        return self._bytes(self._scalar("<u8")).decode("utf-8")

    def _value(self, vtype):
        if vtype == GGUFValueType.STRING:
            return [vtype], self._string()
        if vtype == GGUFValueType.ARRAY:
            etype = GGUFValueType(self._scalar("<u4"))
            count = self._scalar("<u8")
            if etype in _SCALAR:
                dt = np.dtype(_SCALAR[etype])
                arr = np.frombuffer(self._bytes(dt.itemsize * count), dt)
                vals = [bool(v) for v in arr] if etype == GGUFValueType.BOOL else arr.tolist()
                return [vtype, etype], vals
            items, sub = [], [etype]
            for _ in range(count):
                sub, v = self._value(etype)
                items.append(v)
            return [vtype] + sub, items
        v = self._scalar(_SCALAR[vtype])
        return [vtype], bool(v) if vtype == GGUFValueType.BOOL else v


# ------------------------------------------------------------------------------------------------ writing
def _pack_value(vtype, value):
    if vtype == GGUFValueType.STRING:
        raw = value.encode("utf-8")
        return struct.pack("<Q", len(raw)) + raw
    if vtype == GGUFValueType.ARRAY:
        raise ValueError("nested arrays are written with _pack_array")
    return np.array([value], dtype=_SCALAR[vtype]).tobytes()


def _infer(value):
    if isinstance(value, bool):
        return GGUFValueType.BOOL
    if isinstance(value, int):
        return GGUFValueType.INT64 if value < 0 else GGUFValueType.UINT64 if value > 0xFFFFFFFF else GGUFValueType.UINT32
    if isinstance(value, float):
        return GGUFValueType.FLOAT32
    if isinstance(value, str):
        return GGUFValueType.STRING
    if isinstance(value, (list, tuple)):
        return GGUFValueType.ARRAY
    raise ValueError(f"cannot store {type(value).__name__} in GGUF")


def write_gguf(path, fields, tensors, alignment=DEFAULT_ALIGNMENT):
    """Writes a GGUF v3 file. fields: {key: value} (int, float, bool, str, or a list of one scalar kind; a
    (GGUFValueType, value) pair forces the type). tensors: list of (name, tensor_type, shape outermost first, data),
    data the tensor's bytes (numpy array of the plain type, or uint8 blocks)."""
    kv = bytearray()
    items = dict(fields)
    if alignment != DEFAULT_ALIGNMENT:
        items["general.alignment"] = (GGUFValueType.UINT32, alignment)
    for key, value in items.items():
        vtype, v = value if isinstance(value, tuple) and isinstance(value[0], GGUFValueType) else (_infer(value), value)
        kv += _pack_value(GGUFValueType.STRING, key) + struct.pack("<I", vtype)
        if vtype == GGUFValueType.ARRAY:
            etype = _infer(v[0]) if v else GGUFValueType.UINT32
            kv += struct.pack("<IQ", etype, len(v))
            for item in v:
                kv += _pack_value(etype, item)
        else:
            kv += _pack_value(vtype, v)
    infos, blobs, offset = bytearray(), [], 0
    for name, ttype, shape, data in tensors:
        raw = np.ascontiguousarray(data).tobytes()
        values, size = TYPE_SIZE[Q(ttype)]
        n_el = int(np.prod(shape)) if len(shape) else 1
        if len(raw) != n_el // values * size or shape[-1] % values:
            raise ValueError(f"tensor {name}: {len(raw)} bytes do not match its shape and type")
        dims = list(reversed([int(d) for d in shape]))
        infos += _pack_value(GGUFValueType.STRING, name) + struct.pack("<I", len(dims))
        infos += struct.pack(f"<{len(dims)}Q", *dims) + struct.pack("<IQ", int(ttype), offset)
        blobs.append((offset, raw))
        offset = -(-(offset + len(raw)) // alignment) * alignment
    head = GGUF_MAGIC + struct.pack("<IQQ", 3, len(tensors), len(items))
    with open(path, "wb") as f:
        f.write(head + kv + infos)
        f.write(b"\0" * ((-f.tell()) % alignment))
        start = f.tell()
        for off, raw in blobs:
            f.write(b"\0" * (start + off - f.tell()))
            f.write(raw)


# ------------------------------------------------------------------------------------------------ host values
def dequantize(data, tensor_type):
    """fp32 values of a tensor's data (gguf-py's quants.dequantize semantics: plain types widened, block formats
    expanded with the reference's fp32 operations), shaped like the logical tensor, outermost first."""
    t = Q(tensor_type)
    a = np.asarray(data)
    if t in (Q.F32, Q.F16, Q.F64):
        return a.astype(np.float32)
    if t == Q.BF16:
        u = np.ascontiguousarray(a).view("<u2").astype(np.uint32) << 16
        return u.view(np.float32).reshape(a.shape[:-1] + (a.shape[-1] // 2,))
    if t in (Q.Q8_0, Q.Q4_0, Q.Q2_K, Q.Q4_K, Q.Q6_K):
        values, size = TYPE_SIZE[t]
        rows = a.shape[0] if a.ndim == 2 else 1
        row_bytes = a.size // rows
        k = row_bytes // size * values
        from idol_packed import _host_values
        out = _host_values(torch.from_numpy(np.array(a, dtype=np.uint8, copy=True).reshape(-1)), t, rows, k).numpy()
        return out.reshape(a.shape[:-1] + (k,)) if a.ndim == 2 else out.reshape(-1)
    raise NotImplementedError(f"dequantize is not implemented for {t.name}")


# ------------------------------------------------------------------------------------------------ the Idol loader
COMPONENTS = ("denoiser", "octree", "gaussian", "background")
SUPPORTED = {Q.F32, Q.F16, Q.Q8_0, Q.Q4_0, Q.Q2_K, Q.Q4_K, Q.Q6_K, Q.I8, Q.I16, Q.I32, Q.I64}
_INTEGER = {Q.I8, Q.I16, Q.I32, Q.I64}


def validate_tensor_values(tensor):
    """Numeric validity without a dequantized copy (tools/idol_gguf.py:22-49): finite scales for block formats,
    finite values for float tensors, no all-ones exponent for BF16."""
    k_formats = {Q.Q2_K: (84, (80, 82)), Q.Q4_K: (144, (0, 2)), Q.Q6_K: (210, (208,))}
    t = tensor.tensor_type
    if t in k_formats:
        size, offsets = k_formats[t]
        raw = np.asarray(tensor.data).reshape(-1, size)
        return all(np.isfinite(np.ascontiguousarray(raw[:, o:o + 2]).view("<f2")).all() for o in offsets)
    if t in (Q.Q4_0, Q.Q8_0):
        raw = np.asarray(tensor.data).reshape(-1, 18 if t == Q.Q4_0 else 34)
        return bool(np.isfinite(np.ascontiguousarray(raw[:, :2]).view("<f2")).all())
    if t == Q.BF16:
        u = np.ascontiguousarray(tensor.data).view("<u2").reshape(-1)
        return all(not np.any((u[i:i + 1_000_000] & 0x7F80) == 0x7F80) for i in range(0, u.size, 1_000_000))
    if t in (Q.F16, Q.F32):
        v = np.asarray(tensor.data).reshape(-1)
        return all(np.isfinite(v[i:i + 1_000_000]).all() for i in range(0, v.size, 1_000_000))
    return True


def validate_runtime_half_storage(model, module):
    """Fail if a runtime-aware file would downcast a float32 matrix of the module (tools/idol_gguf.py:52-111)."""
    field = model.reader.get_field("idol.quantization.tier")
    if field is None:
        return
    tier = field.contents()
    denoiser_kind, mixed = None, False
    suffixes = {"_DENOISER_Q2K_COV": (Q.Q2_K, False), "_DENOISER_Q4K_COV": (Q.Q4_K, False),
                "_DENOISER_Q6K_COV": (Q.Q6_K, False), "_DENOISER_Q80_COV": (Q.Q8_0, False),
                "_DENOISER_Q2KF16_COV": (Q.Q2_K, True), "_DENOISER_Q4KF16_COV": (Q.Q4_K, True),
                "_DENOISER_Q6KF16_COV": (Q.Q6_K, True), "_DENOISER_Q80F16_COV": (Q.Q8_0, True)}
    for suffix, (kind, is_mixed) in suffixes.items():
        if tier.endswith(suffix):
            tier, denoiser_kind, mixed = tier[:-len(suffix)], kind, is_mixed
            break
    if tier not in ("RUNTIME_F16_Q8", "RUNTIME_F16_GAUSSIAN_Q2K", "RUNTIME_F16_GAUSSIAN_Q4K",
                    "RUNTIME_F16_GAUSSIAN_Q6K", "RUNTIME_F16_GAUSSIAN_Q2K_COV", "RUNTIME_F16_GAUSSIAN_Q4K_COV",
                    "RUNTIME_F16_GAUSSIAN_Q6K_COV", "RUNTIME_F16_GAUSSIAN_Q2Q4_COV"):
        return
    expected = module.state_dict()
    checked, preserved, seen = 0, set(), set()
    if mixed:
        allocation = model.reader.get_field("idol.quantization.denoiser_preserved_blocks")
        if allocation is None:
            raise ValueError("mixed denoiser tier is missing its block allocation")
        values = json.loads(allocation.contents())
        if (not isinstance(values, list) or any(type(v) is not int or v < 0 for v in values)
                or values != sorted(set(values))):
            raise ValueError("invalid mixed denoiser block allocation")
        preserved = set(values)
    for name, tensor in model.tensors["denoiser"].items():
        if (denoiser_kind is not None and name.startswith("blocks.") and name.endswith("weight")
                and len(tensor.shape) == 2 and int(tensor.shape[0]) % 256 == 0):
            checked += 1
            parts = name.split(".")
            if mixed and (len(parts) < 3 or not parts[1].isdigit()):
                raise ValueError("invalid mixed denoiser block name: " + name)
            block = int(parts[1]) if mixed else None
            if mixed:
                seen.add(block)
            required = Q.F16 if block in preserved else denoiser_kind
            if tensor.tensor_type != required or name not in expected or expected[name].dtype != torch.float16:
                raise ValueError("encoded denoiser block is incompatible with the runtime: " + name)
        if (tensor.tensor_type == Q.F16 and len(tensor.shape) == 2
                and (name not in expected or expected[name].dtype != torch.float16)):
            raise ValueError("runtime-aware half-precision matrix is not half precision in this SDK: " + name)
    if denoiser_kind is not None and checked == 0:
        raise ValueError("encoded denoiser tier has no eligible runtime blocks")
    if mixed and (not preserved <= seen or preserved == seen):
        raise ValueError("mixed denoiser block allocation does not match the runtime")


class IdolGGUF:
    """An Idol GGUF file (tools/idol_gguf.py:114-224): `config` (the embedded JSON), `tensors[component][name]`,
    load_module and load_module_packed, with the reference's checks and messages."""

    def __init__(self, path):
        self.path = Path(path)
        self.reader = GGUFReader(self.path)
        arch = self.reader.get_field("general.architecture")
        config = self.reader.get_field("idol.config.json")
        if arch is None or arch.contents() != "idol" or config is None:
            raise ValueError("not an Idol GGUF file with an embedded configuration")
        self.config = json.loads(config.contents())
        if not all(k in self.config for k in ("denoiser", "decoder", "decoder_gs", "image_encoders")):
            raise ValueError("incomplete Idol configuration")
        self.tensors = {name: {} for name in COMPONENTS}
        for tensor in self.reader.tensors:
            parts = tensor.name.split(".", 2)
            if len(parts) != 3 or parts[0] != "idol" or parts[1] not in self.tensors or not parts[2]:
                raise ValueError("unexpected tensor in Idol GGUF: " + tensor.name)
            group = self.tensors[parts[1]]
            if parts[2] in group or tensor.tensor_type not in SUPPORTED:
                raise ValueError("duplicate tensor or unsupported GGUF encoding: " + tensor.name)
            group[parts[2]] = tensor
        if any(not values for values in self.tensors.values()):
            raise ValueError("Idol GGUF is missing a component")

    def load_module(self, component, module):
        """Every tensor of `component` expanded into `module`'s state (tools/idol_gguf.py:131-162)."""
        if component not in self.tensors:
            raise ValueError("unknown component: " + component)
        expected = module.state_dict()
        source = self.tensors[component]
        if set(expected) != set(source):
            missing, extra = sorted(set(expected) - set(source)), sorted(set(source) - set(expected))
            raise ValueError(f"{component} tensor names do not match; missing={missing}, extra={extra}")
        for name, target in expected.items():
            tensor = source[name]
            shape = tuple(reversed(tensor.shape.tolist()))
            if shape != tuple(target.shape):
                raise ValueError(f"{component}.{name} shape {shape} does not match {tuple(target.shape)}")
            if not validate_tensor_values(tensor):
                raise ValueError(f"non-finite value in {component}.{name}")
        with torch.no_grad():
            for name, target in expected.items():
                tensor = source[name]
                shape = tuple(target.shape)
                if tensor.tensor_type in _INTEGER:
                    values = np.asarray(tensor.data).reshape(shape)
                else:
                    values = dequantize(tensor.data, tensor.tensor_type).reshape(shape)
                target.copy_(torch.from_numpy(np.array(values, copy=True)))
        return module

    def load_module_packed(self, component, module, *, include_half=False):
        """A meta-initialized module loaded without expanding its packed matrices: quantized linear weights (and,
        with include_half, F16 ones) become PackedLinear layers (tools/idol_gguf.py:164-224)."""
        from accelerate.utils import set_module_tensor_to_device
        from idol_packed import PackedLinear

        if component not in self.tensors:
            raise ValueError("unknown component: " + component)
        expected, source = module.state_dict(), self.tensors[component]
        if set(expected) != set(source):
            raise ValueError(f"{component} tensor names do not match")
        packed_kinds = {Q.Q8_0, Q.Q4_0, Q.Q2_K, Q.Q4_K, Q.Q6_K}
        selected = {}
        for name, target in expected.items():
            tensor = source[name]
            if tuple(reversed(tensor.shape.tolist())) != tuple(target.shape):
                raise ValueError(f"{component}.{name} shape does not match")
            if not validate_tensor_values(tensor):
                raise ValueError(f"non-finite value in {component}.{name}")
            packed = tensor.tensor_type in packed_kinds or (
                include_half and tensor.tensor_type == Q.F16 and len(tensor.shape) == 2 and name.endswith(".weight"))
            if packed:
                if not name.endswith(".weight"):
                    raise ValueError("quantized tensor is not a linear weight: " + name)
                layer_name = name[:-7]
                try:
                    layer = module.get_submodule(layer_name)
                except AttributeError as exc:
                    raise ValueError("quantized linear layer is missing: " + name) from exc
                if not isinstance(layer, torch.nn.Linear):
                    raise ValueError("quantized tensor is not a linear weight: " + name)
                selected[layer_name] = layer
        skipped = {name + suffix for name in selected for suffix in (".weight", ".bias")}
        for name, target in expected.items():
            if name in skipped:
                continue
            tensor = source[name]
            values = (np.asarray(tensor.data) if tensor.tensor_type in _INTEGER
                      else dequantize(tensor.data, tensor.tensor_type))
            values = torch.from_numpy(np.array(values, copy=True).reshape(target.shape))
            set_module_tensor_to_device(module, name, "cpu", value=values, dtype=target.dtype)
        for name, original in selected.items():
            bias = None
            if original.bias is not None:
                tensor = source[name + ".bias"]
                values = dequantize(tensor.data, tensor.tensor_type)
                bias = torch.from_numpy(np.array(values, copy=True)).reshape(original.bias.shape).to(original.bias.dtype)
            parent_name, _, leaf = name.rpartition(".")
            parent = module.get_submodule(parent_name) if parent_name else module
            setattr(parent, leaf, PackedLinear(source[name + ".weight"], bias))
        if any(value.is_meta for value in list(module.parameters()) + list(module.buffers())):
            raise ValueError("packed module retains uninitialized tensors")
        return module


# ------------------------------------------------------------------------------------------------ decoder bridge
def native_blob(tensor):
    """The panel blob of a Q8_0 or Q4_0 GGUF matrix without re-quantizing (tools/gguf_to_decoder.py:16-40):
    code = q + 128 (8-bit) or the nibble (4-bit), scale = d, minimum = -128 d / -8 d. Returns (blob, bits, shape)."""
    shape = tuple(reversed(tensor.shape.tolist()))
    if len(shape) != 2 or shape[1] % 32:
        raise ValueError("quantized native decoder tensors must be matrices with 32-element groups")
    out, width = shape
    if tensor.tensor_type == Q.Q8_0:
        bits, block_bytes, bias = 8, 34, 128
    elif tensor.tensor_type == Q.Q4_0:
        bits, block_bytes, bias = 4, 18, 8
    else:
        raise ValueError("unsupported quantized decoder tensor")
    blocks = np.asarray(tensor.data).reshape(out, width // 32, block_bytes)
    scales = np.ascontiguousarray(blocks[:, :, :2]).view("<f2").reshape(out, -1).astype(np.float32)
    if not np.isfinite(scales).all():
        raise ValueError("non-finite GGUF scale")
    payload = np.ascontiguousarray(blocks[:, :, 2:])
    if bits == 8:
        codes = (payload.view(np.int8).astype(np.int16) + bias).astype(np.uint8).reshape(out, width)
    else:
        codes = np.concatenate((payload & 15, payload >> 4), axis=-1).reshape(out, width)
    minimum = (-bias * scales).astype(np.float16).astype(np.float32)
    if not np.isfinite(minimum).all() or not np.array_equal(minimum, -bias * scales):
        raise ValueError("GGUF scale cannot be represented exactly in native layout")
    return K.pack_panel(codes, scales, minimum, bits, 32), bits, shape


def _decoder_header(model):
    config = model.config
    oct_args, gs_args = config["decoder"]["args"], config["decoder_gs"]["args"]
    if oct_args["model_channels"] != gs_args["model_channels"] or oct_args["num_heads"] != gs_args["num_heads"]:
        raise ValueError("native decoder requires matching octree and Gaussian dimensions and heads")
    rep = gs_args["representation_config"]
    cfg = E.DecoderConfig(oct_args["model_channels"], oct_args["num_heads"], oct_args["num_blocks"],
                          gs_args["num_blocks"], oct_args["cond_channels"], rep["num_gaussians"])
    return cfg, rep


def _frequency_tables(dim):
    """The embedders' nonpersistent frequency tables, in float32 as PyTorch builds them (tools/gguf_to_decoder.py:81-87)."""
    freq_dim = dim // 3 // 2
    pos = torch.pow(2.0, torch.linspace(0.0, 10.0, steps=freq_dim, dtype=torch.float32)).numpy()
    half = 128
    levels = torch.exp(-np.log(1024) * torch.arange(0, half, dtype=torch.float32) / half).numpy()
    return pos, levels


def _rep_values(rep):
    """The `rep` record in the order the reference's bridge writes it (tools/gguf_to_decoder.py:88-91): the learning
    rates of scaling and opacity in the order (scaling, opacity), which its reader (src/weights.cpp:57-58) takes as
    (opacity, scaling). Kept as the reference has it, so both runtimes see the same values."""
    return (rep["perturbe_size"], rep["3d_filter_kernel_size"], rep["scaling_bias"], rep["opacity_bias"],
            rep["lr"]["_xyz"], rep["lr"]["_features_dc"], rep["lr"]["_scaling"], rep["lr"]["_opacity"],
            rep["lr"]["_rotation"])


def materialize(model, output):
    """Writes the native decoder export of an Idol GGUF (tools/gguf_to_decoder.py:43-91): Q8_0 and Q4_0 matrices as
    panel blobs, every other tensor expanded to fp32, the frequency tables, the `rep` record."""
    output = Path(output)
    cfg, rep = _decoder_header(model)
    header = f"decoders {cfg.dim} {cfg.heads} {cfg.oct_blocks} {cfg.gs_blocks} {cfg.cond} {cfg.per_anchor}"
    manifest = [header]
    output.mkdir(parents=True, exist_ok=False)
    with (output / "weights.bin").open("xb") as stream:
        def place(data):
            stream.write(b"\0" * ((-stream.tell()) % E.ALIGN))
            offset = stream.tell()
            stream.write(data)
            return offset

        def add_dense(name, value):
            array = np.ascontiguousarray(value, dtype="<f4")
            offset = place(array.tobytes())
            dims = " ".join(str(d) for d in value.shape)
            manifest.append(f"{name} {value.ndim} {dims} {offset} {array.nbytes}")

        for component, prefix in (("octree", "oct."), ("gaussian", "gs.")):
            for name, tensor in sorted(model.tensors[component].items()):
                shape = tuple(reversed(tensor.shape.tolist()))
                if tensor.tensor_type in (Q.Q8_0, Q.Q4_0):
                    blob, bits, shape = native_blob(tensor)
                    offset = place(blob.tobytes())
                    manifest.append(f"qtensor {prefix}{name} {shape[0]} {shape[1]} {bits} 32 {offset} {blob.size}")
                else:
                    values = dequantize(tensor.data, tensor.tensor_type).reshape(shape)
                    if not np.isfinite(values).all():
                        raise ValueError("non-finite decoder tensor: " + name)
                    add_dense(prefix + name, values)
        pos, levels = _frequency_tables(cfg.dim)
        for prefix in ("oct.", "gs."):
            add_dense(prefix + "pos_embedder.freqs", pos)
        add_dense("oct.l_embedder.freqs", levels)
    manifest.append("rep " + " ".join(str(v) for v in _rep_values(rep)))
    (output / "manifest.txt").write_text("\n".join(manifest) + "\n", encoding="ascii")


def decoder_export(model):
    """The decoders of an Idol GGUF as an in-memory export (what materialize writes and read_export reads, without
    the files): Q8_0 matrices as their GGUF blocks, Q4_0 matrices re-encoded exactly as Q8_0 blocks, every other
    tensor expanded to fp32. Decoders(decoder_export(IdolGGUF(path))) runs them on the GPU."""
    cfg, rep = _decoder_header(model)
    ex = E.Export(decoders=True, decoder_config=cfg)
    r = _rep_values(rep)
    ex.rep = E.Representation(*(float(np.float32(v)) for v in r))
    for component, prefix in (("octree", "oct."), ("gaussian", "gs.")):
        for name, tensor in sorted(model.tensors[component].items()):
            shape = tuple(reversed(tensor.shape.tolist()))
            if tensor.tensor_type in (Q.Q8_0, Q.Q4_0):
                if len(shape) != 2 or shape[1] % 32:
                    raise ValueError("quantized native decoder tensors must be matrices with 32-element groups")
                raw = np.ascontiguousarray(tensor.data).reshape(-1)
                blocks = raw.copy() if tensor.tensor_type == Q.Q8_0 else _q4_0_as_q8_0(raw)
                scales = blocks.reshape(-1, 34)[:, :2].copy().view("<f2")
                if not np.isfinite(scales).all():
                    raise ValueError("non-finite GGUF scale")
                ex.qtensors[prefix + name] = E.QTensor(shape[0], shape[1], 8, 32, blocks, kind="q8_0")
            else:
                values = dequantize(tensor.data, tensor.tensor_type).reshape(shape)
                if not np.isfinite(values).all():
                    raise ValueError("non-finite decoder tensor: " + name)
                ex.tensors[prefix + name] = E.Tensor(list(shape), np.ascontiguousarray(values, np.float32).reshape(-1))
    pos, levels = _frequency_tables(cfg.dim)
    for prefix in ("oct.", "gs."):
        ex.tensors[prefix + "pos_embedder.freqs"] = E.Tensor([pos.size], pos.astype(np.float32))
    ex.tensors["oct.l_embedder.freqs"] = E.Tensor([levels.size], levels.astype(np.float32))
    return ex


def _q4_0_as_q8_0(raw):
    """Q8_0 blocks holding exactly the values of Q4_0 blocks (same fp16 scale, codes q - 8), on the host."""
    b4 = raw.reshape(-1, 18)
    out = np.empty((b4.shape[0], 34), np.uint8)
    out[:, :2] = b4[:, :2]
    q = np.concatenate([b4[:, 2:] & 15, b4[:, 2:] >> 4], axis=1).astype(np.int16) - 8
    out[:, 2:] = q.astype(np.int8).view(np.uint8)
    return out.reshape(-1)
