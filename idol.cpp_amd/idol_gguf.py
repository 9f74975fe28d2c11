"""The Idol GGUF container without gguf-py: a GGUF v2/v3 reader and writer, host dequantization, the Idol loader on
top (the surface of tools/idol_gguf.py:22-49,114-224: IdolGGUF, validate_tensor_values, load_module,
load_module_packed) and the decoder bridge (the surface of tools/gguf_to_decoder.py:16-91: native_blob,
materialize), each written from its accept/reject cases and messages.

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
import dataclasses
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
# An Idol GGUF names every tensor idol.<component>.<state-dict key>; the embedded JSON configuration holds the four
# model sections. What is accepted and the messages of what is not are the reference loader's
# (tools/idol_gguf.py:22-49,114-224); the code below is organized around two tables: the encodings a file may use,
# and for block formats where each block keeps its fp16 scales.
COMPONENTS = ("denoiser", "octree", "gaussian", "background")
CONFIG_SECTIONS = ("denoiser", "decoder", "decoder_gs", "image_encoders")
_INTEGER = frozenset({Q.I8, Q.I16, Q.I32, Q.I64})
_FLOAT = frozenset({Q.F32, Q.F16})
_BLOCK = frozenset({Q.Q8_0, Q.Q4_0, Q.Q2_K, Q.Q4_K, Q.Q6_K})
SUPPORTED = _INTEGER | _FLOAT | _BLOCK
# block bytes, and the byte offsets of its fp16 scale fields (d, and dmin where the format has one)
_SCALE_FIELDS = {Q.Q8_0: (34, (0,)), Q.Q4_0: (18, (0,)), Q.Q2_K: (84, (80, 82)), Q.Q4_K: (144, (0, 2)),
                 Q.Q6_K: (210, (208,))}
_CHUNK = 1 << 20  # values per finiteness check (bounded temporaries on large tensors)


def _all_finite(values):
    flat = np.asarray(values).reshape(-1)
    return all(bool(np.isfinite(flat[i:i + _CHUNK]).all()) for i in range(0, flat.size, _CHUNK))


def validate_tensor_values(tensor):
    """True when a tensor holds no inf or NaN, checked without expanding it: the fp16 scale fields of every block of
    a block format, the values of F16 / F32 tensors, the exponent fields of BF16 (all ones = inf or NaN). Integer
    tensors are always valid."""
    t = tensor.tensor_type
    if t in _SCALE_FIELDS:
        size, offsets = _SCALE_FIELDS[t]
        blocks = np.asarray(tensor.data).reshape(-1, size)
        return all(_all_finite(np.ascontiguousarray(blocks[:, o:o + 2]).view("<f2")) for o in offsets)
    if t in _FLOAT:
        return _all_finite(tensor.data)
    if t == Q.BF16:
        bits = np.ascontiguousarray(tensor.data).view("<u2").reshape(-1)
        return all(not bool(((bits[i:i + _CHUNK] & 0x7F80) == 0x7F80).any()) for i in range(0, bits.size, _CHUNK))
    return True


def _logical_shape(tensor):
    """The PyTorch shape of a GGUF tensor (GGUF lists dimensions innermost first)."""
    return tuple(int(d) for d in reversed(np.asarray(tensor.shape).tolist()))


def _host_array(tensor, shape):
    """The tensor's values as a fresh host array of `shape`: integers as stored, everything else expanded to fp32."""
    if tensor.tensor_type in _INTEGER:
        values = np.asarray(tensor.data)
    else:
        values = dequantize(tensor.data, tensor.tensor_type)
    return np.array(values, copy=True).reshape(shape)


class IdolGGUF:
    """An Idol GGUF file: `config` (the embedded JSON), `tensors[component][state-dict key]` (reader tensors), and
    load_module / load_module_packed to fill a module of one component."""

    def __init__(self, path):
        self.path = Path(path)
        self.reader = GGUFReader(self.path)
        fields = {key: self.reader.get_field(key) for key in ("general.architecture", "idol.config.json")}
        if fields["idol.config.json"] is None or fields["general.architecture"] is None \
                or fields["general.architecture"].contents() != "idol":
            raise ValueError("not an Idol GGUF file with an embedded configuration")
        self.config = json.loads(fields["idol.config.json"].contents())
        if any(section not in self.config for section in CONFIG_SECTIONS):
            raise ValueError("incomplete Idol configuration")
        self.tensors = {component: {} for component in COMPONENTS}
        for tensor in self.reader.tensors:
            prefix, _, rest = tensor.name.partition(".")
            component, _, key = rest.partition(".")
            if prefix != "idol" or component not in self.tensors or not key:
                raise ValueError("unexpected tensor in Idol GGUF: " + tensor.name)
            held = self.tensors[component]
            if key in held or tensor.tensor_type not in SUPPORTED:
                raise ValueError("duplicate tensor or unsupported GGUF encoding: " + tensor.name)
            held[key] = tensor
        if not all(self.tensors.values()):
            raise ValueError("Idol GGUF is missing a component")

    # -------------------------------------------------------------------------------------------- shared checks
    def _source(self, component):
        if component not in self.tensors:
            raise ValueError("unknown component: " + component)
        return self.tensors[component]

    def _check_mapping(self, component, source, expected, detailed):
        """Same keys on both sides, equal shapes, finite values; `detailed` adds the lists and shapes to the messages
        (load_module's form) where load_module_packed's messages are shorter."""
        if set(source) != set(expected):
            message = f"{component} tensor names do not match"
            if detailed:
                missing, extra = sorted(set(expected) - set(source)), sorted(set(source) - set(expected))
                message += f"; missing={missing}, extra={extra}"
            raise ValueError(message)
        for key, target in expected.items():
            tensor, want = source[key], tuple(target.shape)
            got = _logical_shape(tensor)
            if got != want:
                raise ValueError(f"{component}.{key} shape {got} does not match {want}" if detailed
                                 else f"{component}.{key} shape does not match")
            if not validate_tensor_values(tensor):
                raise ValueError(f"non-finite value in {component}.{key}")

    # -------------------------------------------------------------------------------------------- loaders
    def load_module(self, component, module):
        """Every tensor of `component` expanded to its values and copied into `module` (all checks first)."""
        source = self._source(component)
        state = module.state_dict()
        self._check_mapping(component, source, state, detailed=True)
        values = {key: _host_array(source[key], tuple(target.shape)) for key, target in state.items()}
        with torch.no_grad():
            for key, target in state.items():
                target.copy_(torch.from_numpy(values[key]))
        return module

    def load_module_packed(self, component, module, *, include_half=False):
        """A module built on the meta device, filled without expanding its packed matrices: every block-format linear
        weight (and, with include_half, every F16 matrix weight) becomes a PackedLinear holding the file's bytes;
        the other tensors are materialized on the host."""
        from accelerate.utils import set_module_tensor_to_device
        from idol_packed import PackedLinear

        source = self._source(component)
        state = module.state_dict()
        self._check_mapping(component, source, state, detailed=False)
        layers = {}
        for key in state:
            tensor = source[key]
            if not _packs(key, tensor, include_half):
                continue
            owner = key[:-len(".weight")] if key.endswith(".weight") else None
            layer = _linear_at(module, owner, key)
            layers[owner] = layer
        packed_keys = {owner + suffix for owner in layers for suffix in (".weight", ".bias")}
        for key, target in state.items():
            if key not in packed_keys:
                set_module_tensor_to_device(module, key, "cpu", dtype=target.dtype,
                                            value=torch.from_numpy(_host_array(source[key], tuple(target.shape))))
        for owner, layer in layers.items():
            bias = None
            if layer.bias is not None:
                bias = torch.from_numpy(_host_array(source[owner + ".bias"], tuple(layer.bias.shape)))
                bias = bias.to(layer.bias.dtype)
            parent, _, leaf = owner.rpartition(".")
            setattr(module.get_submodule(parent) if parent else module, leaf,
                    PackedLinear(source[owner + ".weight"], bias))
        if any(t.is_meta for t in list(module.parameters()) + list(module.buffers())):
            raise ValueError("packed module retains uninitialized tensors")
        return module


def _packs(key, tensor, include_half):
    """Whether load_module_packed keeps this tensor packed."""
    if tensor.tensor_type in _BLOCK:
        return True
    return (include_half and tensor.tensor_type == Q.F16 and len(np.asarray(tensor.shape)) == 2
            and key.endswith(".weight"))


def _linear_at(module, owner, key):
    """The nn.Linear a packed weight belongs to, or the reference loader's error for it."""
    if owner is None:
        raise ValueError("quantized tensor is not a linear weight: " + key)
    try:
        layer = module.get_submodule(owner)
    except AttributeError as exc:
        raise ValueError("quantized linear layer is missing: " + key) from exc
    if not isinstance(layer, torch.nn.Linear):
        raise ValueError("quantized tensor is not a linear weight: " + key)
    return layer


# ------------------------------------------------------------------------------------------------ decoder bridge
# The native decoders (src/decoders.cpp) read a manifest + weights.bin export. From an Idol GGUF, the octree and
# Gaussian components become that export: Q8_0 and Q4_0 matrices keep their exact values (as panels on disk, as
# Q8_0 blocks in memory), every other tensor is expanded to fp32, and the frequency tables and the `rep` record of
# the configuration are added (the surface of tools/gguf_to_decoder.py:16-91).
_DECODER_PARTS = (("octree", "oct."), ("gaussian", "gs."))


def _q8_0_blocks(tensor):
    """(blocks uint8 [rows, k / 32, 34], rows, k) of a Q8_0 or Q4_0 matrix as exact Q8_0 blocks: Q4_0's value
    d * (nibble - 8) is the Q8_0 block with the same d and code nibble - 8. Rejects other shapes and inf / NaN
    scales."""
    shape = _logical_shape(tensor)
    if len(shape) != 2 or shape[1] % 32:
        raise ValueError("quantized native decoder tensors must be matrices with 32-element groups")
    rows, k = shape
    raw = np.ascontiguousarray(tensor.data).reshape(-1)
    if tensor.tensor_type == Q.Q8_0:
        blocks = raw.reshape(rows, k // 32, 34).copy()
    elif tensor.tensor_type == Q.Q4_0:
        blocks = _q4_0_as_q8_0(raw).reshape(rows, k // 32, 34)
    else:
        raise ValueError("unsupported quantized decoder tensor")
    if not _all_finite(np.ascontiguousarray(blocks[:, :, :2]).view("<f2")):
        raise ValueError("non-finite GGUF scale")
    return blocks, rows, k


def _q4_0_as_q8_0(raw):
    """Q8_0 blocks with the values of Q4_0 blocks (18 bytes: fp16 d, 16 bytes of nibbles, low nibbles first)."""
    q4 = np.asarray(raw, np.uint8).reshape(-1, 18)
    nibbles = np.concatenate([q4[:, 2:] & 0x0F, q4[:, 2:] >> 4], axis=1)
    q8 = np.empty((q4.shape[0], 34), np.uint8)
    q8[:, :2] = q4[:, :2]
    q8[:, 2:] = (nibbles.astype(np.int8) - np.int8(8)).view(np.uint8)
    return q8.reshape(-1)


def native_blob(tensor):
    """(panel blob, bits, (rows, k)) holding a Q8_0 (8 bits) or Q4_0 (4 bits) matrix's values without re-quantizing:
    per 32-group scale = d and minimum = -2^(bits-1) d, code = q + 2^(bits-1). The minimum must be an exact fp16."""
    blocks, rows, k = _q8_0_blocks(tensor)
    bits = 8 if tensor.tensor_type == Q.Q8_0 else 4
    offset = 1 << (bits - 1)
    d = np.ascontiguousarray(blocks[:, :, :2]).view("<f2")[..., 0].astype(np.float32)
    codes = (blocks[:, :, 2:].view(np.int8).astype(np.int16) + offset).astype(np.uint8).reshape(rows, k)
    minimum = np.float32(-offset) * d
    if not np.array_equal(minimum.astype(np.float16).astype(np.float32), minimum):
        raise ValueError("GGUF scale cannot be represented exactly in native layout")
    return K.pack_panel(codes, d, minimum, bits, 32), bits, (rows, k)


def _decoder_config(model):
    """The export header and the Gaussian representation section of the configuration."""
    octree, gaussian = model.config["decoder"]["args"], model.config["decoder_gs"]["args"]
    if (octree["model_channels"], octree["num_heads"]) != (gaussian["model_channels"], gaussian["num_heads"]):
        raise ValueError("native decoder requires matching octree and Gaussian dimensions and heads")
    rep = gaussian["representation_config"]
    header = E.DecoderConfig(octree["model_channels"], octree["num_heads"], octree["num_blocks"],
                             gaussian["num_blocks"], octree["cond_channels"], rep["num_gaussians"])
    return header, rep


def _representation(rep):
    """The `rep` record the bridge writes. Its scaling and opacity learning rates land in the reader's opacity and
    scaling slots respectively (tools/gguf_to_decoder.py:88-91 against src/weights.cpp:57-58); kept so that this
    build and the reference read the same numbers from the same export."""
    lr = rep["lr"]
    return E.Representation(rep["perturbe_size"], rep["3d_filter_kernel_size"], rep["scaling_bias"],
                            rep["opacity_bias"], lr["_xyz"], lr["_features_dc"], lr["_scaling"], lr["_opacity"],
                            lr["_rotation"])


def _frequencies(dim):
    """The position embedders' frequencies 2^linspace(0, 10, dim / 6) and the level embedder's
    exp(-ln(1024) i / 128), i < 128, in fp32 as PyTorch computes them (the modules' non-persistent buffers)."""
    position = torch.pow(2.0, torch.linspace(0.0, 10.0, steps=dim // 3 // 2, dtype=torch.float32))
    level = torch.exp(-np.log(1024) * torch.arange(0, 128, dtype=torch.float32) / 128)
    return {"oct.pos_embedder.freqs": position.numpy(), "gs.pos_embedder.freqs": position.numpy(),
            "oct.l_embedder.freqs": level.numpy()}


def _decoder_tensors(model):
    """(export name, tensor) of the octree and Gaussian components, each component in key order."""
    for component, prefix in _DECODER_PARTS:
        for key in sorted(model.tensors[component]):
            yield prefix + key, model.tensors[component][key]


def _dense_values(name, tensor):
    values = _host_array(tensor, _logical_shape(tensor)).astype(np.float32)
    if not _all_finite(values):
        raise ValueError("non-finite decoder tensor: " + name.split(".", 1)[1])
    return values


def materialize(model, output):
    """Writes the native decoder export of an Idol GGUF to the new directory `output` (FileExistsError if it exists):
    Q8_0 / Q4_0 matrices as panel blobs (native_blob), the rest as fp32."""
    header, rep = _decoder_config(model)
    dense, panels = {}, {}
    for name, tensor in _decoder_tensors(model):
        if tensor.tensor_type in (Q.Q8_0, Q.Q4_0):
            blob, bits, (rows, k) = native_blob(tensor)
            panels[name] = E.QTensor(rows, k, bits, 32, blob)
        else:
            dense[name] = _dense_values(name, tensor)
    dense.update(_frequencies(header.dim))
    E.write_export(output, header, dense, panels, rep=_representation(rep))


def decoder_export(model):
    """The export materialize writes, in memory: Q8_0 / Q4_0 matrices as exact Q8_0 blocks, the rest fp32.
    Decoders(decoder_export(IdolGGUF(path))) runs a GGUF's decoders without writing files."""
    header, rep = _decoder_config(model)
    ex = E.Export(decoders=True, decoder_config=header)
    r = _representation(rep)
    ex.rep = E.Representation(*(float(np.float32(v)) for v in dataclasses.astuple(r)))
    for name, tensor in _decoder_tensors(model):
        if tensor.tensor_type in (Q.Q8_0, Q.Q4_0):
            blocks, rows, k = _q8_0_blocks(tensor)
            ex.qtensors[name] = E.QTensor(rows, k, 8, 32, blocks.reshape(-1), kind="q8_0")
        else:
            values = _dense_values(name, tensor)
            ex.tensors[name] = E.Tensor(list(values.shape), np.ascontiguousarray(values).reshape(-1))
    for name, values in _frequencies(header.dim).items():
        ex.tensors[name] = E.Tensor([values.size], values.astype(np.float32))
    return ex
