"""The native decoder export: a directory holding manifest.txt and weights.bin (src/weights.cpp:25-121, written by
tools/gguf_to_decoder.py:43-91 and tools/export_idol.py).

manifest.txt, one record per line:
    decoders <dim> <heads> <oct_blocks> <gs_blocks> <cond> <per_anchor>     (first line)
    rep <perturbe> <kernel> <scaling_bias> <opacity_bias> <lr_xyz> <lr_dc> <lr_opacity> <lr_scaling> <lr_rotation>
    case <anchors> <latent> <level>
    qtensor <name> <out> <in> <bits> <group> <offset> <nbytes>             (a panel blob, src/kernels.hpp:33-51)
    <name> <ndim> <dims...> <offset> <nbytes>                               (little-endian fp32)
weights.bin holds the payloads at the byte offsets given (the writers align them to 64 bytes).

The reader accepts and rejects what the reference's read_export does, with the same messages (RuntimeError for its
std::runtime_error); take_qtensor / take_tensor mirror its src/weights.cpp:107-127. Host-side file parsing only:
the tensors are numpy arrays until a decoder moves them to the GPU.
"""
import os
from dataclasses import dataclass, field

import numpy as np

ALIGN = 64  # payload alignment the reference's writers use (tools/idolq.py:21)


@dataclass
class DecoderConfig:
    """The decoders' shape (include/idol/decoders.hpp:13-20)."""
    dim: int = 0
    heads: int = 0
    oct_blocks: int = 0
    gs_blocks: int = 0
    cond: int = 0
    per_anchor: int = 0


def _f32(v):
    return float(np.float32(v))


@dataclass
class Representation:
    """How raw Gaussian features become Gaussians (src/weights.hpp:24-28), with the reference's float defaults."""
    perturbe: float = _f32(1.5)
    kernel: float = _f32(0.0009)
    scaling_bias: float = _f32(0.004)
    opacity_bias: float = _f32(0.1)
    lr_xyz: float = _f32(1.0)
    lr_dc: float = _f32(1.0)
    lr_opacity: float = _f32(1.0)
    lr_scaling: float = _f32(1.0)
    lr_rotation: float = _f32(0.1)


@dataclass
class Tensor:
    shape: list
    data: np.ndarray  # fp32, flat


@dataclass
class QTensor:
    """A quantized weight matrix: a panel blob as manifest.txt records it (kind "panel"), or, for exports built in
    memory from GGUF tensors, the GGUF Q8_0 blocks themselves (kind "q8_0", bits 8, group 32)."""
    out: int
    in_: int
    bits: int
    group: int
    blob: object  # uint8 array (numpy, or a torch tensor for in-memory Q8_0 blocks)
    kind: str = "panel"


@dataclass
class Export:
    decoders: bool = False
    decoder_config: DecoderConfig = field(default_factory=DecoderConfig)
    rep: Representation = field(default_factory=Representation)
    case_anchors: int = 0
    case_latent: int = 0
    case_level: int = 0
    tensors: dict = field(default_factory=dict)
    qtensors: dict = field(default_factory=dict)


def _fail(message):
    raise RuntimeError(message)


class _Fields:
    """Whitespace-separated fields read in order, like an istringstream: a failed read marks the row bad."""

    def __init__(self, line):
        self.items = line.split()
        self.pos = 0
        self.ok = True

    def _next(self, conv):
        if not self.ok or self.pos >= len(self.items):
            self.ok = False
            return conv("0") if conv is not str else ""
        tok = self.items[self.pos]
        self.pos += 1
        try:
            return conv(tok)
        except ValueError:
            self.ok = False
            return conv("0") if conv is not str else ""

    def word(self):
        return self._next(str)

    def int(self):
        return self._next(int)

    def float(self):
        return self._next(_f32)


def read_export(path):
    """Reads path/manifest.txt and path/weights.bin (src/weights.cpp:25-105)."""
    d = str(path)
    try:
        with open(os.path.join(d, "manifest.txt"), "rb") as f:
            text = f.read().decode("latin-1")
    except OSError:
        _fail(f"cannot open {d}/manifest.txt")
    lines = text.split("\n")
    if text == "":
        _fail(f"{d}/manifest.txt is empty")
    ex = Export()
    head = _Fields(lines[0])
    tag = head.word()
    c = ex.decoder_config
    c.dim, c.heads, c.oct_blocks, c.gs_blocks, c.cond, c.per_anchor = (head.int() for _ in range(6))
    if not head.ok or tag != "decoders":
        _fail(f"{d}/manifest.txt: the first line must be 'decoders dim heads oct gs cond per_anchor'")
    ex.decoders = True

    try:
        bin_file = open(os.path.join(d, "weights.bin"), "rb")
    except OSError:
        _fail(f"cannot open {d}/weights.bin")
    with bin_file:
        bin_file.seek(0, os.SEEK_END)
        file_bytes = bin_file.tell()

        def read_at(offset, nbytes):
            bin_file.seek(offset)
            return bin_file.read(nbytes)

        for line in lines[1:] if len(lines) > 1 else []:
            if line.endswith("\r"):
                line = line[:-1]
            if not line:
                continue
            row = _Fields(line)
            name = row.word()
            if name == "rep":
                r = ex.rep
                vals = [row.float() for _ in range(9)]
                if not row.ok:
                    _fail("malformed rep line in manifest.txt")
                (r.perturbe, r.kernel, r.scaling_bias, r.opacity_bias, r.lr_xyz, r.lr_dc, r.lr_opacity, r.lr_scaling,
                 r.lr_rotation) = vals
                continue
            if name == "case":
                vals = [row.int() for _ in range(3)]
                if not row.ok:
                    _fail("malformed case line in manifest.txt")
                ex.case_anchors, ex.case_latent, ex.case_level = vals
                continue
            if name == "qtensor":
                name = row.word()
                out, in_, bits, group, offset, nbytes = (row.int() for _ in range(6))
                if not row.ok or not name:
                    _fail("malformed qtensor line in manifest.txt")
                if offset < 0 or nbytes < 0 or offset + nbytes > file_bytes:
                    _fail(f"qtensor '{name}' lies outside weights.bin")
                raw = read_at(offset, nbytes)
                if len(raw) != nbytes:
                    _fail(f"short read for qtensor '{name}'")
                ex.qtensors[name] = QTensor(out, in_, bits, group, np.frombuffer(raw, np.uint8).copy())
                continue
            ndim = row.int()
            shape = [row.int() for _ in range(max(ndim, 0))]
            offset, nbytes = row.int(), row.int()
            if not row.ok or not name or ndim < 0:
                _fail(f"malformed manifest.txt line for '{name}'")
            count = 1
            for dim in shape:
                if dim < 0:
                    _fail("negative dimension in manifest.txt")
                count *= dim
            if nbytes != count * 4:
                _fail(f"tensor '{name}' has a byte count that does not match its shape")
            if offset < 0 or offset + nbytes > file_bytes:
                _fail(f"tensor '{name}' lies outside weights.bin")
            raw = read_at(offset, nbytes)
            if len(raw) != nbytes:
                _fail(f"short read for tensor '{name}'")
            ex.tensors[name] = Tensor(shape, np.frombuffer(raw, "<f4").astype(np.float32))
    return ex


def take_qtensor(ex, name):
    """Moves the named quantized matrix out of ex; None if the export holds it as fp32 (src/weights.cpp:107-113)."""
    return ex.qtensors.pop(name, None)


def take_tensor(ex, name, expected_count):
    """Moves the named tensor out of ex; RuntimeError if it is missing or holds another count (src/weights.cpp:115-125)."""
    t = ex.tensors.get(name)
    if t is None:
        _fail(f"missing tensor '{name}'")
    if t.data.size != expected_count:
        _fail(f"tensor '{name}' has {t.data.size} values, expected {expected_count}")
    del ex.tensors[name]
    return t


def write_export(path, config, tensors, qtensors=None, rep=None, case=None):
    """Writes an export directory the reader (and the reference's) loads: config a DecoderConfig, tensors
    {name: fp32 array}, qtensors {name: QTensor}, rep a Representation, case (anchors, latent, level) or None.
    Payloads are placed in the order given, each aligned to 64 bytes (tools/gguf_to_decoder.py:53-58)."""
    os.makedirs(path, exist_ok=False)
    c = config
    manifest = [f"decoders {c.dim} {c.heads} {c.oct_blocks} {c.gs_blocks} {c.cond} {c.per_anchor}"]
    with open(os.path.join(path, "weights.bin"), "xb") as f:
        def place(data):
            f.write(b"\0" * ((-f.tell()) % ALIGN))
            offset = f.tell()
            f.write(data)
            return offset

        for name, q in (qtensors or {}).items():
            blob = np.ascontiguousarray(q.blob, np.uint8).tobytes()
            manifest.append(f"qtensor {name} {q.out} {q.in_} {q.bits} {q.group} {place(blob)} {len(blob)}")
        for name, value in tensors.items():
            arr = np.ascontiguousarray(value, dtype="<f4")
            dims = " ".join(str(int(v)) for v in arr.shape)
            manifest.append(f"{name} {arr.ndim} {dims} {place(arr.tobytes())} {arr.nbytes}")
    if rep is not None:
        r = rep
        manifest.append("rep " + " ".join(repr(float(v)) for v in (
            r.perturbe, r.kernel, r.scaling_bias, r.opacity_bias, r.lr_xyz, r.lr_dc, r.lr_opacity, r.lr_scaling,
            r.lr_rotation)))
    if case is not None:
        manifest.append("case " + " ".join(str(int(v)) for v in case))
    with open(os.path.join(path, "manifest.txt"), "w", encoding="ascii") as f:
        f.write("\n".join(manifest) + "\n")
