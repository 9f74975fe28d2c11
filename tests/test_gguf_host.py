"""The GGUF container and the Idol loader on the CPU: a hand-assembled file (bytes packed here, independently of the
writer) pins the reader to the published layout; writer/reader round trips over every type; the reference loader's
checks and messages (tools/idol_gguf.py); load_module / load_module_packed; and the decoder bridge, whose export the
reference's own loader reads (tools/gguf_to_decoder.py)."""
import json
import struct

import numpy as np
import pytest
import torch

import idol_export as E
import idol_gguf as G
import oracle as O
from decoders import Decoders
from ggml_types import GGMLQuantizationType as Q
from gguf_fixture import write_idol_gguf
from idol_packed import PackedLinear


def _s(text):
    raw = text.encode()
    return struct.pack("<Q", len(raw)) + raw


def test_reader_parses_a_hand_assembled_file(tmp_path):
    f32 = np.arange(6, dtype=np.float32).reshape(2, 3)
    q8 = O.q8_0_quantize(np.linspace(-1, 1, 4 * 32, dtype=np.float32).reshape(4, 32))
    kv = (_s("general.architecture") + struct.pack("<I", 8) + _s("idol")
          + _s("n") + struct.pack("<I", 4) + struct.pack("<I", 77)
          + _s("f") + struct.pack("<I", 6) + struct.pack("<f", 0.5)
          + _s("ok") + struct.pack("<I", 7) + b"\x01"
          + _s("names") + struct.pack("<I", 9) + struct.pack("<IQ", 8, 2) + _s("a") + _s("bc")
          + _s("ints") + struct.pack("<I", 9) + struct.pack("<IQ", 5, 3) + struct.pack("<3i", -1, 0, 5))
    infos = (_s("t.f32") + struct.pack("<I", 2) + struct.pack("<2Q", 3, 2) + struct.pack("<IQ", 0, 0)
             + _s("t.q8") + struct.pack("<I", 2) + struct.pack("<2Q", 32, 4) + struct.pack("<IQ", 8, 32))
    head = b"GGUF" + struct.pack("<IQQ", 3, 2, 6)
    body = head + kv + infos
    body += b"\0" * ((-len(body)) % 32)
    data_start = len(body)
    body += f32.tobytes() + b"\0" * 8 + q8.tobytes()  # second tensor at offset 32
    (tmp_path / "h.gguf").write_bytes(body)
    r = G.GGUFReader(tmp_path / "h.gguf")
    assert r.version == 3 and r.alignment == 32 and r.data_start == data_start
    assert r.get_field("general.architecture").contents() == "idol"
    assert r.get_field("n").contents() == 77 and r.get_field("f").contents() == 0.5
    assert r.get_field("ok").contents() is True
    assert r.get_field("names").contents() == ["a", "bc"] and r.get_field("ints").contents() == [-1, 0, 5]
    t0, t1 = r.tensors
    assert t0.name == "t.f32" and t0.tensor_type == Q.F32 and t0.shape.tolist() == [3, 2]
    assert np.array_equal(t0.data, f32) and t0.data_offset == data_start
    assert t1.tensor_type == Q.Q8_0 and t1.shape.tolist() == [32, 4] and t1.data.shape == (4, 34)
    assert np.array_equal(np.asarray(t1.data).reshape(-1), q8) and t1.data_offset == data_start + 32
    assert np.array_equal(G.dequantize(t1.data, t1.tensor_type), O.q8_0_dequant(q8, 4, 32))
    (tmp_path / "bad.gguf").write_bytes(b"GGUF" + struct.pack("<IQQ", 9, 0, 0))
    with pytest.raises(ValueError, match="version"):
        G.GGUFReader(tmp_path / "bad.gguf")
    (tmp_path / "bad2.gguf").write_bytes(b"GGML" + body[4:])
    with pytest.raises(ValueError, match="magic"):
        G.GGUFReader(tmp_path / "bad2.gguf")


def test_writer_reader_round_trip_over_every_type(tmp_path):
    rng = np.random.default_rng(2)
    w = rng.normal(0, 0.3, (8, 256)).astype(np.float32)
    kq = {Q.Q2_K: 84, Q.Q4_K: 144, Q.Q6_K: 210}
    tensors = [("a", Q.F32, (3, 5), rng.standard_normal((3, 5)).astype(np.float32)),
               ("b", Q.F16, (4,), rng.standard_normal(4).astype(np.float16)),
               ("c", Q.BF16, (2, 8), (rng.integers(0, 2 ** 15, (2, 8)) & 0x3FFF).astype(np.uint16)),
               ("d", Q.I32, (7,), np.arange(7, dtype=np.int32)),
               ("e", Q.Q8_0, (8, 256), O.q8_0_quantize(w)),
               ("f", Q.Q4_0, (8, 256), O.q4_0_quantize(w))]
    for t, size in kq.items():
        raw = rng.integers(0, 256, (8, size), dtype=np.uint8)
        raw[:, -4 if t == Q.Q2_K else 0:(None if t == Q.Q2_K else 4)] = 0
        if t == Q.Q6_K:
            raw[:, 208:210] = np.array([np.float16(0.01)]).view(np.uint8)
        tensors.append((f"k{int(t)}", t, (8, 256), raw))
    fields = {"s": "x", "u": 5, "neg": -3, "big": 2 ** 40, "fl": 1.5, "bo": False, "arr": [1, 2, 3], "sarr": ["p"]}
    G.write_gguf(tmp_path / "r.gguf", fields, tensors, alignment=64)
    r = G.GGUFReader(tmp_path / "r.gguf")
    assert r.alignment == 64
    for key, value in fields.items():
        assert r.get_field(key).contents() == value
    by = {t.name: t for t in r.tensors}
    for name, ttype, shape, data in tensors:
        t = by[name]
        assert t.tensor_type == ttype and tuple(reversed(t.shape.tolist())) == tuple(shape)
        assert np.asarray(t.data).tobytes() == np.ascontiguousarray(data).tobytes()
        assert t.data_offset % 64 == 0
    bf = G.dequantize(by["c"].data, Q.BF16)
    assert bf.shape == (2, 8) and np.array_equal(bf.view(np.uint32) >> 16, tensors[2][3].astype(np.uint32))
    for t in (Q.Q4_0, Q.Q2_K, Q.Q4_K, Q.Q6_K):
        name = {Q.Q4_0: "f"}.get(t, f"k{int(t)}")
        got = G.dequantize(by[name].data, t)
        assert np.array_equal(got, O.blocks_values(np.asarray(by[name].data).reshape(-1), int(t), 8, 256))


def test_idol_gguf_checks_match_the_reference(tmp_path):
    write_idol_gguf(tmp_path / "ok.gguf")
    m = G.IdolGGUF(tmp_path / "ok.gguf")
    assert set(m.tensors) == set(G.COMPONENTS) and "in_proj.weight" in m.tensors["octree"]
    assert m.config["decoder"]["args"]["model_channels"] == 64
    G.write_gguf(tmp_path / "a.gguf", {"general.architecture": "llama", "idol.config.json": "{}"}, [])
    with pytest.raises(ValueError, match="not an Idol GGUF file with an embedded configuration"):
        G.IdolGGUF(tmp_path / "a.gguf")
    G.write_gguf(tmp_path / "b.gguf", {"general.architecture": "idol", "idol.config.json": json.dumps({"decoder": 1})}, [])
    with pytest.raises(ValueError, match="incomplete Idol configuration"):
        G.IdolGGUF(tmp_path / "b.gguf")
    cfg = json.dumps({"denoiser": {}, "decoder": {}, "decoder_gs": {}, "image_encoders": {}})
    one = np.zeros((1, 32), np.float32)
    cases = [([("other.octree.x", Q.F32, (1, 32), one)], "unexpected tensor in Idol GGUF: other.octree.x"),
             ([("idol.octree.x", Q.F32, (1, 32), one), ("idol.octree.x", Q.F32, (1, 32), one)], "duplicated"),
             ([("idol.octree.x", Q.Q5_0, (1, 32), np.zeros(22, np.uint8))], "duplicate tensor or unsupported GGUF encoding"),
             ([("idol.octree.x", Q.F32, (1, 32), one)], "Idol GGUF is missing a component")]
    for i, (tensors, message) in enumerate(cases):
        G.write_gguf(tmp_path / f"c{i}.gguf", {"general.architecture": "idol", "idol.config.json": cfg}, tensors)
        with pytest.raises(ValueError, match=message):
            G.IdolGGUF(tmp_path / f"c{i}.gguf")


class _Tiny(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.proj = torch.nn.Linear(64, 48)
        self.norm = torch.nn.LayerNorm(48)
        self.head = torch.nn.Linear(48, 8)


def _tiny_gguf(path, quant=Q.Q8_0, bad=None):
    rng = np.random.default_rng(4)
    w = rng.normal(0, 0.2, (48, 64)).astype(np.float32)
    data = O.q8_0_quantize(w) if quant == Q.Q8_0 else O.q4_0_quantize(w)
    t = [("idol.denoiser.proj.weight", quant, (48, 64), data),
         ("idol.denoiser.proj.bias", Q.F32, (48,), rng.standard_normal(48).astype(np.float32)),
         ("idol.denoiser.norm.weight", Q.F16, (48,), np.ones(48, np.float16)),
         ("idol.denoiser.norm.bias", Q.F32, (48,), np.zeros(48, np.float32)),
         ("idol.denoiser.head.weight", Q.F32, (8, 48), rng.standard_normal((8, 48)).astype(np.float32)),
         ("idol.denoiser.head.bias", Q.F32, (8,), np.zeros(8, np.float32))]
    if bad == "nan":
        t[4] = (t[4][0], Q.F32, (8, 48), np.full((8, 48), np.nan, np.float32))
    if bad == "shape":
        t[4] = (t[4][0], Q.F32, (8, 32), np.zeros((8, 32), np.float32))
    if bad == "name":
        t[5] = ("idol.denoiser.head.bias2", Q.F32, (8,), np.zeros(8, np.float32))
    one = np.zeros((1, 32), np.float32)
    t += [(f"idol.{c}.x", Q.F32, (1, 32), one) for c in ("octree", "gaussian", "background")]
    cfg = json.dumps({"denoiser": {}, "decoder": {}, "decoder_gs": {}, "image_encoders": {}})
    G.write_gguf(path, {"general.architecture": "idol", "idol.config.json": cfg}, t)
    return w, data


def test_load_module_and_load_module_packed(tmp_path):
    for quant in (Q.Q8_0, Q.Q4_0):
        w, data = _tiny_gguf(tmp_path / f"t{int(quant)}.gguf", quant)
        m = G.IdolGGUF(tmp_path / f"t{int(quant)}.gguf")
        net = m.load_module("denoiser", _Tiny())
        want = O.blocks_values(data, int(quant), 48, 64)
        assert torch.equal(net.proj.weight.data, torch.from_numpy(want))
        assert torch.equal(net.norm.weight.data, torch.ones(48))
        with torch.device("meta"):
            meta = _Tiny()
        packed = m.load_module_packed("denoiser", meta)
        assert isinstance(packed.proj, PackedLinear) and packed.proj.kind == quant
        assert isinstance(packed.head, torch.nn.Linear) and not packed.head.weight.is_meta
        assert torch.equal(packed.proj.dequantize(torch.float32), torch.from_numpy(want))
        assert torch.equal(packed.proj.bias.data, net.proj.bias.data)
        x = torch.randn(3, 64)
        assert torch.allclose(packed.head(packed.norm(packed.proj(x))), net.head(net.norm(net.proj(x))), atol=1e-6)
    with pytest.raises(ValueError, match="unknown component: nope"):
        m.load_module("nope", _Tiny())
    for bad, message in (("nan", "non-finite value in denoiser.head.weight"),
                         ("shape", r"denoiser.head.weight shape \(8, 32\) does not match \(8, 48\)"),
                         ("name", "denoiser tensor names do not match")):
        _tiny_gguf(tmp_path / f"{bad}.gguf", bad=bad)
        with pytest.raises(ValueError, match=message):
            G.IdolGGUF(tmp_path / f"{bad}.gguf").load_module("denoiser", _Tiny())


@pytest.mark.parametrize("quant", [Q.Q8_0, Q.Q4_0])
def test_decoder_bridge_matches_materialize(tmp_path, quant):
    # the in-memory export holds exactly what materialize writes and read_export reads back; the reference's own
    # loader accepts the materialized directory
    write_idol_gguf(tmp_path / "d.gguf", quant=quant)
    m = G.IdolGGUF(tmp_path / "d.gguf")
    G.materialize(m, tmp_path / "native")
    with pytest.raises(FileExistsError):
        G.materialize(m, tmp_path / "native")
    a = Decoders(tmp_path / "native", device="cpu")
    b = Decoders(G.decoder_export(m), device="cpu")
    assert a.rep == b.rep and a.cfg == b.cfg
    la, lb = a.oct + a.gs, b.oct + b.gs
    assert len(la) == len(lb)
    for x, y in [(a.oct_input, b.oct_input), (a.gs_out, b.gs_out), (a.oct_in, b.oct_in), (a.oct_l1, b.oct_l1)]:
        if x.q8 is not None:
            assert torch.equal(x.q8, y.q8)
        else:
            assert torch.equal(x.weight, y.weight)
        assert torch.equal(x.bias, y.bias)
    ex = E.read_export(tmp_path / "native")
    assert ex.rep.lr_opacity == np.float32(2.0) and ex.rep.lr_scaling == np.float32(0.5)  # the bridge's order
    if O.ref_available():
        ref = O.RefDecoders(tmp_path / "native")
        assert (ref.dim, ref.heads, ref.oct_blocks, ref.gs_blocks, ref.cond, ref.per_anchor) == (64, 2, 1, 2, 16, 4)
        ref.close()
