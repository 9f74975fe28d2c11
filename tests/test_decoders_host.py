"""The decoder export reader and loader on the CPU: the fixture export reads back as written, and every malformed
export is rejected with the reference's own message (src/weights.cpp:25-127, src/decoders.cpp:126-212), checked
against the reference build when it is present."""
import shutil

import numpy as np
import pytest

import idol_export as E
import idol_kernels as K
import oracle as O
from conftest import GOLDEN
from decoders import Decoders

SMALL = GOLDEN / "decoders_small"


def test_fixture_export_reads_back():
    ex = E.read_export(SMALL)
    assert ex.decoders
    c = ex.decoder_config
    assert (c.dim, c.heads, c.oct_blocks, c.gs_blocks, c.cond, c.per_anchor) == (64, 2, 1, 2, 16, 4)
    assert ex.rep == E.Representation()
    q = ex.qtensors["oct.blocks.0.mlp.mlp.2.weight"]
    assert (q.out, q.in_, q.bits, q.group) == (64, 256, 4, 32)
    assert q.blob.size == 4 * K.quant_panel_bytes(256, 4, 32)
    a = ex.qtensors["gs.blocks.0.self_attn.to_out.weight"]
    assert (a.bits, a.group) == (6, 64)
    t = ex.tensors["oct.in_proj.weight"]
    assert t.shape == [64, 3] and t.data.dtype == np.float32 and t.data.size == 192
    assert ex.tensors["gs.base_offset_scale"].data.tolist() == [0.5]


def test_write_read_round_trip(tmp_path):
    rng = np.random.default_rng(5)
    cfg = E.DecoderConfig(32, 4, 0, 0, 8, 2)
    dense = {"a.weight": rng.standard_normal((5, 7)).astype(np.float32), "s": np.array([1.25], np.float32)}
    codes = rng.integers(0, 8, (20, 64)).astype(np.uint8)
    blob = K.pack_panel(codes, np.full((20, 2), 0.5, np.float32), np.full((20, 2), -2.0, np.float32), 3, 32)
    rep = E.Representation(1.0, 0.5, 0.25, 0.125, 2.0, 3.0, 4.0, 5.0, 6.0)
    E.write_export(tmp_path / "x", cfg, dense, {"q.weight": E.QTensor(20, 64, 3, 32, blob)}, rep=rep, case=(3, 4, 5))
    ex = E.read_export(tmp_path / "x")
    assert ex.decoder_config == cfg and ex.rep == rep
    assert (ex.case_anchors, ex.case_latent, ex.case_level) == (3, 4, 5)
    assert np.array_equal(ex.tensors["a.weight"].data.reshape(5, 7), dense["a.weight"])
    assert ex.tensors["a.weight"].shape == [5, 7]
    assert np.array_equal(ex.qtensors["q.weight"].blob, blob)
    with pytest.raises(FileExistsError):
        E.write_export(tmp_path / "x", cfg, dense)


def test_loader_holds_every_weight_form_on_the_host():
    # symmetric 8- and 4-bit panels become Q8_0 blocks, the asymmetric 6-bit panel and unquantized layers fp32 values
    dec = Decoders(SMALL, device="cpu")
    assert dec.oct_input.q8 is not None and dec.oct_input.qbits == 8
    assert dec.oct[0][2].q8 is not None and dec.oct[0][2].qbits == 4
    sa0 = dec.gs[0][0]
    assert sa0.out.q8 is None and sa0.out.qbits == 6 and sa0.out.weight.shape == (64, 64)
    assert dec.oct_in.q8 is None and dec.oct_in.qbits == 0 and dec.oct_in.weight.shape == (64, 3)
    assert dec.weight_bytes() > 0
    ex = E.read_export(SMALL)
    q = ex.qtensors["oct.blocks.0.mlp.mlp.2.weight"]
    want = K.panel_values(q.blob, 64, 256, 4, 32)
    got = O.q8_0_dequant(dec.oct[0][2].q8.numpy(), 64, 256)
    assert np.array_equal(got, want)
    if O.ref_available():
        assert np.array_equal(want, O.ref_dequantize_panel(q.blob, 64, 256, 4, 32))


def test_panels_of_every_width_unpack_as_the_reference_reads_them():
    if not O.ref_available():
        pytest.skip("reference build absent (make -C oracle ref)")
    rng = np.random.default_rng(9)
    for bits in (2, 3, 4, 5, 6, 8):
        for group in (32, 64, 128):
            out, inp = 21, 256
            codes = rng.integers(0, 1 << bits, (out, inp)).astype(np.uint8)
            s = rng.uniform(0.001, 0.2, (out, inp // group)).astype(np.float16).astype(np.float32)
            m = rng.uniform(-1, 1, (out, inp // group)).astype(np.float16).astype(np.float32)
            blob = K.pack_panel(codes, s, m, bits, group)
            c2, s2, m2 = K.unpack_panel(blob, out, inp, bits, group)
            assert np.array_equal(c2, codes) and np.array_equal(s2, s) and np.array_equal(m2, m)
            assert np.array_equal(K.panel_values(blob, out, inp, bits, group),
                                  O.ref_dequantize_panel(blob, out, inp, bits, group))
            sym = K.pack_panel(codes, s, -float(1 << (bits - 1)) * s, bits, group)
            assert np.array_equal(O.q8_0_dequant(K.panel_to_q8_0(sym, out, inp, bits, group), out, inp),
                                  O.ref_dequantize_panel(sym, out, inp, bits, group))


# ------------------------------------------------------------------------------------------------ malformed exports
def _copy(tmp_path):
    d = tmp_path / "exp"
    shutil.copytree(SMALL, d)
    return d


def _edit_manifest(d, fn):
    lines = (d / "manifest.txt").read_text().split("\n")
    (d / "manifest.txt").write_text("\n".join(fn(lines)))


def _replace(name, new_line):
    def fn(lines):
        return [new_line if ln.split()[:2] in (["qtensor", name],) or (ln.split()[:1] == [name]) else ln
                for ln in lines]
    return fn


CASES = [
    ("missing manifest", lambda d: (d / "manifest.txt").unlink(), "cannot open {d}/manifest.txt"),
    ("empty manifest", lambda d: (d / "manifest.txt").write_text(""), "{d}/manifest.txt is empty"),
    ("bad first line", lambda d: _edit_manifest(d, lambda ls: ["decoders 64 2 1"] + ls[1:]),
     "{d}/manifest.txt: the first line must be 'decoders dim heads oct gs cond per_anchor'"),
    ("wrong tag", lambda d: _edit_manifest(d, lambda ls: ["encoders 64 2 1 2 16 4"] + ls[1:]),
     "{d}/manifest.txt: the first line must be 'decoders dim heads oct gs cond per_anchor'"),
    ("missing weights", lambda d: (d / "weights.bin").unlink(), "cannot open {d}/weights.bin"),
    ("malformed rep", lambda d: _edit_manifest(d, lambda ls: ls + ["rep 1 2 3"]), "malformed rep line in manifest.txt"),
    ("malformed case", lambda d: _edit_manifest(d, lambda ls: ls + ["case 1 x 3"]),
     "malformed case line in manifest.txt"),
    ("malformed qtensor", lambda d: _edit_manifest(d, lambda ls: ls + ["qtensor a.weight 4 32 8 32 0"]),
     "malformed qtensor line in manifest.txt"),
    ("qtensor outside", lambda d: _edit_manifest(d, lambda ls: ls + ["qtensor a.weight 16 32 8 32 0 99999999"]),
     "qtensor 'a.weight' lies outside weights.bin"),
    ("byte count", lambda d: _edit_manifest(d, lambda ls: ls + ["t 2 3 4 0 40"]),
     "tensor 't' has a byte count that does not match its shape"),
    ("tensor outside", lambda d: _edit_manifest(d, lambda ls: ls + ["t 1 4 99999999 16"]),
     "tensor 't' lies outside weights.bin"),
    ("negative dim", lambda d: _edit_manifest(d, lambda ls: ls + ["t 2 -3 4 0 48"]), "negative dimension in manifest.txt"),
    ("malformed tensor", lambda d: _edit_manifest(d, lambda ls: ls + ["t 2 3"]), "malformed manifest.txt line for 't'"),
    ("invalid config", lambda d: _edit_manifest(d, lambda ls: ["decoders 64 3 1 2 16 4"] + ls[1:]),
     "manifest.txt describes an invalid decoder configuration"),
    ("missing tensor", lambda d: _edit_manifest(d, lambda ls: [ln for ln in ls if not ln.startswith("oct.in_proj.bias ")]),
     "missing tensor 'oct.in_proj.bias'"),
    ("wrong count", lambda d: _edit_manifest(d, lambda ls: [ln.replace("oct.l_embedder.freqs 1 128", "oct.l_embedder.freqs 1 64")
                                                         .replace(" 512", " 256") if ln.startswith("oct.l_embedder.freqs") else ln
                                                         for ln in ls]),
     "tensor 'oct.l_embedder.freqs' has 64 values, expected 128"),
    ("qtensor shape", lambda d: _edit_manifest(d, lambda ls: [ln.replace("qtensor oct.input_layer.weight 64 64",
                                                                         "qtensor oct.input_layer.weight 32 64")
                                                              for ln in ls]),
     "quantized tensor 'oct.input_layer.weight' has the wrong shape"),
]


@pytest.mark.parametrize("name,mutate,message", CASES, ids=[c[0] for c in CASES])
def test_malformed_exports_fail_with_the_reference_message(tmp_path, name, mutate, message):
    d = _copy(tmp_path)
    mutate(d)
    want = message.format(d=d)
    with pytest.raises(RuntimeError) as err:
        Decoders(d, device="cpu")
    assert str(err.value) == want
    if O.ref_available():
        with pytest.raises(RuntimeError) as ref_err:
            O.RefDecoders(d)
        assert str(ref_err.value) == want


def test_rejected_panel_fails_like_the_reference(tmp_path):
    d = _copy(tmp_path)
    _edit_manifest(d, lambda ls: [ln.replace("qtensor oct.input_layer.weight 64 64 8 32",
                                             "qtensor oct.input_layer.weight 64 64 7 32") for ln in ls])
    with pytest.raises(ValueError, match="quantized layers use 2, 3, 4, 5, 6 or 8 bits"):
        Decoders(d, device="cpu")
    if O.ref_available():
        with pytest.raises(RuntimeError, match="quantized layers use 2, 3, 4, 5, 6 or 8 bits"):
            O.RefDecoders(d)


def test_decoders_refuse_host_tensors():
    dec = Decoders(SMALL, device="cpu")
    with pytest.raises(ValueError, match="GPU tensors"):
        dec.gaussian_features(np.zeros((4, 3), np.float32), 4, np.zeros((5, 16), np.float32), 5)
