"""Writes the decoder fixtures: a small synthetic decoders export (tests/golden/decoders_small/: manifest.txt +
weights.bin) and the reference's outputs on it (tests/golden/decoders_small.npz).

The export mixes every weight form the reference's loader accepts (src/decoders.cpp:136-148): 8-bit panels from the
GGUF Q8_0 bridge (minimum -128 * scale), 4-bit panels from the Q4_0 bridge (minimum -8 * scale), an asymmetric
6-bit panel with 64-wide groups (a search quantizer's form), and fp32 layers (k = 3 input projections, the k = 16
latent projections, one dense d x d layer). The outputs come from the reference's own idol::Decoders, compiled from
its sources (oracle/_ref/libidolref.so, `make -C oracle ref`), with its float kernel and, where the CPU has AVX-VNNI,
its integer kernel.

Run from the repository root: python tests/golden/make_decoders.py
"""
import shutil
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path[:0] = [str(ROOT / "idol.cpp_amd"), str(ROOT / "oracle")]
import idol_export as E  # noqa: E402
import idol_kernels as K  # noqa: E402
import oracle as O  # noqa: E402

OUT_DIR = Path(__file__).resolve().parent
CFG = E.DecoderConfig(dim=64, heads=2, oct_blocks=1, gs_blocks=2, cond=16, per_anchor=4)
ROWS, TOKENS, LEVEL = 37, 29, 3


def symmetric_panel(w, bits):
    """The bridges' form: per row and 32-group d = amax / (2^(bits-1) - 1) in fp16, code = q + 2^(bits-1)."""
    out, inp = w.shape
    half = 1 << (bits - 1)
    g = w.reshape(out, inp // 32, 32)
    d = (np.abs(g).max(axis=2) / (half - 1)).astype(np.float16).astype(np.float32)
    d = np.where(d == 0, np.float32(1.0), d)
    q = np.clip(np.round(g / d[..., None]), -half, half - 1).astype(np.int16)
    codes = (q + half).astype(np.uint8).reshape(out, inp)
    return E.QTensor(out, inp, bits, 32, K.pack_panel(codes, d, -half * d, bits, 32))


def asymmetric_panel(w, bits, group):
    """min/max form: scale = (max - min) / (2^bits - 1), minimum = min, both fp16."""
    out, inp = w.shape
    g = w.reshape(out, inp // group, group)
    lo = g.min(axis=2).astype(np.float16).astype(np.float32)
    s = ((g.max(axis=2) - lo) / ((1 << bits) - 1)).astype(np.float16).astype(np.float32)
    codes = np.clip(np.round((g - lo[..., None]) / s[..., None]), 0, (1 << bits) - 1).astype(np.uint8)
    return E.QTensor(out, inp, bits, group, K.pack_panel(codes.reshape(out, inp), s, lo, bits, group))


def build_export(path, cfg, seed, forms):
    """A decoders export of random weights; forms maps a layer prefix to 'q8', 'q4', 'a6' or (default) dense."""
    rng = np.random.default_rng(seed)
    D, C = cfg.dim, cfg.cond
    tensors, qtensors = {}, {}

    def linear(prefix, out, inp):
        w = (rng.standard_normal((out, inp)) / np.sqrt(inp)).astype(np.float32)
        b = (0.02 * rng.standard_normal(out)).astype(np.float32)
        form = forms.get(prefix, "dense")
        if form == "q8":
            qtensors[prefix + ".weight"] = symmetric_panel(w, 8)
        elif form == "q4":
            qtensors[prefix + ".weight"] = symmetric_panel(w, 4)
        elif form == "a6":
            qtensors[prefix + ".weight"] = asymmetric_panel(w, 6, 64)
        else:
            tensors[prefix + ".weight"] = w
        tensors[prefix + ".bias"] = b

    def gamma(name, n):
        tensors[name] = (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)

    def attn(p, cross):
        if cross:
            linear(p + ".to_q", D, D)
            linear(p + ".to_kv", 2 * D, C)
        else:
            linear(p + ".to_qkv", 3 * D, D)
        linear(p + ".to_out", D, D)
        gamma(p + ".q_rms_norm.gamma", D)
        gamma(p + ".k_rms_norm.gamma", D)

    linear("oct.in_proj", D, 3)
    linear("oct.input_layer", D, D)
    linear("oct.l_embedder.mlp.0", D, 256)
    linear("oct.l_embedder.mlp.2", D, D)
    linear("oct.adaLN_modulation.1", 6 * D, D)
    linear("oct.out_proj", 8, D)
    for i in range(cfg.oct_blocks):
        p = f"oct.blocks.{i}."
        attn(p + "cross_attn", True)
        linear(p + "mlp.mlp.0", 4 * D, D)
        linear(p + "mlp.mlp.2", D, 4 * D)
    linear("gs.in_proj", D, 3)
    linear("gs.input_layer", D, D)
    linear("gs.out_proj", cfg.per_anchor * 15, D)
    tensors["gs.points_offset_perturbation"] = (0.1 * rng.standard_normal(cfg.per_anchor * 3)).astype(np.float32)
    tensors["gs.base_offset_scale"] = np.array([0.5], np.float32)
    for i in range(cfg.gs_blocks):
        p = f"gs.blocks.{i}."
        attn(p + "self_attn", False)
        attn(p + "cross_attn", True)
        gamma(p + "norm2.weight", D)
        tensors[p + "norm2.bias"] = (0.05 * rng.standard_normal(D)).astype(np.float32)
        linear(p + "mlp.mlp.0", 4 * D, D)
        linear(p + "mlp.mlp.2", D, 4 * D)
    fd = D // 3 // 2
    freqs = np.power(np.float32(2.0), np.linspace(0.0, 10.0, fd, dtype=np.float32)).astype(np.float32)
    tensors["oct.pos_embedder.freqs"] = freqs
    tensors["gs.pos_embedder.freqs"] = freqs
    tensors["oct.l_embedder.freqs"] = np.exp(-np.log(np.float32(1024)) * np.arange(128, dtype=np.float32) / 128,
                                             dtype=np.float32)
    E.write_export(path, cfg, tensors, qtensors, rep=E.Representation())


SMALL_FORMS = {
    "oct.input_layer": "q8", "oct.l_embedder.mlp.0": "q8", "oct.adaLN_modulation.1": "q8", "oct.out_proj": "q8",
    "oct.blocks.0.cross_attn.to_q": "q8", "oct.blocks.0.cross_attn.to_out": "q8",
    "oct.blocks.0.mlp.mlp.0": "q8", "oct.blocks.0.mlp.mlp.2": "q4",
    "gs.input_layer": "q8", "gs.out_proj": "q8",
    "gs.blocks.0.self_attn.to_qkv": "q8", "gs.blocks.0.self_attn.to_out": "a6",
    "gs.blocks.0.cross_attn.to_q": "q8", "gs.blocks.0.cross_attn.to_out": "q8",
    "gs.blocks.0.mlp.mlp.0": "q8", "gs.blocks.0.mlp.mlp.2": "q8",
    "gs.blocks.1.self_attn.to_qkv": "q4", "gs.blocks.1.self_attn.to_out": "q8",
    "gs.blocks.1.cross_attn.to_q": "q8", "gs.blocks.1.cross_attn.to_out": "q8",
    "gs.blocks.1.mlp.mlp.0": "q4", "gs.blocks.1.mlp.mlp.2": "q8",
}  # oct.l_embedder.mlp.2, the in_proj and to_kv layers stay dense

# The same weights with the asymmetric panel quantized symmetrically instead: the reference's integer kernel and the
# INT8 Q8_0 GEMM share their arithmetic on symmetric panels only (an asymmetric panel runs on the float path here),
# so the integer-kernel outputs are recorded for this variant, which build_export rebuilds from the same seed.
SYM_FORMS = {k: ("q8" if v == "a6" else v) for k, v in SMALL_FORMS.items()}


def main():
    export = OUT_DIR / "decoders_small"
    if export.exists():
        shutil.rmtree(export)
    build_export(export, CFG, 11, SMALL_FORMS)
    rng = np.random.default_rng(12)
    anchors = rng.uniform(0, 1, (ROWS, 3)).astype(np.float32)
    cond = rng.standard_normal((TOKENS, CFG.cond)).astype(np.float32)
    ref = O.RefDecoders(export)
    lib = O.ref_lib()
    out = {"anchors": anchors, "cond": cond, "resolution": np.float32(1 << LEVEL)}
    lib.ref_set_quant_kernel(0)
    out["ref_oct"] = ref.octree_logits(anchors, float(1 << LEVEL), cond)
    out["ref_gs"] = ref.gaussian_features(anchors, cond)
    ref.close()
    if O.ref_int8_supported():
        sym = OUT_DIR / "_decoders_small_sym"
        if sym.exists():
            shutil.rmtree(sym)
        build_export(sym, CFG, 11, SYM_FORMS)
        ref = O.RefDecoders(sym)
        lib.ref_set_quant_kernel(1)
        out["sym_oct_int8"] = ref.octree_logits(anchors, float(1 << LEVEL), cond)
        out["sym_gs_int8"] = ref.gaussian_features(anchors, cond)
        lib.ref_set_quant_kernel(0)
        out["sym_oct"] = ref.octree_logits(anchors, float(1 << LEVEL), cond)
        out["sym_gs"] = ref.gaussian_features(anchors, cond)
        ref.close()
        shutil.rmtree(sym)
    lib.ref_set_quant_kernel(-1)
    np.savez_compressed(OUT_DIR / "decoders_small.npz", **out)
    print({k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    main()
