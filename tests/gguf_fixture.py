"""Builds small Idol GGUF files for the tests: the four components the reference's loader requires, the decoders'
PyTorch tensor names (tools/gguf_to_decoder.py:43-91 reads them), and weights in a chosen mix of encodings."""
import json

import numpy as np

import oracle as O
from ggml_types import GGMLQuantizationType as Q
from idol_gguf import write_gguf


def decoder_state(dim, heads, oct_blocks, gs_blocks, cond, per_anchor, seed):
    """(octree, gaussian) state dicts of random fp32 tensors with the SDK modules' names and shapes."""
    rng = np.random.default_rng(seed)
    D = dim

    def lin(d, name, out, inp):
        d[name + ".weight"] = (rng.standard_normal((out, inp)) / np.sqrt(inp)).astype(np.float32)
        d[name + ".bias"] = (0.02 * rng.standard_normal(out)).astype(np.float32)

    def attn(d, p, cross):
        if cross:
            lin(d, p + ".to_q", D, D)
            lin(d, p + ".to_kv", 2 * D, cond)
        else:
            lin(d, p + ".to_qkv", 3 * D, D)
        lin(d, p + ".to_out", D, D)
        d[p + ".q_rms_norm.gamma"] = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
        d[p + ".k_rms_norm.gamma"] = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)

    octree, gs = {}, {}
    lin(octree, "in_proj", D, 3)
    lin(octree, "input_layer", D, D)
    lin(octree, "l_embedder.mlp.0", D, 256)
    lin(octree, "l_embedder.mlp.2", D, D)
    lin(octree, "adaLN_modulation.1", 6 * D, D)
    lin(octree, "out_proj", 8, D)
    for i in range(oct_blocks):
        attn(octree, f"blocks.{i}.cross_attn", True)
        lin(octree, f"blocks.{i}.mlp.mlp.0", 4 * D, D)
        lin(octree, f"blocks.{i}.mlp.mlp.2", D, 4 * D)
    lin(gs, "in_proj", D, 3)
    lin(gs, "input_layer", D, D)
    lin(gs, "out_proj", per_anchor * 15, D)
    gs["points_offset_perturbation"] = (0.1 * rng.standard_normal(per_anchor * 3)).astype(np.float32)
    gs["base_offset_scale"] = np.array([0.5], np.float32)
    for i in range(gs_blocks):
        attn(gs, f"blocks.{i}.self_attn", False)
        attn(gs, f"blocks.{i}.cross_attn", True)
        gs[f"blocks.{i}.norm2.weight"] = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
        gs[f"blocks.{i}.norm2.bias"] = (0.05 * rng.standard_normal(D)).astype(np.float32)
        lin(gs, f"blocks.{i}.mlp.mlp.0", 4 * D, D)
        lin(gs, f"blocks.{i}.mlp.mlp.2", D, 4 * D)
    return octree, gs


def encode(name, value, quant):
    """(name, type, shape, data) of one tensor: 2-D weights whose width is a multiple of 32 in `quant` (Q8_0 or Q4_0),
    everything else F32 (vectors of the norms in F16 when quant is Q4_0, to exercise that encoding)."""
    if value.ndim == 2 and value.shape[1] % 32 == 0 and name.endswith(".weight") and quant is not None:
        data = O.q8_0_quantize(value) if quant == Q.Q8_0 else O.q4_0_quantize(value)
        return name, quant, value.shape, data
    if quant == Q.Q4_0 and value.ndim == 1 and name.endswith("gamma"):
        return name, Q.F16, value.shape, value.astype(np.float16)
    return name, Q.F32, value.shape, value


def config(dim, heads, oct_blocks, gs_blocks, cond, per_anchor):
    rep = {"num_gaussians": per_anchor, "lr": {"_xyz": 1.0, "_features_dc": 1.0, "_opacity": 0.5, "_scaling": 2.0,
                                               "_rotation": 1.0},
           "perturbe_size": 1.5, "3d_filter_kernel_size": 0.0009, "scaling_bias": 0.004, "opacity_bias": 0.1}
    oct_args = {"model_channels": dim, "cond_channels": cond, "num_blocks": oct_blocks, "num_heads": heads,
                "mlp_ratio": 4}
    gs_args = {"in_channels": 3, **oct_args, "num_blocks": gs_blocks, "representation_config": rep}
    return {"decoder": {"args": oct_args}, "decoder_gs": {"args": gs_args}, "denoiser": {}, "image_encoders": {}}


def write_idol_gguf(path, dim=64, heads=2, oct_blocks=1, gs_blocks=2, cond=16, per_anchor=4, seed=7,
                    quant=Q.Q8_0, extra=()):
    cfg = config(dim, heads, oct_blocks, gs_blocks, cond, per_anchor)
    octree, gs = decoder_state(dim, heads, oct_blocks, gs_blocks, cond, per_anchor, seed)
    tensors = [encode(f"idol.octree.{k}", v, quant) for k, v in octree.items()]
    tensors += [encode(f"idol.gaussian.{k}", v, quant) for k, v in gs.items()]
    tensors += [("idol.denoiser.dummy.weight", Q.F32, (2, 32), np.zeros((2, 32), np.float32)),
                ("idol.background.dummy.weight", Q.F32, (2, 32), np.zeros((2, 32), np.float32))]
    tensors += list(extra)
    fields = {"general.architecture": "idol", "general.name": "Idol",
              "idol.config.json": json.dumps(cfg, sort_keys=True, separators=(",", ":"))}
    write_gguf(path, fields, tensors)
    return octree, gs
