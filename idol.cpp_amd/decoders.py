"""idol::Decoders on MI355X: the octree decoder and the Gaussian decoder of the real Idol model (src/decoders.cpp,
include/idol/decoders.hpp), loaded from the native export (manifest.txt + weights.bin) and run on the GPU.

Every operator is a libidolq HIP kernel, on fp32 activations like the reference's CPU path:
  linears       Q8_0 GEMM (quantized layers; EXACT mode, or INT8 when the reference would use its integer kernel)
                or the dense fp32 GEMM in the reference's summation order (unquantized layers, asymmetric panels);
                the reference's separate SiLU / tanh-GELU passes are fused into the GEMM epilogue (the same fp32
                operations on the same values: bias, then residual, then the activation)
  layer norm    fp64 statistics (src/decoders.cpp:23-42), adaLN shift/scale from the level MLP
  rms_heads, add_gated, the level embedding, the position embedding   one kernel each
  attention     the fp32 attention kernel (src/kernels.cpp:735-746 semantics)
Buffers are allocated per call from PyTorch's caching allocator. Inputs and outputs are fp32 GPU tensors; numpy
arrays are accepted and copied to the device.

The order of operations follows src/decoders.cpp:232-316 step by step. Output tolerance against the reference's
float kernel is the one its own decoder check uses (norm-relative 2e-5, tests/python/test_gguf_decoder.py:63-65).
"""
import numpy as np
import torch

import idol_export as E
import idol_kernels as K
import idolq_lib as L


class _Attn:
    __slots__ = ("q", "kv", "qkv", "out", "q_gamma", "k_gamma")


class Decoders:
    """The reference's idol::Decoders (include/idol/decoders.hpp:36-77) on one GPU.

    Decoders(path) reads an export directory; Decoders(export) takes an already-read idol_export.Export. Raises
    RuntimeError for a missing or malformed export, with the reference's messages."""

    def __init__(self, source, device="cuda"):
        ex = source if isinstance(source, E.Export) else E.read_export(source)
        self.device = torch.device(device)
        if not ex.decoders:
            raise RuntimeError("this export is not a decoders export (tools/export_idol.py)")
        cfg = ex.decoder_config
        D, H4 = cfg.dim, 4 * cfg.dim
        if (D <= 0 or cfg.heads <= 0 or D % cfg.heads != 0 or cfg.cond <= 0 or cfg.per_anchor <= 0
                or cfg.oct_blocks < 0 or cfg.gs_blocks < 0):
            raise RuntimeError("manifest.txt describes an invalid decoder configuration")
        self.cfg, self.rep = cfg, ex.rep
        dev = self.device

        def linear(prefix, out, in_):
            q = E.take_qtensor(ex, prefix + ".weight")
            if q is not None:
                if q.out != out or q.in_ != in_:
                    raise RuntimeError(f"quantized tensor '{prefix}.weight' has the wrong shape")
                b = E.take_tensor(ex, prefix + ".bias", out)
                if q.kind == "q8_0":
                    return K.q8_0_linear(q.blob, b.data, out, in_, device=dev)
                return K.quantized_linear(q.blob, b.data, out, in_, q.bits, q.group, device=dev)
            w = E.take_tensor(ex, prefix + ".weight", out * in_)
            b = E.take_tensor(ex, prefix + ".bias", out)
            return K.pack_linear(w.data, b.data, out, in_, device=dev)

        def vec(name, count):
            return torch.from_numpy(E.take_tensor(ex, name, count).data.copy()).to(dev)

        def attn(p, cross):
            a = _Attn()
            a.q = a.kv = a.qkv = None
            if cross:
                a.q = linear(p + ".to_q", D, D)
                a.kv = linear(p + ".to_kv", 2 * D, cfg.cond)
            else:
                a.qkv = linear(p + ".to_qkv", 3 * D, D)
            a.out = linear(p + ".to_out", D, D)
            a.q_gamma = vec(p + ".q_rms_norm.gamma", D)
            a.k_gamma = vec(p + ".k_rms_norm.gamma", D)
            return a

        self.oct_in = linear("oct.in_proj", D, 3)
        self.oct_input = linear("oct.input_layer", D, D)
        self.oct_l1 = linear("oct.l_embedder.mlp.0", D, 256)
        self.oct_l2 = linear("oct.l_embedder.mlp.2", D, D)
        self.oct_ada = linear("oct.adaLN_modulation.1", 6 * D, D)
        self.oct_out = linear("oct.out_proj", 8, D)
        self.oct = []
        for i in range(cfg.oct_blocks):
            p = f"oct.blocks.{i}."
            self.oct.append((attn(p + "cross_attn", True), linear(p + "mlp.mlp.0", H4, D), linear(p + "mlp.mlp.2", D, H4)))

        outs = cfg.per_anchor * 15
        self.gs_in = linear("gs.in_proj", D, 3)
        self.gs_input = linear("gs.input_layer", D, D)
        self.gs_out = linear("gs.out_proj", outs, D)
        self.perturbation = vec("gs.points_offset_perturbation", cfg.per_anchor * 3)
        self.base_offset_scale = float(E.take_tensor(ex, "gs.base_offset_scale", 1).data[0])
        self.gs = []
        for i in range(cfg.gs_blocks):
            p = f"gs.blocks.{i}."
            self_attn, cross_attn = attn(p + "self_attn", False), attn(p + "cross_attn", True)
            g2, b2 = vec(p + "norm2.weight", D), vec(p + "norm2.bias", D)
            self.gs.append((self_attn, cross_attn, g2, b2, linear(p + "mlp.mlp.0", H4, D), linear(p + "mlp.mlp.2", D, H4)))

        # the embedders' frequency tables as the export holds them (PyTorch's float32 values)
        self.oct_pos_freqs = vec("oct.pos_embedder.freqs", D // 3 // 2)
        self.gs_pos_freqs = vec("gs.pos_embedder.freqs", D // 3 // 2)
        self.level_freqs = vec("oct.l_embedder.freqs", 128)

        layers = [self.oct_in, self.oct_input, self.oct_l1, self.oct_l2, self.oct_ada, self.oct_out, self.gs_in,
                  self.gs_input, self.gs_out]
        for a, f1, f2 in self.oct:
            layers += [a.q, a.kv, a.out, f1, f2]
        for sa, ca, _, _, f1, f2 in self.gs:
            layers += [sa.qkv, sa.out, ca.q, ca.kv, ca.out, f1, f2]
        self._weight_bytes = sum(layer.bytes() for layer in layers)

    # ---------------------------------------------------------------------------------------------------- queries
    def config(self):
        return self.cfg

    def weight_bytes(self):
        """Bytes the layers hold on the device (weights as stored here plus padded biases)."""
        return self._weight_bytes

    # ---------------------------------------------------------------------------------------------------- helpers
    def _f32(self, a, name):
        t = torch.as_tensor(a) if not isinstance(a, torch.Tensor) else a
        if t.dtype != torch.float32:
            raise ValueError(f"{name} must be fp32")
        return t.to(self.device).contiguous()

    @staticmethod
    def _linear(a, w, out, residual=None, act=L.ACT_NONE):
        """out = act(a @ W^T + bias + residual): gemm_packed (src/kernels.hpp:73-76) with the activation fused."""
        if w.q8 is None:
            return L.gemm_f32(a, w.weight, bias=w.bias[:w.out], residual=residual, act=act, out=out)
        mode = L.MODE_INT8 if K._use_int8() else L.MODE_EXACT
        return L.gemm(a, w.q8, w.out, 0, w.out, bias=w.bias[:w.out], residual=residual, act=act, mode=mode, out=out)

    def _embed_points(self, freqs, x, rows, lin_in, lin_input, X, H):
        """X = input_layer(in_proj(x) + pos_embed(x)) (src/decoders.cpp:247-250 and 283-286)."""
        D = self.cfg.dim
        fd = freqs.numel()
        if 6 * fd < D:
            H[:, 6 * fd:].zero_()
        L.pos_embed(x, freqs, H[:, :6 * fd], ldo=D)
        self._linear(x, lin_in, X, residual=H)
        self._linear(X, lin_input, H)
        return H, X  # the reference swaps X and H

    def _cross_attention(self, a, h, rows, cond, cond_rows, Q, KV, A):
        """src/decoders.cpp:232-240."""
        D, heads = self.cfg.dim, self.cfg.heads
        hd = D // heads
        self._linear(h, a.q, Q)
        L.rms_heads(Q, heads, hd, a.q_gamma)
        self._linear(cond, a.kv, KV)
        L.rms_heads(KV, heads, hd, a.k_gamma)
        K.attention(Q, rows, D, KV, KV[:, D:], cond_rows, 2 * D, heads, hd, A, D)

    # ---------------------------------------------------------------------------------------------------- decoders
    def octree_logits(self, x, rows, resolution, cond, cond_rows, out=None):
        """Octree decoder (src/decoders.cpp:242-279): x [rows, 3] cell centres, resolution 2^level, cond
        [cond_rows, cond]. Returns (or writes) out [rows, 8]."""
        cfg = self.cfg
        D, H4 = cfg.dim, 4 * cfg.dim
        x = self._f32(x, "x")[:rows]
        cond = self._f32(cond, "cond")[:cond_rows]
        dev = self.device
        if out is None:
            out = torch.empty((rows, 8), device=dev, dtype=torch.float32)
        if rows == 0:
            return out
        X = torch.empty((rows, D), device=dev)
        H = torch.empty_like(X)
        Q, A = torch.empty_like(X), torch.empty_like(X)
        F = torch.empty((rows, H4), device=dev)
        KV = torch.empty((cond_rows, 2 * D), device=dev)

        X, H = self._embed_points(self.oct_pos_freqs, x, rows, self.oct_in, self.oct_input, X, H)

        # the octree level, embedded and turned into the shared adaLN modulation
        emb = L.level_embed(resolution, self.level_freqs).view(1, -1)
        l1 = torch.empty((1, D), device=dev)
        l2 = torch.empty((1, D), device=dev)
        mod = torch.empty((1, 6 * D), device=dev)
        self._linear(emb, self.oct_l1, l1, act=L.ACT_SILU)
        self._linear(l1, self.oct_l2, l2, act=L.ACT_SILU)
        self._linear(l2, self.oct_ada, mod)
        m = mod.view(-1)
        shift_a, scale_a, gate_a = m[0:D], m[D:2 * D], m[2 * D:3 * D]
        shift_m, scale_m, gate_m = m[3 * D:4 * D], m[4 * D:5 * D], m[5 * D:6 * D]

        for a, ff1, ff2 in self.oct:
            L.layernorm(X, 1e-6, shift=shift_a, scale=scale_a, out=H)
            self._cross_attention(a, H, rows, cond, cond_rows, Q, KV, A)
            self._linear(A, a.out, H)
            L.add_gated(X, H, gate_a)
            L.layernorm(X, 1e-6, shift=shift_m, scale=scale_m, out=H)
            self._linear(H, ff1, F, act=L.ACT_GELU_TANH)
            self._linear(F, ff2, H)
            L.add_gated(X, H, gate_m)
        L.layernorm(X, 1e-5, out=H)
        self._linear(H, self.oct_out, out)
        return out

    def gaussian_features(self, points, rows, cond, cond_rows, out=None):
        """Gaussian decoder (src/decoders.cpp:281-316): points [rows, 3] anchors, cond [cond_rows, cond]. Returns (or
        writes) out [rows, per_anchor * 15] raw values."""
        cfg = self.cfg
        D, H4, heads = cfg.dim, 4 * cfg.dim, cfg.heads
        hd = D // heads
        points = self._f32(points, "points")[:rows]
        cond = self._f32(cond, "cond")[:cond_rows]
        dev = self.device
        if out is None:
            out = torch.empty((rows, cfg.per_anchor * 15), device=dev, dtype=torch.float32)
        if rows == 0:
            return out
        X = torch.empty((rows, D), device=dev)
        H = torch.empty_like(X)
        Q, A = torch.empty_like(X), torch.empty_like(X)
        F = torch.empty((rows, H4), device=dev)
        QKV = torch.empty((rows, 3 * D), device=dev)
        KV = torch.empty((cond_rows, 2 * D), device=dev)

        X, H = self._embed_points(self.gs_pos_freqs, points, rows, self.gs_in, self.gs_input, X, H)

        for sa, ca, g2, b2, ff1, ff2 in self.gs:
            L.layernorm(X, 1e-6, out=H)
            self._linear(H, sa.qkv, QKV)
            L.rms_heads(QKV, heads, hd, sa.q_gamma)
            L.rms_heads(QKV[:, D:], heads, hd, sa.k_gamma)
            K.attention(QKV, rows, 3 * D, QKV[:, D:], QKV[:, 2 * D:], rows, 3 * D, heads, hd, A, D)
            self._linear(A, sa.out, X, residual=X)

            L.layernorm(X, 1e-6, gamma=g2, beta=b2, out=H)
            self._cross_attention(ca, H, rows, cond, cond_rows, Q, KV, A)
            self._linear(A, ca.out, X, residual=X)

            L.layernorm(X, 1e-6, out=H)
            self._linear(H, ff1, F, act=L.ACT_GELU_TANH)
            self._linear(F, ff2, X, residual=X)
        L.layernorm(X, 1e-5, out=H)
        self._linear(H, self.gs_out, out)
        return out


def synthetic_export(cfg, seed=0, device="cuda"):
    """An in-memory export of randomly initialised decoders with the weight forms of the real model's GGUF export:
    every matrix whose input width is a multiple of 256 as Q8_0 blocks (quantized on the GPU), the k = 3 input
    projections and the k = cond latent projections as fp32 (tools/export_full_gguf.py:91 quantizes only those).
    Weights ~ N(0, 1/in), biases ~ N(0, 0.02^2), norm and RMS gains ~ 1 + N(0, 0.1^2). For benchmarks."""
    gen = torch.Generator(device="cpu").manual_seed(seed)
    D, C = cfg.dim, cfg.cond
    ex = E.Export(decoders=True, decoder_config=cfg)

    def randn(*shape):
        return torch.randn(*shape, generator=gen, dtype=torch.float32)

    def linear(prefix, out, in_):
        w = randn(out, in_) / float(np.sqrt(in_))
        if in_ % 256 == 0:
            ex.qtensors[prefix + ".weight"] = E.QTensor(out, in_, 8, 32, L.quantize_q8_0(w.to(device)), kind="q8_0")
        else:
            ex.tensors[prefix + ".weight"] = E.Tensor([out, in_], w.numpy().reshape(-1))
        ex.tensors[prefix + ".bias"] = E.Tensor([out], (0.02 * randn(out)).numpy())

    def vec(name, values):
        ex.tensors[name] = E.Tensor([values.size], np.ascontiguousarray(values, np.float32).reshape(-1))

    def attn(p, cross):
        if cross:
            linear(p + ".to_q", D, D)
            linear(p + ".to_kv", 2 * D, C)
        else:
            linear(p + ".to_qkv", 3 * D, D)
        linear(p + ".to_out", D, D)
        vec(p + ".q_rms_norm.gamma", (1 + 0.1 * randn(D)).numpy())
        vec(p + ".k_rms_norm.gamma", (1 + 0.1 * randn(D)).numpy())

    linear("oct.in_proj", D, 3)
    linear("oct.input_layer", D, D)
    linear("oct.l_embedder.mlp.0", D, 256)
    linear("oct.l_embedder.mlp.2", D, D)
    linear("oct.adaLN_modulation.1", 6 * D, D)
    linear("oct.out_proj", 8, D)
    for i in range(cfg.oct_blocks):
        attn(f"oct.blocks.{i}.cross_attn", True)
        linear(f"oct.blocks.{i}.mlp.mlp.0", 4 * D, D)
        linear(f"oct.blocks.{i}.mlp.mlp.2", D, 4 * D)
    linear("gs.in_proj", D, 3)
    linear("gs.input_layer", D, D)
    linear("gs.out_proj", cfg.per_anchor * 15, D)
    vec("gs.points_offset_perturbation", (0.1 * randn(cfg.per_anchor * 3)).numpy())
    vec("gs.base_offset_scale", np.array([0.5], np.float32))
    for i in range(cfg.gs_blocks):
        p = f"gs.blocks.{i}."
        attn(p + "self_attn", False)
        attn(p + "cross_attn", True)
        vec(p + "norm2.weight", (1 + 0.1 * randn(D)).numpy())
        vec(p + "norm2.bias", (0.05 * randn(D)).numpy())
        linear(p + "mlp.mlp.0", 4 * D, D)
        linear(p + "mlp.mlp.2", D, 4 * D)
    fd = D // 3 // 2
    freqs = torch.pow(2.0, torch.linspace(0.0, 10.0, fd, dtype=torch.float32)).numpy()
    vec("oct.pos_embedder.freqs", freqs)
    vec("gs.pos_embedder.freqs", freqs)
    vec("oct.l_embedder.freqs", torch.exp(-np.log(1024) * torch.arange(0, 128, dtype=torch.float32) / 128).numpy())
    return ex


# ------------------------------------------------------------------------------------------------ sampling
class MT19937_64:
    """std::mt19937_64 (the 64-bit Mersenne Twister of Matsumoto and Nishimura, as the C++ standard specifies it:
    n = 312, m = 156, r = 31, a = 0xB5026F5AA96619E9, tempering (29, 0x5555555555555555), (17, 0x71D67FFFEDA60000),
    (37, 0xFFF7EEE000000000), 43; seeding multiplier 6364136223846793005), generated 312 outputs at a time with
    numpy, and std::uniform_real_distribution<float>(0, 1) on top as libstdc++ computes it (generate_canonical: one
    64-bit draw, float(x) / 2^64, 1 mapped to the float below 1)."""
    _N, _M = 312, 156
    _A = np.uint64(0xB5026F5AA96619E9)
    _UPPER, _LOWER = np.uint64(0xFFFFFFFF80000000), np.uint64(0x7FFFFFFF)

    def __init__(self, seed):
        mt = np.empty(self._N, np.uint64)
        mt[0] = np.uint64(seed & 0xFFFFFFFFFFFFFFFF)
        with np.errstate(over="ignore"):
            for i in range(1, self._N):
                prev = int(mt[i - 1])
                mt[i] = np.uint64((6364136223846793005 * (prev ^ (prev >> 62)) + i) & 0xFFFFFFFFFFFFFFFF)
        self.mt = mt
        self.buf = np.empty(0, np.uint64)
        self.pos = 0

    def _twist(self):
        mt, N, M = self.mt, self._N, self._M
        one = np.uint64(1)

        def mix(cur, nxt, far):
            x = (cur & self._UPPER) | (nxt & self._LOWER)
            return far ^ (x >> one) ^ np.where((x & one) != 0, self._A, np.uint64(0))

        mt[:N - M] = mix(mt[:N - M], mt[1:N - M + 1], mt[M:])            # far values not yet replaced
        mt[N - M:N - 1] = mix(mt[N - M:N - 1], mt[N - M + 1:], mt[:M - 1])  # far values of this round
        mt[N - 1] = mix(mt[N - 1:], mt[:1], mt[M - 1:M])[0]
        y = mt.copy()
        y ^= (y >> np.uint64(29)) & np.uint64(0x5555555555555555)
        y ^= (y << np.uint64(17)) & np.uint64(0x71D67FFFEDA60000)
        y ^= (y << np.uint64(37)) & np.uint64(0xFFF7EEE000000000)
        y ^= y >> np.uint64(43)
        self.buf, self.pos = y, 0

    def raw(self, count):
        """The next `count` 64-bit outputs."""
        out = np.empty(count, np.uint64)
        filled = 0
        while filled < count:
            if self.pos == self.buf.size:
                self._twist()
            take = min(count - filled, self.buf.size - self.pos)
            out[filled:filled + take] = self.buf[self.pos:self.pos + take]
            self.pos += take
            filled += take
        return out

    def uniform(self, count):
        """The next `count` uniform floats in [0, 1)."""
        f = self.raw(count).astype(np.float32) * np.float32(2.0 ** -64)
        return np.where(f >= np.float32(1.0), np.nextafter(np.float32(1.0), np.float32(0.0)), f).astype(np.float32)


_BELOW_ONE = np.float32(1.0) - np.float32(1e-7)


def _expf(x):
    """float32 exp, rounded from the double result."""
    return np.exp(x.astype(np.float64)).astype(np.float32)


def descend_octree(logits_fn, num_points, level, seed):
    """The octree descent of Decoders::sample_anchors (src/decoders.cpp:335-391): from the root cell, per level, the
    children's logits of every occupied cell (logits_fn(centres [cells, 3] fp32, resolution) -> [cells, 8]), a
    softmax, and systematic resampling of the cell's points among its children with one uniform draw per cell; then
    each point placed uniformly inside its leaf cell. Host arithmetic in fp32 with the reference's operation order;
    the draws come from MT19937_64(seed) in the reference's order. Returns num_points x 3 fp32."""
    if num_points < 1 or level < 1 or level > 20:
        raise ValueError("sample_anchors: bad num_points or level")
    rng = MT19937_64(seed)
    coords = np.zeros((1, 3), np.uint32)
    counts = np.array([num_points], np.int64)
    bits = np.array([[c & 1, (c >> 1) & 1, (c >> 2) & 1] for c in range(8)], np.uint32)
    for lv in range(1, level + 1):
        res_p = np.float32(1 << (lv - 1))
        centres = ((coords.astype(np.float32) + np.float32(0.5)) / res_p).astype(np.float32)
        logits = np.asarray(logits_fn(centres, float(1 << lv)), np.float32).reshape(-1, 8)
        mx = logits.max(axis=1)
        e = _expf(logits - mx[:, None])
        total = np.zeros(len(counts), np.float32)
        for c in range(8):
            total = (total + e[:, c]).astype(np.float32)
        cdf = np.empty_like(e)
        acc = np.zeros(len(counts), np.float32)
        for c in range(8):
            acc = (acc + (e[:, c] / total).astype(np.float32)).astype(np.float32)
            cdf[:, c] = np.minimum(acc, _BELOW_ONE)
        n = counts.astype(np.float32)
        u0 = (rng.uniform(len(counts)) / n).astype(np.float32)
        owner = np.repeat(np.arange(len(counts)), counts)
        k = (np.arange(owner.size) - np.repeat(np.cumsum(counts) - counts, counts)).astype(np.float32)
        u = np.minimum((u0[owner] + (k / n[owner]).astype(np.float32)).astype(np.float32), _BELOW_ONE)
        child = np.minimum(7, (cdf[owner] < u[:, None]).sum(axis=1))
        got = np.zeros((len(counts), 8), np.int64)
        np.add.at(got, (owner, child), 1)
        parent, which = np.nonzero(got)
        coords = coords[parent] * np.uint32(2) + bits[which]
        counts = got[parent, which]
    cells = np.float32(1 << level)
    cell_of = np.repeat(np.arange(len(counts)), counts)
    draws = rng.uniform(3 * num_points).reshape(num_points, 3)
    return ((coords[cell_of].astype(np.float32) + draws) / cells).astype(np.float32)


class GaussianCloud:
    """Activated Gaussians (include/idol/decoders.hpp:22-30): xyz, f_dc, scale [n, 3], rotation [n, 4] (w first),
    opacity [n], fp32 tensors (on the GPU as decode returns them)."""

    def __init__(self, xyz, f_dc, scale, rotation, opacity):
        self.xyz, self.f_dc, self.scale, self.rotation, self.opacity = xyz, f_dc, scale, rotation, opacity

    def size(self):
        return int(self.opacity.numel())


def _rep_vector(dec):
    """The to_gaussians constants: the rep fields, the inverse softplus of the scaling bias and the inverse sigmoid
    of the opacity bias (computed in double, as the reference does), and the base offset scale."""
    r = dec.rep
    sb, ob = float(r.scaling_bias), float(r.opacity_bias)
    scale_offset = np.float32(sb + np.log(-np.expm1(-sb)))
    opacity_offset = np.float32(np.log(ob / (1.0 - ob)))
    return torch.tensor([r.perturbe, r.kernel, r.lr_xyz, r.lr_dc, r.lr_opacity, r.lr_scaling, r.lr_rotation,
                         scale_offset, opacity_offset, dec.base_offset_scale], dtype=torch.float32, device=dec.device)


def _sample_anchors(self, cond, cond_rows, num_points, level, seed):
    """Decoders::sample_anchors: the octree descent with this module's octree_logits on the GPU (num_points x 3 fp32,
    on the host). The draws follow the reference's generator, so given the same logits the anchors are the
    reference's; logits differing in the last bits can move a point to a sibling cell where a draw falls on a
    cumulative-probability boundary."""
    cond_t = self._f32(cond, "cond")[:cond_rows]

    def logits(centres, resolution):
        x = torch.from_numpy(centres).to(self.device)
        return self.octree_logits(x, x.shape[0], resolution, cond_t, cond_rows).cpu().numpy()

    return descend_octree(logits, num_points, level, seed)


def _to_gaussians(self, anchors, rows, features):
    """Decoders::to_gaussians on the GPU: anchors [rows, 3], features [rows, per_anchor * 15] -> GaussianCloud."""
    a = self._f32(anchors, "anchors")[:rows]
    f = self._f32(features, "features")[:rows]
    out = L.to_gaussians(a, f, self.cfg.per_anchor, self.perturbation, _rep_vector(self))
    return GaussianCloud(out["xyz"], out["f_dc"], out["scale"], out["rotation"], out["opacity"])


def _decode(self, cond, cond_rows, num_gaussians, level, seed):
    """Decoders::decode (src/decoders.cpp:434-442): sample_anchors, gaussian_features, to_gaussians; num_gaussians
    rounded down to a multiple of per_anchor (at least one anchor)."""
    G = self.cfg.per_anchor
    anchors = max(1, num_gaussians // G)
    points = torch.from_numpy(self.sample_anchors(cond, cond_rows, anchors, level, seed)).to(self.device)
    cond_t = self._f32(cond, "cond")[:cond_rows]
    features = self.gaussian_features(points, anchors, cond_t, cond_rows)
    return self.to_gaussians(points, anchors, features)


Decoders.sample_anchors = _sample_anchors
Decoders.to_gaussians = _to_gaussians
Decoders.decode = _decode


def write_gaussian_ply(cloud, path):
    """A binary little-endian 3DGS PLY of the cloud, turned from z-up to y-up ((x, y, z) -> (x, -z, y), the rotation
    premultiplied by +90 degrees about x), opacity as a logit and scales as logs (src/decoders.cpp:444-476)."""
    xyz, f_dc, scale, rot, op = (np.asarray(t.detach().cpu() if isinstance(t, torch.Tensor) else t, np.float32)
                                 for t in (cloud.xyz, cloud.f_dc, cloud.scale, cloud.rotation, cloud.opacity))
    n = op.size
    names = ["x", "y", "z", "nx", "ny", "nz", "f_dc_0", "f_dc_1", "f_dc_2", "opacity", "scale_0", "scale_1",
             "scale_2", "rot_0", "rot_1", "rot_2", "rot_3"]
    head = "ply\nformat binary_little_endian 1.0\nelement vertex %d\n" % n
    head += "".join(f"property float {name}\n" for name in names) + "end_header\n"
    row = np.zeros((n, 17), np.float32)
    xyz, rot = xyz.reshape(n, 3), rot.reshape(n, 4)
    row[:, 0], row[:, 1], row[:, 2] = xyz[:, 0], -xyz[:, 2], xyz[:, 1]
    row[:, 6:9] = f_dc.reshape(n, 3)
    o = np.minimum(np.maximum(op, np.float32(1e-6)), np.float32(1.0) - np.float32(1e-6)).astype(np.float32)
    row[:, 9] = np.log((o / (np.float32(1.0) - o)).astype(np.float64)).astype(np.float32)
    row[:, 10:13] = np.log(np.maximum(scale.reshape(n, 3), np.float32(1e-6)).astype(np.float64)).astype(np.float32)
    h = np.sqrt(np.float32(0.5))
    row[:, 13] = h * rot[:, 0] - h * rot[:, 1]
    row[:, 14] = h * rot[:, 1] + h * rot[:, 0]
    row[:, 15] = h * rot[:, 2] - h * rot[:, 3]
    row[:, 16] = h * rot[:, 3] + h * rot[:, 2]
    with open(path, "wb") as f:
        f.write(head.encode("ascii"))
        f.write(row.astype("<f4").tobytes())
