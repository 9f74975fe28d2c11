"""The decoders' tall-skinny per-point MLP on libidolq: point features and a sine/cosine position embedding of the
point coordinates, three Q8_0 linears with ReLU, and a dense fp32 head.

Shape (the per-point heads of the octree / Gaussian decoders, src/decoders.cpp:232-316, at the synthetic size):
    x   = [features (256) | pos_embed(coords) (3 x 16 x (sin, cos) = 96)]         K = 352 per point
    h1  = relu(x  @ W1^T + b1)     W1 Q8_0 [256 x 352]
    h2  = relu(h1 @ W2^T + b2)     W2 Q8_0 [256 x 256]
    h3  = relu(h2 @ W3^T + b3)     W3 Q8_0 [64 x 256]
    out = h3 @ Wh^T + bh           Wh fp32 [14 x 64] (opacity, scale, rotation, colour)
The embedding follows src/decoders.cpp:215-230 (coordinate by coordinate, sines then cosines, angle (v * f) * pi)
with the frequencies 2^linspace(0, 10, 16) of tools/gguf_to_decoder.py:82-84.

On the GPU the activations between layers are bf16 (the Q8_0 linears run in DEQUANT arithmetic) and the head is fp32.
The first layer's depth is padded from 352 to 384 with zero blocks (and zero input columns) so that the 256-wide layers
read the tiled weight layout (256-column tiles); the padding adds exact zeros. The 64-wide third layer reads the GGUF
row-major blocks, whose kernel tiles 128 (or 64) columns. All buffers are allocated once per point count.

forward() runs all of it in one launch (idolq_point_mlp: 32 points per workgroup, the activations in LDS, the
weights as the bf16 values of their Q8_0 blocks in MFMA fragment order), with the same roundings; forward_layers() is the six-launch route.
"""
import torch

import idolq_lib as L

FEAT, NFREQ, HIDDEN, MID, OUT = 256, 16, 256, 64, 14


def _q8(gen, n, k, std, device):
    return L.quantize_q8_0(torch.randn((n, k), device=device, generator=gen) * std)


class PointMLP:
    def __init__(self, seed=0, device="cuda", feat=FEAT, nfreq=NFREQ, hidden=HIDDEN, mid=MID, out=OUT, wstd=0.05,
                 bstd=0.01):
        gen = torch.Generator(device=device).manual_seed(seed)
        self.device = device
        self.feat, self.nfreq, self.hidden, self.mid, self.out = feat, nfreq, hidden, mid, out
        self.k1 = feat + 6 * nfreq
        self.k1pad = (self.k1 + 63) // 64 * 64
        self.freqs = torch.pow(2.0, torch.linspace(0.0, 10.0, nfreq, dtype=torch.float32)).to(device)
        # Q8_0 weights as GGUF row-major blocks (w) and, for the 256-wide layers, in the tiled layout (wt); layer 1
        # zero-padded in depth
        self.shape = {"l1": (hidden, self.k1), "l2": (hidden, hidden), "l3": (mid, hidden)}
        self.w, self.b = {}, {}
        for name, (n, k) in self.shape.items():
            self.w[name] = _q8(gen, n, k, wstd, device)
            self.b[name] = torch.randn(n, device=device, generator=gen) * bstd
        self.head_w = (torch.randn((out, mid), device=device, generator=gen) * wstd).contiguous()
        self.head_b = torch.randn(out, device=device, generator=gen) * bstd
        pad_blocks = (self.k1pad - self.k1) // 32
        w1 = self.w["l1"].view(hidden, self.k1 // 32, 34)
        w1pad = torch.cat([w1, torch.zeros((hidden, pad_blocks, 34), dtype=torch.uint8, device=device)], dim=1)
        self.wt = {"l1": L.tile_q8_0(w1pad.reshape(-1).contiguous(), hidden, self.k1pad),
                   "l2": L.tile_q8_0(self.w["l2"], hidden, hidden)}
        # the fused kernel's operands: the bf16 values of the Q8_0 weights (the DEQUANT arithmetic's weights)
        self._fusable = (feat, nfreq, hidden, mid) == (FEAT, NFREQ, HIDDEN, MID) and out <= 16
        self.wv = {name: L.dequant(self.w[name], n, k, torch.bfloat16) for name, (n, k) in self.shape.items()}
        self.wp = L.point_mlp_pack(self.wv["l1"], self.wv["l2"], self.wv["l3"]) if self._fusable else None
        self._m = None

    def _buffers(self, m):
        if self._m != m:
            bf16 = torch.bfloat16
            self.x = torch.zeros((m, self.k1pad), device=self.device, dtype=bf16)  # padding columns stay zero
            self.h1 = torch.empty((m, self.hidden), device=self.device, dtype=bf16)
            self.h2 = torch.empty((m, self.hidden), device=self.device, dtype=bf16)
            self.h3 = torch.empty((m, self.mid), device=self.device, dtype=bf16)
            self.y = torch.empty((m, self.out), device=self.device, dtype=torch.float32)
            self._m = m

    def embed(self, feats, coords):
        """x = [features | pos_embed(coords)] as bf16 rows of width k1pad (zero padding)."""
        m = feats.shape[0]
        self._buffers(m)
        L.copy2d(feats, self.x[:, :self.feat])
        L.pos_embed(coords, self.freqs, self.x[:, self.feat:], ldo=self.k1pad)
        return self.x

    def forward(self, feats, coords):
        """[m, 14] fp32 head outputs for fp32 features [m, 256] and coordinates [m, 3]: one launch
        (idolq_point_mlp) for the synthetic size, else the layer-by-layer route."""
        if not self._fusable:
            return self.forward_layers(feats, coords)
        return L.point_mlp(feats, coords, self.freqs, self.wp[0], self.b["l1"], self.wp[1], self.b["l2"], self.wp[2],
                           self.b["l3"], self.head_w, self.head_b)

    def forward_layers(self, feats, coords):
        """The same outputs layer by layer: embedding, three Q8_0 GEMMs, the fp32 head (six launches)."""
        x = self.embed(feats, coords)
        relu, dq = L.ACT_RELU, L.MODE_DEQUANT
        L.gemm(x, self.wt["l1"], self.hidden, bias=self.b["l1"], act=relu, mode=dq, out=self.h1, tiled=True)
        L.gemm(self.h1, self.wt["l2"], self.hidden, bias=self.b["l2"], act=relu, mode=dq, out=self.h2, tiled=True)
        L.gemm(self.h2, self.w["l3"], self.mid, bias=self.b["l3"], act=relu, mode=dq, out=self.h3)
        return L.linear_f32(self.h3, self.head_w, self.head_b, out=self.y)

    def flop(self, m):
        return 2.0 * m * (self.k1 * self.hidden + self.hidden * self.hidden + self.hidden * self.mid + self.mid * self.out)

    def min_bytes(self, m):
        """Bytes a fused implementation must move: fp32 features and coordinates in, fp32 outputs out."""
        return m * (self.feat * 4 + 3 * 4 + self.out * 4)


def inputs(m, seed=1, device="cuda"):
    gen = torch.Generator(device=device).manual_seed(seed)
    feats = torch.randn((m, FEAT), device=device, generator=gen)
    coords = torch.rand((m, 3), device=device, generator=gen) * 2.0 - 1.0
    return feats, coords
