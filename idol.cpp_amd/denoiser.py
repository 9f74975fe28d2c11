"""A synthetic flow-matching denoiser step built only from libidolq's kernels (Q8_0 GEMMs with fused epilogues,
layer norm, attention), standing in for the external idol-sdk denoiser whose linears the reference's fused path
replaces (tools/idol_packed.py PackedLinear -> tools/idol_triton.py fused_linear).

Shape (per layer, hidden D = 1536, 24 heads of 64, MLP 6144, context 1024 tokens of 1280 channels):
    h = adaLN-LN(x)          eps 1e-6, v * (1 + scale[b]) + shift[b] per guidance branch b
    x = x + out(self_attn(qkv(h)))                 Q8_0 qkv [4608 x 1536], out [1536 x 1536]
    h = LN(x)                eps 1e-6
    x = x + cout(cross_attn(cq(h), ckv(ctx)))      Q8_0 cq, cout [1536 x 1536], ckv [3072 x 1280] (K and V rows)
    h = LN(x)                eps 1e-6
    x = x + down(gelu_tanh(up(h)))                 Q8_0 up [6144 x 1536], down [1536 x 6144]
The layer layout follows the Gaussian decoder block of the reference (src/decoders.cpp:284-316: norm, self
attention, norm, cross attention, norm, MLP), with the adaLN modulation of its octree block (:265-276).

Batched guidance: the cond and uncond branches are two sequences of one batch (tools/idol_generate.py:186-193), so
every linear runs on M = 2 * 4096 rows and reads each weight once; attention runs per branch (batch 2).
Activations are bf16; all buffers are allocated once, so a step allocates nothing.
"""
import torch

import idolq_lib as L

D, HEADS, HEAD_DIM, MLP, CTX_DIM = 1536, 24, 64, 6144, 1280


def _q8(gen, n, k, std, device):
    w = torch.randn((n, k), device=device, generator=gen) * std
    return L.quantize_q8_0(w)


class DenoiserLayer:
    """Q8_0 weights (GGUF row-major blocks in `w`; the same blocks in the tiled GEMM layout in `wt`, made once at
    build time) and fp32 biases of one layer."""

    def __init__(self, gen, device, dim=D, mlp=MLP, ctx_dim=CTX_DIM, wstd=0.02, bstd=0.01):
        self.dim, self.mlp, self.ctx_dim = dim, mlp, ctx_dim
        shapes = {"qkv": (3 * dim, dim), "out": (dim, dim), "cq": (dim, dim), "ckv": (2 * dim, ctx_dim),
                  "cout": (dim, dim), "up": (mlp, dim), "down": (dim, mlp)}
        self.w, self.wt, self.b, self.shape = {}, {}, {}, shapes
        for name, (n, k) in shapes.items():
            self.w[name] = _q8(gen, n, k, wstd, device)
            self.b[name] = torch.randn(n, device=device, generator=gen) * bstd
            if k % 64 == 0:
                self.wt[name] = L.tile_q8_0(self.w[name], n, k)

    def linear(self, name, x, out, act=L.ACT_NONE, residual=None, mode=L.MODE_DEQUANT):
        n, _ = self.shape[name]
        if mode == L.MODE_DEQUANT and name in self.wt:
            return L.gemm(x, self.wt[name], n, bias=self.b[name], act=act, residual=residual, mode=mode, out=out,
                          tiled=True, split=True)
        return L.gemm(x, self.w[name], n, bias=self.b[name], act=act, residual=residual, mode=mode, out=out)


class SyntheticDenoiser:
    """layers x DenoiserLayer over a batch of `batch` sequences of `seq` tokens and `ctx_len` context tokens."""

    def __init__(self, layers, batch=2, seq=4096, ctx_len=1024, heads=HEADS, head_dim=HEAD_DIM, mlp=MLP,
                 ctx_dim=CTX_DIM, device="cuda"):
        self.layers = layers
        self.batch, self.seq, self.ctx_len = batch, seq, ctx_len
        self.heads, self.head_dim = heads, head_dim
        self.dim = heads * head_dim
        self.mlp, self.ctx_dim = mlp, ctx_dim
        self.device = device
        self.shift = self.scale = None
        rows, crow = batch * seq, batch * ctx_len
        bf16 = torch.bfloat16
        self.h = torch.empty((rows, self.dim), device=device, dtype=bf16)
        self.qkv = torch.empty((rows, 3 * self.dim), device=device, dtype=bf16)
        self.attn = torch.empty((rows, self.dim), device=device, dtype=bf16)
        self.q = torch.empty((rows, self.dim), device=device, dtype=bf16)
        self.kv = torch.empty((crow, 2 * self.dim), device=device, dtype=bf16)
        self.f = torch.empty((rows, mlp), device=device, dtype=bf16)
        # every layer's context K/V projection in one GEMM per step (see batch_context_kv)
        self.ckv_w = self.ckv_b = self.kv_all = None

    @classmethod
    def build(cls, layers=24, seed=0, batch=2, seq=4096, ctx_len=1024, heads=HEADS, head_dim=HEAD_DIM, mlp=MLP,
              ctx_dim=CTX_DIM, device="cuda"):
        model = cls(None, batch, seq, ctx_len, heads, head_dim, mlp, ctx_dim, device)
        gen = torch.Generator(device=device).manual_seed(seed)
        model.layers = [DenoiserLayer(gen, device, model.dim, mlp, ctx_dim) for _ in range(layers)]
        model.shift = torch.randn((batch, model.dim), device=device, generator=gen) * 0.1
        model.scale = torch.randn((batch, model.dim), device=device, generator=gen) * 0.1
        model.batch_context_kv()
        return model

    def batch_context_kv(self):
        """Every layer reads the same context, so a step projects it for all layers in one GEMM: the layers' tiled
        ckv weights side by side (the tiled layout is whole 32-row groups, so concatenated groups are the tiled
        layout of the stacked matrix) and their biases, into one [batch * ctx_len, layers * 2 * dim] buffer whose
        column slices the layers' cross-attentions read. One launch of len(layers) x 192 tiles fills the CUs where
        each layer's 2048-row projection alone leaves a quarter of them idle; the sums are those of the per-layer
        GEMMs (whole tiles, the same depth order)."""
        if not self.layers or any("ckv" not in layer.wt for layer in self.layers):
            return
        self.ckv_w = torch.cat([layer.wt["ckv"] for layer in self.layers])
        self.ckv_b = torch.cat([layer.b["ckv"] for layer in self.layers])
        self.kv_all = torch.empty((self.batch * self.ctx_len, len(self.layers) * 2 * self.dim), device=self.device,
                                  dtype=torch.bfloat16)

    def inputs(self, seed=1):
        gen = torch.Generator(device=self.device).manual_seed(seed)
        x = torch.randn((self.batch * self.seq, self.dim), device=self.device, generator=gen).bfloat16()
        ctx = torch.randn((self.batch * self.ctx_len, self.ctx_dim), device=self.device, generator=gen).bfloat16()
        return x, ctx

    # ---------------------------------------------------------------------------------------------------- blocks
    def attention_block(self, layer, x, ctx, ada=True, kv=None):
        """Pre-LN self attention and cross attention with residuals, updating x in place. kv: the layer's context
        K and V ([batch * ctx_len, 2 * dim], any row stride) when already projected; otherwise projected here."""
        B, S, Lc, D3 = self.batch, self.seq, self.ctx_len, 3 * self.dim
        D = self.dim
        if ada:
            L.layernorm(x, 1e-6, shift=self.shift, scale=self.scale, rows_per_batch=S, out=self.h)
        else:
            L.layernorm(x, 1e-6, out=self.h)
        layer.linear("qkv", self.h, self.qkv)
        L.attention(self.qkv[:, :D], self.qkv[:, D:2 * D], self.qkv[:, 2 * D:], B, S, S, self.heads,
                    self.head_dim, D3, D3, S * D3, S * D3, self.attn, D, S * D)
        layer.linear("out", self.attn, x, residual=x)
        L.layernorm(x, 1e-6, out=self.h)
        layer.linear("cq", self.h, self.q)
        if kv is None:
            layer.linear("ckv", ctx, self.kv)
            kv = self.kv
        ldkv = kv.stride(0)
        L.attention(self.q, kv[:, :D], kv[:, D:], B, S, Lc, self.heads, self.head_dim, D, ldkv,
                    S * D, Lc * ldkv, self.attn, D, S * D)
        layer.linear("cout", self.attn, x, residual=x)
        return x

    def mlp_block(self, layer, x):
        L.layernorm(x, 1e-6, out=self.h)
        layer.linear("up", self.h, self.f, act=L.ACT_GELU_TANH)
        layer.linear("down", self.f, x, residual=x)
        return x

    def step(self, x, ctx):
        """One denoising step over all layers; x (bf16 [batch * seq, dim]) is updated in place and returned."""
        D2 = 2 * self.dim
        if self.kv_all is not None:
            L.gemm(ctx, self.ckv_w, self.kv_all.shape[1], bias=self.ckv_b, out=self.kv_all, tiled=True, split=True)
        for i, layer in enumerate(self.layers):
            kv = self.kv_all[:, i * D2:(i + 1) * D2] if self.kv_all is not None else None
            self.attention_block(layer, x, ctx, kv=kv)
            self.mlp_block(layer, x)
        return x

    # ---------------------------------------------------------------------------------------------------- work
    def flop_per_layer(self):
        rows, crow, D = self.batch * self.seq, self.batch * self.ctx_len, self.dim
        gemm = 2 * rows * D * (3 * D + D + D + D + 2 * self.mlp) + 2 * crow * self.ctx_dim * 2 * D
        attn = 4 * self.batch * self.heads * self.head_dim * self.seq * (self.seq + self.ctx_len)
        return gemm + attn

    def flop_per_step(self):
        return len(self.layers) * self.flop_per_layer()
