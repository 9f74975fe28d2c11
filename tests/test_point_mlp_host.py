"""The fused per-point MLP's weight packing (idolq_lib.point_mlp_pack), checked element by element against the
fragment order the kernel reads: fragment (row tile t, 16-deep chunk c), 16-byte piece l = 32 h + r holding row
32 t + r, depth 16 c + 8 h .. + 8; the third layer's rows permuted so that each lane half holds 32 consecutive
features."""
import numpy as np
import torch

import idolq_lib as L


def _frag_value(packed, k, t, c, lane, j):
    return packed[((t * (k // 16) + c) * 64 + lane) * 8 + j]


def test_point_mlp_pack_fragment_order():
    gen = torch.Generator().manual_seed(0)
    w1 = torch.randn((256, 352), generator=gen).bfloat16()
    w2 = torch.randn((256, 256), generator=gen).bfloat16()
    w3 = torch.randn((64, 256), generator=gen).bfloat16()
    p1, p2, p3 = L.point_mlp_pack(w1, w2, w3)
    assert p1.numel() == w1.numel() and p2.numel() == w2.numel() and p3.numel() == w3.numel()
    rng = np.random.default_rng(1)
    for w, p in ((w1, p1), (w2, p2)):
        n, k = w.shape
        for _ in range(2000):
            t, c, lane, j = rng.integers(n // 32), rng.integers(k // 16), rng.integers(64), rng.integers(8)
            r, h = lane % 32, lane // 32
            assert _frag_value(p, k, t, c, lane, j) == w[32 * t + r, 16 * c + 8 * h + j]
    # third layer: D row i of tile b (element e = 4 (i / 8) + i % 4 of lane half (i / 4) % 2) is feature 32 h + 16 b + e
    for b in range(2):
        for i in range(32):
            h, e = (i // 4) % 2, 4 * (i // 8) + i % 4
            feature = 32 * h + 16 * b + e
            for c in range(16):
                for hh in range(2):
                    lane = 32 * hh + i
                    got = torch.stack([_frag_value(p3, 256, b, c, lane, j) for j in range(8)])
                    assert torch.equal(got, w3[feature, 16 * c + 8 * hh:16 * c + 8 * hh + 8])
    # every feature appears once
    i = np.arange(32)
    feats = np.concatenate([32 * ((i // 4) % 2) + 16 * b + 4 * (i // 8) + i % 4 for b in range(2)])
    assert sorted(feats.tolist()) == list(range(64))
