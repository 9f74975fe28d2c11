"""The fused MLP launch (idolq_q8_0_mlp): h bit-identical to the up-projection GEMM, y within the split plans' fp32
reassociation of the two-launch result and within the DEQUANT bar of an fp32 reference, repeatable, the workspace's
counters left at zero, and the argument checks."""
import numpy as np
import pytest
import torch

import idolq_lib as L
from conftest import norm_rel

# A one-launch fused MLP (up tiles and down k-parts taken from one queue, down parts waiting on per-row-block counts
# of finished up tiles) hung on its first GPU run, at m=4096 d=1536 hdim=6144, with no cause shown by reading the
# code; the entry point is not in the library, and these cases stay skipped until a cause is found and fixed.
pytestmark = [pytest.mark.gpu, pytest.mark.skip(reason="fused MLP hung on its first GPU run; cause not found, entry point removed")]
DEV = "cuda"


def _weights(n, k, gen):
    w = 0.02 * torch.randn(n, k, device=DEV, generator=gen)
    q8 = L.quantize_q8_0(w)
    return w, q8, L.tile_q8_0(q8, n, k)


@pytest.mark.parametrize("m,d,hdim,act,res,dtype", [
    (4096, 1536, 6144, L.ACT_GELU_TANH, True, torch.bfloat16),
    (300, 256, 512, L.ACT_GELU_TANH, True, torch.bfloat16),
    (513, 128, 384, L.ACT_RELU, False, torch.float16),
    (64, 64, 128, L.ACT_NONE, True, torch.bfloat16),
    (1000, 512, 2048, L.ACT_GELU_TANH, True, torch.float16),
])
def test_fused_mlp_matches_two_launches(m, d, hdim, act, res, dtype):
    print(f"fused MLP m={m} d={d} hdim={hdim}", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(m + d)
    x = torch.randn(m, d, device=DEV, generator=gen).to(dtype)
    wu, qu, tu = _weights(hdim, d, gen)
    wd, qd, td = _weights(d, hdim, gen)
    bu = 0.01 * torch.randn(hdim, device=DEV, generator=gen)
    bd = 0.01 * torch.randn(d, device=DEV, generator=gen)
    r = x if res else None
    h_ref = L.gemm(x, tu, hdim, bias=bu, act=act, mode=L.MODE_DEQUANT, tiled=True, split=True)
    y_ref = L.gemm(h_ref, td, d, bias=bd, residual=r, mode=L.MODE_DEQUANT, tiled=True, split=True)
    h, y = L.mlp(x, tu, hdim, bu, act, td, bd, residual=r)
    torch.cuda.synchronize()
    assert torch.equal(h, h_ref)
    assert norm_rel(y.float().cpu().numpy(), y_ref.float().cpu().numpy()) < 2e-3
    # the DEQUANT bar against fp32 arithmetic on the dequantized weights
    deq_u = L.dequant(qu, hdim, d, torch.float32)
    deq_d = L.dequant(qd, d, hdim, torch.float32)
    hf = x.float() @ deq_u.T + bu
    if act == L.ACT_GELU_TANH:
        hf = torch.nn.functional.gelu(hf, approximate="tanh")
    elif act == L.ACT_RELU:
        hf = torch.relu(hf)
    yf = hf.to(dtype).float() @ deq_d.T + bd + (x.float() if res else 0)
    assert norm_rel(y.float().cpu().numpy(), yf.cpu().numpy()) < 2e-2
    # repeatable (the last part to arrive adds the others, so sums may differ in the last fp32 bits)
    _, y2 = L.mlp(x, tu, hdim, bu, act, td, bd, residual=r)
    assert norm_rel(y2.float().cpu().numpy(), y.float().cpu().numpy()) < 1e-3
    ws = L._mlp_workspaces[x.device]
    assert int(ws[:4096].sum()) == 0  # queue, counts and error flag back at zero


def test_fused_mlp_argument_checks():
    x = torch.randn(8, 96, device=DEV).bfloat16()
    with pytest.raises(ValueError, match="multiples of 64"):
        L.mlp(x, torch.zeros(10, dtype=torch.uint8, device=DEV), 128, None, L.ACT_NONE,
              torch.zeros(10, dtype=torch.uint8, device=DEV), None)
