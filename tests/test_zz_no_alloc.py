"""idolq_q8_0_gemm_noalloc (the GEMM entry point that allocates nothing; INT8 scratch in a static device array)
through the C ABI against idolq_q8_0_gemm with a caller workspace: the same kernels, so bit-identical outputs, on
two calls in a row (the second smaller, reusing the array the first filled), and the size limit is an error."""
import ctypes

import numpy as np
import pytest
import torch

import idolq_lib as L
import oracle as O

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _call_noalloc(x, w, n_total, n, bias, mode, out, flags=0):
    lib = L.load()
    m, k = x.shape
    return lib.idolq_q8_0_gemm_noalloc(
        ctypes.c_void_p(x.data_ptr()), L.DTYPE_CODE[x.dtype], m, k, x.stride(0), ctypes.c_void_p(w.data_ptr()),
        n_total, 0, n, ctypes.c_void_p(bias.data_ptr()), L.F32, None, 0, 0, L.ACT_GELU_ERF, mode, flags,
        ctypes.c_void_p(out.data_ptr()), L.DTYPE_CODE[out.dtype], out.stride(0),
        ctypes.c_void_p(torch.cuda.current_stream(DEV).cuda_stream))


@pytest.mark.parametrize("mode", [L.MODE_INT8, L.MODE_DEQUANT, L.MODE_EXACT])
def test_noalloc_gemm_matches_the_workspace_gemm(mode):
    rng = np.random.default_rng(40 + mode)
    for m, n, k in ((1024, 768, 2048), (300, 200, 512)):   # the second call smaller than the first
        x32 = rng.standard_normal((m, k)).astype(np.float32)
        x = torch.from_numpy(x32).to(DEV)
        if mode == L.MODE_DEQUANT:
            x = x.bfloat16()
        w = torch.from_numpy(O.q8_0_quantize(rng.normal(0, 0.02, (n, k)).astype(np.float32))).to(DEV)
        b = torch.from_numpy(rng.normal(0, 0.01, n).astype(np.float32)).to(DEV)
        want = L.gemm(x, w, n, bias=b, act=L.ACT_GELU_ERF, mode=mode, out_dtype=torch.float32)
        got = torch.full((m, n), float("nan"), device=DEV)
        assert _call_noalloc(x, w, n, n, b, mode, got) == 0, L.load().idolq_last_error()
        torch.cuda.synchronize()
        assert torch.equal(got, want), (m, n, k)


def test_noalloc_int8_on_tiled_weights_matches_the_workspace_gemm():
    # INT8 on tiled weights takes its codes and scales from the array too (whole tiles): the same bits as the
    # workspace call without split, on two calls in a row, the second smaller
    rng = np.random.default_rng(47)
    for m, n, k in ((1024, 768, 2048), (300, 224, 512)):
        x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(DEV).bfloat16()
        w = torch.from_numpy(O.q8_0_quantize(rng.normal(0, 0.02, (n, k)).astype(np.float32))).to(DEV)
        wt = L.tile_q8_0(w, n, k)
        b = torch.from_numpy(rng.normal(0, 0.01, n).astype(np.float32)).to(DEV)
        want = L.gemm(x, wt, n, bias=b, act=L.ACT_GELU_ERF, mode=L.MODE_INT8, out_dtype=torch.float32, tiled=True)
        got = torch.full((m, n), float("nan"), device=DEV)
        assert _call_noalloc(x, wt, n, n, b, L.MODE_INT8, got, L.FLAG_TILED_WEIGHTS) == 0, L.load().idolq_last_error()
        torch.cuda.synchronize()
        assert torch.equal(got, want), (m, n, k)


def test_noalloc_exact_on_tiled_weights_matches_the_workspace_gemm():
    # EXACT on tiled weights takes its bf16 high and low parts from the array (whole tiles): the same bits as the
    # workspace call without split, on two calls in a row, the second smaller
    rng = np.random.default_rng(48)
    for m, n, k in ((1024, 768, 2048), (300, 224, 512)):
        x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(DEV)
        w = torch.from_numpy(O.q8_0_quantize(rng.normal(0, 0.02, (n, k)).astype(np.float32))).to(DEV)
        wt = L.tile_q8_0(w, n, k)
        b = torch.from_numpy(rng.normal(0, 0.01, n).astype(np.float32)).to(DEV)
        want = L.gemm(x, wt, n, bias=b, act=L.ACT_GELU_ERF, mode=L.MODE_EXACT, out_dtype=torch.float32, tiled=True)
        got = torch.full((m, n), float("nan"), device=DEV)
        assert _call_noalloc(x, wt, n, n, b, L.MODE_EXACT, got, L.FLAG_TILED_WEIGHTS) == 0, L.load().idolq_last_error()
        torch.cuda.synchronize()
        assert torch.equal(got, want), (m, n, k)


def test_noalloc_gemm_rejects_inputs_beyond_its_scratch():
    lib = L.load()
    cap = int(lib.idolq_q8_0_gemm_noalloc_max_bytes())
    assert cap == 32 << 20
    k = 4096
    m = cap // (k * 9 // 8) + 32      # m * k * 9 / 8 bytes exceed the array
    x = torch.zeros((m, k), device=DEV)
    w = torch.zeros(O.q8_0_quantize(np.zeros((32, k), np.float32)).size, device=DEV, dtype=torch.uint8)
    b = torch.zeros(32, device=DEV)
    out = torch.empty((m, 32), device=DEV)
    assert _call_noalloc(x, w, 32, 32, b, L.MODE_INT8, out) == L.EINVAL
    assert b"scratch" in lib.idolq_last_error()
    # EXACT on tiled weights needs m * k * 4 bytes
    m = cap // (4 * k) + 32
    x = torch.zeros((m, k), device=DEV)
    wt = torch.zeros(int(lib.idolq_q8_0_tiled_bytes(32, k)), device=DEV, dtype=torch.uint8)
    out = torch.empty((m, 32), device=DEV)
    assert _call_noalloc(x, wt, 32, 32, b, L.MODE_EXACT, out, L.FLAG_TILED_WEIGHTS) == L.EINVAL
    assert b"EXACT" in lib.idolq_last_error()
