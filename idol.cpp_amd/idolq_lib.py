"""ctypes binding of libidolq.so (include/idolq.h) over PyTorch-ROCm tensors.

PyTorch supplies device memory and the current HIP stream; every computation runs in the library's HIP kernels.
There is no fallback: if the library is missing or a call fails, a Python exception is raised.
"""
import ctypes
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libidolq.so"

F32, F16, BF16 = 0, 1, 2
ACT_NONE, ACT_GELU_ERF, ACT_GELU_TANH, ACT_RELU, ACT_SILU = 0, 1, 2, 3, 4
MODE_AUTO, MODE_DEQUANT, MODE_EXACT, MODE_INT8 = 0, 1, 2, 3
FLAG_ROUND_BEFORE_BIAS, FLAG_TILED_WEIGHTS = 1, 2
EINVAL, ELAUNCH, ENOSUPPORT = -1, -2, -3
KIND_F16, KIND_Q4_0, KIND_Q8_0, KIND_Q2_K, KIND_Q4_K, KIND_Q6_K = 1, 2, 8, 10, 12, 14

DTYPE_CODE = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}
Q8_0_BLOCK, Q8_0_BYTES = 32, 34

_vp, _i64, _int, _sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_size_t

# name: (restype, argtypes)
_SIGNATURES = {
    "idolq_last_error": (ctypes.c_char_p, []),
    "idolq_version": (ctypes.c_char_p, []),
    "idolq_q8_0_bytes": (_i64, [_i64, _i64]),
    "idolq_q8_0_gemm": (_int, [_vp, _int, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _int, _vp, _int, _i64, _int,
                               _int, _int, _vp, _int, _i64, _vp, _sz, _vp]),
    "idolq_q8_0_gemm_workspace": (_sz, [_i64, _i64, _int]),
    "idolq_q8_0_gemm_noalloc": (_int, [_vp, _int, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _int, _vp, _int, _i64,
                                       _int, _int, _int, _vp, _int, _i64, _vp]),
    "idolq_q8_0_gemm_noalloc_max_bytes": (_sz, []),
    "idolq_q8_0_quantize": (_int, [_vp, _i64, _i64, _i64, _vp, _vp]),
    "idolq_q8_0_tiled_bytes": (_i64, [_i64, _i64]),
    "idolq_linear_f32": (_int, [_vp, _int, _i64, _i64, _i64, _vp, _i64, _vp, _int, _vp, _int, _i64, _vp]),
    "idolq_q8_0_tile": (_int, [_vp, _i64, _i64, _vp, _vp]),
    "idolq_q8_0_dequant": (_int, [_vp, _i64, _i64, _vp, _int, _vp]),
    "idolq_quantize_act_q8": (_int, [_vp, _int, _i64, _i64, _i64, _vp, _vp, _vp, _vp]),
    "idolq_q8_0_block_dots": (_int, [_vp, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _vp]),
    "idolq_layernorm": (_int, [_vp, _int, _i64, _i64, _i64, ctypes.c_float, _vp, _vp, _vp, _vp, _i64, _vp, _int, _i64,
                               _vp]),
    "idolq_attention": (_int, [_vp, _vp, _vp, _int, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _int,
                               _i64, _i64, _vp]),
    "idolq_attention_ws": (_int, [_vp, _vp, _vp, _int, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp,
                                  _int, _i64, _i64, _vp, _sz, _vp]),
    "idolq_attention_workspace": (_sz, [_int, _i64, _i64, _i64, _i64]),
    "idolq_activation": (_int, [_vp, _int, _i64, _int, _vp]),
    "idolq_pos_embed": (_int, [_vp, _i64, _vp, _i64, _vp, _int, _i64, _vp]),
    "idolq_point_mlp": (_int, [_vp, _i64, _i64, _vp, _vp, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _vp,
                               _i64, _vp]),
    "idolq_copy2d": (_int, [_vp, _int, _i64, _vp, _int, _i64, _i64, _i64, _vp]),
    "idolq_gemm_f32": (_int, [_vp, _i64, _i64, _i64, _vp, _i64, _vp, _vp, _i64, _int, _vp, _i64, _vp]),
    "idolq_rms_heads": (_int, [_vp, _int, _i64, _i64, _i64, _i64, _vp, _vp]),
    "idolq_add_gated": (_int, [_vp, _int, _i64, _vp, _int, _i64, _i64, _i64, _vp, _vp]),
    "idolq_level_embed": (_int, [ctypes.c_float, _vp, _i64, _vp, _vp]),
    "idolq_blocks_bytes": (_i64, [_int, _i64, _i64]),
    "idolq_to_gaussians": (_int, [_vp, _i64, _vp, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "idolq_blocks_dequant": (_int, [_vp, _int, _i64, _i64, _vp, _int, _vp]),
    "idolq_q4_0_to_q8_0": (_int, [_vp, _i64, _i64, _vp, _vp]),
    "idolq_q4_k_bytes": (_i64, [_i64, _i64]),
    "idolq_q4_k_gemm": (_int, [_vp, _int, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _int, _vp, _int, _i64, _int,
                               _int, _vp, _int, _i64, _vp, _sz, _vp]),
    "idolq_panel_bytes": (_i64, [_i64, _i64, _int, _int]),
    "idolq_panel_expand_f32": (_int, [_vp, _i64, _i64, _i64, _int, _int, _vp, _i64, _vp]),
    "idolq_panel_to_q8_0": (_int, [_vp, _i64, _i64, _i64, _int, _int, _vp, _vp, _vp]),
}

_lib = None


class IdolqError(RuntimeError):
    """A failed library call that is not an argument error (launch failure, unsupported combination)."""


def load():
    """Load libidolq.so (built in-tree by `make -C idol.cpp_amd`); raises if it is absent."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"libidolq is not built: {LIB_PATH} is missing (run `make -C idol.cpp_amd`)")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def exported_symbols():
    return list(_SIGNATURES)


def _check(rc):
    if rc != 0:
        msg = load().idolq_last_error().decode()
        if rc == EINVAL:
            raise ValueError(msg)
        raise IdolqError(msg)


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _code(t):
    try:
        return DTYPE_CODE[t.dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {t.dtype}") from None


def _row_stride(t):
    """Row stride (elements) of a 2-D tensor whose last dimension is unit-stride."""
    if t.dim() != 2 or (t.shape[1] > 1 and t.stride(1) != 1):
        raise ValueError("expected a 2-D tensor with a unit-stride last dimension")
    return max(t.stride(0), t.shape[1]) if t.shape[0] > 1 else t.shape[1]


def _require_shape(t, rows, cols, name):
    """A 2-D [rows, cols] tensor with unit-stride rows: the extent the library reads or writes through its pointer and
    row stride, so a shorter or narrower view cannot send the kernel past the end of its memory."""
    if t is None:
        return
    if t.dim() != 2 or tuple(t.shape) != (rows, cols):
        raise ValueError(f"{name} must be a [{rows}, {cols}] tensor, got {list(t.shape)}")
    if cols > 1 and t.stride(1) != 1:
        raise ValueError(f"{name} needs a unit-stride last dimension")
    if rows > 1 and t.stride(0) < cols:
        raise ValueError(f"{name} rows overlap (row stride {t.stride(0)} < {cols})")


def _require_cuda(*tensors):
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("libidolq works on GPU tensors")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError("all tensors must be on the same device")
    return dev


def q8_0_bytes(n, k):
    return int(load().idolq_q8_0_bytes(n, k))


_split_workspaces = {}


def _split_workspace(device, nbytes):
    """The zero-filled DEQUANT workspace (tile counters, then partial tiles of the split k stages) of the current
    stream of a device, kept for the process: the library leaves it ready for the next call. Each stream has its own,
    so calls on different streams never share counters; calls on one stream run one after another."""
    key = (device, torch.cuda.current_stream(device).cuda_stream)
    ws = _split_workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(nbytes, device=device, dtype=torch.uint8)
        _split_workspaces[key] = ws
    return ws


def split_workspace_of(device):
    """The split workspace of the current stream of `device` (None before the first split call on it)."""
    return _split_workspaces.get((device, torch.cuda.current_stream(device).cuda_stream))


def gemm(x, w, n_total, n_offset=0, n=None, bias=None, residual=None, act=ACT_NONE, mode=MODE_AUTO, flags=0,
         out=None, out_dtype=None, workspace=None, split=False, tiled=False):
    """y = epilogue(x @ W[n_offset:n_offset+n]^T) with W Q8_0 blocks, row-major (GGUF) or, with tiled=True, in the
    layout of tile_q8_0. x is [m, k] (unit-stride rows).

    In DEQUANT mode split=True passes the device's cached workspace, which lets the library split the tiles' k range
    over the CUs (partial tiles); by default whole tiles per workgroup. INT8 mode, and EXACT mode on tiled weights,
    need a workspace (allocated here when none is given); on tiled weights split=True lets them use the rest of that
    workspace the same way."""
    lib = load()
    if x.dim() != 2:
        raise ValueError("x must be a 2-D [m, k] tensor")
    m, k = x.shape
    if n is None:
        n = n_total - n_offset
    _require_shape(out, m, n, "out")
    _require_shape(residual, m, n, "residual")
    dev = _require_cuda(x, w, bias, residual, out, workspace)
    if w.dtype != torch.uint8:
        raise ValueError("Q8_0 weights are a uint8 tensor")
    wbytes = int(lib.idolq_q8_0_tiled_bytes(n_total, k)) if tiled else q8_0_bytes(n_total, k)
    if w.numel() != wbytes or not w.is_contiguous():
        raise ValueError("Q8_0 weight size does not match its shape")
    if tiled:
        flags |= FLAG_TILED_WEIGHTS
    if out is None:
        out = torch.empty((m, n), device=x.device, dtype=out_dtype or x.dtype)
    if bias is not None and (bias.dim() != 1 or bias.numel() != n_total or not bias.is_contiguous()):
        raise ValueError("bias must be a contiguous vector of n_total values")
    eff_mode = mode if mode != MODE_AUTO else (MODE_EXACT if x.dtype == torch.float32 else MODE_DEQUANT)
    ws_bytes = int(lib.idolq_q8_0_gemm_workspace(m, k, eff_mode))
    if eff_mode == MODE_EXACT and not tiled:
        ws_bytes = 0   # the row-major EXACT kernel takes none
    elif eff_mode in (MODE_INT8, MODE_EXACT) and not (tiled and split):
        # the INT8 codes and scales or the EXACT high and low parts alone (the rest of the workspace is the tiled
        # path's split room)
        ws_bytes -= int(lib.idolq_q8_0_gemm_workspace(m, k, MODE_DEQUANT))
    if ws_bytes and (workspace is None or workspace.numel() * workspace.element_size() < ws_bytes):
        if eff_mode == MODE_DEQUANT:
            workspace = _split_workspace(x.device, ws_bytes) if split else None
        else:
            workspace = torch.empty(ws_bytes, device=x.device, dtype=torch.uint8)
    ldr = _row_stride(residual) if residual is not None else 0
    _check(lib.idolq_q8_0_gemm(_ptr(x), _code(x), m, k, _row_stride(x), _ptr(w), n_total, n_offset, n, _ptr(bias),
                               _code(bias) if bias is not None else 0, _ptr(residual),
                               _code(residual) if residual is not None else 0, ldr, act, mode, flags, _ptr(out),
                               _code(out), _row_stride(out), _ptr(workspace) if workspace is not None else None,
                               ws_bytes if workspace is not None else 0,
                               _stream(dev)))
    return out


def q4_k_gemm(x, w, n_total, n_offset=0, n=None, bias=None, residual=None, act=ACT_NONE, flags=0, out=None,
              out_dtype=None, split=False):
    """y = epilogue(x @ W[n_offset:n_offset+n]^T) with W GGUF Q4_K super-blocks, row-major, decoded inside the GEMM
    (idolq_q4_k_gemm). x is bf16 or fp16 [m, k] with unit-stride rows; split=True passes the stream's DEQUANT
    workspace (stream-K)."""
    lib = load()
    if x.dim() != 2:
        raise ValueError("x must be a 2-D [m, k] tensor")
    m, k = x.shape
    if n is None:
        n = n_total - n_offset
    _require_shape(out, m, n, "out")
    _require_shape(residual, m, n, "residual")
    dev = _require_cuda(x, w, bias, residual, out)
    if w.dtype != torch.uint8 or w.numel() != int(lib.idolq_q4_k_bytes(n_total, k)) or not w.is_contiguous():
        raise ValueError("Q4_K weight size does not match its shape")
    if bias is not None and (bias.dim() != 1 or bias.numel() != n_total or not bias.is_contiguous()):
        raise ValueError("bias must be a contiguous vector of n_total values")
    if out is None:
        out = torch.empty((m, n), device=x.device, dtype=out_dtype or x.dtype)
    ws = None
    if split:
        nbytes = int(lib.idolq_q8_0_gemm_workspace(m, k, MODE_DEQUANT))
        ws = _split_workspace(x.device, nbytes)
    ldr = _row_stride(residual) if residual is not None else 0
    _check(lib.idolq_q4_k_gemm(_ptr(x), _code(x), m, k, _row_stride(x), _ptr(w), n_total, n_offset, n, _ptr(bias),
                               _code(bias) if bias is not None else 0, _ptr(residual),
                               _code(residual) if residual is not None else 0, ldr, act, flags, _ptr(out), _code(out),
                               _row_stride(out), _ptr(ws), ws.numel() if ws is not None else 0, _stream(dev)))
    return out


def tiled_q8_0_bytes(n, k):
    """Bytes of the tiled layout of an [n, k] Q8_0 matrix (rows padded to a multiple of 32; 0 unless k % 64 == 0)."""
    return int(load().idolq_q8_0_tiled_bytes(n, k))


def tile_q8_0(w, n, k):
    """The tiled layout (idolq_q8_0_tile) of GGUF Q8_0 blocks of an [n, k] weight: the same blocks, reordered once so
    that each GEMM stage reads contiguous bytes. Needs k % 64 == 0."""
    lib = load()
    _require_cuda(w)
    if w.dtype != torch.uint8 or w.numel() != q8_0_bytes(n, k) or not w.is_contiguous():
        raise ValueError("Q8_0 weight size does not match its shape")
    nbytes = int(lib.idolq_q8_0_tiled_bytes(n, k))
    if nbytes == 0:
        raise ValueError("the tiled layout needs k a multiple of 64")
    out = torch.empty(nbytes, device=w.device, dtype=torch.uint8)
    _check(lib.idolq_q8_0_tile(_ptr(w), n, k, _ptr(out), _stream(w.device)))
    return out


def linear_f32(x, w, bias=None, act=ACT_NONE, out=None, out_dtype=None):
    """Dense fp32 layer y = act(x @ w^T + bias) (narrow heads: n <= 32); x [m, k] any float dtype, w [n, k] fp32."""
    lib = load()
    dev = _require_cuda(x, w, bias, out)
    m, k = x.shape
    n = w.shape[0]
    if w.dtype != torch.float32 or w.shape[1] != k or not w.is_contiguous():
        raise ValueError("w must be a contiguous fp32 [n, k] matrix")
    if bias is not None and (bias.dtype != torch.float32 or bias.numel() != n or not bias.is_contiguous()):
        raise ValueError("bias must be n contiguous fp32 values")
    if out is None:
        out = torch.empty((m, n), device=x.device, dtype=out_dtype or torch.float32)
    _check(lib.idolq_linear_f32(_ptr(x), _code(x), m, k, _row_stride(x), _ptr(w), n, _ptr(bias), act, _ptr(out),
                                _code(out), _row_stride(out), _stream(dev)))
    return out


def quantize_q8_0(w):
    """Q8_0 blocks (uint8, n * k / 32 * 34 bytes) of an fp32 [n, k] GPU matrix."""
    lib = load()
    _require_cuda(w)
    if w.dtype != torch.float32 or w.dim() != 2:
        raise ValueError("quantize_q8_0 takes an fp32 matrix")
    n, k = w.shape
    out = torch.empty(q8_0_bytes(n, k), device=w.device, dtype=torch.uint8)
    _check(lib.idolq_q8_0_quantize(_ptr(w), n, k, _row_stride(w), _ptr(out), _stream(w.device)))
    return out


def dequant(w, n, k, dtype):
    lib = load()
    _require_cuda(w)
    out = torch.empty((n, k), device=w.device, dtype=dtype)
    if w.numel() != q8_0_bytes(n, k):
        raise ValueError("Q8_0 weight size does not match its shape")
    _check(lib.idolq_q8_0_dequant(_ptr(w), n, k, _ptr(out), _code(out), _stream(w.device)))
    return out


def quantize_act(x, with_qsum=True):
    """(qa int8 [m, k], scale fp32 [m, k/32], qsum int32 [m, k/32] or None) of the integer kernel."""
    lib = load()
    _require_cuda(x)
    m, k = x.shape
    qa = torch.empty((m, k), device=x.device, dtype=torch.int8)
    sa = torch.empty((m, k // Q8_0_BLOCK), device=x.device, dtype=torch.float32)
    qs = torch.empty((m, k // Q8_0_BLOCK), device=x.device, dtype=torch.int32) if with_qsum else None
    _check(lib.idolq_quantize_act_q8(_ptr(x), _code(x), m, k, _row_stride(x), _ptr(qa), _ptr(sa), _ptr(qs),
                                     _stream(x.device)))
    return qa, sa, qs


def block_dots(qa, w, n_total, n_offset=0, n=None):
    lib = load()
    _require_cuda(qa, w)
    m, k = qa.shape
    if n is None:
        n = n_total - n_offset
    if w.numel() != q8_0_bytes(n_total, k):
        raise ValueError("Q8_0 weight size does not match its shape")
    dots = torch.empty((m, n, k // Q8_0_BLOCK), device=qa.device, dtype=torch.int32)
    _check(lib.idolq_q8_0_block_dots(_ptr(qa), m, k, _ptr(w), n_total, n_offset, n, _ptr(dots), _stream(qa.device)))
    return dots


def layernorm(x, eps, gamma=None, beta=None, shift=None, scale=None, rows_per_batch=0, out=None, out_dtype=None):
    lib = load()
    if x.dim() != 2:
        raise ValueError("x must be a 2-D [rows, dim] tensor")
    rows, dim = x.shape
    _require_shape(out, rows, dim, "out")
    _require_cuda(x, gamma, beta, shift, scale, out)
    for v in (gamma, beta, shift, scale):
        if v is not None and (v.dtype != torch.float32 or not v.is_contiguous()):
            raise ValueError("gamma, beta, shift and scale are contiguous fp32 tensors")
    batches = (rows + rows_per_batch - 1) // rows_per_batch if rows_per_batch > 0 and rows else 1
    for v, need in ((gamma, dim), (beta, dim), (shift, batches * dim), (scale, batches * dim)):
        if v is not None and v.numel() < need:
            raise ValueError(f"gamma and beta need {dim} values, shift and scale {batches * dim}")
    if out is None:
        out = torch.empty((rows, dim), device=x.device, dtype=out_dtype or x.dtype)
    _check(lib.idolq_layernorm(_ptr(x), _code(x), rows, dim, _row_stride(x), eps, _ptr(gamma), _ptr(beta),
                               _ptr(shift), _ptr(scale), rows_per_batch, _ptr(out), _code(out), _row_stride(out),
                               _stream(x.device)))
    return out


def _attention_workspace(device, nbytes):
    """The attention workspace of the current stream of a device (grown as needed, kept for the process): each call
    writes its V^T tiles before the attention reads them, and calls on one stream run one after another."""
    key = (device, torch.cuda.current_stream(device).cuda_stream)
    ws = _attention_workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(nbytes, device=device, dtype=torch.uint8)
        _attention_workspaces[key] = ws
    return ws


_attention_workspaces = {}


STAGED_V_MIN_KEYS = 2048  # measured: staging V pays from about 32 key tiles (its launch costs ~5 us)


def attention(q, k, v, batch, lq, lk, heads, head_dim, ldq, ldkv, q_bs, kv_bs, out, ldo, o_bs, staged_v=None):
    """Multi-head attention over flat buffers; q/k/v/out may be views into wider projection buffers. bf16 inputs
    with head_dim 64 can stage V once per call as fp16 V^T tiles in the stream's cached workspace (the same output
    bits as converting V in every query workgroup); staged_v=None stages from STAGED_V_MIN_KEYS keys on, True or
    False forces the choice."""
    lib = load()
    dev = _require_cuda(q, k, v, out)
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError("q, k and v must share a dtype")
    if staged_v is None:
        staged_v = lk >= STAGED_V_MIN_KEYS
    need = int(lib.idolq_attention_workspace(_code(q), batch, lk, heads, head_dim)) if staged_v else 0
    ws = _attention_workspace(q.device, need) if need else None
    _check(lib.idolq_attention_ws(_ptr(q), _ptr(k), _ptr(v), _code(q), batch, lq, lk, heads, head_dim, ldq, ldkv,
                                  q_bs, kv_bs, _ptr(out), _code(out), ldo, o_bs, _ptr(ws), need, _stream(dev)))
    return out


def activation(x, act):
    lib = load()
    _require_cuda(x)
    if not x.is_contiguous():
        raise ValueError("activation works in place on a contiguous tensor")
    _check(lib.idolq_activation(_ptr(x), _code(x), x.numel(), act, _stream(x.device)))
    return x


def pos_embed(coords, freqs, out, ldo=None):
    lib = load()
    _require_cuda(coords, freqs, out)
    rows = coords.shape[0]
    if coords.dtype != torch.float32 or freqs.dtype != torch.float32:
        raise ValueError("coords and freqs are fp32")
    if ldo is None:
        ldo = _row_stride(out)
    _check(lib.idolq_pos_embed(_ptr(coords), rows, _ptr(freqs), freqs.numel(), _ptr(out), _code(out), ldo,
                               _stream(coords.device)))
    return out


def _point_mlp_fragments(w):
    """[n, k] bf16 -> MFMA fragment order: fragment (n-tile t, 16-deep chunk c) is 1 KB at (t * k / 16 + c) KB, lane
    l = 32 h + r holding row 32 t + r, depth 16 c + 8 h .. + 8 in its 16 bytes."""
    n, k = w.shape
    return w.reshape(n // 32, 32, k // 16, 2, 8).permute(0, 2, 3, 1, 4).contiguous().reshape(-1)


def point_mlp_pack(w1, w2, w3):
    """The fused per-point MLP's weight operands from the bf16 values of the three Q8_0 layers (w1 [256, 352],
    w2 [256, 256], w3 [64, 256]): each in MFMA fragment order; w3's rows first permuted so that row 32 b + i is
    feature 32 ((i / 4) % 2) + 16 b + 4 (i / 8) + i % 4 (each lane half then holds 32 consecutive features)."""
    for w, shape in ((w1, (256, 352)), (w2, (256, 256)), (w3, (64, 256))):
        if w.dtype != torch.bfloat16 or tuple(w.shape) != shape:
            raise ValueError(f"weights must be bf16 {shape}")
    i = torch.arange(32)
    feat = 32 * ((i >> 2) & 1) + 4 * (i >> 3) + (i & 3)
    order = torch.cat([feat, feat + 16]).to(w3.device)
    return _point_mlp_fragments(w1), _point_mlp_fragments(w2), _point_mlp_fragments(w3[order])


def point_mlp(feats, coords, freqs, w1, b1, w2, b2, w3, b3, wh, bh=None, out=None):
    """The decoders' per-point MLP in one launch: fp32 features [m, 256] and coordinates [m, 3], a 16-frequency
    sine/cosine embedding, three ReLU layers on bf16 weight values packed by point_mlp_pack (from w1 [256, 352],
    w2 [256, 256], w3 [64, 256]; fp32 biases) and an fp32 head wh [nout, 64] (nout <= 16). Returns fp32 [m, nout]."""
    lib = load()
    dev = _require_cuda(feats, coords, freqs, w1, b1, w2, b2, w3, b3, wh, bh, out)
    m = feats.shape[0]
    for w, size in ((w1, 256 * 352), (w2, 256 * 256), (w3, 64 * 256)):
        if w.dtype != torch.bfloat16 or w.numel() != size or not w.is_contiguous():
            raise ValueError("weights must be the contiguous bf16 operands of point_mlp_pack")
    for t in (feats, coords, freqs, b1, b2, b3, wh) + ((bh,) if bh is not None else ()):
        if t.dtype != torch.float32:
            raise ValueError("features, coordinates, frequencies, biases and the head are fp32")
    if (feats.shape[1] != 256 or feats.stride(1) != 1 or not coords.is_contiguous() or tuple(coords.shape) != (m, 3)
            or not (wh.is_contiguous() and wh.shape[1] == 64)):
        raise ValueError("features [m, 256], contiguous coordinates [m, 3] and a contiguous head [nout, 64]")
    nout = wh.shape[0]
    for t, size, name in ((b1, 256, "b1"), (b2, 256, "b2"), (b3, 64, "b3"), (freqs, 16, "freqs")) + \
            (((bh, nout, "bh"),) if bh is not None else ()):
        if t.dim() != 1 or t.numel() != size or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous vector of {size} values")
    if out is None:
        out = torch.empty((m, nout), device=feats.device, dtype=torch.float32)
    elif (out.dtype != torch.float32 or out.dim() != 2 or tuple(out.shape) != (m, nout)
          or (nout > 1 and out.stride(1) != 1) or out.stride(0) < nout):
        raise ValueError(f"out must be fp32 [{m}, {nout}] with unit column stride")
    _check(lib.idolq_point_mlp(_ptr(feats), m, feats.stride(0), _ptr(coords), _ptr(freqs), freqs.numel(), _ptr(w1),
                               _ptr(b1), _ptr(w2), _ptr(b2), _ptr(w3), _ptr(b3), _ptr(wh), _ptr(bh), nout, _ptr(out),
                               out.stride(0), _stream(dev)))
    return out


def copy2d(src, dst):
    lib = load()
    _require_cuda(src, dst)
    rows, cols = src.shape
    if dst.shape != src.shape:
        raise ValueError("copy2d needs equal shapes")
    _check(lib.idolq_copy2d(_ptr(src), _code(src), _row_stride(src), _ptr(dst), _code(dst), _row_stride(dst), rows,
                            cols, _stream(src.device)))
    return dst


def gemm_f32(x, w, bias=None, residual=None, act=ACT_NONE, out=None):
    """Dense fp32 y = act(x @ w^T + bias + residual) in the reference's summation order; residual may be out."""
    lib = load()
    dev = _require_cuda(x, w, bias, residual, out)
    m, k = x.shape
    n = w.shape[0]
    for t, name in ((x, "x"), (w, "w"), (bias, "bias"), (residual, "residual"), (out, "out")):
        if t is not None and t.dtype != torch.float32:
            raise ValueError(f"gemm_f32: {name} must be fp32")
    if w.dim() != 2 or w.shape[1] != k or not w.is_contiguous():
        raise ValueError("w must be a contiguous fp32 [n, k] matrix")
    if bias is not None and (bias.numel() != n or not bias.is_contiguous()):
        raise ValueError("bias must be n contiguous fp32 values")
    _require_shape(out, m, n, "out")
    if out is None:
        out = torch.empty((m, n), device=x.device, dtype=torch.float32)
    if residual is not None and residual.shape != (m, n):
        raise ValueError("residual must be [m, n]")
    ldr = _row_stride(residual) if residual is not None else 0
    _check(lib.idolq_gemm_f32(_ptr(x), m, k, _row_stride(x), _ptr(w), n, _ptr(bias), _ptr(residual), ldr, act,
                              _ptr(out), _row_stride(out), _stream(dev)))
    return out


def rms_heads(x, heads, head_dim, gamma):
    """In place: each head of each row of x [rows, >= heads * head_dim] scaled to norm sqrt(head_dim), times gamma."""
    lib = load()
    _require_cuda(x, gamma)
    if gamma.dtype != torch.float32 or gamma.numel() != heads * head_dim or not gamma.is_contiguous():
        raise ValueError("gamma must be heads * head_dim contiguous fp32 values")
    _check(lib.idolq_rms_heads(_ptr(x), _code(x), x.shape[0], _row_stride(x), heads, head_dim, _ptr(gamma),
                               _stream(x.device)))
    return x


def add_gated(x, h, gate):
    """In place: x += h * gate (gate per column)."""
    lib = load()
    _require_cuda(x, h, gate)
    if h.shape != x.shape:
        raise ValueError("add_gated needs x and h of one shape")
    if gate.dtype != torch.float32 or gate.numel() != x.shape[1] or not gate.is_contiguous():
        raise ValueError("gate must be one contiguous fp32 value per column")
    _check(lib.idolq_add_gated(_ptr(x), _code(x), _row_stride(x), _ptr(h), _code(h), _row_stride(h), x.shape[0],
                               x.shape[1], _ptr(gate), _stream(x.device)))
    return x


def level_embed(resolution, freqs, out=None):
    """[cos | sin] of ((resolution * freqs) * 2) * pi, fp32 [2 * len(freqs)]."""
    lib = load()
    _require_cuda(freqs, out)
    if freqs.dtype != torch.float32 or not freqs.is_contiguous():
        raise ValueError("freqs must be contiguous fp32")
    half = freqs.numel()
    if out is None:
        out = torch.empty(2 * half, device=freqs.device, dtype=torch.float32)
    _check(lib.idolq_level_embed(float(resolution), _ptr(freqs), half, _ptr(out), _stream(freqs.device)))
    return out


def blocks_bytes(kind, n, k):
    return int(load().idolq_blocks_bytes(kind, n, k))


def blocks_dequant(w, kind, n, k, dtype, out=None):
    """The dense [n, k] matrix in `dtype` of GGUF blocks of format `kind` (KIND_*) on the GPU."""
    lib = load()
    _require_cuda(w, out)
    if w.dtype != torch.uint8 or not w.is_contiguous() or w.numel() != blocks_bytes(kind, n, k) or w.numel() == 0:
        raise ValueError("packed weight size does not match its shape and format")
    if out is None:
        out = torch.empty((n, k), device=w.device, dtype=dtype)
    _check(lib.idolq_blocks_dequant(_ptr(w), kind, n, k, _ptr(out), _code(out), _stream(w.device)))
    return out


def q4_0_to_q8_0(w, n, k, out=None):
    """Q8_0 blocks holding exactly the values of Q4_0 blocks [n, k]."""
    lib = load()
    _require_cuda(w, out)
    if w.dtype != torch.uint8 or not w.is_contiguous() or w.numel() != blocks_bytes(KIND_Q4_0, n, k):
        raise ValueError("Q4_0 weight size does not match its shape")
    if out is None:
        out = torch.empty(q8_0_bytes(n, k), device=w.device, dtype=torch.uint8)
    _check(lib.idolq_q4_0_to_q8_0(_ptr(w), n, k, _ptr(out), _stream(w.device)))
    return out


def to_gaussians(anchors, features, per_anchor, perturbation, rep):
    """Activated Gaussians of raw features: dict of xyz, f_dc, scale [n, 3], rotation [n, 4], opacity [n] (fp32)."""
    lib = load()
    _require_cuda(anchors, features, perturbation, rep)
    for t in (anchors, features, perturbation, rep):
        if t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError("to_gaussians takes contiguous fp32 tensors")
    rows = anchors.shape[0]
    if features.shape != (rows, per_anchor * 15) or perturbation.numel() != per_anchor * 3 or rep.numel() != 10:
        raise ValueError("to_gaussians: shapes do not match")
    n = rows * per_anchor
    dev = anchors.device
    out = {"xyz": torch.empty((n, 3), device=dev), "f_dc": torch.empty((n, 3), device=dev),
           "scale": torch.empty((n, 3), device=dev), "rotation": torch.empty((n, 4), device=dev),
           "opacity": torch.empty(n, device=dev)}
    _check(lib.idolq_to_gaussians(_ptr(anchors), rows, _ptr(features), per_anchor, _ptr(perturbation), _ptr(rep),
                                  _ptr(out["xyz"]), _ptr(out["f_dc"]), _ptr(out["scale"]), _ptr(out["rotation"]),
                                  _ptr(out["opacity"]), _stream(dev)))
    return out


def panel_bytes(out, in_, bits, group):
    """Bytes of a native panel blob (0 for an invalid bit width or group)."""
    return int(load().idolq_panel_bytes(out, in_, bits, group))


def panel_expand_f32(blob, out, in_, bits, group, w=None):
    """fp32 [out, in_] values fma(code, scale, min) of a panel blob held on the device (uint8)."""
    lib = load()
    dev = _require_cuda(blob, w)
    if blob.dtype != torch.uint8 or not blob.is_contiguous():
        raise ValueError("a panel blob is a contiguous uint8 tensor")
    if w is None:
        w = torch.empty((out, in_), device=dev, dtype=torch.float32)
    elif w.dtype != torch.float32 or tuple(w.shape) != (out, in_) or (in_ > 1 and w.stride(1) != 1):
        raise ValueError(f"w must be fp32 [{out}, {in_}] with unit column stride")
    _check(lib.idolq_panel_expand_f32(_ptr(blob), blob.numel(), out, in_, bits, group, _ptr(w),
                                      max(w.stride(0), in_), _stream(dev)))
    return w


def panel_to_q8_0(blob, out, in_, bits, group, inexact=None):
    """(Q8_0 blocks, inexact) of a panel blob on the device: the blocks hold the panel's values when the device
    int32 `inexact` (zeroed here unless passed in) ends at zero."""
    lib = load()
    dev = _require_cuda(blob, inexact)
    if blob.dtype != torch.uint8 or not blob.is_contiguous():
        raise ValueError("a panel blob is a contiguous uint8 tensor")
    if in_ % 32:
        raise ValueError("the quantization group must be a multiple of 32 that divides the input size")
    q8 = torch.empty(out * (in_ // 32) * Q8_0_BYTES, device=dev, dtype=torch.uint8)
    if inexact is None:
        inexact = torch.zeros(1, device=dev, dtype=torch.int32)
    _check(lib.idolq_panel_to_q8_0(_ptr(blob), blob.numel(), out, in_, bits, group, _ptr(q8), _ptr(inexact),
                                   _stream(dev)))
    return q8, inexact
