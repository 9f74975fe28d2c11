"""ctypes bindings for the CPU oracle (liboracle.so) and the reference build (_ref/libidolref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, to check
results against. The product (idol.cpp_amd/) never imports this module.

All functions take and return numpy arrays (C-contiguous). Q8_0 weights are uint8 arrays of n * (k / 32) * 34
bytes; panel blobs are the native layout of the reference's src/kernels.hpp:33-51.
"""
import ctypes
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_LIB = HERE / "liboracle.so"
REF_LIB = HERE / "_ref" / "libidolref.so"

ACT_NONE, ACT_GELU_ERF, ACT_GELU_TANH, ACT_RELU = 0, 1, 2, 3

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_i64 = ctypes.c_int64
_int = ctypes.c_int
_vp = ctypes.c_void_p


def _ptr(a):
    """A raw pointer for optional arguments (None -> NULL)."""
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


_oracle = None
_ref = None


def oracle_lib():
    global _oracle
    if _oracle is None:
        if not ORACLE_LIB.exists():
            raise RuntimeError(f"{ORACLE_LIB} is not built: run `make -C oracle oracle`")
        lib = ctypes.CDLL(str(ORACLE_LIB))
        lib.orc_half_to_float_n.argtypes = [_u16p, _i64, _f32p]
        lib.orc_float_to_half_n.argtypes = [_f32p, _i64, _u16p]
        lib.orc_q8_0_quantize.argtypes = [_f32p, _i64, _i64, _u8p]
        lib.orc_q8_0_dequant.argtypes = [_u8p, _i64, _i64, _f32p]
        lib.orc_q8_0_to_panel.argtypes = [_u8p, _i64, _i64, _u8p]
        lib.orc_q8_0_to_panel.restype = _int
        lib.orc_panel_bytes.argtypes = [_i64, _i64]
        lib.orc_panel_bytes.restype = _i64
        gemm_args = [_f32p, _i64, _u8p, _i64, _i64, _vp, _i64, _i64, _vp, _int, _f32p]
        lib.orc_gemm_q8_float.argtypes = gemm_args
        lib.orc_gemm_q8_int8.argtypes = gemm_args
        lib.orc_gemm_dense.argtypes = [_f32p, _i64, _f32p, _i64, _i64, _vp, _i64, _i64, _int, _f32p]
        lib.orc_quantize_act.argtypes = [_f32p, _i64, _i64, _i8p, _f32p, _i32p]
        lib.orc_block_dots.argtypes = [_i8p, _i64, _u8p, _i64, _i64, _i64, _i32p]
        lib.orc_layer_norm.argtypes = [_f32p, _i64, _i64, _f32p, _f32p, _f32p]
        lib.orc_norm_rows.argtypes = [_f32p, _f32p, _i64, _i64, ctypes.c_float, _vp, _vp, _vp, _vp, _i64]
        lib.orc_attention.argtypes = [_vp, _i64, _i64, _vp, _vp, _i64, _i64, _i64, _i64, _f32p, _i64]
        lib.orc_exp256.argtypes = [_f32p, _i64, _f32p]
        lib.orc_gelu_erf.argtypes = [_f32p, _i64, _f32p]
        lib.orc_gelu_scalar.argtypes = [_f32p, _i64, _f32p]
        lib.orc_gelu_tanh.argtypes = [_f32p, _i64]
        lib.orc_pos_embed.argtypes = [_f32p, _i64, _f32p, _i64, _vp, _i64]
        _oracle = lib
    return _oracle


def ref_available():
    return REF_LIB.exists()


def ref_lib():
    global _ref
    if _ref is None:
        if not REF_LIB.exists():
            raise RuntimeError(f"{REF_LIB} is not built (needs the reference checkout): `make -C oracle ref`")
        lib = ctypes.CDLL(str(REF_LIB))
        lib.ref_quant_int8_supported.restype = _int
        lib.ref_gemm_panel.argtypes = [_f32p, _int, _u8p, _i64, _f32p, _int, _int, _int, _int, _int, _int, _vp, _int,
                                       _f32p, _int]
        lib.ref_gemm_panel.restype = _int
        lib.ref_gemm_dense.argtypes = [_f32p, _int, _f32p, _f32p, _int, _int, _int, _int, _vp, _int, _f32p]
        lib.ref_gemm_dense.restype = _int
        lib.ref_dequantize_panel.argtypes = [_u8p, _i64, _int, _int, _int, _int, _f32p]
        lib.ref_dequantize_panel.restype = _int
        lib.ref_quant_panel_bytes.argtypes = [_int, _int, _int]
        lib.ref_quant_panel_bytes.restype = _i64
        lib.ref_quantize_activations.argtypes = [_f32p, _int, _int, _i8p, _f32p, _i32p]
        lib.ref_quantize_activations.restype = _int
        lib.ref_layer_norm.argtypes = [_f32p, _int, _int, _f32p, _f32p, _f32p]
        lib.ref_norm_rows.argtypes = [_f32p, _f32p, _int, _int, ctypes.c_float, _vp, _vp, _vp, _vp]
        lib.ref_attention.argtypes = [_vp, _int, _int, _vp, _vp, _int, _int, _int, _int, _f32p, _int]
        lib.ref_gelu_tanh.argtypes = [_f32p, _i64]
        lib.ref_exp256.argtypes = [_f32p, _i64, _f32p]
        lib.ref_gelu256.argtypes = [_f32p, _i64, _f32p]
        lib.ref_gelu_scalar.argtypes = [_f32p, _i64, _f32p]
        lib.ref_last_error.restype = ctypes.c_char_p
        lib.ref_set_quant_kernel.argtypes = [_int]
        lib.ref_uniform_floats.argtypes = [ctypes.c_uint64, _i64, _f32p, _vp]
        lib.ref_decoders_sample_anchors.argtypes = [_vp, _f32p, _int, _int, _int, ctypes.c_uint64, _f32p]
        lib.ref_decoders_sample_anchors.restype = _int
        lib.ref_decoders_to_gaussians.argtypes = [_vp, _f32p, _int, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p]
        lib.ref_decoders_to_gaussians.restype = _int
        lib.ref_write_gaussian_ply.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, _i64, ctypes.c_char_p]
        lib.ref_write_gaussian_ply.restype = _int
        lib.ref_rms_heads.argtypes = [_f32p, _int, _int, _int, _int, _f32p]
        lib.ref_add_gated.argtypes = [_f32p, _f32p, _int, _int, _f32p]
        lib.ref_decoders_open.argtypes = [ctypes.c_char_p]
        lib.ref_decoders_open.restype = _vp
        lib.ref_decoders_close.argtypes = [_vp]
        lib.ref_decoders_config.argtypes = [_vp, _i32p]
        lib.ref_decoders_weight_bytes.argtypes = [_vp]
        lib.ref_decoders_weight_bytes.restype = _i64
        lib.ref_decoders_octree_logits.argtypes = [_vp, _f32p, _int, ctypes.c_float, _f32p, _int, _f32p]
        lib.ref_decoders_octree_logits.restype = _int
        lib.ref_decoders_gaussian_features.argtypes = [_vp, _f32p, _int, _f32p, _int, _f32p]
        lib.ref_decoders_gaussian_features.restype = _int
        _ref = lib
    return _ref


# ------------------------------------------------------------------------------------------------ oracle wrappers
def half_to_float(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    oracle_lib().orc_half_to_float_n(h.reshape(-1), h.size, out.reshape(-1))
    return out


def float_to_half(f):
    f = _f32(f)
    out = np.empty(f.shape, np.uint16)
    oracle_lib().orc_float_to_half_n(f.reshape(-1), f.size, out.reshape(-1))
    return out


def q8_0_quantize(w):
    w = _f32(w)
    n, k = w.shape
    if k % 32:
        raise ValueError("Q8_0 needs k % 32 == 0")
    out = np.empty(n * (k // 32) * 34, np.uint8)
    oracle_lib().orc_q8_0_quantize(w, n, k, out)
    return out


def q8_0_dequant(blocks, n, k):
    out = np.empty((n, k), np.float32)
    oracle_lib().orc_q8_0_dequant(np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1), n, k, out)
    return out


def panel_bytes(n, k):
    return int(oracle_lib().orc_panel_bytes(n, k))


def q8_0_to_panel(blocks, n, k):
    out = np.empty(panel_bytes(n, k), np.uint8)
    rc = oracle_lib().orc_q8_0_to_panel(np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1), n, k, out)
    if rc != 0:
        raise ValueError("GGUF scale cannot be represented exactly in native layout")
    return out


def _gemm(fn, a, w, n_total, k, bias, n_offset, n, residual, gelu):
    a = _f32(a)
    m = a.shape[0]
    if n is None:
        n = n_total - n_offset
    bias = None if bias is None else _f32(bias)
    residual = None if residual is None else _f32(residual)
    c = np.empty((m, n), np.float32)
    fn(a, m, np.ascontiguousarray(w, dtype=np.uint8).reshape(-1), n_total, k, _ptr(bias), n_offset, n,
       _ptr(residual), int(gelu), c)
    return c


def gemm_q8_float(a, w, n_total, k, bias=None, n_offset=0, n=None, residual=None, gelu=False):
    """Reference float kernel semantics (gemm_packed, IDOL_QUANT_KERNEL=float) on Q8_0 blocks."""
    return _gemm(oracle_lib().orc_gemm_q8_float, a, w, n_total, k, bias, n_offset, n, residual, gelu)


def gemm_dense(a, weight, bias=None, gelu=False):
    """Reference dense gemm_packed semantics (unquantized fp32 weight [n, k]): 32-deep chunked FMA sums."""
    a, weight = _f32(a), _f32(weight)
    m, k = a.shape
    n = weight.shape[0]
    c = np.empty((m, n), np.float32)
    b = _f32(bias) if bias is not None else None
    oracle_lib().orc_gemm_dense(a, m, weight, n, k, _ptr(b), 0, n, int(gelu), c)
    return c


def gemm_q8_int8(a, w, n_total, k, bias=None, n_offset=0, n=None, residual=None, gelu=False):
    """Reference integer kernel semantics (gemm_packed with AVX-VNNI) on Q8_0 blocks."""
    return _gemm(oracle_lib().orc_gemm_q8_int8, a, w, n_total, k, bias, n_offset, n, residual, gelu)


def quantize_act(a):
    a = _f32(a)
    m, k = a.shape
    qa = np.empty((m, k), np.int8)
    sa = np.empty((m, k // 32), np.float32)
    qs = np.empty((m, k // 32), np.int32)
    oracle_lib().orc_quantize_act(a, m, k, qa, sa, qs)
    return qa, sa, qs


def block_dots(qa, w, k, n_offset, n):
    qa = np.ascontiguousarray(qa, dtype=np.int8)
    m = qa.shape[0]
    out = np.empty((m, n, k // 32), np.int32)
    oracle_lib().orc_block_dots(qa, m, np.ascontiguousarray(w, dtype=np.uint8).reshape(-1), n_offset, n, k, out)
    return out


def layer_norm(x, gamma, beta):
    x = _f32(x)
    y = np.empty_like(x)
    oracle_lib().orc_layer_norm(x, x.shape[0], x.shape[1], _f32(gamma), _f32(beta), y)
    return y


def norm_rows(x, eps, gamma=None, beta=None, shift=None, scale=None, rows_per_batch=0):
    x = _f32(x)
    y = np.empty_like(x)
    args = [None if v is None else _f32(v) for v in (gamma, beta, shift, scale)]
    oracle_lib().orc_norm_rows(x, y, x.shape[0], x.shape[1], eps, *[_ptr(v) for v in args], rows_per_batch)
    return y


def attention(q, k, v, lq, lk, ldq, ldkv, heads, head_dim):
    """q, k, v are flat fp32 buffers of lq * ldq and lk * ldkv values. Returns [lq, heads * head_dim]."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    dim = heads * head_dim
    if q.size < (lq - 1) * ldq + dim or k.size < (lk - 1) * ldkv + dim or v.size < (lk - 1) * ldkv + dim:
        raise ValueError("attention buffers are smaller than their rows and strides")
    out = np.empty((lq, dim), np.float32)
    oracle_lib().orc_attention(_ptr(q), lq, ldq, _ptr(k), _ptr(v), lk, ldkv, heads, head_dim, out, dim)
    return out


def exp256(x):
    x = _f32(x).reshape(-1)
    y = np.empty_like(x)
    oracle_lib().orc_exp256(x, x.size, y)
    return y


def gelu_erf(x):
    x = _f32(x).reshape(-1)
    y = np.empty_like(x)
    oracle_lib().orc_gelu_erf(x, x.size, y)
    return y


def gelu_scalar(x):
    x = _f32(x).reshape(-1)
    y = np.empty_like(x)
    oracle_lib().orc_gelu_scalar(x, x.size, y)
    return y


def gelu_tanh(x):
    y = _f32(x).copy()
    oracle_lib().orc_gelu_tanh(y.reshape(-1), y.size)
    return y


def pos_embed(freqs, coords, out=None, ldo=None):
    freqs, coords = _f32(freqs), _f32(coords)
    rows = coords.shape[0]
    width = 6 * freqs.size
    if out is None:
        out = np.zeros((rows, width), np.float32)
        ldo = width
    oracle_lib().orc_pos_embed(freqs, freqs.size, coords.reshape(-1), rows, _ptr(out), ldo)
    return out


# ------------------------------------------------------------------------------------------------ reference wrappers
def ref_int8_supported():
    return bool(ref_lib().ref_quant_int8_supported())


def ref_gemm_panel(a, blob, bias, out, inp, n_offset=0, n=None, residual=None, gelu=False, mode=0, bits=8, group=32):
    a = _f32(a)
    m = a.shape[0]
    if n is None:
        n = out - n_offset
    bias = _f32(np.zeros(out) if bias is None else bias)
    residual = None if residual is None else _f32(residual)
    c = np.empty((m, n), np.float32)
    blob = np.ascontiguousarray(blob, dtype=np.uint8)
    rc = ref_lib().ref_gemm_panel(a, m, blob, blob.size, bias, out, inp, bits, group, n_offset, n, _ptr(residual),
                                  int(gelu), c, mode)
    if rc != 0:
        raise ValueError("reference quantized_linear rejected the blob")
    return c


def ref_gemm_dense(a, weight, bias, n_offset=0, n=None, residual=None, gelu=False):
    a, weight, bias = _f32(a), _f32(weight), _f32(bias)
    m = a.shape[0]
    out, inp = weight.shape
    if n is None:
        n = out - n_offset
    residual = None if residual is None else _f32(residual)
    c = np.empty((m, n), np.float32)
    ref_lib().ref_gemm_dense(a, m, weight, bias, out, inp, n_offset, n, _ptr(residual), int(gelu), c)
    return c


def ref_dequantize_panel(blob, out, inp, bits=8, group=32):
    w = np.empty((out, inp), np.float32)
    blob = np.ascontiguousarray(blob, dtype=np.uint8)
    if ref_lib().ref_dequantize_panel(blob, blob.size, out, inp, bits, group, w) != 0:
        raise ValueError("reference quantized_linear rejected the blob")
    return w


def ref_quantize_activations(a):
    a = _f32(a)
    m, k = a.shape
    qa = np.empty((m, k), np.int8)
    sa = np.empty((m, k // 32), np.float32)
    qs = np.empty((m, k // 32), np.int32)
    if ref_lib().ref_quantize_activations(a, m, k, qa, sa, qs) != 0:
        raise RuntimeError("reference built without the integer kernel")
    return qa, sa, qs


def ref_layer_norm(x, gamma, beta):
    x = _f32(x)
    y = np.empty_like(x)
    ref_lib().ref_layer_norm(x, x.shape[0], x.shape[1], _f32(gamma), _f32(beta), y)
    return y


def ref_norm_rows(x, eps, gamma=None, beta=None, shift=None, scale=None):
    x = _f32(x)
    y = np.empty_like(x)
    args = [None if v is None else _f32(v) for v in (gamma, beta, shift, scale)]
    ref_lib().ref_norm_rows(x, y, x.shape[0], x.shape[1], eps, *[_ptr(v) for v in args])
    return y


def ref_attention(q, k, v, lq, lk, ldq, ldkv, heads, head_dim):
    q, k, v = _f32(q), _f32(k), _f32(v)
    dim = heads * head_dim
    if q.size < (lq - 1) * ldq + dim or k.size < (lk - 1) * ldkv + dim or v.size < (lk - 1) * ldkv + dim:
        raise ValueError("attention buffers are smaller than their rows and strides")
    out = np.empty((lq, dim), np.float32)
    ref_lib().ref_attention(_ptr(q), lq, ldq, _ptr(k), _ptr(v), lk, ldkv, heads, head_dim, out, dim)
    return out


def ref_gelu_tanh(x):
    y = _f32(x).copy()
    ref_lib().ref_gelu_tanh(y.reshape(-1), y.size)
    return y


def ref_exp256(x):
    x = _f32(x).reshape(-1)
    y = np.empty_like(x)
    ref_lib().ref_exp256(x, x.size, y)
    return y


def ref_gelu256(x):
    x = _f32(x).reshape(-1)
    y = np.empty_like(x)
    ref_lib().ref_gelu256(x, x.size, y)
    return y


def ref_gelu_scalar(x):
    x = _f32(x).reshape(-1)
    y = np.empty_like(x)
    ref_lib().ref_gelu_scalar(x, x.size, y)
    return y


def set_threads(n):
    """OpenMP threads for both libraries (read at the next parallel region)."""
    os.environ["OMP_NUM_THREADS"] = str(n)


def ref_rms_heads(x, heads, head_dim, gamma):
    """src/decoders.cpp:74-86 on a copy of x [rows, ld]."""
    y = _f32(x).copy()
    ref_lib().ref_rms_heads(y, y.shape[0], y.shape[1], heads, head_dim, _f32(gamma))
    return y


def ref_add_gated(x, h, gate):
    """src/decoders.cpp:45-52 on a copy of x [rows, dim]."""
    y = _f32(x).copy()
    ref_lib().ref_add_gated(y, _f32(h), y.shape[0], y.shape[1], _f32(gate))
    return y


class RefDecoders:
    """The reference's idol::Decoders (src/decoders.cpp) over an export directory, on the CPU."""

    def __init__(self, path):
        lib = ref_lib()
        self._h = lib.ref_decoders_open(str(path).encode())
        if not self._h:
            raise RuntimeError(lib.ref_last_error().decode())
        cfg = np.zeros(6, np.int32)
        lib.ref_decoders_config(self._h, cfg)
        self.dim, self.heads, self.oct_blocks, self.gs_blocks, self.cond, self.per_anchor = (int(v) for v in cfg)

    def close(self):
        if self._h:
            ref_lib().ref_decoders_close(self._h)
            self._h = None

    __del__ = close

    def weight_bytes(self):
        return int(ref_lib().ref_decoders_weight_bytes(self._h))

    def octree_logits(self, x, resolution, cond):
        x, cond = _f32(x), _f32(cond)
        out = np.empty((x.shape[0], 8), np.float32)
        if ref_lib().ref_decoders_octree_logits(self._h, x, x.shape[0], resolution, cond, cond.shape[0], out):
            raise RuntimeError(ref_lib().ref_last_error().decode())
        return out

    def sample_anchors(self, cond, num_points, level, seed):
        cond = _f32(cond)
        out = np.empty((num_points, 3), np.float32)
        if ref_lib().ref_decoders_sample_anchors(self._h, cond, cond.shape[0], num_points, level, seed, out):
            raise RuntimeError(ref_lib().ref_last_error().decode())
        return out

    def to_gaussians(self, anchors, features):
        anchors, features = _f32(anchors), _f32(features)
        n = anchors.shape[0] * self.per_anchor
        out = {"xyz": np.empty((n, 3), np.float32), "f_dc": np.empty((n, 3), np.float32),
               "scale": np.empty((n, 3), np.float32), "rotation": np.empty((n, 4), np.float32),
               "opacity": np.empty(n, np.float32)}
        if ref_lib().ref_decoders_to_gaussians(self._h, anchors, anchors.shape[0], features, out["xyz"], out["f_dc"],
                                               out["scale"], out["rotation"], out["opacity"]):
            raise RuntimeError(ref_lib().ref_last_error().decode())
        return out

    def gaussian_features(self, points, cond):
        points, cond = _f32(points), _f32(cond)
        out = np.empty((points.shape[0], self.per_anchor * 15), np.float32)
        if ref_lib().ref_decoders_gaussian_features(self._h, points, points.shape[0], cond, cond.shape[0], out):
            raise RuntimeError(ref_lib().ref_last_error().decode())
        return out


# ------------------------------------------------------------------------------------------------ other block formats
# GGUF block formats restated element by element from the ggml layouts (ggml-quants.c dequantize_row_*), the layouts
# the reference's expansion (tools/idol_packed.py:25-71) and fused kernel (tools/idol_triton.py:48-82) decode: for
# every element e of a block, the byte and bit position of its code and the index of its scale group. Values are
# products and differences in fp32 without fused multiply-adds.
KIND_F16, KIND_Q4_0, KIND_Q8_0, KIND_Q2_K, KIND_Q4_K, KIND_Q6_K = 1, 2, 8, 10, 12, 14
BLOCK_SHAPE = {KIND_Q4_0: (32, 18), KIND_Q8_0: (32, 34), KIND_Q2_K: (256, 84), KIND_Q4_K: (256, 144),
               KIND_Q6_K: (256, 210)}


def _f16(blocks, off):
    return np.ascontiguousarray(blocks[:, off:off + 2]).view("<f2").astype(np.float32)[:, 0]


def blocks_values(raw, kind, n, k):
    """fp32 [n, k] values of GGUF blocks of format `kind` (a uint8 array of n * k / values * bytes)."""
    values, size = BLOCK_SHAPE[kind]
    blocks = np.asarray(raw, np.uint8).reshape(-1, size)
    nb = blocks.shape[0]
    out = np.empty((nb, values), np.float32)
    e = np.arange(values)
    if kind == KIND_Q8_0:
        d = _f16(blocks, 0)
        q = blocks[:, 2:].view(np.int8).astype(np.float32)
        out[:] = d[:, None] * q
    elif kind == KIND_Q4_0:
        d = _f16(blocks, 0)
        byte = blocks[:, 2 + (e % 16)]
        q = np.where(e < 16, byte & 15, byte >> 4).astype(np.int32) - 8
        out[:] = d[:, None] * q.astype(np.float32)
    elif kind == KIND_Q2_K:
        d, dmin = _f16(blocks, 80), _f16(blocks, 82)
        h, s, l = e // 128, (e % 128) // 32, e % 32
        q = (blocks[:, 16 + 32 * h + l] >> (2 * s)) & 3
        pair = blocks[:, e // 16]
        sd = d[:, None] * (pair & 15).astype(np.float32)
        sm = dmin[:, None] * (pair >> 4).astype(np.float32)
        out[:] = sd * q.astype(np.float32) - sm
    elif kind == KIND_Q4_K:
        d, dmin = _f16(blocks, 0), _f16(blocks, 2)
        j = e // 32
        sc = np.empty((nb, 8), np.int32)
        mn = np.empty((nb, 8), np.int32)
        s = blocks[:, 4:16].astype(np.int32)
        for g in range(8):
            if g < 4:
                sc[:, g] = s[:, g] & 63
                mn[:, g] = s[:, g + 4] & 63
            else:
                sc[:, g] = (s[:, g + 4] & 15) | ((s[:, g - 4] >> 6) << 4)
                mn[:, g] = (s[:, g + 4] >> 4) | ((s[:, g] >> 6) << 4)
        byte = blocks[:, 16 + 32 * (j // 2) + e % 32]
        q = np.where(j % 2 == 0, byte & 15, byte >> 4).astype(np.float32)
        sd = d[:, None] * sc[:, j].astype(np.float32)
        sm = dmin[:, None] * mn[:, j].astype(np.float32)
        out[:] = sd * q - sm
    elif kind == KIND_Q6_K:
        d = _f16(blocks, 208)
        h, t, l = e // 128, (e % 128) // 32, e % 32
        lo_byte = blocks[:, 64 * h + 32 * (t % 2) + l]
        lo = np.where(t >= 2, lo_byte >> 4, lo_byte & 15).astype(np.int32)
        hi = ((blocks[:, 128 + 32 * h + l] >> (2 * t)) & 3).astype(np.int32)
        sc = blocks[:, 192:208].view(np.int8).astype(np.float32)
        sd = d[:, None] * sc[:, e // 16]
        out[:] = sd * ((lo | (hi << 4)) - 32).astype(np.float32)
    else:
        raise ValueError("unsupported block format")
    return out.reshape(n, k)


def q4_0_to_q8_0(raw, n, k):
    """Q8_0 blocks with the values of Q4_0 blocks: the same fp16 scale, codes q - 8."""
    b4 = np.asarray(raw, np.uint8).reshape(-1, 18)
    out = np.empty((b4.shape[0], 34), np.uint8)
    out[:, :2] = b4[:, :2]
    q = np.concatenate([b4[:, 2:] & 15, b4[:, 2:] >> 4], axis=1).astype(np.int16) - 8
    out[:, 2:] = q.astype(np.int8).view(np.uint8)
    return out.reshape(-1)


def q4_0_quantize(w):
    """Q4_0 blocks of fp32 w [n, k] by ggml's rule: per 32 values, m = the value of largest magnitude, d = m / -8,
    q = min(15, trunc(x / d + 8.5)) (quantize_row_q4_0_ref), d stored as fp16."""
    w = np.asarray(w, np.float32)
    n, k = w.shape
    g = w.reshape(-1, 32)
    idx = np.argmax(np.abs(g), axis=1)
    m = g[np.arange(g.shape[0]), idx]
    d = (m / np.float32(-8.0)).astype(np.float32)
    inv = np.where(d != 0, np.float32(1.0) / np.where(d != 0, d, np.float32(1.0)), np.float32(0.0)).astype(np.float32)
    q = np.minimum(15, np.trunc(g * inv[:, None] + np.float32(8.5)).astype(np.int32)).astype(np.uint8)
    out = np.empty((g.shape[0], 18), np.uint8)
    out[:, :2] = d.astype(np.float16).reshape(-1, 1).view(np.uint8)
    out[:, 2:] = q[:, :16] | (q[:, 16:] << 4)
    return out.reshape(-1)


def ref_uniform_floats(seed, count):
    """(floats, raw 64-bit outputs) of std::mt19937_64(seed) with std::uniform_real_distribution<float>(0, 1)."""
    out = np.empty(count, np.float32)
    raw = np.empty(count, np.uint64)
    ref_lib().ref_uniform_floats(seed, count, out, raw.ctypes.data_as(ctypes.c_void_p))
    return out, raw


def ref_write_gaussian_ply(cloud, path):
    c = {k: _f32(v) for k, v in cloud.items()}
    if ref_lib().ref_write_gaussian_ply(c["xyz"], c["f_dc"], c["scale"], c["rotation"], c["opacity"],
                                        c["opacity"].size, str(path).encode()):
        raise RuntimeError(ref_lib().ref_last_error().decode())
