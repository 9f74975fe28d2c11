"""Writes the golden fixtures in this directory from the reference's own CPU kernels.

The reference build is oracle/_ref/libidolref.so (oracle/Makefile compiles the reference's src/kernels.cpp,
src/decoders.cpp and src/weights.cpp where they lie, with the reference's flags, plus -DIDOL_VNNI_PATH=1 for the
integer kernel). Inputs are seeded; each fixture stores its inputs and the reference outputs, so the tests need
neither the reference checkout nor its build.

    make -C oracle && python tests/golden/make_golden.py [fixture names, default all]
"""
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1] / "oracle"))
import oracle as O  # noqa: E402

# (m, n, k, n_offset, n_count, residual, gelu): the reference test's shapes (tests/test_kernels.cpp:111-263), K tails
# around the 32-deep chunk, a column window with residual before GELU, a ragged 14-wide head and K = 352.
GEMM_CASES = [
    (7, 37, 64, 0, 37, False, False),
    (19, 37, 128, 0, 37, False, False),
    (19, 37, 128, 16, 16, True, True),
    (5, 20, 32, 0, 20, False, False),
    (5, 20, 96, 0, 20, True, False),
    (6, 37, 160, 16, 21, True, True),
    (64, 64, 1024, 0, 64, True, True),
    (33, 14, 64, 0, 14, False, True),
    (30, 48, 352, 0, 48, False, False),
    (48, 256, 256, 32, 192, True, False),
]

# (m, n, k, gelu): dense fp32 heads (src/kernels.cpp:566-596), the decoders' 64 -> 14 head among them, K tails.
DENSE_CASES = [(300, 14, 64, False), (37, 5, 100, False), (64, 33, 352, True), (9, 1, 7, False), (40, 32, 512, True)]

ATTN_CASES = [(5, 9, 3, 4), (37, 53, 2, 32), (3, 16, 1, 16), (70, 130, 2, 64), (40, 77, 3, 20), (64, 96, 2, 64)]


def gemm_fixture(rng):
    out = {}
    for i, (m, n, k, off, cnt, res, gelu) in enumerate(GEMM_CASES):
        w = O.q8_0_quantize(rng.normal(0, 0.25, (n, k)).astype(np.float32))
        blob = O.q8_0_to_panel(w, n, k)
        a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
        bias = rng.uniform(-0.5, 0.5, n).astype(np.float32)
        r = rng.uniform(-0.5, 0.5, (m, cnt)).astype(np.float32) if res else None
        y_float = O.ref_gemm_panel(a, blob, bias, n, k, off, cnt, r, gelu, mode=0)
        y_int8 = O.ref_gemm_panel(a, blob, bias, n, k, off, cnt, r, gelu, mode=1)
        case = dict(shape=np.array([m, n, k, off, cnt, int(res), int(gelu)]), a=a, w=w, bias=bias, y_float=y_float,
                    y_int8=y_int8, w_dense=O.ref_dequantize_panel(blob, n, k))
        if r is not None:
            case["residual"] = r
        for key, val in case.items():
            out[f"c{i}_{key}"] = val
    out["cases"] = np.array(len(GEMM_CASES))
    return out


def gemm_dense_fixture(rng):
    out = {}
    for i, (m, n, k, gelu) in enumerate(DENSE_CASES):
        w = rng.normal(0, 0.1, (n, k)).astype(np.float32)
        a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
        bias = rng.uniform(-0.5, 0.5, n).astype(np.float32)
        out[f"c{i}_shape"] = np.array([m, n, k, int(gelu)])
        out[f"c{i}_a"], out[f"c{i}_w"], out[f"c{i}_bias"] = a, w, bias
        out[f"c{i}_y"] = O.ref_gemm_dense(a, w, bias, gelu=gelu)
    out["cases"] = np.array(len(DENSE_CASES))
    return out


def quantize_act_fixture(rng):
    a = np.concatenate([rng.normal(0, 1, (16, 256)), rng.uniform(-3, 3, (16, 256)),
                        np.zeros((1, 256)), np.full((1, 256), 0.5)]).astype(np.float32)
    a[5, 32:64] = 0.0  # an all-zero block inside a row
    a[6, :32] = np.linspace(-127, 127, 32)  # ties after scaling
    qa, sa, qs = O.ref_quantize_activations(a)
    return dict(a=a, qa=qa, sa=sa, qsum=qs)


def norm_fixture(rng):
    x = rng.normal(0.3, 2.0, (9, 1536)).astype(np.float32)
    small = rng.uniform(-2, 2, (5, 24)).astype(np.float32)
    g24, b24 = rng.uniform(-1, 1, 24).astype(np.float32), rng.uniform(-0.5, 0.5, 24).astype(np.float32)
    g, b = rng.normal(1, 0.1, 1536).astype(np.float32), rng.normal(0, 0.1, 1536).astype(np.float32)
    sh, sc = rng.normal(0, 0.1, 1536).astype(np.float32), rng.normal(0, 0.1, 1536).astype(np.float32)
    return dict(x=x, small=small, g24=g24, b24=b24, gamma=g, beta=b, shift=sh, scale=sc,
                layer_norm_small=O.ref_layer_norm(small, g24, b24), layer_norm=O.ref_layer_norm(x, g, b),
                norm_plain=O.ref_norm_rows(x, 1e-6), norm_affine=O.ref_norm_rows(x, 1e-6, gamma=g, beta=b),
                norm_ada=O.ref_norm_rows(x, 1e-6, shift=sh, scale=sc), norm_eps5=O.ref_norm_rows(x, 1e-5))


def attention_fixture(rng):
    out = {}
    for i, (lq, lk, heads, hd) in enumerate(ATTN_CASES):
        dim = heads * hd
        ldq, ldkv = dim + 3, dim + 1  # strided rows as in tests/test_kernels.cpp:184-228
        q = rng.uniform(-1, 1, lq * ldq).astype(np.float32)
        k = rng.uniform(-1, 1, lk * ldkv).astype(np.float32)
        v = rng.uniform(-1, 1, lk * ldkv).astype(np.float32)
        out[f"c{i}_shape"] = np.array([lq, lk, heads, hd, ldq, ldkv])
        out[f"c{i}_q"], out[f"c{i}_k"], out[f"c{i}_v"] = q, k, v
        out[f"c{i}_out"] = O.ref_attention(q, k, v, lq, lk, ldq, ldkv, heads, hd)
    out["cases"] = np.array(len(ATTN_CASES))
    return out


def elementwise_fixture(rng):
    xe = np.concatenate([np.linspace(-20, 20, 4000), rng.uniform(-90, 90, 96)]).astype(np.float32)
    xg = np.concatenate([np.linspace(-6, 6, 1200), rng.normal(0, 3, 1000)]).astype(np.float32)
    xt = rng.normal(0, 3, 1003).astype(np.float32)  # 1003 = 125 * 8 + a scalar tail of 3
    return dict(x_exp=xe, exp256=O.ref_exp256(xe), x_gelu=xg, gelu256=O.ref_gelu256(xg),
                gelu_scalar=O.ref_gelu_scalar(xg), x_tanh=xt, gelu_tanh=O.ref_gelu_tanh(xt))


def main():
    if not O.ref_available():
        raise SystemExit("oracle/_ref/libidolref.so is not built (needs the reference checkout): make -C oracle ref")
    if not O.ref_int8_supported():
        raise SystemExit("this CPU has no AVX-VNNI: the reference's integer kernel cannot run")
    rng = np.random.default_rng(20261201)
    fixtures = {
        "gemm_q8": gemm_fixture(rng),
        "quantize_act": quantize_act_fixture(rng),
        "norm": norm_fixture(rng),
        "attention": attention_fixture(rng),
        "elementwise": elementwise_fixture(rng),
    }
    # added later with a seed of its own, so the fixtures above keep their bytes
    fixtures["gemm_dense"] = gemm_dense_fixture(np.random.default_rng(20261202))
    only = set(sys.argv[1:])
    for name, arrays in fixtures.items():
        if only and name not in only:
            continue
        path = HERE / f"{name}.npz"
        np.savez_compressed(path, **arrays)
        print(f"wrote {path.name}: {path.stat().st_size} bytes")


if __name__ == "__main__":
    main()
