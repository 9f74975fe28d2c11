"""Benchmark of the Q8_0 linear path on one MI355X.

A step is one pass of the MLP block the metric is quoted on, on synthetic seeded data resident in HBM:
    x bf16 [4096, 1536] ~ N(0, 1)
    h = gelu_tanh(x @ W_up^T + b_up)      W_up   Q8_0 [6144 x 1536]  (bias and tanh-GELU fused in the epilogue)
    y = h @ W_down^T + b_down + x         W_down Q8_0 [1536 x 6144]  (bias and residual fused in the epilogue)
Weights ~ N(0, 0.02) and biases ~ N(0, 0.01), quantized to Q8_0 on the GPU. value = 2 * 2 * 4096 * 1536 * 6144 FLOP
per step / measured time, in TFLOP/s.

Also reported, in the same JSON line:
  roofline       the GEMM kernel's average launch time from HIP events on its stream over the timed steps;
                 achieved = 2 * M * N * K / launch time against the MFMA peak of the arithmetic it runs; traffic =
                 HBM bytes per launch from the committed rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE summary of the
                 --traffic-probe run (profiles/q8_gemm_mlp_block_traffic.md), scaled by a copy kernel of known size
  pct_int8_peak  value as a fraction of the gfx950 dense int8 MFMA peak (5.0 POP/s), as the metric asks
  denoiser_step_ms  one full synthetic denoiser step (24 layers, batch 2 x 4096 tokens), unless --no-denoiser
  fused_*        fused_linear per fused kind (Q8_0, Q4_0, Q4_K) at the up-projection shape, with bias
  decoders_*     the real model's octree and Gaussian decoders (dim 1024, 16 heads, 4 and 16 blocks, 32 Gaussians per
                 anchor) on 1024 anchors and 8192 latent tokens, fp32 activations, the reference's float-kernel
                 numerics, unless --no-decoders; with the reference's own decoders timed on the host beside them;
  decode_ms      Decoders.decode end to end: 262144 Gaussians (8192 anchors), octree descent to level 8
  int8_*         the same block in INT8 mode (the reference's integer-kernel semantics on int8 MFMA), per GEMM
  layernorm_*    idolq_layernorm at 8192 x 1536 bf16 over rotating buffers larger than the Infinity Cache (HBM GB/s)
  gemv_*         the small-m form at m = 1 and 16 on 4096 x 4096 Q8_0 weights rotating over 428 MB (HBM GB/s)
  cpu_baseline   the reference's own CPU kernels (oracle/_ref, float kernel, its OpenMP threads) on the same MLP block;
                 cpu_baseline_int8 the same with its integer (AVX-VNNI) kernel
"""
import argparse
import json
import os
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "idol.cpp_amd"))

METRIC = "Q8_0 GEMM TFLOP/s (% int8 MFMA peak) + denoiser-step ms at seq 4096, 1 GPU"
PEAK_TFLOPS = {"bf16": 2500.0, "fp16": 2500.0, "int8": 5000.0}
HBM_GBS = 8000.0
M, D, H = 4096, 1536, 6144
# Minimum HBM bytes of one launch: Q8_0 weights (34 B per 32 weights) + bf16 activations in + out (+ bias fp32,
# + residual for the down projection)
ALG_BYTES_UP = H * D // 32 * 34 + M * D * 2 + M * H * 2 + H * 4
ALG_BYTES_DOWN = D * H // 32 * 34 + M * H * 2 + M * D * 2 * 2 + D * 4


def parse():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=30)
    p.add_argument("--mode", choices=["dequant", "exact", "int8"], default="dequant",
                   help="GEMM arithmetic: bf16-dequant MFMA (the reference GPU path's numerics), exact-code bf16 "
                        "MFMA with per-block fp32 scaling, or int8 MFMA on quantized activations")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-denoiser", action="store_true")
    p.add_argument("--no-decoder-mlp", action="store_true")
    p.add_argument("--no-decoders", action="store_true",
                   help="skip the real-size octree and Gaussian decoders (dim 1024, 16 heads, 4 + 16 blocks)")
    p.add_argument("--denoiser-layers", type=int, default=24)
    p.add_argument("--cpu-rows", type=int, default=1024, help="rows of the MLP block the CPU baseline runs")
    p.add_argument("--counter-probe", action="store_true",
                   help="launch only the MLP block's GEMMs in DEQUANT and INT8 mode and the config-2 self- and "
                        "cross-attention, 3 times each, untimed: the program the rocprofv3 --pmc counter passes "
                        "(MFMA busy cycles and ops, VALU instructions) run")
    p.add_argument("--size-sweep", action="store_true",
                   help="time idolq_layernorm (adaLN, bf16, dim 1536), the copy kernel (bf16, width 1536) and the "
                        "small-m GEMV (m = 1, square Q8_0 weights) over a range of sizes, each on rotating buffers "
                        "larger than the Infinity Cache, one JSON line per point: the per-launch fixed cost and the "
                        "rate each kernel approaches")
    p.add_argument("--traffic-probe", action="store_true",
                   help="launch only the calibration copy (512 MiB bf16) and the two GEMMs, 3 times each, untimed: the "
                        "program rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs to measure HBM bytes per launch")
    return p.parse_args()


def cpu_threads():
    """Threads the reference's OpenMP kernels run with: OMP_NUM_THREADS when set, else the cores this process may
    run on (its affinity mask), which is libgomp's default."""
    env = os.environ.get("OMP_NUM_THREADS", "")
    return int(env) if env.isdigit() and int(env) > 0 else len(os.sched_getaffinity(0))


def cpu_note():
    return f"{cpu_threads()} OpenMP threads on {len(os.sched_getaffinity(0))} cores of the process's affinity mask"


def mlp_inputs(torch, L, seed=0):
    gen = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn((M, D), device="cuda", generator=gen).bfloat16()
    w_up = L.quantize_q8_0(torch.randn((H, D), device="cuda", generator=gen) * 0.02)
    w_down = L.quantize_q8_0(torch.randn((D, H), device="cuda", generator=gen) * 0.02)
    b_up = torch.randn(H, device="cuda", generator=gen) * 0.01
    b_down = torch.randn(D, device="cuda", generator=gen) * 0.01
    return x, w_up, w_down, b_up, b_down


class MlpBlock:
    """The MLP block on preallocated buffers. DEQUANT and INT8 read the weights in the tiled Q8_0 layout (the same
    blocks, reordered once at load time; INT8 with its workspace); EXACT reads the GGUF row-major blocks."""

    def __init__(self, torch, L, mode, inputs):
        self.L, self.mode = L, mode
        self.x, w_up, w_down, self.b_up, self.b_down = inputs
        self.tiled = mode in (L.MODE_DEQUANT, L.MODE_INT8)
        self.w_up = L.tile_q8_0(w_up, H, D) if self.tiled else w_up
        self.w_down = L.tile_q8_0(w_down, D, H) if self.tiled else w_down
        self.h = torch.empty((M, H), device="cuda", dtype=torch.bfloat16)
        self.y = torch.empty((M, D), device="cuda", dtype=torch.bfloat16)
        self.ws = None
        if mode == L.MODE_INT8:
            self.ws = torch.empty(L.load().idolq_q8_0_gemm_workspace(M, H, mode), device="cuda", dtype=torch.uint8)

    def up(self):
        self.L.gemm(self.x, self.w_up, H, bias=self.b_up, act=self.L.ACT_GELU_TANH, mode=self.mode, out=self.h,
                    workspace=self.ws, tiled=self.tiled, split=self.tiled)

    def down(self):
        self.L.gemm(self.h, self.w_down, D, bias=self.b_down, residual=self.x, mode=self.mode, out=self.y,
                    workspace=self.ws, tiled=self.tiled, split=self.tiled)


TRAFFIC_FILE = ROOT / "profiles" / "q8_gemm_mlp_block_traffic.md"
COPY_ROWS, COPY_COLS = 16384, 16384  # bf16: 512 MiB read + 512 MiB written, twice the 256 MB Infinity Cache


def run_traffic_probe(args):
    import torch
    import idolq_lib as L

    mode = {"dequant": L.MODE_DEQUANT, "exact": L.MODE_EXACT, "int8": L.MODE_INT8}[args.mode]
    blk = MlpBlock(torch, L, mode, mlp_inputs(torch, L))
    src = torch.empty((COPY_ROWS, COPY_COLS), device="cuda", dtype=torch.bfloat16).fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(3):
        L.copy2d(src, dst)
    torch.cuda.synchronize()
    for _ in range(3):
        blk.up()
        blk.down()
    torch.cuda.synchronize()
    print(json.dumps({"traffic_probe": "done", "copy_bytes": COPY_ROWS * COPY_COLS * 2}), flush=True)


def run_counter_probe(args):
    import torch
    import idolq_lib as L

    inputs = mlp_inputs(torch, L)
    for mode in (L.MODE_DEQUANT, L.MODE_INT8):
        blk = MlpBlock(torch, L, mode, inputs)
        for _ in range(3):
            blk.up()
            blk.down()
        torch.cuda.synchronize()
        del blk
    # config 2's attention: batch 2 x 4096 queries, 24 heads of 64; self over 4096 keys (q, k, v column slices of the
    # [8192, 4608] projection), cross over 1024 context keys (k, v slices of the [2048, 3072] projection)
    gen = torch.Generator(device="cuda").manual_seed(6)
    B, S, Lc, heads, hd = 2, 4096, 1024, 24, 64
    qkv = torch.randn((B * S, 3 * D), device="cuda", generator=gen).bfloat16()
    kv = torch.randn((B * Lc, 2 * D), device="cuda", generator=gen).bfloat16()
    out = torch.empty((B * S, D), device="cuda", dtype=torch.bfloat16)
    for _ in range(3):
        L.attention(qkv[:, :D], qkv[:, D:2 * D], qkv[:, 2 * D:], B, S, S, heads, hd, 3 * D, 3 * D, S * 3 * D,
                    S * 3 * D, out, D, S * D)
    for _ in range(3):
        L.attention(qkv[:, :D], kv[:, :D], kv[:, D:], B, S, Lc, heads, hd, 3 * D, 2 * D, S * 3 * D, Lc * 2 * D,
                    out, D, S * D)
    torch.cuda.synchronize()
    print(json.dumps({"counter_probe": "done"}), flush=True)


def run_size_sweep(args):
    """us per call and GB/s of layer norm, copy and GEMV at growing sizes (rotating buffers of >= 600 MB in total, so
    every call reads HBM): where the rate stops growing with size, the remaining time is per-launch."""
    import torch
    import idolq_lib as L

    gen = torch.Generator(device="cuda").manual_seed(5)
    shift = torch.randn((2, D), device="cuda", generator=gen) * 0.1
    scale = torch.randn((2, D), device="cuda", generator=gen) * 0.1
    for rows in (1024, 2048, 4096, 8192, 16384, 32768, 65536):
        nb = max(2, int(600e6 // (rows * D * 4)))
        xs = [torch.randn((rows, D), device="cuda", generator=gen).bfloat16() for _ in range(nb)]
        ys = [torch.empty_like(x) for x in xs]
        turn = [0]

        def ln():
            i = turn[0] % nb
            turn[0] += 1
            L.layernorm(xs[i], 1e-6, shift=shift, scale=scale, rows_per_batch=rows // 2, out=ys[i])

        def cp():
            i = turn[0] % nb
            turn[0] += 1
            L.copy2d(xs[i], ys[i])

        for name, fn in (("layernorm_adaln_bf16", ln), ("copy_bf16", cp)):
            for _ in range(nb):
                fn()
            us = gpu_time_us(torch, fn, max(20, 3 * nb))
            nbytes = 2 * rows * D * 2
            print(json.dumps({"sweep": name, "rows": rows, "dim": D, "bytes": nbytes, "us": round(us, 2),
                              "gbs": round(nbytes / (us * 1e-6) / 1e9, 1)}), flush=True)
        del xs, ys
    for nk in (2048, 4096, 8192, 16384):
        per = nk * nk // 32 * 34
        nb = max(2, int(600e6 // per))
        ws = [L.quantize_q8_0(torch.randn((nk, nk), device="cuda", generator=gen) * 0.02) for _ in range(nb)]
        x = torch.randn((1, nk), device="cuda", generator=gen).bfloat16()
        y = torch.empty((1, nk), device="cuda", dtype=torch.bfloat16)
        turn = [0]

        def gemv():
            L.gemm(x, ws[turn[0] % nb], nk, mode=L.MODE_DEQUANT, out=y)
            turn[0] += 1

        for _ in range(nb):
            gemv()
        us = gpu_time_us(torch, gemv, max(20, 3 * nb))
        nbytes = per + 4 * nk
        print(json.dumps({"sweep": "gemv_q8_0_m1", "n": nk, "k": nk, "bytes": nbytes, "us": round(us, 2),
                          "gbs": round(nbytes / (us * 1e-6) / 1e9, 1)}), flush=True)
        del ws
    a = torch.zeros((1, 8), device="cuda", dtype=torch.bfloat16)
    b = torch.empty_like(a)
    us = gpu_time_us(torch, lambda: L.copy2d(a, b), 200)
    print(json.dumps({"sweep": "copy_16_bytes", "us": round(us, 2)}), flush=True)


def measured_traffic():
    """HBM bytes per GEMM launch from the committed --pmc summary (lines 'traffic_bytes up=<B> down=<B>'), or None."""
    try:
        text = TRAFFIC_FILE.read_text()
    except OSError:
        return None
    m = re.search(r"traffic_bytes up=(\d+) down=(\d+)", text)
    if not m:
        return None
    up, down = int(m.group(1)), int(m.group(2))
    return {"up": up, "down": down, "mean": (up + down) / 2}


def run_gpu(args):
    import torch
    import idolq_lib as L

    mode = {"dequant": L.MODE_DEQUANT, "exact": L.MODE_EXACT, "int8": L.MODE_INT8}[args.mode]
    inputs = mlp_inputs(torch, L)
    blk = MlpBlock(torch, L, mode, inputs)

    def step(before_up=None, before_down=None):
        if before_up is not None:
            before_up.record()
        blk.up()
        if before_down is not None:
            before_down.record()
        blk.down()

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # Events on the stream the kernels are launched on (torch's current stream, which idolq_lib passes down): one
    # before each up launch, one before each down launch and one after the last step, so that step i's up GEMM is
    # ev[2 i] -> ev[2 i + 1] and its down GEMM ev[2 i + 1] -> ev[2 i + 2] (two markers per step in the queue).
    stream = torch.cuda.current_stream()
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(2 * args.steps + 1)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        for i in range(args.steps):
            step(evs[2 * i], evs[2 * i + 1])
        evs[-1].record()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    up_ms = sum(evs[2 * i].elapsed_time(evs[2 * i + 1]) for i in range(args.steps)) / args.steps
    down_ms = sum(evs[2 * i + 1].elapsed_time(evs[2 * i + 2]) for i in range(args.steps)) / args.steps
    flop_gemm = 2.0 * M * D * H
    ms_per_step = elapsed * 1e3 / args.steps
    value = 2 * flop_gemm / (ms_per_step * 1e-3) / 1e12
    arith = {"dequant": "bf16", "exact": "bf16", "int8": "int8"}[args.mode]
    gemm_ms = (up_ms + down_ms) / 2
    traffic = measured_traffic() if args.mode == "dequant" else None
    achieved = flop_gemm / (gemm_ms * 1e-3) / 1e12
    out = {
        "value": value,
        "ms_per_step": ms_per_step,
        "dtype": arith,
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": PEAK_TFLOPS[arith], "unit": "TFLOP/s",
                     "frac": achieved / PEAK_TFLOPS[arith], "traffic": traffic["mean"] if traffic else None,
                     "traffic_per_launch": traffic,
                     "algorithmic_bytes": {"up": ALG_BYTES_UP, "down": ALG_BYTES_DOWN},
                     "kernel": "q8_gemm_kernel" if args.mode == "exact" else "q8_wide_kernel",
                     "launch_ms": {"up": up_ms, "down": down_ms},
                     "flop_per_launch": flop_gemm},
        "pct_int8_peak": value / PEAK_TFLOPS["int8"],
    }
    del blk
    return out, inputs


def run_int8_block(args, inputs):
    """The MLP block in INT8 mode (the reference's integer kernel semantics: activations quantized per row and
    32-block, int8 MFMA block dots, per-block fp32 scale fold; tiled weights, stream-K allowed) on the same inputs:
    per-GEMM launch time from HIP
    events on the launch stream (activation quantization included, it is part of the mode), as TFLOP/s-equivalent
    and as a fraction of the int8 MFMA peak."""
    import torch
    import idolq_lib as L

    blk = MlpBlock(torch, L, L.MODE_INT8, inputs)
    for _ in range(3):
        blk.up()
        blk.down()
    torch.cuda.synchronize()
    steps = max(5, args.steps // 2)
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    for e in evs:
        e[0].record()
        blk.up()
        e[1].record()
        blk.down()
        e[2].record()
    torch.cuda.synchronize()
    up = sum(e[0].elapsed_time(e[1]) for e in evs) / steps
    down = sum(e[1].elapsed_time(e[2]) for e in evs) / steps
    flop = 2.0 * M * D * H
    gemm_ms = (up + down) / 2
    tops = flop / (gemm_ms * 1e-3) / 1e12
    del blk
    return {"int8_gemm_ms": round(gemm_ms, 4), "int8_gemm_ms_up": round(up, 4), "int8_gemm_ms_down": round(down, 4),
            "int8_tops": round(tops, 1), "int8_pct_int8_peak": round(tops / PEAK_TFLOPS["int8"], 4)}


def gpu_time_us(torch, fn, reps):
    """Average GPU microseconds of fn() over `reps` back-to-back calls. The calls are queued behind a GPU spin long
    enough for the host to enqueue all of them, so the events time the GPU's work, not the host's call overhead."""
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(int(2e6 + reps * 1e5))  # clock cycles: ~1 ms + 40 us per call at 2.4 GHz
    start.record()
    for _ in range(reps):
        fn()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / reps * 1e3


LN_ROWS, LN_BUFFERS = 8192, 12  # 12 x (8192 x 1536 bf16 in + out) = 604 MB rotating, over twice the 256 MB cache


def run_layernorm_hbm(args):
    """idolq_layernorm on the denoiser's activation shape (8192 x 1536 bf16, adaLN) over LN_BUFFERS input/output
    pairs used in turn, so successive calls miss the Infinity Cache: ms per call and GB/s of its 2 * rows * dim * 2
    bytes against the 8 TB/s HBM peak."""
    import torch
    import idolq_lib as L

    gen = torch.Generator(device="cuda").manual_seed(5)
    xs = [torch.randn((LN_ROWS, D), device="cuda", generator=gen).bfloat16() for _ in range(LN_BUFFERS)]
    ys = [torch.empty_like(x) for x in xs]
    shift = torch.randn((2, D), device="cuda", generator=gen) * 0.1
    scale = torch.randn((2, D), device="cuda", generator=gen) * 0.1
    turn = [0]

    def call():
        i = turn[0] % LN_BUFFERS
        turn[0] += 1
        L.layernorm(xs[i], 1e-6, shift=shift, scale=scale, rows_per_batch=LN_ROWS // 2, out=ys[i])

    for _ in range(LN_BUFFERS):
        call()
    ms = gpu_time_us(torch, call, 5 * LN_BUFFERS) * 1e-3
    nbytes = 2 * LN_ROWS * D * 2
    return {"layernorm_ms": round(ms, 4), "layernorm_gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "layernorm_hbm_frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_GBS, 3),
            "layernorm_config": f"{LN_ROWS} x {D} bf16 adaLN, {LN_BUFFERS} rotating buffer pairs "
                                f"({LN_BUFFERS * nbytes / 1e6:.0f} MB)"}


GEMV_N, GEMV_K, GEMV_SETS = 4096, 4096, 24  # 24 x 17.8 MB of Q8_0 weights (428 MB), over the 256 MB Infinity Cache


def run_gemv_hbm(args):
    """The small-m form (q8_gemv_kernel) at m = 1 and m = 16, bf16 x, DEQUANT, on GGUF row-major Q8_0 weights
    [4096 x 4096] taken in turn from GEMV_SETS matrices: us per call and GB/s of the bytes a call must move (weights,
    activations, output) against the 8 TB/s HBM peak."""
    import torch
    import idolq_lib as L

    gen = torch.Generator(device="cuda").manual_seed(7)
    ws = [L.quantize_q8_0(torch.randn((GEMV_N, GEMV_K), device="cuda", generator=gen) * 0.02)
          for _ in range(GEMV_SETS)]
    out = {}
    for m in (1, 16):
        x = torch.randn((m, GEMV_K), device="cuda", generator=gen).bfloat16()
        y = torch.empty((m, GEMV_N), device="cuda", dtype=torch.bfloat16)
        turn = [0]

        def call():
            L.gemm(x, ws[turn[0] % GEMV_SETS], GEMV_N, mode=L.MODE_DEQUANT, out=y)
            turn[0] += 1

        for _ in range(GEMV_SETS):
            call()
        us = gpu_time_us(torch, call, 4 * GEMV_SETS)
        nbytes = GEMV_N * GEMV_K // 32 * 34 + m * GEMV_K * 2 + m * GEMV_N * 2
        gbs = nbytes / (us * 1e-6) / 1e9
        out.update({f"gemv_m{m}_us": round(us, 2), f"gemv_m{m}_gbs": round(gbs, 1),
                    f"gemv_m{m}_hbm_frac": round(gbs / HBM_GBS, 3)})
    out["gemv_config"] = (f"Q8_0 [{GEMV_N} x {GEMV_K}] row-major GGUF blocks, bf16 x, DEQUANT, {GEMV_SETS} weight "
                          f"matrices in turn ({GEMV_SETS * GEMV_N * GEMV_K // 32 * 34 / 1e6:.0f} MB)")
    del ws
    return out


def run_denoiser(args):
    """One synthetic denoiser step: 24 layers, batch 2 (guidance pair) x 4096 tokens, context 2 x 1024 x 1280."""
    import torch
    import denoiser

    model = denoiser.SyntheticDenoiser.build(layers=args.denoiser_layers, seed=0)
    x0, ctx = model.inputs(seed=1)
    x = x0.clone()
    for _ in range(2):
        x.copy_(x0)
        model.step(x, ctx)
    torch.cuda.synchronize()
    reps = 5
    times = []
    for _ in range(reps):
        x.copy_(x0)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        model.step(x, ctx)
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    ms = sorted(times)[reps // 2] * 1e3
    flop = model.flop_per_step()
    out = {"denoiser_step_ms": round(ms, 3), "denoiser_tflops": round(flop / (ms * 1e-3) / 1e12, 2),
           "denoiser_layers": args.denoiser_layers}
    return out, model, ctx


DECODER_POINTS = 262144


def run_decoder_mlp(args):
    """The decoders' tall-skinny per-point MLP (352 -> 256 -> 256 -> 64 Q8_0 with ReLU, fp32 64 -> 14 head) on 262144
    points: ms per pass (one launch; the layer-by-layer route beside it), GB/s of the bytes a fused pass must move (fp32 features, coordinates and outputs), TFLOP/s."""
    import torch
    import decoder_mlp

    model = decoder_mlp.PointMLP(seed=0)
    feats, coords = decoder_mlp.inputs(DECODER_POINTS, seed=1)

    def timed(fn, reps=20):
        for _ in range(3):
            fn(feats, coords)
        torch.cuda.synchronize()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(reps):
            fn(feats, coords)
        stop.record()
        torch.cuda.synchronize()
        return start.elapsed_time(stop) / reps

    # one launch (idolq_point_mlp), and the six-launch layer-by-layer route for comparison
    ms = timed(model.forward)
    layers_ms = timed(model.forward_layers)
    out = {"decoder_mlp_ms": round(ms, 4), "decoder_mlp_layers_ms": round(layers_ms, 4),
           "decoder_mlp_points": DECODER_POINTS,
           "decoder_mlp_gbs": round(model.min_bytes(DECODER_POINTS) / (ms * 1e-3) / 1e9, 1),
           "decoder_mlp_tflops": round(model.flop(DECODER_POINTS) / (ms * 1e-3) / 1e12, 2)}
    return out, model


DEC_ROWS, DEC_TOKENS, DEC_LEVEL, DEC_GAUSSIANS = 1024, 8192, 8, 262144


def _decoder_config(oct_blocks=4, gs_blocks=16):
    import idol_export as E
    return E.DecoderConfig(dim=1024, heads=16, oct_blocks=oct_blocks, gs_blocks=gs_blocks, cond=16, per_anchor=32)


def decoder_flop(cfg, rows, tokens):
    """FLOP of one octree_logits and one gaussian_features call (matrix products and attention only)."""
    D, C, H4 = cfg.dim, cfg.cond, 4 * cfg.dim
    kv = 2 * tokens * C * 2 * D
    cross = 2 * rows * D * D * 2 + kv + 4 * rows * tokens * D  # q, out, kv, QK^T and PV
    mlp = 2 * rows * D * H4 * 2
    embed = 2 * rows * (3 * D + D * D)
    oct_ = embed + cfg.oct_blocks * (cross + mlp) + 2 * rows * D * 8
    self_attn = 2 * rows * D * 3 * D + 2 * rows * D * D + 4 * rows * rows * D
    gs = embed + cfg.gs_blocks * (self_attn + cross + mlp) + 2 * rows * D * cfg.per_anchor * 15
    return oct_, gs


def run_decoders(args):
    """The real decoders at the model's size on 1024 anchors and 8192 latent tokens: median ms of 5 calls after a
    warm-up, with the reference's float-kernel numerics (EXACT Q8_0 GEMMs, fp32 attention)."""
    import torch
    import idol_kernels as K
    from decoders import Decoders, synthetic_export

    cfg = _decoder_config()
    dec = Decoders(synthetic_export(cfg, seed=0))
    gen = torch.Generator().manual_seed(1)
    anchors = torch.rand(DEC_ROWS, 3, generator=gen).cuda()
    cond = torch.randn(DEC_TOKENS, cfg.cond, generator=gen).cuda()
    res = float(1 << DEC_LEVEL)
    K.set_quant_kernel(0)
    out = {}
    try:
        for name, fn in (("oct", lambda: dec.octree_logits(anchors, DEC_ROWS, res, cond, DEC_TOKENS)),
                         ("gs", lambda: dec.gaussian_features(anchors, DEC_ROWS, cond, DEC_TOKENS))):
            fn()
            torch.cuda.synchronize()
            times = []
            for _ in range(5):
                t0 = time.perf_counter()
                fn()
                torch.cuda.synchronize()
                times.append(time.perf_counter() - t0)
            out[name] = sorted(times)[2] * 1e3
    finally:
        K.set_quant_kernel(-1)
    # decode end to end (octree descent to level 8 with systematic resampling, the Gaussian decoder on the anchors,
    # activation): 262144 Gaussians = 8192 anchors of 32
    cond_np = cond.cpu().numpy()
    K.set_quant_kernel(0)
    try:
        dec.decode(cond_np, DEC_TOKENS, DEC_GAUSSIANS, DEC_LEVEL, 7)
        torch.cuda.synchronize()
        times = []
        for _ in range(3):
            t0 = time.perf_counter()
            cloud = dec.decode(cond_np, DEC_TOKENS, DEC_GAUSSIANS, DEC_LEVEL, 7)
            torch.cuda.synchronize()
            times.append(time.perf_counter() - t0)
    finally:
        K.set_quant_kernel(-1)
    out["decode"] = sorted(times)[1] * 1e3
    f_oct, f_gs = decoder_flop(cfg, DEC_ROWS, DEC_TOKENS)
    return {"decoders_oct_ms": round(out["oct"], 3), "decoders_gs_ms": round(out["gs"], 3),
            "decode_ms": round(out["decode"], 1), "decode_gaussians": cloud.size(),
            "decoders_tflops": round((f_oct + f_gs) / ((out["oct"] + out["gs"]) * 1e-3) / 1e12, 2),
            "decoders_config": f"dim 1024, 16 heads, 4 octree + 16 Gaussian blocks, 32 per anchor; {DEC_ROWS} anchors, "
                               f"{DEC_TOKENS} latent tokens, fp32, float-kernel numerics"}


def run_fused_kinds(args):
    """The packed-linear surface for each fused kind at the MLP block's up-projection shape, bf16 x [4096, 1536] ->
    [4096, 6144] with bias: PackedLinear layers with the fused path enabled (the reference pipeline's call,
    tools/idol_packed.py:73-82), ms per call (20 calls after 3 warm-ups) and TFLOP/s; beside them fused_linear called
    directly on the GGUF bytes (fused_q8_0_direct_ms) and the tiled-weight GEMM with the same bias and no activation
    (fused_q8_0_tiled_gemm_ms), the kernel the layer's tiled copy runs."""
    from types import SimpleNamespace

    import numpy as np
    import torch
    import idolq_lib as L
    from ggml_types import GGMLQuantizationType as T
    from idol_hip import fused_linear
    from idol_packed import PackedLinear, enable_fused_packed

    gen = torch.Generator(device="cuda").manual_seed(3)
    x = torch.randn(M, D, device="cuda", dtype=torch.bfloat16, generator=gen)
    bias = (0.01 * torch.randn(H, device="cuda", generator=gen)).bfloat16()
    w = 0.02 * torch.randn(H, D, device="cuda", generator=gen)
    q8 = L.quantize_q8_0(w)
    rng = np.random.default_rng(4)
    q4k = rng.integers(0, 256, size=(H * D // 256, 144), dtype=np.uint8)
    q4k[:, :4] = np.frombuffer(np.array([0.001, 0.0005], np.float16).tobytes(), np.uint8)
    # Q4_0 blocks of the same weights: scale = max-magnitude value / -8, codes clipped to 0..15 (ggml's rule)
    g = w.reshape(-1, 32)
    m = g.gather(1, g.abs().argmax(1, keepdim=True))
    d = (m / -8.0).half()
    inv = torch.where(d != 0, 1.0 / d.float(), torch.zeros_like(d, dtype=torch.float32))
    q = torch.clamp(torch.trunc(g * inv + 8.5), max=15).to(torch.uint8)
    q4 = torch.cat([d.view(torch.uint8).reshape(-1, 2), q[:, :16] | (q[:, 16:] << 4)], dim=1).reshape(-1)

    def timed(fn):
        with torch.no_grad():
            for _ in range(3):
                fn()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(20):
                fn()
            torch.cuda.synchronize()
        return (time.perf_counter() - t0) / 20 * 1e3

    out = {}
    for name, kind, packed in (("q8_0", T.Q8_0, q8), ("q4_0", T.Q4_0, q4), ("q4_k", T.Q4_K, torch.from_numpy(q4k))):
        layer = PackedLinear(SimpleNamespace(shape=np.array([D, H]), tensor_type=kind,
                                             data=packed.cpu().numpy().reshape(-1)), bias).to("cuda")
        enable_fused_packed(layer)
        ms = timed(lambda: layer(x))
        out[f"fused_{name}_ms"] = round(ms, 4)
        out[f"fused_{name}_tflops"] = round(2.0 * M * D * H / (ms * 1e-3) / 1e12, 1)
    out["fused_q8_0_direct_ms"] = round(timed(lambda: fused_linear(x, q8, (H, D), 8, bias)), 4)
    tiled, b32 = L.tile_q8_0(q8, H, D), bias.float()
    y = torch.empty((M, H), device="cuda", dtype=torch.bfloat16)
    out["fused_q8_0_tiled_gemm_ms"] = round(timed(lambda: L.gemm(x, tiled, H, bias=b32, mode=L.MODE_DEQUANT, out=y,
                                                                  flags=L.FLAG_ROUND_BEFORE_BIAS, tiled=True)), 4)
    out["fused_note"] = ("PackedLinear layers (fused path enabled) at bf16 [4096, 1536] -> 6144 with bias; Q8_0 and "
                         "Q4_0 run their tiled Q8_0 copy, Q4_K its GGUF super-blocks")
    return out


def run_cpu_decoders():
    """The reference's own idol::Decoders (oracle/_ref) on the host, same rows and tokens, all host cores. A bounded
    sample: exports of the model's width with 1 and with 2 blocks per decoder are timed (median of 3 after a
    warm-up); the per-block time is their difference, and the 4 + 16-block time is extrapolated from it."""
    import tempfile
    import numpy as np
    import torch
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as O
    import idol_export as E
    from decoders import synthetic_export

    if not O.ref_available():
        return {}
    gen = torch.Generator().manual_seed(1)
    anchors = torch.rand(DEC_ROWS, 3, generator=gen).numpy()
    cond = torch.randn(DEC_TOKENS, 16, generator=gen).numpy()
    res = float(1 << DEC_LEVEL)
    times = {}
    with tempfile.TemporaryDirectory(prefix="idolq-dec-") as tmp:
        for nb in (1, 2):
            ex = synthetic_export(_decoder_config(nb, nb), seed=0)
            q = {name: E.QTensor(t.out, t.in_, 8, 32, O.q8_0_to_panel(t.blob.cpu().numpy(), t.out, t.in_))
                 for name, t in ex.qtensors.items()}
            dense = {name: t.data.reshape(t.shape) for name, t in ex.tensors.items()}
            path = Path(tmp) / f"b{nb}"
            E.write_export(path, ex.decoder_config, dense, q, rep=E.Representation())
            del ex, q, dense
            ref = O.RefDecoders(path)
            O.ref_lib().ref_set_quant_kernel(0)
            for name, fn in (("oct", lambda: ref.octree_logits(anchors, res, cond)),
                             ("gs", lambda: ref.gaussian_features(anchors, cond))):
                fn()
                ts = []
                for _ in range(3):
                    t0 = time.perf_counter()
                    fn()
                    ts.append(time.perf_counter() - t0)
                times[(name, nb)] = float(np.median(ts))
            O.ref_lib().ref_set_quant_kernel(-1)
            ref.close()
    oct_s = times[("oct", 1)] + 3 * (times[("oct", 2)] - times[("oct", 1)])
    gs_s = times[("gs", 1)] + 15 * (times[("gs", 2)] - times[("gs", 1)])
    return {"decoders_cpu_oct_ms_est": round(oct_s * 1e3, 1), "decoders_cpu_gs_ms_est": round(gs_s * 1e3, 1),
            "decoders_cpu_cores": cpu_threads(),
            "decoders_cpu_note": "reference idol::Decoders, float kernel, model width with 1 and 2 blocks timed "
                                 "(median of 3 after 1 warm-up), 4 + 16 blocks extrapolated from the per-block time"}


def run_cpu_decoder_mlp(model, sample=16384):
    """The reference's CPU kernels (oracle/_ref: gemm_packed float kernel on the three Q8_0 layers, dense gemm_packed
    head; the position embedding from the oracle) on `sample` points, all host cores; scaled to 262144 points."""
    import numpy as np
    import torch
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as O
    import decoder_mlp

    if not O.ref_available():
        return {}
    feats, coords = decoder_mlp.inputs(sample, seed=2)
    f, c = feats.cpu().numpy(), coords.cpu().numpy()
    blobs = {k: O.q8_0_to_panel(v.cpu().numpy(), *model.shape[k]) for k, v in model.w.items()}
    b = {k: v.cpu().numpy() for k, v in model.b.items()}
    hw, hb = model.head_w.cpu().numpy(), model.head_b.cpu().numpy()
    freqs = model.freqs.cpu().numpy()

    def run():
        h = np.concatenate([f, O.pos_embed(freqs, c)], axis=1)
        for name in ("l1", "l2", "l3"):
            n, k = model.shape[name]
            h = np.maximum(O.ref_gemm_panel(h, blobs[name], b[name], n, k, mode=0), 0.0)
        return O.ref_gemm_dense(h, hw, hb)

    run()
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    t = float(np.median(times)) * DECODER_POINTS / sample
    return {"decoder_mlp_cpu_ms_est": round(t * 1e3, 2), "decoder_mlp_cpu_cores": cpu_threads(),
            "decoder_mlp_cpu_note": f"reference kernels.cpp float kernel (3 Q8_0 layers) + dense head on {sample} "
                                    f"points, median of 3 after 1 warm-up, scaled to {DECODER_POINTS} points"}


def run_cpu_denoiser_layer(model, ctx):
    """The reference's CPU kernels (oracle/_ref: gemm_packed float kernel, norm_rows, attention, gelu_tanh) on one
    full-size denoiser layer, all host cores; the step estimate is 24 x the layer."""
    import numpy as np
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as O

    if not O.ref_available():
        return {}
    layer = model.layers[0]
    B, S, Lc, H, hd = model.batch, model.seq, model.ctx_len, model.heads, model.head_dim
    Dm = model.dim
    w = {k: v.cpu().numpy() for k, v in layer.w.items()}
    b = {k: v.cpu().numpy() for k, v in layer.b.items()}
    blobs = {k: O.q8_0_to_panel(w[k], *layer.shape[k]) for k in w}
    gen = np.random.default_rng(0)
    x = gen.standard_normal((B * S, Dm), dtype=np.float32)
    c = ctx.float().cpu().numpy()
    shift, scale = model.shift.cpu().numpy(), model.scale.cpu().numpy()

    def lin(name, a, residual=None):
        n, k = layer.shape[name]
        return O.ref_gemm_panel(a, blobs[name], b[name], n, k, residual=residual, mode=0)

    def one_layer(x):
        h = np.concatenate([O.ref_norm_rows(x[i * S:(i + 1) * S], 1e-6, shift=shift[i], scale=scale[i]) for i in range(B)])
        qkv = lin("qkv", h)
        # q, k and v are column ranges of the [S, 3D] projection rows: flat slices at offsets 0, D and 2D
        att = np.concatenate([O.ref_attention(qkv[i * S:(i + 1) * S].reshape(-1), qkv[i * S:(i + 1) * S].reshape(-1)[Dm:],
                                              qkv[i * S:(i + 1) * S].reshape(-1)[2 * Dm:], S, S, 3 * Dm, 3 * Dm, H, hd)
                              for i in range(B)])
        x = lin("out", att, residual=x)
        q = lin("cq", O.ref_norm_rows(x, 1e-6))
        kv = lin("ckv", c)
        att = np.concatenate([O.ref_attention(q[i * S:(i + 1) * S], kv[i * Lc:(i + 1) * Lc].reshape(-1),
                                              kv[i * Lc:(i + 1) * Lc].reshape(-1)[Dm:], S, Lc, Dm, 2 * Dm, H, hd)
                              for i in range(B)])
        x = lin("cout", att, residual=x)
        f = O.ref_gelu_tanh(lin("up", O.ref_norm_rows(x, 1e-6)))
        return lin("down", f, residual=x)

    one_layer(x)
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        one_layer(x)
        times.append(time.perf_counter() - t0)
    t = float(np.median(times))
    return {"denoiser_cpu_layer_ms": round(t * 1e3, 1), "denoiser_cpu_step_ms_est": round(24 * t * 1e3, 1),
            "denoiser_cpu_cores": cpu_threads(),
            "denoiser_cpu_note": "reference kernels.cpp float kernel + attention + norm_rows + gelu_tanh on one "
                                 "full-size layer (batch 2 x 4096 tokens), median of 3 after 1 warm-up, step = 24 x "
                                 "layer; " + cpu_note()}


def run_cpu_baseline(args, inputs):
    """The reference's kernels.cpp float kernel (oracle/_ref, all host cores) on args.cpu_rows rows of the block."""
    import numpy as np
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as O

    x, w_up, w_down, b_up, b_down = inputs
    rows = min(args.cpu_rows, M)
    xs = x[:rows].float().cpu().numpy()
    wu, wd = w_up.cpu().numpy(), w_down.cpu().numpy()
    bu, bd = b_up.cpu().numpy(), b_down.cpu().numpy()
    kind = "reference" if O.ref_available() else "port"
    flop = 2 * 2.0 * rows * D * H

    def timed(block):
        block()
        times = []
        for _ in range(3):
            t0 = time.perf_counter()
            block()
            times.append(time.perf_counter() - t0)
        return float(np.median(times))

    def result(t, what):
        return {"value": flop / t / 1e12, "unit": "TFLOP/s", "cores": cpu_threads(), "kind": kind,
                "sample": f"MLP block (up + tanh-GELU + down + residual) on {rows} of {M} rows, fp32, {what}, median "
                          f"of 3 after 1 warm-up, {t * 1e3:.1f} ms per block; {cpu_note()}"}

    if kind == "reference":
        blob_up, blob_down = O.q8_0_to_panel(wu, H, D), O.q8_0_to_panel(wd, D, H)

        def block(mode):
            hh = O.ref_gemm_panel(xs, blob_up, bu, H, D, mode=mode)
            hh = O.ref_gelu_tanh(hh)
            return O.ref_gemm_panel(hh, blob_down, bd, D, H, residual=xs, mode=mode)

        out = result(timed(lambda: block(0)), "float kernel (IDOL_QUANT_KERNEL=float)")
        if O.ref_int8_supported():
            out8 = result(timed(lambda: block(1)), "integer kernel (AVX-VNNI vpdpbusd, the reference's default "
                                                   "where the host has avxvnni)")
        else:
            out8 = {"value": None, "unit": "TFLOP/s", "kind": kind,
                    "sample": "absent: this host has no avxvnni, so the reference build has no integer kernel"}
        return out, out8

    def port_block():
        hh = O.gelu_tanh(O.gemm_q8_float(xs, wu, H, D, bu))
        return O.gemm_q8_float(hh, wd, D, H, bd, residual=xs)

    out = result(timed(port_block), "the oracle's scalar restatement of the float kernel")
    out["cores"] = 1
    return out, {"value": None, "unit": "TFLOP/s", "kind": "port", "sample": "absent: no reference build"}


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py runs on exactly one GPU: the library has no multi-GPU path (--gpus must be 1)", file=sys.stderr)
        sys.exit(2)
    if args.traffic_probe:
        run_traffic_probe(args)
        return
    if args.counter_probe:
        run_counter_probe(args)
        return
    if args.size_sweep:
        run_size_sweep(args)
        return
    # The sections beside the headline run first: each is measured on its own, and the GPU has then been busy for a
    # while when the headline's warm-up steps start (its clocks ramp up over the first milliseconds of sustained
    # work), so the timed steps measure the MLP block at its steady clock however few warm-up steps are asked for.
    # The CPU baselines run last, after all GPU timing.
    side = {}
    side.update(run_layernorm_hbm(args))
    side.update(run_gemv_hbm(args))
    dec_model = None
    if not args.no_decoder_mlp:
        dec, dec_model = run_decoder_mlp(args)
        side.update(dec)
    side.update(run_fused_kinds(args))
    if not args.no_decoders:
        side.update(run_decoders(args))
    model = ctx = None
    if not args.no_denoiser:
        dn, model, ctx = run_denoiser(args)
        side.update(dn)
    gpu, inputs = run_gpu(args)
    result = {
        "metric": METRIC,
        "value": round(gpu["value"], 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(gpu["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": gpu["dtype"],
        "data": "synthetic (seeded N(0,1) activations, N(0,0.02) weights quantized to Q8_0, N(0,0.01) biases)",
        "config": {"workload": "Q8_0 MLP block: x bf16 [4096,1536] -> up Q8_0 [6144x1536] + bias + tanh-GELU -> "
                               "down Q8_0 [1536x6144] + bias + residual",
                   "m": M, "k_up": D, "n_up": H, "gemm_mode": args.mode},
        "roofline": gpu["roofline"],
        "pct_int8_peak": round(gpu["pct_int8_peak"], 4),
    }
    if args.mode == "dequant":
        result.update(run_int8_block(args, inputs))
    result.update(side)
    if not args.no_cpu_baseline:
        result["cpu_baseline"], result["cpu_baseline_int8"] = run_cpu_baseline(args, inputs)
        if model is not None:
            cpu = run_cpu_denoiser_layer(model, ctx)
            result.update(cpu)
            if cpu:
                result["denoiser_speedup_vs_cpu"] = round(cpu["denoiser_cpu_step_ms_est"] / result["denoiser_step_ms"], 1)
        if not args.no_decoders:
            cpu = run_cpu_decoders()
            result.update(cpu)
            if cpu:
                result["decoders_speedup_vs_cpu"] = round(
                    (cpu["decoders_cpu_oct_ms_est"] + cpu["decoders_cpu_gs_ms_est"])
                    / (result["decoders_oct_ms"] + result["decoders_gs_ms"]), 1)
        if dec_model is not None:
            cpu = run_cpu_decoder_mlp(dec_model)
            result.update(cpu)
            if cpu:
                result["decoder_mlp_speedup_vs_cpu"] = round(cpu["decoder_mlp_cpu_ms_est"] / result["decoder_mlp_ms"], 1)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
