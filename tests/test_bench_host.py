"""bench.py's contract on the host: the one-GPU rule, the algorithmic bytes of the two GEMM launches (recomputed
from the shapes) and the committed FETCH/WRITE summary it reads for the roofline's traffic."""
import importlib.util
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def _bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and not r.stdout.strip()


def test_algorithmic_bytes_of_the_mlp_block_launches():
    b = _bench()
    m, d, h = 4096, 1536, 6144
    assert (b.M, b.D, b.H) == (m, d, h)
    q8 = lambda rows, cols: rows * cols // 32 * 34  # 34-byte blocks of 32 weights
    # up: W_up, x in, h out (bf16), fp32 bias; down: W_down, h in, y out and the residual x (bf16), fp32 bias
    assert b.ALG_BYTES_UP == q8(h, d) + 2 * m * d + 2 * m * h + 4 * h == 72_966_144
    assert b.ALG_BYTES_DOWN == q8(d, h) + 2 * m * h + 2 * 2 * m * d + 4 * d == 85_530_624
    # one step's FLOP: two products of 2 m d h each
    assert 2 * 2 * m * d * h == 154_618_822_656


def test_traffic_summary_is_committed_and_read():
    b = _bench()
    t = b.measured_traffic()
    assert t is not None, "the FETCH/WRITE summary the roofline's traffic comes from is missing"
    assert t["mean"] == (t["up"] + t["down"]) / 2
    # at least the algorithmic bytes, and within a small multiple of them (re-reads served from L2 or MALL)
    assert b.ALG_BYTES_UP <= t["up"] <= 8 * b.ALG_BYTES_UP
    assert b.ALG_BYTES_DOWN <= t["down"] <= 8 * b.ALG_BYTES_DOWN
