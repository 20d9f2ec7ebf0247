"""bench.py on the CPU: the byte models it prices the roofline with, and the
one-GPU contract of its command line (no GPU is touched)."""
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def test_bytes_alg_matches_the_config_table():
    # C2: M = K = 1e6, nnz = 15,946,412, N = 128, fp32 everywhere
    assert bench.bytes_alg(1_000_000, 1_000_000, 15_946_412, 128) == 1_155_571_300
    # rowptr + (colind, vals) + B once + C once, by hand
    M, K, nnz, N = 7, 5, 11, 3
    assert bench.bytes_alg(M, K, nnz, N) == 4 * 8 + 11 * 8 + 5 * 3 * 4 + 7 * 3 * 4
    assert bench.bytes_alg(M, K, nnz, N, s_val=2, s_b=2) == 4 * 8 + 11 * 6 + 5 * 3 * 2 + 7 * 3 * 4


def test_bytes_edgewise_is_the_reference_model():
    # 12*nnz + 4*nnz*N + 4*M*N (ra_eval_utils.py:647-651)
    assert bench.bytes_edgewise(10, 100, 8) == 12 * 100 + 4 * 100 * 8 + 4 * 10 * 8


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr)
    assert r.stdout.strip() == "" or not r.stdout.strip().startswith("{")
