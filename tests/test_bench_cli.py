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


def test_cpu_sample_rows_bounds_the_sample():
    import numpy as np
    from ra_spmm import synthetic as S
    g = S.random_csr(5000, 4000, 20.0, seed=1)
    assert bench.cpu_sample_rows(g, 128, flops=1e12) is None  # whole matrix
    rows = bench.cpu_sample_rows(g, 128, flops=2.0 * 128 * 10_000)
    assert rows is not None and 0 < rows < g.M
    assert g.rowptr[rows] >= 10_000 and g.rowptr[rows - 1] < 10_000


def test_block_of_carries_the_driver_fields():
    res = {"path": "ZERO_OVERHEAD_CSR", "ms_per_step": 1.0, "gflops": 4000.0, "kernel": "zo_fused_kernel",
           "kernel_ms": 0.9, "bytes_alg": 1_000_000_000, "cold_route_ms": 0.03, "cold_build_ms": 0.7,
           "cold_first_exec_ms": 1.1, "baseline_ms": 27.0, "speedup_vs_baseline": 27.0,
           "max_rel_err_vs_baseline": 3e-7, "rocsparse": {"ms": 1.5, "alg": "csr_nnz_split"},
           "speedup_vs_rocsparse": 1.5, "torch_sparse_gpu": {"ms": 30.0}, "speedup_vs_torch_sparse_gpu": 30.0,
           "cpu_torch_sparse": {"value": 33.0, "sample": "full matrix"},
           "gather_ceiling": {"csr_order": {"ms": 0.81}, "uniform": {"ms": 1.1}},
           "cold_speedup_vs_rocsparse": 0.9,
           "deployed_cold": {"path": "ZERO_OVERHEAD_CSR", "ms": 2.0, "speedup_vs_rocsparse": 0.8}}
    res["rocsparse"]["cold_ms"] = 1.6
    b = bench.block_of(res)
    assert b["roofline"]["frac"] == round(1e9 / 0.9e-3 / 1e9 / 8000.0, 4)
    assert b["roofline"]["frac_of_gather_probe"] == round(0.81 / 0.9, 4)
    assert b["speedup_vs_rocsparse"] == 1.5 and b["rocsparse_alg"] == "csr_nnz_split"
    assert set(b["cold"]) == {"route_ms", "build_ms", "first_exec_ms", "rocsparse_cold_ms", "speedup_vs_rocsparse",
                              "deployed_path", "deployed_ms", "deployed_speedup_vs_rocsparse"}
    assert b["cold"]["deployed_speedup_vs_rocsparse"] == 0.8 and b["cold"]["rocsparse_cold_ms"] == 1.6
    # a tile plan's probe walks its vector columns and is keyed plan_order
    res["gather_ceiling"] = {"plan_order": {"ms": 0.45, "gathers": 10}}
    assert bench.block_of(res)["roofline"]["frac_of_gather_probe"] == round(0.45 / 0.9, 4)


def test_order_study_counts_the_plans_vectors():
    """The study's gathered-row count for the identity and leading-column
    orders at 8-row windows equals the vector count of the oracle's
    TC_DIRECT and COMMUNITY_TC formats (a vector = one gathered B row)."""
    import numpy as np
    from oracle import oracle as O
    from ra_spmm import synthetic as S
    g = S.random_csr(301, 280, 6.0, seed=1, skew=1.1, empty_frac=0.05)
    study = bench.order_study(heights=(8,), g=g)["rows"]
    for kind, name in ((0, "identity (TC_DIRECT)"), (1, "leading column (COMMUNITY_TC)")):
        fmt = O.tile_format(kind, g.rowptr, g.colind, g.vals, g.M)
        vectors = int(np.count_nonzero(np.any(fmt["blocks"] != 0, axis=1)))
        assert study[f"{name} | H=8"]["gathered_rows"] == vectors, name
