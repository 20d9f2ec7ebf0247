"""Device tile-format build (hipCUB sorts and scans) against the host builder.

Both builders must emit the same plan bit for bit: every array of the format
(win_rows, block_offsets, atox, fp16/bf16 value bits, segment and merge
tables) and every count in the plan info.  The host builder is itself pinned
against the oracle's tile_format (tests/test_oracle_structures.py), so
equality here carries that pin over to the device build.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

import ra_spmm  # noqa: E402
from ra_spmm import synthetic as S  # noqa: E402

MAKE = {0: ra_spmm.make_tc_direct_plan, 1: ra_spmm.make_community_tc_plan,
        2: ra_spmm.make_segment_hybrid_plan}
ARRAYS = ("win_rows", "block_offsets", "atox", "vals", "seg_window", "seg_bbegin", "seg_bend",
          "seg_slot", "split_windows", "split_offsets")
INFO = ("active", "num_windows", "num_blocks", "num_segments", "num_split_windows",
        "num_split_segs", "nnz", "num_vectors", "plan_bytes", "avg_tc_tile_density",
        "value_scale_log2", "max_window_blocks")


def _dups(seed=21):
    """CSR with repeated (row, column) entries, unsorted columns and empty windows."""
    rng = np.random.default_rng(seed)
    M, K = 300, 120
    deg = rng.integers(0, 30, M)
    deg[40:72] = 0                                      # four empty windows
    rp = np.concatenate([[0], np.cumsum(deg)]).astype(np.int32)
    ci = rng.integers(0, K // 3, rp[-1]).astype(np.int32)   # many duplicates
    vl = rng.standard_normal(rp[-1]).astype(np.float32)
    return S.Graph(rp, ci, vl, M, K, "dups")


GRAPHS = {
    "skewed": lambda: S.random_csr(1003, 900, 9.0, seed=3, skew=1.1, empty_frac=0.05),
    "community": lambda: S.sbm(64, 50, 12.0, 0.9, seed=6),
    "hub_windows": lambda: S.random_csr(40, 40000, 2500.0, seed=8),
    "dense_rows": lambda: S.random_csr(200, 3000, 150.0, seed=4),
    "duplicates": _dups,
    "one_row": lambda: S.random_csr(1, 50, 20.0, seed=2),
}


def _compare(g, kind, value_dtype, N=64):
    rp, ci, vl = (torch.from_numpy(np.ascontiguousarray(a)) for a in (g.rowptr, g.colind, g.vals))
    host = MAKE[kind](rp, ci, vl, g.M, g.K, N, value_dtype, build="host")
    dev = MAKE[kind](rp.cuda(), ci.cuda(), vl.cuda(), g.M, g.K, N, value_dtype, build="gpu", rows_per_window=8)
    for f in INFO:
        assert getattr(host, f) == getattr(dev, f), f
    for a in ARRAYS:
        h = ra_spmm.export_tile_plan(host, a).numpy()
        d = ra_spmm.export_tile_plan(dev, a).numpy()
        np.testing.assert_array_equal(h, d, err_msg=a)
    return host, dev


@pytest.mark.parametrize("gname", list(GRAPHS))
@pytest.mark.parametrize("kind", [0, 1, 2])
@pytest.mark.parametrize("value_dtype", ["fp16", "bf16"])
def test_device_build_matches_host(gname, kind, value_dtype):
    print(f"[tile-build] {gname} kind={kind} {value_dtype}", flush=True)
    host, dev = _compare(GRAPHS[gname](), kind, value_dtype)
    assert host.active


def test_device_build_runs_identically():
    g = GRAPHS["skewed"]()
    B = torch.randn(g.K, 96, device="cuda")
    for kind in (0, 1, 2):
        host, dev = _compare(g, kind, "fp16", 96)
        for route in ("fp16", "fp32"):
            assert torch.equal(ra_spmm.run_tile_plan_route(host, B, route),
                               ra_spmm.run_tile_plan_route(dev, B, route))


def test_device_build_inactive_and_invalid():
    g = GRAPHS["skewed"]()
    rp, ci, vl = g.torch("cuda")
    p = ra_spmm.make_tc_direct_plan(rp, ci, vl, g.M, g.K, 8, build="gpu", rows_per_window=8)
    assert p.valid and not p.active
    bad = ci.clone()
    bad[5] = g.K
    with pytest.raises(RuntimeError, match="out of range"):
        ra_spmm.make_tc_direct_plan(rp, bad, vl, g.M, g.K, 64, build="gpu")


def test_c3_device_build_matches_host():
    g = S.CONFIGS["C3"]()
    for kind in (0, 1):
        _compare(g, kind, "fp16", 256)


@pytest.mark.parametrize("seed", range(16))
def test_device_build_matches_host_random(seed):
    """Seeded shapes, densities, skew, empty rows and duplicates: the device
    build equals the host build array for array."""
    rng = np.random.default_rng(500 + seed)
    M, K = int(rng.integers(1, 2500)), int(rng.integers(1, 4000))
    d = float(rng.choice([1.0, 6.0, 30.0, 120.0]))
    g = S.random_csr(M, K, min(d, K), seed=int(rng.integers(1 << 30)), skew=float(rng.choice([0.0, 1.1])),
                     empty_frac=float(rng.choice([0.0, 0.2])), max_deg=K)
    if rng.random() < 0.4 and g.nnz > 1:  # repeated (row, column) entries
        ci = g.colind.copy()
        ci[1::3] = ci[0:-1:3][: len(ci[1::3])]
        g = S.Graph(g.rowptr, ci, g.vals, M, K, "dups")
    kind = int(rng.integers(0, 3))
    value_dtype = "bf16" if rng.random() < 0.3 else "fp16"
    print(f"[tile-build] random seed={seed} M={M} K={K} nnz={g.nnz} kind={kind} {value_dtype}", flush=True)
    _compare(g, kind, value_dtype, N=int(rng.choice([16, 64, 200])))
