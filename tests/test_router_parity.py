"""Product router parity: Python mirror (ra_spmm.router) == C++ router
(ra_route_dispatch through the binding) bit for bit, on the golden rows and on
a dense grid that straddles every threshold; and the reference table
reproduces the published decisions.
(Reference contract: ra_router_parity_test.py:61-121.)
"""
import csv
import itertools
from pathlib import Path

import numpy as np
import pytest

import ra_spmm
from ra_spmm.router import route_with_rules, features_from_moments

GOLDEN = Path(__file__).resolve().parent / "golden" / "router_golden.csv"


def _cpp(M, N, nnz, s2, table):
    d = ra_spmm.route_features(M, M, N, nnz, s2, 0, 0, "MAIN", table)
    return ra_spmm.route_label(d), d


def _moments_for(M, d, cv):
    """Integer (nnz, sum d^2) realising mean d and population CV cv on M rows."""
    nnz = int(round(d * M))
    mean = nnz / M
    s2 = int(round(M * ((cv * mean) ** 2 + mean * mean)))
    return nnz, s2


def test_reference_table_reproduces_golden_rows():
    bad = []
    with open(GOLDEN) as f:
        for r in csv.DictReader(f):
            M, N = int(r["M"]), int(r["N"])
            d, cv = float(r["avg_nnz_per_row"]), float(r["cv_d"])
            py = route_with_rules(d, cv, M, N, int(r["nnz"]), table="reference")
            if py != r["router_kernel"]:
                bad.append((r["dataset"], N, r["router_kernel"], py))
    assert not bad, bad[:10]


@pytest.mark.parametrize("table", ["reference", "mi355x"])
def test_python_equals_cpp_on_threshold_grid(table):
    Ms = [5_000, 19_999, 20_000, 25_000, 25_001, 249_999, 250_000, 1_000_000]
    ds = [1.0, 4.49, 4.5, 4.51, 4.99, 5.0, 6.99, 7.0, 8.99, 9.0, 16.0, 24.99, 25.0, 39.99, 40.0, 500.0]
    cvs = [0.0, 0.19, 0.2, 0.21, 0.69, 0.7, 0.71, 1.09, 1.1, 1.45, 1.46, 1.49, 1.5, 1.79, 1.8,
           2.99, 3.0, 4.99, 5.0, 13.4]
    Ns = [8, 15, 16, 47, 64, 65, 95, 96, 128, 129, 255, 256, 257, 512]
    n = 0
    for M, d, cv in itertools.product(Ms, ds, cvs):
        nnz, s2 = _moments_for(M, d, cv)
        d32, cv32 = features_from_moments(M, nnz, s2)
        for N in Ns:
            cpp, dd = _cpp(M, N, nnz, s2, table)
            assert dd["feature_values"]["avg_nnz_per_row"] == d32
            assert dd["feature_values"]["degree_cv"] == cv32
            py = route_with_rules(d32, cv32, M, N, nnz, table=table)
            assert py == cpp, (M, d, cv, N, py, cpp)
            n += 1
    assert n == len(Ms) * len(ds) * len(cvs) * len(Ns)


def test_python_equals_cpp_on_exact_threshold_values():
    """Features that land exactly on a float32 threshold (cv == 0.7f, d == 25)."""
    for table in ("reference", "mi355x"):
        for M in (1000, 4000, 250_000):
            for nnz in (25 * M, 40 * M, 9 * M, int(4.5 * M)):
                for s2 in (nnz * nnz // M, nnz * nnz // M + M, nnz * nnz // M * 2):
                    d32, cv32 = features_from_moments(M, nnz, s2)
                    for N in (64, 128, 256):
                        assert route_with_rules(d32, cv32, M, N, nnz, table=table) == \
                            _cpp(M, N, nnz, s2, table)[0]


def test_production_features_match_cpp_host_features():
    from ra_spmm import synthetic as S
    import torch
    for seed in range(3):
        g = S.random_csr(3000, 3000, 6.0 + seed, seed=seed, skew=1.1, empty_frac=0.02)
        py = ra_spmm.production_features(g.rowptr, form="two_pass")
        c = ra_spmm.compute_features(torch.from_numpy(g.rowptr), g.M, g.K, 64)
        for k in ("nnz", "sum_deg_sq", "max_deg", "avg_nnz_per_row", "degree_cv"):
            assert py[k] == c[k], k


def test_plan_dict_schema():
    import torch
    rp = torch.tensor([0, 2, 3, 3, 7], dtype=torch.int32)
    d = ra_spmm.make_router_plan(rp, rp, rp, 4, 4, 64)
    for key in ("chosen_path", "use_tf32", "chosen_path_int", "decision_reason", "estimated_risk",
                "planning_time_ms", "gate_margin_raw", "gate_margin_norm", "path_count",
                "path_names", "feasible", "feasible_by_path", "rejection_codes",
                "rejection_details", "feature_values", "scores", "feature_set",
                "feature_backend"):
        assert key in d, key
    assert d["path_count"] == 15 and len(d["path_names"]) == 15
    assert d["feature_set"] == "production_4" and d["feature_backend"] == "cpu_rowptr"
    assert d["rejection_codes"][d["chosen_path"]] == "CHOSEN"
    small = ra_spmm.make_router_plan(rp, rp, rp, 4, 4, 8)
    assert not small["feasible_by_path"]["TC_DIRECT"]
    assert small["chosen_path"] not in ("TC_DIRECT", "COMMUNITY_TC", "SEGMENT_HYBRID")
    with pytest.raises(RuntimeError):
        ra_spmm.make_router_plan(rp, rp, rp, 4, 4, 64, "MAIN", "bogus")
