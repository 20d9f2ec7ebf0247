"""Oracle router and features pinned on the reference's published decisions.

tests/golden/router_golden.csv holds 420 decisions the reference itself
published (router_quality_v8.csv on RTX 3090, the RTX 4090 rerun, and the 36
held-out graphs), with the per-graph (avg_nnz_per_row, cv_d) of
final_fair_v3.csv.  Both restatements of the reference router (its Python
mirror, ra_router_eval.py:37-124, and its C++ deployed block,
router/router_dispatch.cpp:979-1110) must reproduce every row.
"""
import csv
from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden" / "router_golden.csv"


def _rows():
    with open(GOLDEN) as f:
        return list(csv.DictReader(f))


def test_golden_file_shape():
    rows = _rows()
    assert len(rows) == 420
    assert sum(r["source"] == "tf32_v8" for r in rows) == 192
    labels = {r["router_kernel"] for r in rows}
    assert {"TC_DIRECT", "COMMUNITY_TC", "ZERO_OVERHEAD_CSR", "CUSPARSE",
            "SEGMENT_HYBRID", "CSR_DIRECT", "TC_DIRECT_TF32", "COMMUNITY_TC_TF32"} <= labels


def test_oracle_routers_reproduce_golden(oracle):
    bad = []
    for r in _rows():
        d, cv = float(r["avg_nnz_per_row"]), float(r["cv_d"])
        M, N, nnz = int(r["M"]), int(r["N"]), int(r["nnz"])
        py = oracle.route_python_reference(d, cv, M, N, nnz)
        cpp = oracle.route_cpp_reference(d, cv, M, N)
        if py != r["router_kernel"] or cpp != r["router_kernel"]:
            bad.append((r["dataset"], N, r["router_kernel"], py, cpp))
    assert not bad, bad[:10]


def test_rule_ablation_changes_decisions(oracle):
    # Disabling rule 1 must move an extreme-skew graph off ZERO_OVERHEAD_CSR.
    assert oracle.route_python_reference(5.0, 9.7, 1_157_827, 128, 5_975_248) == "ZERO_OVERHEAD_CSR"
    assert oracle.route_python_reference(5.0, 9.7, 1_157_827, 128, 5_975_248,
                                         disabled_rules=(1,)) != "ZERO_OVERHEAD_CSR"


def test_feature_forms_agree(oracle):
    """Moment form (GPU reference) vs two-pass form (CPU reference): the same
    population CV up to rounding; golden avg matches nnz/M to 6 decimals."""
    from ra_spmm import synthetic as S
    for seed in range(4):
        g = S.random_csr(5000, 5000, 7.0, seed=seed, skew=1.2, empty_frac=0.05)
        nnz, avg, std, a32, s32, cv_m = oracle.features_gpu_reference(g.rowptr, g.M)
        nnz2, a32b, s32b, cv_t = oracle.features_cpu_reference(g.rowptr, g.M)
        deg = np.diff(g.rowptr).astype(np.float64)
        assert nnz == nnz2 == g.nnz
        assert a32 == a32b
        assert abs(cv_m - deg.std() / deg.mean()) <= 1e-6 * cv_m
        assert abs(cv_m - cv_t) <= 1e-6 * cv_m
    for r in _rows():
        assert abs(int(r["nnz"]) / int(r["M"]) - float(r["avg_nnz_per_row"])) < 1e-5
