"""Diagnostic feature extractor (analyze_matrix, router_features.cpp:113-432):
closed forms on structured matrices, then bit-for-bit agreement with the
pure-Python restatement (oracle/diagnostics_oracle.py) on random matrices."""
import numpy as np
import pytest
import torch

import ra_spmm
from ra_spmm import synthetic as S
from oracle import diagnostics_oracle as DO


def _analyze(rowptr, colind, M, K, N):
    return ra_spmm.analyze_matrix(torch.from_numpy(np.asarray(rowptr, np.int32)),
                                  torch.from_numpy(np.asarray(colind, np.int32)), M, K, N)


def _csr_from_dense(A):
    rp = np.concatenate([[0], np.cumsum((A != 0).sum(1))]).astype(np.int32)
    ci = np.concatenate([np.flatnonzero(r) for r in A]).astype(np.int32) if A.any() else np.zeros(0, np.int32)
    return rp, ci


def test_identity_closed_form():
    rp, ci = _csr_from_dense(np.eye(64))
    d = _analyze(rp, ci, 64, 64, 128)
    assert d["avg_nnz_per_row"] == 1.0 and d["degree_cv"] == 0.0 and d["std_nnz_per_row"] == 0.0
    # four diagonal 16x16 tiles of 16 nonzeros each, out of 16 tiles
    assert d["tile_fill_mean"] == pytest.approx(16 / 256) and d["tile_fill_max"] == pytest.approx(16 / 256)
    assert d["tile_fill_variance"] == 0.0 and d["tile_occupancy"] == pytest.approx(0.25)
    assert d["avg_nnz_per_tile"] == 16.0 and d["actual_nnz_coverage"] == 0.0 and d["tc_candidate_tiles"] == 0
    # one distinct signature bucket per row: adjacent rows never overlap
    assert d["local_row_similarity_proxy"] == 0.0
    assert d["top_1_row_nnz_fraction"] == pytest.approx(1 / 64) and d["top_5_row_nnz_fraction"] == pytest.approx(5 / 64)


def test_dense_block_closed_form():
    rp, ci = _csr_from_dense(np.ones((32, 32)))
    d = _analyze(rp, ci, 32, 32, 128)
    assert d["tile_fill_mean"] == 1.0 and d["tc_candidate_ratio"] == 1.0 and d["actual_nnz_coverage"] == 1.0
    assert d["tc_candidate_tiles"] == 4 and d["avg_nnz_per_tile"] == 256.0
    assert d["local_row_similarity_proxy"] == 1.0 and d["reordered_locality_proxy"] == 1.0
    assert d["row_window_colspan_compactness"] == 1.0
    # every window is a tensor-core window: tc_score = .35 + .30 + .20 + .15*(1 - 32/129) >= 0.55
    assert d["estimated_tc_partition_ratio"] == 1.0 and d["estimated_cuda_partition_ratio"] == 0.0
    assert d["long_row_fraction"] == 0.0 and d["frac_dense_rows"] == 0.0


def test_one_hub_row_closed_form():
    # row 0 holds all 100 columns, rows 1..99 one column each
    A = np.zeros((100, 100))
    A[0, :] = 1
    A[np.arange(1, 100), np.arange(1, 100)] = 1
    rp, ci = _csr_from_dense(A)
    d = _analyze(rp, ci, 100, 100, 64)
    nnz = 199
    assert d["top_1_row_nnz_fraction"] == pytest.approx(100 / nnz)
    assert d["max_to_mean_ratio"] == pytest.approx(100 / (nnz / 100), rel=1e-6)
    # long rows: len >= max(32, 2*avg) -> only row 0
    assert d["long_row_fraction"] == pytest.approx(0.01) and d["long_row_nnz_fraction"] == pytest.approx(100 / nnz)


def test_empty_and_degenerate():
    d = _analyze([0, 0, 0], [], 2, 5, 64)
    assert d["nnz"] == 0 and d["avg_nnz_per_row"] == 0.0
    d = _analyze([0], [], 0, 5, 64)
    assert d["avg_nnz_per_row"] == 0.0


@pytest.mark.parametrize("seed", range(5))
def test_matches_reference_restatement_bitwise(seed):
    rng = np.random.default_rng(seed)
    kind = seed % 3
    if kind == 0:
        g = S.random_csr(int(rng.integers(50, 400)), int(rng.integers(40, 500)), 8.0, seed=seed, skew=1.1,
                         empty_frac=0.1)
    elif kind == 1:
        g = S.sbm(12, 20, 9.0, 0.85, seed=seed)
    else:
        g = S.random_csr(300, 300, 40.0, seed=seed)
    for N in (16, 128, 512):
        got = _analyze(g.rowptr, g.colind, g.M, g.K, N)
        ref = DO.analyze_reference(g.rowptr, g.colind, g.M, g.K, N)
        for k in DO.KEYS:
            assert np.float32(got[k]) == ref[k], (k, got[k], ref[k])
        assert got["tc_candidate_tiles"] == ref["tc_candidate_tiles"]


def test_full_portfolio_plan_carries_diagnostics():
    g = S.random_csr(200, 200, 10.0, seed=3)
    rp, ci, vl = (torch.from_numpy(a) for a in (g.rowptr, g.colind, g.vals))
    plan = ra_spmm.make_router_plan(rp, ci, vl, g.M, g.K, 64, "FULL")
    main = ra_spmm.make_router_plan(rp, ci, vl, g.M, g.K, 64, "MAIN")
    assert plan["feature_set"] == "full" and main["feature_set"] == "production_4"
    d = _analyze(g.rowptr, g.colind, g.M, g.K, 64)
    for k in DO.KEYS:
        assert plan["feature_values"][k] == d[k]
    assert plan["chosen_path"] == main["chosen_path"]
