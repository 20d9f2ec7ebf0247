"""GPU feature pass (ra_features_device, make_router_plan on device tensors)
and host feature path against the oracle's restatements of the reference's
two forms.

Bar: device features == oracle.features_gpu_reference (moment form,
router/router_features_cuda.cu:78-91) bit for bit; host features ==
oracle.features_cpu_reference (two-pass form, router/router_features.cpp:79-111)
bit for bit; the two forms' degree_cv differ by at most one float32 ulp, and
the routed decisions agree.  Inputs: random CSRs, degree sequences with
closed-form CV at the router's thresholds, the committed one-ulp sequence,
and the full rowptrs of configs C1, C2 and C5.
"""
import numpy as np
import pytest
import torch

import ra_spmm
from ra_spmm import synthetic as S
from test_features_forms import EXACT, ULP_CASE, _rowptr, exact_cv_rowptr, ulps

pytestmark = pytest.mark.gpu


def _inputs():
    yield "ulp_case", _rowptr(ULP_CASE)
    # 65,536 rows is the largest matrix the one-block reduction takes
    for seed, (M, d, skew) in enumerate([(1, 3.0, 0), (1000, 5.0, 1.0), (200_003, 12.0, 1.1),
                                         (65_536, 6.0, 1.2), (65_537, 6.0, 1.2)]):
        yield f"random{seed}", S.random_csr(M, 5000, d, seed=seed, skew=skew, empty_frac=0.01).rowptr
    for (num, den), cv in EXACT:
        yield f"cv{cv}", exact_cv_rowptr(num, den, 1001, 37)
    for name in ("C1", "C2", "C5"):
        yield name, S.CONFIGS[name]().rowptr


def test_feature_forms_against_oracle(oracle):
    gaps = {}
    for name, rp in _inputs():
        print(f"[features] {name} M={rp.size - 1}", flush=True)
        M = rp.size - 1
        K = max(M, 1)
        g = oracle.features_gpu_reference(rp, M, K)
        c = oracle.features_cpu_reference(rp, M, K)
        rpt = torch.from_numpy(rp)
        fd = ra_spmm.compute_features(rpt.cuda(), M, K, 128)
        assert fd["nnz"] == g[0], name
        assert (fd["avg_nnz_per_row"], fd["std_nnz_per_row"], fd["degree_cv"]) == (g[3], g[4], g[5]), name
        assert fd["sum_deg_sq"] == oracle.degree_moments(rp)[1], name
        fh = ra_spmm.compute_features(rpt, M, K, 128)
        assert (fh["nnz"], fh["avg_nnz_per_row"], fh["std_nnz_per_row"], fh["degree_cv"]) == c, name
        for N in (64, 128):
            pd = ra_spmm.make_router_plan(rpt.cuda(), rpt.cuda(), rpt.cuda(), M, K, N)
            ph = ra_spmm.make_router_plan(rpt, rpt, rpt, M, K, N)
            assert pd["feature_backend"] == "cuda_rowptr_moments"
            assert ph["feature_backend"] == "cpu_rowptr"
            assert pd["feature_values"]["degree_cv"] == g[5]
            assert pd["feature_values"]["avg_nnz_per_row"] == g[3]
            assert ph["feature_values"]["degree_cv"] == c[3]
            assert (pd["chosen_path"], pd["use_tf32"]) == (ph["chosen_path"], ph["use_tf32"]), name
            py = ra_spmm.route_with_rules(g[3], g[5], M, N, g[0])
            assert py == ra_spmm.route_label(pd), name
        gaps[name] = ulps(g[5], c[3])
    print("cv32 ulp gap moment vs two-pass:", gaps, flush=True)
    assert max(gaps.values()) <= 1
    assert gaps["ulp_case"] == 1


def test_feature_pass_behind_queued_work(oracle):
    """The feature pass polls the result its kernel publishes and falls back to
    a stream synchronisation after ~200 us: with ~tens of ms of SpMM queued
    ahead of it on the same stream it takes the fallback, and the features are
    the same as on an idle stream (both block sizes of the reduction)."""
    big = S.CONFIGS["C2"]()
    rp_b, ci_b, vl_b = big.torch("cuda")
    B = torch.randn(big.K, 128, device="cuda")
    for M in (10_000, 200_003):
        rp = S.random_csr(M, 5000, 8.0, seed=M, skew=1.1).rowptr
        want = oracle.features_gpu_reference(rp, M, M)
        rpd = torch.from_numpy(rp).cuda()
        torch.cuda.synchronize()
        for _ in range(2):  # ~25 ms each: the baseline kernel on config C2
            ra_spmm.spmm_csr_baseline(rp_b, ci_b, vl_b, B)
        fd = ra_spmm.compute_features(rpd, M, M, 128)
        assert (fd["nnz"], fd["avg_nnz_per_row"], fd["std_nnz_per_row"], fd["degree_cv"]) == \
            (want[0], want[3], want[4], want[5])
        idle = ra_spmm.compute_features(rpd, M, M, 128)
        assert idle == fd
