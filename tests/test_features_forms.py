"""The routing features in the reference's two forms, pinned to the oracle.

ra_features_host is the reference host path's two-pass form
(router/router_features.cpp:79-111); the finalisation of the device pass,
ra_features_from_moments, is the reference GPU path's moment form
(router/router_features_cuda.cu:78-91).  Each is compared bit for bit with its
oracle restatement (oracle.features_cpu_reference / features_gpu_reference),
and the oracle itself is pinned by degree sequences whose CV is known in
closed form and by numpy's population standard deviation.  The gap between
the two forms is measured: at most one float32 ulp of degree_cv, seen only
where the moment form's cancellation error reaches a float32 rounding
boundary (the committed sequence below is one such case).
"""
import ctypes

import numpy as np
import pytest
import torch

import ra_spmm
from ra_spmm import capi
from ra_spmm import synthetic as S

# 61 rows with CV ~ 0.0086: the moment form's cv32 is one ulp above the
# two-pass form's (found by a search over near-uniform degree sequences).
ULP_CASE = [5423, 5410, 5387, 5346, 5452, 5312, 5481, 5462, 5437, 5368, 5407, 5389, 5397, 5464,
            5464, 5438, 5442, 5455, 5332, 5435, 5300, 5451, 5430, 5385, 5383, 5417, 5473, 5422,
            5426, 5447, 5411, 5369, 5449, 5462, 5393, 5440, 5408, 5448, 5430, 5428, 5448, 5308,
            5453, 5391, 5477, 5400, 5345, 5426, 5470, 5460, 5476, 5425, 5419, 5473, 5353, 5407,
            5429, 5439, 5512, 5517, 5475]


def _rowptr(deg):
    return np.concatenate([[0], np.cumsum(np.asarray(deg, np.int64))]).astype(np.int32)


def exact_cv_rowptr(cv_sq_num, cv_sq_den, a, t):
    """Rows of degree a (k of them) and empty rows (M - k) with
    cv^2 = (M - k) / k = num/den exactly: k = den*t, M = (num + den)*t."""
    k = cv_sq_den * t
    M = (cv_sq_num + cv_sq_den) * t
    deg = np.zeros(M, np.int64)
    deg[:k] = a
    return _rowptr(deg)


# cv = 5, 3, 1.5 (the router's float32-exact CV thresholds) and 0.5.
EXACT = [((25, 1), 5.0), ((9, 1), 3.0), ((9, 4), 1.5), ((1, 4), 0.5)]


def ulps(a, b):
    return abs(int(np.float32(a).view(np.int32)) - int(np.float32(b).view(np.int32)))


def cases():
    out = [_rowptr(ULP_CASE)]
    for seed, (M, d, skew) in enumerate([(1, 3.0, 0), (1000, 5.0, 1.0), (20_003, 12.0, 1.1),
                                         (7, 0.0, 0.0)]):
        out.append(S.random_csr(M, 5000, d, seed=seed, skew=skew, empty_frac=0.01).rowptr)
    for (num, den), _ in EXACT:
        for a, t in ((7, 3), (13, 11), (1001, 37)):
            out.append(exact_cv_rowptr(num, den, a, t))
    out.append(S.CONFIGS["C1"]().rowptr)
    return out


def test_oracle_forms_closed_form_cv(oracle):
    for (num, den), cv in EXACT:
        for a, t in ((7, 3), (13, 11), (1001, 37), (50_000, 5)):
            rp = exact_cv_rowptr(num, den, a, t)
            M = rp.size - 1
            assert oracle.features_gpu_reference(rp, M)[5] == np.float32(cv)
            assert oracle.features_cpu_reference(rp, M)[3] == np.float32(cv)


def test_oracle_forms_numpy_std_and_edges(oracle):
    rng = np.random.default_rng(0)
    for _ in range(50):
        M = int(rng.integers(1, 3000))
        deg = rng.integers(0, int(rng.integers(1, 300)), M)
        rp = _rowptr(deg)
        ref = np.float32(deg.std() / deg.mean()) if deg.sum() > 0 else np.float32(0)
        g = oracle.features_gpu_reference(rp, M)
        c = oracle.features_cpu_reference(rp, M)
        assert g[0] == c[0] == deg.sum()
        assert g[3] == c[1] == np.float32(deg.mean())
        assert ulps(g[5], ref) <= 1 and ulps(c[3], ref) <= 1
    rp = _rowptr([3, 0, 2])
    assert oracle.features_gpu_reference(rp, 3, K=0) == (0, 0.0, 0.0, 0.0, 0.0, 0.0)
    assert oracle.features_cpu_reference(rp, 3, K=0) == (0, 0.0, 0.0, 0.0)
    z = _rowptr([0, 0, 0])
    assert oracle.features_cpu_reference(z, 3)[3] == 0.0
    assert oracle.features_gpu_reference(z, 3)[5] == 0.0


def test_forms_differ_by_one_ulp_on_the_committed_case(oracle):
    rp = _rowptr(ULP_CASE)
    M = rp.size - 1
    g = oracle.features_gpu_reference(rp, M)[5]
    c = oracle.features_cpu_reference(rp, M)[3]
    assert ulps(g, c) == 1


def _host(rp, M, K=None, N=64):
    f = ra_spmm.compute_features(torch.from_numpy(rp), M, M if K is None else K, N)
    return f


@pytest.mark.parametrize("i", range(len(cases())))
def test_host_features_equal_two_pass_oracle(oracle, i):
    rp = cases()[i]
    M = rp.size - 1
    f = _host(rp, M)
    nnz, a32, s32, cv32 = oracle.features_cpu_reference(rp, M)
    assert f["nnz"] == nnz
    assert f["avg_nnz_per_row"] == a32
    assert f["std_nnz_per_row"] == s32
    assert f["degree_cv"] == cv32
    py = ra_spmm.production_features(rp, form="two_pass")
    assert (py["avg_nnz_per_row"], py["degree_cv"]) == (a32, cv32)


@pytest.mark.parametrize("i", range(len(cases())))
def test_moment_finalisation_equals_gpu_oracle(oracle, i):
    rp = cases()[i]
    M = rp.size - 1
    nnz, s2, mx, em = oracle.degree_moments(rp)
    lib = capi.load()
    f = capi.Features()
    assert lib.ra_features_from_moments(M, M, 64, nnz, s2, mx, em, ctypes.byref(f)) == 0
    g = oracle.features_gpu_reference(rp, M)
    assert f.nnz == g[0]
    assert f.avg_nnz_per_row == g[3] and f.std_nnz_per_row == g[4] and f.degree_cv == g[5]
    py = ra_spmm.production_features(rp, form="moments")
    assert (py["avg_nnz_per_row"], py["degree_cv"]) == (g[3], g[5])
    assert ulps(f.degree_cv, oracle.features_cpu_reference(rp, M)[3]) <= 1


def test_empty_shapes_give_zero_features():
    rp = _rowptr([3, 0, 2])
    f = _host(rp, 3, K=0)
    assert f["nnz"] == 0 and f["avg_nnz_per_row"] == 0.0 and f["degree_cv"] == 0.0
    lib = capi.load()
    m = capi.Features()
    assert lib.ra_features_from_moments(3, 0, 64, 5, 13, 3, 1, ctypes.byref(m)) == 0
    assert m.nnz == 0 and m.degree_cv == 0.0 and m.K == 0 and m.M == 3
    z = _host(_rowptr([0, 0]), 2)
    assert z["avg_nnz_per_row"] == 0.0 and z["degree_cv"] == 0.0


def test_decisions_agree_across_forms_on_threshold_sequences(oracle):
    """At the float32-exact CV thresholds both forms give the threshold itself,
    so both reach the same rule; the 1-ulp case sits far from any threshold."""
    for rp in cases():
        M = rp.size - 1
        if M == 0:
            continue
        g = oracle.features_gpu_reference(rp, M)
        c = oracle.features_cpu_reference(rp, M)
        for N in (32, 64, 128, 256):
            for table in ("reference", "mi355x"):
                a = ra_spmm.route_with_rules(g[3], g[5], M, N, g[0], table=table)
                b = ra_spmm.route_with_rules(c[1], c[3], M, N, c[0], table=table)
                assert a == b
