"""Degenerate shapes through every entry point: M = 0, N = 0, nnz = 0, K = 1,
a single dense row, B with N = 1 and N = 16 (the tile minimum)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

import ra_spmm  # noqa: E402


def _dev(rp, ci, vl):
    return (torch.tensor(rp, dtype=torch.int32, device="cuda"), torch.tensor(ci, dtype=torch.int32, device="cuda"),
            torch.tensor(vl, dtype=torch.float32, device="cuda"))


def _all_paths(rp, ci, vl, M, K, B):
    outs = {"csr_direct": ra_spmm.spmm_csr_direct(rp, ci, vl, B),
            "baseline": ra_spmm.spmm_csr_baseline(rp, ci, vl, B)}
    z = ra_spmm.make_zero_overhead_plan(rp, M, K)
    outs["zo"] = ra_spmm.run_zero_overhead_plan(z, rp, ci, vl, B)
    N = B.shape[1]
    if N >= 16 and M > 0:
        for name, mk, run in (("tc", ra_spmm.make_tc_direct_plan, ra_spmm.run_tc_direct_plan_tf32),
                              ("comm", ra_spmm.make_community_tc_plan, ra_spmm.run_community_tc_plan_tf32)):
            p = mk(rp, ci, vl, M, K, N)
            outs[name] = run(p, B)
        p = ra_spmm.make_segment_hybrid_plan(rp, ci, vl, M, K, N)
        outs["seg"] = ra_spmm.run_segment_hybrid_plan_tf32(p, ci, vl, B)
    return outs


@pytest.mark.parametrize("N", [1, 16, 64])
def test_all_rows_empty(N):
    M, K = 37, 20
    rp, ci, vl = _dev([0] * (M + 1), [], [])
    B = torch.randn(K, N, device="cuda")
    for name, C in _all_paths(rp, ci, vl, M, K, B).items():
        assert C.shape == (M, N), name
        assert torch.count_nonzero(C) == 0, name


def test_zero_rows():
    rp, ci, vl = _dev([0], [], [])
    B = torch.randn(10, 32, device="cuda")
    for name, C in _all_paths(rp, ci, vl, 0, 10, B).items():
        assert C.shape == (0, 32), name


def test_zero_columns_of_B():
    rp, ci, vl = _dev([0, 2, 3], [0, 1, 1], [1.0, 2.0, 3.0])
    B = torch.randn(2, 0, device="cuda")
    for name in ("csr_direct", "baseline", "zo"):
        C = _all_paths(rp, ci, vl, 2, 2, B)[name]
        assert C.shape == (2, 0), name


@pytest.mark.parametrize("N", [1, 3, 16, 17, 130])
def test_single_column_matrix_and_dense_row(oracle, N):
    # K = 1: every row gathers the same B row; row 2 is dense over K = 1.
    rp, ci, vl = _dev([0, 1, 1, 2, 3], [0, 0, 0], [2.0, -1.0, 0.5])
    B = torch.randn(1, N, device="cuda")
    ref = oracle.spmm_seq_f32(np.array([0, 1, 1, 2, 3], np.int32), np.zeros(3, np.int32),
                              np.array([2.0, -1.0, 0.5], np.float32), B.cpu().numpy())
    for name, C in _all_paths(rp, ci, vl, 4, 1, B).items():
        np.testing.assert_allclose(C.cpu().numpy(), ref, rtol=1e-3 if name in ("tc", "comm", "seg") else 0,
                                   atol=0, err_msg=name)


def test_one_long_row(oracle):
    K = 70000
    cols = np.arange(0, K, 1, dtype=np.int32)
    vals = np.random.default_rng(0).standard_normal(K).astype(np.float32)
    rp, ci, vl = _dev([0, K], cols, vals)
    B = torch.randn(K, 64, device="cuda")
    ref = oracle.spmm_f64(np.array([0, K], np.int32), cols, vals, B.cpu().numpy())
    scale = oracle.spmm_f64(np.array([0, K], np.int32), cols, np.abs(vals), np.abs(B.cpu().numpy()))
    for name, C in _all_paths(rp, ci, vl, 1, K, B).items():
        tol = 2.0 ** -10 if name in ("tc", "comm", "seg") else 1e-5
        assert np.all(np.abs(C.cpu().numpy() - ref) <= tol * scale), name


def test_B_with_too_few_rows_is_rejected():
    """A B shorter than the plan's K would make the gathers read past B: the
    plan runs refuse it instead of launching."""
    from ra_spmm import synthetic as S
    g = S.random_csr(100, 80, 6.0, seed=1)
    rp, ci, vl = g.torch("cuda")
    short = torch.randn(40, 32, device="cuda")
    z = ra_spmm.make_zero_overhead_plan(rp, g.M, g.K)
    with pytest.raises(RuntimeError, match="rows"):
        ra_spmm.run_zero_overhead_plan(z, rp, ci, vl, short)
    t = ra_spmm.make_tc_direct_plan(rp, ci, vl, g.M, g.K, 32)
    with pytest.raises(RuntimeError, match="rows"):
        ra_spmm.run_tc_direct_plan(t, short)


def test_allocation_failures_raise_cleanly_and_leak_nothing(monkeypatch):
    """Failure taxonomy (the OOM case): with RA_MAX_ALLOC_BYTES capping every
    library allocation, each plan build and each run that grows plan scratch
    raises RuntimeError (RA_ERR_OUT_OF_MEMORY); the plans stay usable once the
    cap is lifted.  Repeating the whole cycle leaves device memory outside
    torch's caching allocator unchanged (the first cycle absorbs one-time
    runtime allocations)."""
    from ra_spmm import synthetic as S
    g = S.random_csr(6000, 6000, 14.0, seed=31, skew=0.9, max_deg=3000)
    assert int(np.diff(g.rowptr).max()) > 512  # split ZO chunks: partial slots are allocated per N
    rp, ci, vl = g.torch("cuda")
    B = torch.randn(g.K, 64, device="cuda")
    ref = ra_spmm.spmm_csr_baseline(rp, ci, vl, B)
    scale = ra_spmm.spmm_csr_baseline(rp, ci, vl.abs(), B.abs())
    makers = [lambda: ra_spmm.make_zero_overhead_plan(rp, g.M, g.K),
              lambda: ra_spmm.make_zero_overhead_plan(rp.cpu(), g.M, g.K, build="host"),
              lambda: ra_spmm.make_tc_direct_plan(rp, ci, vl, g.M, g.K, 64),
              lambda: ra_spmm.make_community_tc_plan(rp.cpu(), ci.cpu(), vl.cpu(), g.M, g.K, 64, build="host")]

    def cycle():
        monkeypatch.setenv("RA_MAX_ALLOC_BYTES", "4096")
        for mk in makers:
            with pytest.raises(RuntimeError, match="RA_ERR_OUT_OF_MEMORY"):
                mk()
        monkeypatch.delenv("RA_MAX_ALLOC_BYTES")
        zo, tc = makers[0](), makers[2]()
        monkeypatch.setenv("RA_MAX_ALLOC_BYTES", "4096")
        with pytest.raises(RuntimeError, match="RA_ERR_OUT_OF_MEMORY"):
            ra_spmm.run_zero_overhead_plan(zo, rp, ci, vl, B)       # partial slots
        with pytest.raises(RuntimeError, match="RA_ERR_OUT_OF_MEMORY"):
            ra_spmm.run_tc_direct_plan(tc, B)                      # fp16 copy of B
        with pytest.raises(RuntimeError, match="RA_ERR_OUT_OF_MEMORY"):
            ra_spmm.run_tc_direct_plan_tf32(tc, B)                 # CSR of the stored values
        monkeypatch.delenv("RA_MAX_ALLOC_BYTES")
        assert bool(((ra_spmm.run_zero_overhead_plan(zo, rp, ci, vl, B) - ref).abs() <= 1e-5 * scale + 1e-30).all())
        # FP32 route: exact products of the fp16-rounded values (2^-11 relative each).
        assert bool(((ra_spmm.run_tc_direct_plan_tf32(tc, B) - ref).abs() <= 2.0 ** -10 * scale + 1e-30).all())
        assert bool(ra_spmm.run_tc_direct_plan(tc, B).isfinite().all())
        del zo, tc
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        return torch.cuda.mem_get_info()[0] + torch.cuda.memory_reserved()

    free0 = cycle()
    for _ in range(3):
        free1 = cycle()
    assert abs(free1 - free0) < (2 << 20), (free0, free1)
