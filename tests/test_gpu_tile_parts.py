"""Column-partitioned tile plans: windows cut into P cells by column range, one
launch per partition adding into C in partition order.  The FP16/BF16 routes
keep the 8-row format's bar (1e-5 of |A||B| against fp64 of the quantised
inputs); the FP32 route is no longer one fma chain per row (each partition
starts its own), so it is held to 1e-5 as well.  Results are identical from run
to run."""
import os

import numpy as np
import pytest
import torch

from conftest import assert_close_scaled, assert_fp32_route

pytestmark = pytest.mark.gpu

import ra_spmm  # noqa: E402
from ra_spmm import synthetic as S  # noqa: E402

MAKE = {0: ra_spmm.make_tc_direct_plan, 1: ra_spmm.make_community_tc_plan,
        2: ra_spmm.make_segment_hybrid_plan}


def _build(kind, g, N, parts, rows=0):
    rp, ci, vl = g.torch("cuda")
    old = os.environ.get("RA_TILE_COL_PARTS")
    os.environ["RA_TILE_COL_PARTS"] = str(parts)
    try:
        return MAKE[kind](rp, ci, vl, g.M, g.K, N, rows_per_window=rows)
    finally:
        if old is None:
            del os.environ["RA_TILE_COL_PARTS"]
        else:
            os.environ["RA_TILE_COL_PARTS"] = old


GRAPHS = {
    "skewed": lambda: S.random_csr(1003, 900, 9.0, seed=3, skew=1.1, empty_frac=0.05),
    "dense_rows": lambda: S.random_csr(200, 3000, 150.0, seed=4),
    "hub_windows": lambda: S.random_csr(40, 40000, 2500.0, seed=8),
    "community": lambda: S.sbm(64, 50, 12.0, 0.9, seed=6),
}


@pytest.mark.parametrize("gname", list(GRAPHS))
@pytest.mark.parametrize("kind", [0, 1, 2])
@pytest.mark.parametrize("parts", [2, 8])
@pytest.mark.parametrize("rows", [8, 32])
def test_partitioned_routes(oracle, gname, kind, parts, rows):
    print(f"[parts] {gname} kind={kind} P={parts} rows={rows}", flush=True)
    g = GRAPHS[gname]()
    N = 96
    B = np.random.default_rng(parts + kind).standard_normal((g.K, N)).astype(np.float32)
    Bd = torch.from_numpy(B).cuda()
    plan = _build(kind, g, N, parts, rows)
    assert plan.col_parts == parts and plan.rows_per_window == rows
    C = ra_spmm.run_tile_plan_route(plan, Bd, "fp16").cpu().numpy()
    qv, qb = oracle.quantize_f16(g.vals), oracle.quantize_f16(B)
    assert_close_scaled(C, oracle.spmm_tile_f64(g.rowptr, g.colind, g.vals, B, "f16"),
                        oracle.spmm_f64(g.rowptr, g.colind, np.abs(qv), np.abs(qb)), 1e-5, "parts f16")
    qs = oracle.quantize_f16_scaled(g.vals, oracle.tile_value_scale_log2(g.vals))
    C32 = ra_spmm.run_tile_plan_route(plan, Bd, "fp32").cpu().numpy()
    assert_fp32_route(C32, g.rowptr, g.colind, qs, B, oracle, f"parts fp32 parts={parts} rows={rows}")
    np.testing.assert_array_equal(ra_spmm.run_tile_plan_route(plan, Bd, "fp16").cpu().numpy(), C)


def test_auto_partitions_long_rows_over_wide_B():
    wide = S.random_csr(400, 70000, 150.0, seed=5)
    narrow = S.random_csr(400, 3000, 150.0, seed=5)
    for g, parts in ((wide, 8), (narrow, 1)):
        rp, ci, vl = g.torch("cuda")
        assert ra_spmm.make_tc_direct_plan(rp, ci, vl, g.M, g.K, 64).col_parts == parts
