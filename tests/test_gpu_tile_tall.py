"""Tall tile windows (16 or 32 rows, blocks of 32 vectors): the device build
decodes back to the matrix (values rounded and scaled as in the 8-row format),
and the MFMA / FP32 routes meet the 8-row format's bars:
  FP16 / BF16 route  vs fp64 of the quantised inputs: 1e-5 (scaled by |A||B|);
  FP32 route         the CSR of the stored values, as for 8-row plans
                     (conftest.assert_fp32_route).
The automatic height picks a tall layout where rows of a window share columns
(community graphs) and keeps 8 rows where they do not."""
import numpy as np
import pytest
import torch

from conftest import assert_close_scaled, assert_fp32_route

pytestmark = pytest.mark.gpu

import ra_spmm  # noqa: E402
from ra_spmm import synthetic as S  # noqa: E402

MAKE = {0: ra_spmm.make_tc_direct_plan, 1: ra_spmm.make_community_tc_plan,
        2: ra_spmm.make_segment_hybrid_plan}
GRAPHS = {
    "skewed": lambda: S.random_csr(1003, 900, 9.0, seed=3, skew=1.1, empty_frac=0.05),
    "community": lambda: S.sbm(64, 50, 12.0, 0.9, seed=6),
    "dense_rows": lambda: S.random_csr(200, 3000, 150.0, seed=4),
    "hub_windows": lambda: S.random_csr(40, 40000, 2500.0, seed=8),
}


def _decode(plan, M, K, bf16=False):
    """Dense matrix of a tall plan's arrays (stored values, scale removed)."""
    H = plan.rows_per_window
    boff = ra_spmm.export_tile_plan(plan, "block_offsets").numpy()
    atox = ra_spmm.export_tile_plan(plan, "atox").numpy()
    vals = ra_spmm.export_tile_plan(plan, "vals").numpy().view(np.uint16)
    wr = ra_spmm.export_tile_plan(plan, "win_rows").numpy()
    if not bf16:
        v = vals.view(np.float16).astype(np.float64) * 2.0 ** -plan.value_scale_log2
    else:
        v = (vals.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    D = np.zeros((M, K))
    for w in range(len(boff) - 1):
        for b in range(boff[w], boff[w + 1]):
            for kk in range(32):
                c = atox[b * 32 + kk]
                if c < 0:
                    continue
                for slot in range(H):
                    x = v[b * H * 32 + (((slot >> 4) * 4 + (kk >> 3)) * 16 + (slot & 15)) * 8 + (kk & 7)]
                    if x != 0:
                        r = wr[w * H + slot]
                        assert r >= 0
                        D[r, c] += x
    return D


@pytest.mark.parametrize("rows", [16, 32])
@pytest.mark.parametrize("kind", [0, 1, 2])
@pytest.mark.parametrize("gname", ["skewed", "community"])
def test_tall_plan_decodes_to_matrix(oracle, rows, kind, gname):
    g = GRAPHS[gname]()
    rp, ci, vl = g.torch("cuda")
    plan = MAKE[kind](rp, ci, vl, g.M, g.K, 64, rows_per_window=rows)
    assert plan.rows_per_window == rows and plan.active
    got = _decode(plan, g.M, g.K)
    q = oracle.quantize_f16_scaled(g.vals, oracle.tile_value_scale_log2(g.vals)).astype(np.float64)
    ref = np.zeros((g.M, g.K))
    np.add.at(ref, (np.repeat(np.arange(g.M), np.diff(g.rowptr)), g.colind), q)
    np.testing.assert_array_equal(got, ref)


@pytest.mark.parametrize("gname", list(GRAPHS))
@pytest.mark.parametrize("kind", [0, 1, 2])
@pytest.mark.parametrize("rows", [16, 32])
@pytest.mark.parametrize("N", [16, 47, 128, 256, 520])
def test_tall_routes(oracle, gname, kind, rows, N):
    print(f"[tall] {gname} kind={kind} rows={rows} N={N}", flush=True)
    g = GRAPHS[gname]()
    rp, ci, vl = g.torch("cuda")
    B = np.random.default_rng(N + kind).standard_normal((g.K, N)).astype(np.float32)
    Bd = torch.from_numpy(B).cuda()
    plan = MAKE[kind](rp, ci, vl, g.M, g.K, N, rows_per_window=rows)
    assert plan.rows_per_window == rows
    C = ra_spmm.run_tile_plan_route(plan, Bd, "fp16").cpu().numpy()
    qv, qb = oracle.quantize_f16(g.vals), oracle.quantize_f16(B)
    assert_close_scaled(C, oracle.spmm_tile_f64(g.rowptr, g.colind, g.vals, B, "f16"),
                        oracle.spmm_f64(g.rowptr, g.colind, np.abs(qv), np.abs(qb)), 1e-5, "tall f16")
    C32 = ra_spmm.run_tile_plan_route(plan, Bd, "fp32").cpu().numpy()
    qs = oracle.quantize_f16_scaled(g.vals, oracle.tile_value_scale_log2(g.vals))
    assert_fp32_route(C32, g.rowptr, g.colind, qs, B, oracle, f"tall fp32 {gname} kind={kind} rows={rows}")
    np.testing.assert_array_equal(ra_spmm.run_tile_plan_route(plan, Bd, "fp16").cpu().numpy(), C)


@pytest.mark.parametrize("rows", [16, 32])
@pytest.mark.parametrize("N", [128, 512])  # 32-row windows at N >= 512 run on the 32x32x16 MFMA kernel
def test_tall_bf16_and_lowp(oracle, rows, N):
    g = GRAPHS["community"]()
    rp, ci, vl = g.torch("cuda")
    B = np.random.default_rng(9).standard_normal((g.K, N)).astype(np.float32)
    Bd = torch.from_numpy(B).cuda()
    plan = ra_spmm.make_tc_direct_plan(rp, ci, vl, g.M, g.K, N, "bf16", rows_per_window=rows)
    C = ra_spmm.run_tile_plan_route(plan, Bd, "bf16").cpu().numpy()
    qv, qb = oracle.quantize_bf16(g.vals), oracle.quantize_bf16(B)
    assert_close_scaled(C, oracle.spmm_tile_f64(g.rowptr, g.colind, g.vals, B, "bf16"),
                        oracle.spmm_f64(g.rowptr, g.colind, np.abs(qv), np.abs(qb)), 1e-5, "tall bf16")
    np.testing.assert_array_equal(C, ra_spmm.run_tc_direct_plan(plan, Bd.to(torch.bfloat16)).cpu().numpy())


def test_auto_height_follows_column_sharing():
    comm = S.sbm(200, 60, 20.0, 0.95, seed=2)     # rows of a window share columns
    rnd = S.random_csr(5000, 200000, 16.0, seed=3)  # they do not
    for g, tall in ((comm, True), (rnd, False)):
        rp, ci, vl = g.torch("cuda")
        p = ra_spmm.make_tc_direct_plan(rp, ci, vl, g.M, g.K, 128)
        assert (p.rows_per_window > 8) == tall, (g.name, p.rows_per_window)
    with pytest.raises(RuntimeError):
        ra_spmm.make_tc_direct_plan(rp.cpu(), ci.cpu(), vl.cpu(), g.M, g.K, 128, build="host", rows_per_window=32)


def _model_rows(g):
    """The height the build's cost model picks from exact distinct (row / h,
    column) counts: 10 per 32 vectors at h = 8 and 16, 11 at h = 32, a tall
    layout only when it saves >= 15%."""
    rows = np.repeat(np.arange(g.M, dtype=np.int64), np.diff(g.rowptr.astype(np.int64)))
    c = g.colind.astype(np.int64)
    v = {h: np.unique((rows // h) * g.K + c).size for h in (8, 16, 32)}
    c8, c16, c32 = 10.0 * v[8], 10.0 * v[16], 11.0 * v[32]
    if c32 <= 0.85 * c8 and c32 <= c16:
        return 32
    if c16 <= 0.85 * c8:
        return 16
    return 8


@pytest.mark.parametrize("gname", ["sbm_large", "random_large", "mixed_large", "mixed_weak"])
def test_sampled_height_matches_exact_model(gname):
    """Large matrices count vectors on every S-th 32-row window only; the
    height chosen equals the exact model's on community, random and mixed
    graphs."""
    graphs = {
        "sbm_large": lambda: S.sbm(512, 128, 96.0, 0.9, seed=12),            # 65k rows, 5.4M nnz
        "random_large": lambda: S.random_csr(70000, 300000, 80.0, seed=13),   # 5.6M nnz
        "mixed_large": lambda: S.sbm(1024, 96, 60.0, 0.7, seed=14),          # weaker communities (model: 0.78)
        "mixed_weak": lambda: S.sbm(1024, 96, 60.0, 0.4, seed=14),           # model: 0.92 -> 8 rows
    }
    g = graphs[gname]()
    assert g.nnz >= (1 << 21) * 2  # sampling is on (S >= 2)
    rp, ci, vl = g.torch("cuda")
    p = ra_spmm.make_tc_direct_plan(rp, ci, vl, g.M, g.K, 128)
    assert p.rows_per_window == _model_rows(g), (gname, p.rows_per_window)
