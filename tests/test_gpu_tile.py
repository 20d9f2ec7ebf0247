"""GPU parity of the tile family (TC_DIRECT, COMMUNITY_TC, SEGMENT_HYBRID).

Stated tolerances (elementwise, scaled by |A||B| so cancellation cannot
inflate them):
  FP16 MFMA route   vs fp64 of the fp16-quantised inputs: 1e-5 (fp16 x fp16
                    products are exact in fp32; only summation order differs);
                    vs fp64 of the unquantised inputs: 2^-10 (two fp16
                    roundings of 2^-11 each).
  BF16 MFMA route   vs fp64 of the bf16-quantised inputs: 1e-5; unquantised: 2^-7.
  FP32-FMA route    (replaces the reference TF32 path) every kind:
                    bit-identical to the sequential fp32 fma chain over the
                    fp16-stored values in column order; on skewed rows (CV >=
                    1.5) rows of <= 256 stored nonzeros bit-identical and the
                    rest 1e-5 (conftest.assert_fp32_route).
The reference's own gate is 1e-2 * sqrt(max row nnz) absolute for tile paths
(ra_real_graph_eval.py:41-51, 478-495); every bound above is tighter.
"""
import numpy as np
import pytest
import torch

from conftest import assert_close_scaled, assert_fp32_route

pytestmark = pytest.mark.gpu

import ra_spmm  # noqa: E402
from ra_spmm import synthetic as S  # noqa: E402

MAKE = {0: ra_spmm.make_tc_direct_plan, 1: ra_spmm.make_community_tc_plan,
        2: ra_spmm.make_segment_hybrid_plan}


def run(kind, plan, B, route, g_dev):
    rp, ci, vl = g_dev
    if kind == 0:
        return (ra_spmm.run_tc_direct_plan_tf32 if route == "fp32" else ra_spmm.run_tc_direct_plan)(plan, B)
    if kind == 1:
        return (ra_spmm.run_community_tc_plan_tf32 if route == "fp32" else ra_spmm.run_community_tc_plan)(plan, B)
    fn = ra_spmm.run_segment_hybrid_plan_tf32 if route == "fp32" else ra_spmm.run_segment_hybrid_plan
    return fn(plan, ci, vl, B)


GRAPHS = {
    "skewed": lambda: S.random_csr(1003, 900, 9.0, seed=3, skew=1.1, empty_frac=0.05),
    "dense_rows": lambda: S.random_csr(200, 3000, 150.0, seed=4),    # > 64 blocks per window
    "community": lambda: S.sbm(64, 50, 12.0, 0.9, seed=6),
    "hub_windows": lambda: S.random_csr(40, 40000, 2500.0, seed=8),  # > 512 blocks: every kind splits
}


@pytest.mark.parametrize("gname", list(GRAPHS))
@pytest.mark.parametrize("kind", [0, 1, 2])
@pytest.mark.parametrize("N", [16, 32, 47, 64, 128, 256, 512])
def test_tile_routes(oracle, gname, kind, N):
    print(f"[tile] {gname} kind={kind} N={N}", flush=True)
    g = GRAPHS[gname]()
    gd = g.torch("cuda")
    B = np.random.default_rng(N + kind).standard_normal((g.K, N)).astype(np.float32)
    Bd = torch.from_numpy(B).cuda()
    exact = oracle.spmm_f64(g.rowptr, g.colind, g.vals, B)
    scale = oracle.spmm_f64(g.rowptr, g.colind, np.abs(g.vals), np.abs(B))

    plan = MAKE[kind](gd[0].cpu(), gd[1].cpu(), gd[2].cpu(), g.M, g.K, N)
    assert plan.valid and plan.active
    C = run(kind, plan, Bd, "f16", gd).cpu().numpy()
    qv, qb = oracle.quantize_f16(g.vals), oracle.quantize_f16(B)
    assert_close_scaled(C, oracle.spmm_tile_f64(g.rowptr, g.colind, g.vals, B, "f16"),
                        oracle.spmm_f64(g.rowptr, g.colind, np.abs(qv), np.abs(qb)), 1e-5, "f16 vs quantised")
    assert_close_scaled(C, exact, scale, 2.0 ** -10, "f16 vs exact")

    C32 = run(kind, plan, Bd, "fp32", gd).cpu().numpy()
    qv = oracle.quantize_f16_scaled(g.vals, oracle.tile_value_scale_log2(g.vals))
    assert_fp32_route(C32, g.rowptr, g.colind, qv, B, oracle, f"fp32 {gname} kind={kind}")
    np.testing.assert_array_equal(run(kind, plan, Bd, "fp32", gd).cpu().numpy(), C32)

    # Deterministic across runs.
    np.testing.assert_array_equal(run(kind, plan, Bd, "f16", gd).cpu().numpy(), C)


@pytest.mark.parametrize("kind", [0, 1, 2])
def test_tiny_values_keep_fp16_precision(oracle, kind):
    """GCN-style values far below 1 (hub pairs give 1/sqrt(d_i d_j) ~ 1e-5):
    the plan's power-of-two value scale keeps them out of the fp16 subnormal
    range, so the FP16 route stays within 2^-10 of the exact product."""
    g = S.random_csr(600, 500, 20.0, seed=12)
    g.vals = (np.abs(g.vals) * 3e-6).astype(np.float32)
    gd = g.torch("cuda")
    B = np.random.default_rng(1).standard_normal((g.K, 64)).astype(np.float32)
    plan = MAKE[kind](gd[0].cpu(), gd[1].cpu(), gd[2].cpu(), g.M, g.K, 64)
    C = run(kind, plan, torch.from_numpy(B).cuda(), "f16", gd).cpu().numpy()
    exact = oracle.spmm_f64(g.rowptr, g.colind, g.vals, B)
    scale = oracle.spmm_f64(g.rowptr, g.colind, np.abs(g.vals), np.abs(B))
    assert_close_scaled(C, exact, scale, 2.0 ** -10, "tiny values")


@pytest.mark.parametrize("kind", [0, 1, 2])
def test_bf16_plan_and_lowp_entry(oracle, kind):
    g = GRAPHS["skewed"]()
    gd = g.torch("cuda")
    N = 128
    B = np.random.default_rng(9).standard_normal((g.K, N)).astype(np.float32)
    Bd = torch.from_numpy(B).cuda()
    plan = MAKE[kind](gd[0].cpu(), gd[1].cpu(), gd[2].cpu(), g.M, g.K, N, "bf16")
    C = run(kind, plan, Bd, "bf16", gd).cpu().numpy()
    qv, qb = oracle.quantize_bf16(g.vals), oracle.quantize_bf16(B)
    assert_close_scaled(C, oracle.spmm_tile_f64(g.rowptr, g.colind, g.vals, B, "bf16"),
                        oracle.spmm_f64(g.rowptr, g.colind, np.abs(qv), np.abs(qb)), 1e-5, "bf16")
    assert_close_scaled(C, oracle.spmm_f64(g.rowptr, g.colind, g.vals, B),
                        oracle.spmm_f64(g.rowptr, g.colind, np.abs(g.vals), np.abs(B)), 2.0 ** -7, "bf16 exact")
    # Native bf16 B: no conversion pass, identical result.
    C2 = run(kind, plan, Bd.to(torch.bfloat16), "bf16", gd).cpu().numpy()
    np.testing.assert_array_equal(C, C2)
    # fp16 plan with native fp16 B.
    p16 = MAKE[kind](gd[0].cpu(), gd[1].cpu(), gd[2].cpu(), g.M, g.K, N)
    np.testing.assert_array_equal(run(kind, p16, Bd, "f16", gd).cpu().numpy(),
                                  run(kind, p16, Bd.half(), "f16", gd).cpu().numpy())


def test_inactive_plan_raises_and_families_agree(oracle):
    g = GRAPHS["community"]()
    gd = g.torch("cuda")
    p = ra_spmm.make_tc_direct_plan(gd[0].cpu(), gd[1].cpu(), gd[2].cpu(), g.M, g.K, 8)
    assert not p.active
    with pytest.raises(RuntimeError):
        ra_spmm.run_tc_direct_plan(p, torch.randn(g.K, 64, device="cuda"))
    B = torch.randn(g.K, 64, device="cuda")
    outs = [run(k, MAKE[k](gd[0].cpu(), gd[1].cpu(), gd[2].cpu(), g.M, g.K, 64), B, "fp32", gd)
            for k in (0, 1, 2)]
    # One CSR of the stored values for every kind: the FP32 route agrees bit for bit.
    np.testing.assert_array_equal(outs[0].cpu().numpy(), outs[1].cpu().numpy())
    np.testing.assert_array_equal(outs[0].cpu().numpy(), outs[2].cpu().numpy())


@pytest.mark.parametrize("N", [256, 512])  # 32-row windows run on the 32x32x16 MFMA kernel at N >= 512
def test_c3_full_size_properties(oracle, N):
    """config C3 (SBM, fp16 values) at full size through TC_DIRECT and
    COMMUNITY_TC: a row sample against the oracle, and all-ones row sums."""
    print(f"[c3 full] N={N}", flush=True)
    g = S.CONFIGS["C3"]()
    gd = g.torch("cuda")
    rng = np.random.default_rng(2)
    B = rng.standard_normal((g.K, N)).astype(np.float16).astype(np.float32)
    Bd = torch.from_numpy(B).cuda()
    deg = np.diff(g.rowptr)
    rows = np.arange(0, g.M, 1021)
    sub_rp = np.concatenate([[0], np.cumsum(deg[rows])]).astype(np.int32)
    sub_ci = np.concatenate([g.colind[g.rowptr[r]:g.rowptr[r + 1]] for r in rows])
    sub_vl = np.concatenate([g.vals[g.rowptr[r]:g.rowptr[r + 1]] for r in rows])
    ref = oracle.spmm_f64(sub_rp, sub_ci, sub_vl, B)
    scale = oracle.spmm_f64(sub_rp, sub_ci, np.abs(sub_vl), np.abs(B))
    for kind in (0, 1, 2):
        plan = MAKE[kind](gd[0].cpu(), gd[1].cpu(), gd[2].cpu(), g.M, g.K, N)
        C = run(kind, plan, Bd, "f16", gd)
        assert_close_scaled(C.cpu().numpy()[rows], ref, scale, 1e-5, f"C3 kind {kind}")
        ones = torch.ones(g.K, 16, device="cuda")
        rs = run(kind, plan, ones, "f16", gd)[:, 0].double().cpu().numpy()
        exact = np.add.reduceat(np.append(g.vals.astype(np.float64), 0), g.rowptr[:-1])
        exact[deg == 0] = 0
        assert np.all(np.abs(rs - exact) <= 1e-5 * np.maximum(1, np.abs(exact)))
        del plan


def test_c4_full_size_properties(oracle):
    """config C4 (log-normal degrees to 20k, fp16 values) at full size through
    the routed COMMUNITY_TC, TC_DIRECT and SEGMENT_HYBRID with the automatic 8
    column partitions: a row sample (including the 20 longest rows) against
    the oracle at N=512 on the FP16 route (1e-5) and the FP32 route
    (bit-exact), the all-ones row sums on every row, and a second call
    bit-identical to the first (the split windows' merge is deterministic)."""
    g = S.CONFIGS["C4"]()
    gd = g.torch("cuda")
    N = 512
    rng = np.random.default_rng(4)
    B = rng.standard_normal((g.K, N)).astype(np.float16).astype(np.float32)
    Bd = torch.from_numpy(B).cuda()
    deg = np.diff(g.rowptr)
    rows = np.unique(np.concatenate([np.arange(0, g.M, 2003), np.argsort(deg)[-20:]]))
    sub_rp = np.concatenate([[0], np.cumsum(deg[rows])]).astype(np.int32)
    sub_ci = np.concatenate([g.colind[g.rowptr[r]:g.rowptr[r + 1]] for r in rows])
    sub_vl = np.concatenate([g.vals[g.rowptr[r]:g.rowptr[r + 1]] for r in rows])
    ref = oracle.spmm_f64(sub_rp, sub_ci, sub_vl, B)
    scale = oracle.spmm_f64(sub_rp, sub_ci, np.abs(sub_vl), np.abs(B))
    exact = np.add.reduceat(np.append(g.vals.astype(np.float64), 0), g.rowptr[:-1])
    exact[deg == 0] = 0
    for kind in (1, 0, 2):
        print(f"[c4 full] kind={kind}", flush=True)
        plan = MAKE[kind](gd[0], gd[1], gd[2], g.M, g.K, N)
        assert plan.col_parts == 8 and plan.rows_per_window == 8
        C = run(kind, plan, Bd, "f16", gd)
        assert_close_scaled(C.cpu().numpy()[rows], ref, scale, 1e-5, f"C4 kind {kind}")
        assert torch.equal(C, run(kind, plan, Bd, "f16", gd)), f"C4 kind {kind}: second call differs"
        del C
        # FP32 route over the 8 column ranges: one fma chain per element in
        # ascending column order (values are fp16-representable: stored exactly).
        C32 = run(kind, plan, Bd, "fp32", gd).cpu().numpy()[rows]
        np.testing.assert_array_equal(C32, oracle.spmm_seq_f32(sub_rp, sub_ci, sub_vl, B), err_msg=f"C4 fp32 {kind}")
        ones = torch.ones(g.K, 16, device="cuda")
        rs = run(kind, plan, ones, "f16", gd)[:, 0].double().cpu().numpy()
        assert np.all(np.abs(rs - exact) <= 1e-5 * np.maximum(1, np.abs(exact)))
        del plan
        torch.cuda.empty_cache()


def test_c4_full_size_bf16(oracle):
    """config C4 at full size with bf16-valued plans of every kind (bf16 B,
    N=512, 8 column partitions): a row sample with the 20 longest rows against
    the fp64 product of the bf16-quantised inputs (1e-5), the all-ones row sums
    against the bf16-rounded values (1e-5), and a repeated call bit-identical."""
    g = S.CONFIGS["C4"]()
    gd = g.torch("cuda")
    N = 512
    B = np.random.default_rng(5).standard_normal((g.K, N)).astype(np.float32)
    Bd = torch.from_numpy(oracle.quantize_bf16(B).astype(np.float32)).cuda().to(torch.bfloat16)
    deg = np.diff(g.rowptr)
    rows = np.unique(np.concatenate([np.arange(0, g.M, 2003), np.argsort(deg)[-20:]]))
    sub_rp = np.concatenate([[0], np.cumsum(deg[rows])]).astype(np.int32)
    sub_ci = np.concatenate([g.colind[g.rowptr[r]:g.rowptr[r + 1]] for r in rows])
    sub_vl = np.concatenate([g.vals[g.rowptr[r]:g.rowptr[r + 1]] for r in rows])
    ref = oracle.spmm_tile_f64(sub_rp, sub_ci, sub_vl, B, "bf16")
    scale = oracle.spmm_f64(sub_rp, sub_ci, np.abs(oracle.quantize_bf16(sub_vl)), np.abs(oracle.quantize_bf16(B)))
    qv = oracle.quantize_bf16(g.vals).astype(np.float64)
    exact = np.add.reduceat(np.append(qv, 0), g.rowptr[:-1])
    exact[deg == 0] = 0
    for kind in (1, 0, 2):
        print(f"[c4 full bf16] kind={kind}", flush=True)
        plan = MAKE[kind](gd[0], gd[1], gd[2], g.M, g.K, N, "bf16")
        assert plan.col_parts == 8
        C = run(kind, plan, Bd, "bf16", gd)
        assert_close_scaled(C.cpu().numpy()[rows], ref, scale, 1e-5, f"C4 bf16 kind {kind}")
        assert torch.equal(C, run(kind, plan, Bd, "bf16", gd)), f"C4 bf16 kind {kind}: second call differs"
        del C
        ones = torch.ones(g.K, 16, device="cuda", dtype=torch.bfloat16)
        rs = run(kind, plan, ones, "bf16", gd)[:, 0].double().cpu().numpy()
        assert np.all(np.abs(rs - exact) <= 1e-5 * np.maximum(1, np.abs(exact)))
        del plan
        torch.cuda.empty_cache()


@pytest.mark.parametrize("N", [1024, 2000])
@pytest.mark.parametrize("kind", [0, 1, 2])
def test_wide_B(oracle, kind, N):
    """Many column slices: N=1024 (8 slices of 128, slice-major order with
    the window remap) and N=2000 (not a multiple of 8: B is padded to ldb in
    the fp16 copy, the tail columns are masked)."""
    g = GRAPHS["skewed"]()
    gd = g.torch("cuda")
    B = np.random.default_rng(N + kind).standard_normal((g.K, N)).astype(np.float32)
    Bd = torch.from_numpy(B).cuda()
    plan = MAKE[kind](gd[0], gd[1], gd[2], g.M, g.K, N)
    C = run(kind, plan, Bd, "f16", gd).cpu().numpy()
    qv, qb = oracle.quantize_f16(g.vals), oracle.quantize_f16(B)
    assert_close_scaled(C, oracle.spmm_tile_f64(g.rowptr, g.colind, g.vals, B, "f16"),
                        oracle.spmm_f64(g.rowptr, g.colind, np.abs(qv), np.abs(qb)), 1e-5, f"wide f16 N={N}")
    qs = oracle.quantize_f16_scaled(g.vals, oracle.tile_value_scale_log2(g.vals))
    assert_fp32_route(run(kind, plan, Bd, "fp32", gd).cpu().numpy(), g.rowptr, g.colind, qs, B, oracle,
                      f"wide fp32 N={N}")
