"""The C ABI driven directly through ctypes (no torch binding): routing from a
device rowptr, device-built ZERO_OVERHEAD_CSR and tile plans (every height and
both column schedules), runs on the current stream, and the diagnostic
features, each checked against the oracle."""
import ctypes

import numpy as np
import pytest
import torch

from conftest import assert_close_scaled

pytestmark = pytest.mark.gpu

import ra_spmm  # noqa: E402,F401  (loads torch's HIP runtime first)
from ra_spmm import capi  # noqa: E402
from ra_spmm import synthetic as S  # noqa: E402

P = capi.ptr


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def test_route_and_zero_overhead_through_the_abi(oracle):
    lib = capi.load()
    g = S.random_csr(5000, 4000, 12.0, seed=31, skew=0.9, empty_frac=0.05, max_deg=2000)
    rp, ci, vl = g.torch("cuda")
    f = capi.Features()
    capi.check(lib.ra_features_device(P(rp), g.M, g.K, 128, _stream(), ctypes.byref(f)))
    r = capi.Route()
    capi.check(lib.ra_route_dispatch(ctypes.byref(f), 0, 1, ctypes.byref(r)))  # MAIN, MI355X table
    py = ra_spmm.route_with_rules(f.avg_nnz_per_row, f.degree_cv, g.M, 128)
    assert lib.ra_path_name(r.chosen_path).decode() == py.replace("_TF32", "")
    plan = ctypes.c_void_p()
    capi.check(lib.ra_zo_plan_create_device(P(rp), g.M, g.K, _stream(), ctypes.byref(plan)))
    B = np.random.default_rng(1).standard_normal((g.K, 128)).astype(np.float32)
    Bd = torch.from_numpy(B).cuda()
    C = torch.empty(g.M, 128, device="cuda")
    capi.check(lib.ra_zo_plan_run(plan, P(rp), P(ci), P(vl), P(Bd), P(C), 128, _stream()))
    torch.cuda.synchronize()
    lib.ra_zo_plan_destroy(plan)
    short = np.diff(g.rowptr) <= 256
    seq = oracle.spmm_seq_f32(g.rowptr, g.colind, g.vals, B)
    np.testing.assert_array_equal(C.cpu().numpy()[short], seq[short])
    assert_close_scaled(C.cpu().numpy(), oracle.spmm_f64(g.rowptr, g.colind, g.vals, B),
                        oracle.spmm_f64(g.rowptr, g.colind, np.abs(g.vals), np.abs(B)), 1e-5, "zo abi")


@pytest.mark.parametrize("rows", [0, 8, 16, 32])
@pytest.mark.parametrize("kind", [0, 1, 2])
def test_tile_plans_through_the_abi(oracle, rows, kind):
    lib = capi.load()
    g = S.sbm(40, 40, 14.0, 0.9, seed=kind + rows)
    rp, ci, vl = g.torch("cuda")
    plan = ctypes.c_void_p()
    capi.check(lib.ra_tile_plan_create_device(kind, P(rp), P(ci), P(vl), g.M, g.K, 96, 1, rows, _stream(),  # RA_DTYPE_F16
                                              ctypes.byref(plan)))
    info = capi.TileInfo()
    capi.check(lib.ra_tile_plan_get_info(plan, ctypes.byref(info)))
    assert info.active == 1 and (rows == 0 or info.rows_per_window == rows)
    B = np.random.default_rng(2).standard_normal((g.K, 96)).astype(np.float32)
    Bd = torch.from_numpy(B).cuda()
    C = torch.empty(g.M, 96, device="cuda")
    capi.check(lib.ra_tile_plan_run(plan, P(Bd), P(C), 96, 0, _stream()))  # FP16 route
    torch.cuda.synchronize()
    qv, qb = oracle.quantize_f16(g.vals), oracle.quantize_f16(B)
    assert_close_scaled(C.cpu().numpy(), oracle.spmm_tile_f64(g.rowptr, g.colind, g.vals, B, "f16"),
                        oracle.spmm_f64(g.rowptr, g.colind, np.abs(qv), np.abs(qb)), 1e-5, "tile abi")
    n = ctypes.c_int64()
    capi.check(lib.ra_tile_plan_export(plan, b"atox", None, ctypes.byref(n)))
    assert n.value == info.num_blocks * (8 if info.rows_per_window == 8 else 32)
    lib.ra_tile_plan_destroy(plan)


def test_analyze_matrix_through_the_abi():
    from oracle import diagnostics_oracle as DO
    lib = capi.load()
    g = S.random_csr(300, 250, 9.0, seed=4, skew=1.0)
    d = capi.DiagFeatures()
    capi.check(lib.ra_analyze_matrix(P(g.rowptr), P(g.colind), g.M, g.K, 128, ctypes.byref(d)))
    ref = DO.analyze_reference(g.rowptr, g.colind, g.M, g.K, 128)
    for k in DO.KEYS:
        assert np.float32(getattr(d, k)) == ref[k], k
