"""Seeded random matrices through every path, each against its bar:
  CSR_DIRECT, baseline            bit-identical to the oracle's fma chain
  fp16 guardrail                  bit-identical to the chain on fp16-rounded A values and B
  ZERO_OVERHEAD_CSR               rows <= 256 nnz bit-identical, all within 1e-5 of |A||B|
  tile FP16 route (any layout)    1e-5 of |Aq||Bq| against fp64 of the quantised inputs
  tile FP32 route (any layout)    1e-5 of |Aq||B| against fp64 of the stored values
Shapes, densities, skew, empty rows, duplicate entries, N (1..520, ragged),
window heights, column partitions and the stored value type (fp16 / bf16)
vary with the seed."""
import os

import numpy as np
import pytest
import torch

from conftest import assert_close_scaled, assert_fp32_route

pytestmark = pytest.mark.gpu

import ra_spmm  # noqa: E402
from ra_spmm import synthetic as S  # noqa: E402


def _graph(rng):
    M = int(rng.integers(1, 3000))
    K = int(rng.integers(1, 3000))
    d = float(rng.choice([0.5, 3.0, 12.0, 40.0]))
    g = S.random_csr(M, K, min(d, K), seed=int(rng.integers(1 << 30)), skew=float(rng.choice([0.0, 1.0, 1.4])),
                     empty_frac=float(rng.choice([0.0, 0.1])), max_deg=K)
    if rng.random() < 0.3 and g.nnz > 0:  # duplicate some (row, column) entries
        deg = np.diff(g.rowptr)
        ci = g.colind.copy()
        for r in np.flatnonzero(deg >= 2)[:50]:
            a = g.rowptr[r]
            ci[a + 1] = ci[a]
        rows = np.repeat(np.arange(M), deg)
        order = np.lexsort((ci, rows))
        g = S.Graph(g.rowptr, ci[order].astype(np.int32), g.vals[order], M, K, "dups")
    return g


@pytest.mark.parametrize("seed", range(64))
def test_random_parity(oracle, seed):
    rng = np.random.default_rng(1000 + seed)
    g = _graph(rng)
    N = int(rng.choice([1, 7, 16, 33, 64, 100, 128, 260, 300, 512, 520]))
    print(f"[random] seed={seed} M={g.M} K={g.K} nnz={g.nnz} N={N}", flush=True)
    rp, ci, vl = g.torch("cuda")
    B = rng.standard_normal((g.K, N)).astype(np.float32)
    Bd = torch.from_numpy(B).cuda()
    seq = oracle.spmm_seq_f32(g.rowptr, g.colind, g.vals, B)
    exact = oracle.spmm_f64(g.rowptr, g.colind, g.vals, B)
    scale = oracle.spmm_f64(g.rowptr, g.colind, np.abs(g.vals), np.abs(B))
    np.testing.assert_array_equal(ra_spmm.spmm_csr_direct(rp, ci, vl, Bd).cpu().numpy(), seq)
    np.testing.assert_array_equal(ra_spmm.spmm_csr_baseline(rp, ci, vl, Bd).cpu().numpy(), seq)
    np.testing.assert_array_equal(
        ra_spmm.spmm_cusparse_fp16(rp, ci, vl, Bd).cpu().numpy(),
        oracle.spmm_seq_f32(g.rowptr, g.colind, oracle.quantize_f16(g.vals), oracle.quantize_f16(B)))
    z = ra_spmm.make_zero_overhead_plan(rp, g.M, g.K)
    C = ra_spmm.run_zero_overhead_plan(z, rp, ci, vl, Bd).cpu().numpy()
    short = np.diff(g.rowptr) <= 256
    np.testing.assert_array_equal(C[short], seq[short])
    assert_close_scaled(C, exact, scale, 1e-5, "zo")
    if N < 16:
        return
    rows = int(rng.choice([0, 8, 16, 32]))
    parts = str(int(rng.choice([1, 1, 2, 8])))
    vdt = "bf16" if rng.random() < 0.25 else "fp16"
    quant = oracle.quantize_bf16 if vdt == "bf16" else oracle.quantize_f16
    qv, qb = quant(g.vals), quant(B)
    mrp, mci, mvl = oracle.merge_duplicates(g.rowptr, g.colind, g.vals)  # what a plan stores
    qs = (oracle.quantize_bf16(mvl) if vdt == "bf16"
          else oracle.quantize_f16_scaled(mvl, oracle.tile_value_scale_log2(g.vals)))
    old = os.environ.get("RA_TILE_COL_PARTS")
    os.environ["RA_TILE_COL_PARTS"] = parts
    try:
        for kind, mk in enumerate((ra_spmm.make_tc_direct_plan, ra_spmm.make_community_tc_plan,
                                   ra_spmm.make_segment_hybrid_plan)):
            p = mk(rp, ci, vl, g.M, g.K, N, vdt, rows_per_window=rows)
            C16 = ra_spmm.run_tile_plan_route(p, Bd, vdt).cpu().numpy()
            assert_close_scaled(C16, oracle.spmm_tile_f64(g.rowptr, g.colind, g.vals, B,
                                                          "bf16" if vdt == "bf16" else "f16"),
                                oracle.spmm_f64(g.rowptr, g.colind, np.abs(qv), np.abs(qb)), 1e-5,
                                f"tile {vdt} kind={kind} rows={p.rows_per_window} parts={p.col_parts}")
            C32 = ra_spmm.run_tile_plan_route(p, Bd, "fp32").cpu().numpy()
            assert_fp32_route(C32, mrp, mci, qs, B, oracle,
                              f"tile fp32 kind={kind} rows={p.rows_per_window} parts={p.col_parts}")
    finally:
        if old is None:
            del os.environ["RA_TILE_COL_PARTS"]
        else:
            os.environ["RA_TILE_COL_PARTS"] = old
