"""Config C1 (Erdos-Renyi, M=10,000, avg degree 8, GCN-normalised fp32
values, B ~ N(0,1) fp32) on the GPU, through the routed path and every
deployed path, at N=64 (the config's width) and N=128.

References: oracle.spmm_seq_f32 (the sequential fma chain of
csr/csr_direct.cu:201-228) and torch.sparse CPU SpMM, which the benchmark
names as C1's bit-level reference (the reference harness checks against a
sparse library product the same way, test_ra.py:493-523).
Bars: CSR_DIRECT, the baseline guardrail and ZERO_OVERHEAD_CSR (every C1 row
has <= 64 nonzeros) bit-identical to the oracle; every FP32 path within 1e-5
of |A||B| of torch.sparse CPU (and bit-equality with it is reported);
the FP16 MFMA tile paths within 2^-10 of |A||B| of the exact product; the
FP32 route of the tile plans per conftest.assert_fp32_route.
"""
import numpy as np
import pytest
import torch

from conftest import assert_close_scaled, assert_fp32_route

pytestmark = pytest.mark.gpu

import ra_spmm  # noqa: E402
from ra_spmm import synthetic as S  # noqa: E402

CSR_FAMILY = ("CSR_DIRECT", "CSR_BASELINE", "CUSPARSE", "ZERO_OVERHEAD_CSR")


@pytest.fixture(scope="module")
def c1():
    return S.CONFIGS["C1"]()


@pytest.mark.parametrize("N", [64, 128])
def test_c1_every_path(oracle, c1, N):
    g = c1
    assert g.M == 10_000 and int(np.diff(g.rowptr).max()) <= 64
    B = np.random.default_rng(100 + N).standard_normal((g.K, N)).astype(np.float32)
    seq = oracle.spmm_seq_f32(g.rowptr, g.colind, g.vals, B)
    exact = oracle.spmm_f64(g.rowptr, g.colind, g.vals, B)
    scale = oracle.spmm_f64(g.rowptr, g.colind, np.abs(g.vals), np.abs(B))
    A_cpu = torch.sparse_csr_tensor(torch.from_numpy(g.rowptr).long(), torch.from_numpy(g.colind).long(),
                                    torch.from_numpy(g.vals), (g.M, g.K))
    ts = torch.sparse.mm(A_cpu, torch.from_numpy(B)).numpy()
    print(f"[C1] N={N} torch.sparse CPU == oracle bits: {np.array_equal(ts, seq)}", flush=True)
    assert_close_scaled(ts, exact, scale, 1e-5, "torch.sparse CPU")

    rp, ci, vl = g.torch("cuda")
    Bd = torch.from_numpy(B).cuda()
    qv = oracle.quantize_f16_scaled(g.vals, oracle.tile_value_scale_log2(g.vals))
    cache = {}
    agree = {}
    for name in ra_spmm.DEPLOYED_KERNELS + ["CSR_BASELINE", "CUSPARSE"]:
        print(f"[C1] N={N} {name}", flush=True)
        C = ra_spmm.run_kernel(name, rp, ci, vl, Bd, cache, name).cpu().numpy()
        if name in CSR_FAMILY:
            np.testing.assert_array_equal(C, seq, err_msg=name)
            assert_close_scaled(C, ts.astype(np.float64), scale, 1e-5, f"{name} vs torch.sparse")
            agree[name] = bool(np.array_equal(C, ts))
        elif name.endswith("_TF32"):
            assert_fp32_route(C, g.rowptr, g.colind, qv, B, oracle, name)
        else:
            assert_close_scaled(C, exact, scale, 2.0 ** -10, name)
            assert_close_scaled(C, ts.astype(np.float64), scale, 2.0 ** -10, f"{name} vs torch.sparse")
    print(f"[C1] N={N} bit-equal to torch.sparse CPU: {agree}", flush=True)

    plan = ra_spmm.make_router_plan(rp, ci, vl, g.M, g.K, N)
    label = ra_spmm.route_label(plan)
    C = ra_spmm.run_router_plan(plan, rp, ci, vl, Bd).cpu().numpy()
    print(f"[C1] N={N} routed {label}", flush=True)
    if label in CSR_FAMILY:
        np.testing.assert_array_equal(C, seq, err_msg=f"routed {label}")
    assert_close_scaled(C, ts.astype(np.float64), scale,
                        1e-5 if label not in ra_spmm.TILE_KERNELS or label.endswith("_TF32") else 2.0 ** -10,
                        f"routed {label} vs torch.sparse")
