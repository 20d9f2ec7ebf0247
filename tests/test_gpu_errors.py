"""Argument checks of the `ra_spmm` boundary raise RuntimeError before any
launch, as the reference's TORCH_CHECKs do (bindings/ra_bindings.cpp:288-306
check_csr_tensors: device-resident, contiguous, int32/int32/fp32; run
functions check device and contiguity; an unknown name is a TORCH_CHECK
failure, :1881)."""
import pytest
import torch

pytestmark = pytest.mark.gpu

import ra_spmm  # noqa: E402
from ra_spmm import synthetic as S  # noqa: E402


@pytest.fixture(scope="module")
def case():
    g = S.random_csr(300, 200, 6.0, seed=4)
    rp, ci, vl = g.torch("cuda")
    B = torch.randn(g.K, 32, device="cuda")
    host = (rp.cpu(), ci.cpu(), vl.cpu())
    z = ra_spmm.make_zero_overhead_plan(host[0], g.M, g.K)
    t = ra_spmm.make_tc_direct_plan(*host, g.M, g.K, 32)
    return dict(g=g, rp=rp, ci=ci, vl=vl, B=B, host=host, z=z, t=t)


CASES = {
    "B on the host": (lambda c: ra_spmm.spmm_csr_direct(c["rp"], c["ci"], c["vl"], c["B"].cpu()), "CUDA"),
    "B not contiguous": (lambda c: ra_spmm.spmm_csr_direct(c["rp"], c["ci"], c["vl"],
                                                           torch.randn(32, c["g"].K, device="cuda").t()),
                         "contiguous"),
    "B float64": (lambda c: ra_spmm.spmm_csr_direct(c["rp"], c["ci"], c["vl"], c["B"].double()), "float32"),
    "B 1-D": (lambda c: ra_spmm.spmm_csr_direct(c["rp"], c["ci"], c["vl"], c["B"][:, 0].contiguous()), "2-D"),
    "colind int64": (lambda c: ra_spmm.spmm_csr_direct(c["rp"], c["ci"].long(), c["vl"], c["B"]), "int32"),
    "vals float16": (lambda c: ra_spmm.spmm_csr_direct(c["rp"], c["ci"], c["vl"].half(), c["B"]), "float32"),
    "rowptr on the host": (lambda c: ra_spmm.spmm_csr_baseline(c["rp"].cpu(), c["ci"], c["vl"], c["B"]), "CUDA"),
    "ZO plan, rowptr of another M": (lambda c: ra_spmm.run_zero_overhead_plan(
        c["z"], c["rp"][:100].contiguous(), c["ci"], c["vl"], c["B"]), "M"),
    "ZO plan, B too short": (lambda c: ra_spmm.run_zero_overhead_plan(
        c["z"], c["rp"], c["ci"], c["vl"], c["B"][:10]), "rows"),
    "tile plan, B too short": (lambda c: ra_spmm.run_tc_direct_plan(c["t"], c["B"][:10]), "rows"),
    "tile plan, unknown route": (lambda c: ra_spmm.run_tile_plan_route(c["t"], c["B"], "fp8"), "route"),
    "tile plan, fp16 B with N % 8 != 0": (lambda c: ra_spmm.run_tile_plan_route(
        c["t"], torch.randn(c["g"].K, 20, device="cuda").half(), "fp16"), "N % 8"),
    "tile plan, unknown value dtype": (lambda c: ra_spmm.make_tc_direct_plan(
        *c["host"], c["g"].M, c["g"].K, 32, "fp8"), "value_dtype"),
    "tile plan, unknown build": (lambda c: ra_spmm.make_tc_direct_plan(
        *c["host"], c["g"].M, c["g"].K, 32, "fp16", "cpu"), "build"),
    "plan builder, rowptr shorter than M+1": (lambda c: ra_spmm.make_zero_overhead_plan(
        c["host"][0][:50], c["g"].M, c["g"].K), "M\\+1"),
    "router, unknown table": (lambda c: ra_spmm.make_router_plan(
        c["rp"], c["ci"], c["vl"], c["g"].M, c["g"].K, 32, "MAIN", "h100"), "table"),
}


@pytest.mark.parametrize("name", list(CASES))
def test_bad_arguments_raise(case, name):
    fn, match = CASES[name]
    print(f"[errors] {name}", flush=True)
    with pytest.raises(RuntimeError, match=match):
        fn(case)
    torch.cuda.synchronize()  # nothing was launched that could fail later


def test_calls_after_errors_still_work(case, oracle):
    """An argument error leaves no sticky state: the next valid call is exact."""
    for fn, _ in CASES.values():
        with pytest.raises(RuntimeError):
            fn(case)
    g = case["g"]
    C = ra_spmm.spmm_csr_direct(case["rp"], case["ci"], case["vl"], case["B"])
    ref = oracle.spmm_seq_f32(g.rowptr, g.colind, g.vals, case["B"].cpu().numpy())
    assert (C.cpu().numpy() == ref).all()
