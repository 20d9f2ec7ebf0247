"""Stream semantics: every launch of every path goes on the caller's current
torch stream (the binding passes it down to the C ABI), so work queued before
it on that stream is seen, and plans on different streams run independently.

A non-default stream is made busy (a bounded spin kernel), then B is doubled
on that stream and the SpMM is queued behind it with no synchronisation: a
launch on any other stream would read B before the doubling.  Doubling is
exact, so every path must return exactly twice its own eager result.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

import ra_spmm  # noqa: E402
from ra_spmm import synthetic as S  # noqa: E402

LABELS = ["CSR_BASELINE"] + ra_spmm.DEPLOYED_KERNELS
SPIN = 20_000_000  # cycles of torch.cuda._sleep: a few ms


def _setup(seed=21, M=3000, N=64):
    g = S.random_csr(M, M, 12.0, seed=seed, skew=1.2)
    rp, ci, vl = g.torch("cuda")
    host = (rp.cpu(), ci.cpu(), vl.cpu())
    B = torch.randn(g.K, N, device="cuda", generator=torch.Generator(device="cuda").manual_seed(seed))
    # no magnitudes near the fp16 subnormal range, where rounding 2x and x differ
    B = torch.where(B.abs() < 1e-3, torch.full_like(B, 1e-3), B)
    return g, rp, ci, vl, host, B


@pytest.mark.parametrize("label", LABELS + ["FP16_GUARDRAIL"])
def test_launch_follows_the_current_stream(label):
    g, rp, ci, vl, host, B = _setup()
    if label == "FP16_GUARDRAIL":
        run = lambda X: ra_spmm.spmm_cusparse_fp16(rp, ci, vl, X)  # noqa: E731
    else:
        plan = ra_spmm.build_kernel_plan(label, *host, g.M, g.K, B.shape[1])
        run = lambda X: ra_spmm.run_planned_kernel(label, plan, rp, ci, vl, X)  # noqa: E731
    ref = run(B)  # eager, default stream; also sizes scratch and derives lazy state
    torch.cuda.synchronize()
    print(f"[streams] {label}", flush=True)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        B2 = B.clone()
        torch.cuda._sleep(SPIN)
        B2.mul_(2.0)
        C = run(B2)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(C.cpu().numpy(), 2.0 * ref.cpu().numpy(), err_msg=label)


def test_two_plans_on_two_streams():
    g1, rp1, ci1, vl1, host1, B1 = _setup(seed=31)
    g2, rp2, ci2, vl2, host2, B2 = _setup(seed=32, M=2500, N=128)
    z = ra_spmm.build_kernel_plan("ZERO_OVERHEAD_CSR", *host1, g1.M, g1.K, B1.shape[1])
    t = ra_spmm.build_kernel_plan("COMMUNITY_TC", *host2, g2.M, g2.K, B2.shape[1])
    run1 = lambda: ra_spmm.run_planned_kernel("ZERO_OVERHEAD_CSR", z, rp1, ci1, vl1, B1)  # noqa: E731
    run2 = lambda: ra_spmm.run_planned_kernel("COMMUNITY_TC", t, rp2, ci2, vl2, B2)  # noqa: E731
    ref1, ref2 = run1(), run2()
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    for s in (s1, s2):
        s.wait_stream(torch.cuda.current_stream())
    outs1, outs2 = [], []
    for _ in range(5):
        with torch.cuda.stream(s1):
            outs1.append(run1())
        with torch.cuda.stream(s2):
            outs2.append(run2())
    for s in (s1, s2):
        torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for c in outs1:
        assert torch.equal(c, ref1)
    for c in outs2:
        assert torch.equal(c, ref2)
