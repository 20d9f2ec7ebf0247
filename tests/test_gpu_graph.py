"""Graph capture: every routed path, run once eagerly (plan scratch is sized
then), captured into a HIP graph through torch.cuda.graph, and replayed several
times with eager work and synchronisations in between.  Each replay must equal
the eager result bit for bit (the kernels are deterministic and no path records
a memset into the graph)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

import ra_spmm  # noqa: E402
from ra_spmm import synthetic as S  # noqa: E402

CASES = [("CSR_DIRECT", 64), ("CSR_DIRECT", 256),  # 256: XCD-dealt column slices (small matrix)
         ("ZERO_OVERHEAD_CSR", 128), ("ZERO_OVERHEAD_CSR", 512), ("TC_DIRECT", 128), ("COMMUNITY_TC", 96),
         ("SEGMENT_HYBRID", 64), ("TC_DIRECT_TF32", 64), ("SEGMENT_HYBRID_TF32", 48)]


@pytest.mark.parametrize("label,N", CASES)
def test_capture_and_replay(label, N):
    print(f"[graph] {label} N={N}", flush=True)
    g = S.random_csr(3000, 2500, 14.0, seed=7, skew=0.9, max_deg=1500)  # hub rows: chunks and splits
    rp, ci, vl = g.torch("cuda")
    plan = ra_spmm.build_kernel_plan(label, rp.cpu(), ci.cpu(), vl.cpu(), g.M, g.K, N)
    B = torch.randn(g.K, N, device="cuda")
    run = lambda: ra_spmm.run_planned_kernel(label, plan, rp, ci, vl, B)  # noqa: E731
    eager = run()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run()  # warm on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = run()
    for i in range(3):
        junk = torch.randn(1000, 1000, device="cuda") @ torch.randn(1000, 1000, device="cuda")
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), (label, i)
        del junk
