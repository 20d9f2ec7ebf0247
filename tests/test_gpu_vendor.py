"""The measurement helpers bench.py relies on: the rocSPARSE comparator
(ra_spmm.vendor, every CSR algorithm) against the oracle, the gather probe
(ra_spmm.measure) against torch, and the device sort of the synthetic
generators against the host sort."""
import numpy as np
import pytest
import torch

from conftest import assert_close_scaled

pytestmark = pytest.mark.gpu

from ra_spmm import synthetic as S  # noqa: E402
from ra_spmm import vendor  # noqa: E402


@pytest.mark.parametrize("alg", list(vendor.ALGS))
def test_rocsparse_comparator_matches_oracle(oracle, alg):
    g = S.random_csr(3000, 2500, 12.0, seed=7, skew=1.1, empty_frac=0.02)
    N = 128
    B = np.random.default_rng(3).standard_normal((g.K, N)).astype(np.float32)
    rp, ci, vl = g.torch("cuda")
    Bd = torch.from_numpy(B).cuda()
    C = torch.full((g.M, N), float("nan"), device="cuda")
    v = vendor.RocsparseSpMM(rp, ci, vl, Bd, C, alg)
    v.run()
    torch.cuda.synchronize()
    assert_close_scaled(C.cpu().numpy(), oracle.spmm_f64(g.rowptr, g.colind, g.vals, B),
                        oracle.spmm_f64(g.rowptr, g.colind, np.abs(g.vals), np.abs(B)), 1e-5, alg)
    v.close()


def test_device_sort_generates_the_same_graphs():
    try:
        for make in (lambda: S.chung_lu(20_000, 9.0, 2.2, 2000, seed=3),
                     lambda: S.lognormal_social(5000, 60.0, 1.0, 1, 900, seed=4),
                     lambda: S.sbm(16, 100, 10.0, 0.9, seed=2)):
            S.use_device_sort(None)
            a = make()
            S.use_device_sort("cuda")
            b = make()
            np.testing.assert_array_equal(a.rowptr, b.rowptr)
            np.testing.assert_array_equal(a.colind, b.colind)
            np.testing.assert_array_equal(a.vals, b.vals)
    finally:
        S.use_device_sort(None)


@pytest.mark.parametrize("N,span", [(128, 32), (256, 256), (16, 32)])
def test_gather_probe_reads_every_indexed_row(N, span):
    """The gather probe's lanes add up exactly the B rows the index stream
    names: the column sums of its output equal those of B[idx]."""
    from ra_spmm import measure
    gen = torch.Generator(device="cuda").manual_seed(N)
    B = torch.randn(5000, N, device="cuda", generator=gen)
    idx = torch.randint(0, 5000, (77_777,), device="cuda", dtype=torch.int32, generator=gen)
    p = measure.GatherProbe(B, idx, span)
    out = p.run().view(-1, 4)
    torch.cuda.synchronize()
    packets = N // 4
    lanes = out.shape[0]
    # lane l of a wave covers packet l % packets of its group's rows
    per_packet = out.view(lanes // packets, packets, 4).sum(0).reshape(-1)
    want = B[idx.long()].double().sum(0)
    torch.testing.assert_close(per_packet.double(), want, rtol=1e-4, atol=1e-2)
