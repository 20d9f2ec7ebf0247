"""The GCN aggregation operator (CPU): build_aggregation_operator (scipy,
gnn_bench/router_vs_baselines_gcn.py:89-126) and the synthetic generator's
gcn_operator agree, and both satisfy the closed form D^-1/2 (A+I) D^-1/2."""
import numpy as np
import scipy.sparse as sp

from ra_spmm import synthetic as S
from ra_spmm.gnn import build_aggregation_operator, operator_descriptors


def test_gcn_operator_closed_form_and_agreement():
    g = S.chung_lu(3000, 6.0, 2.3, 300, seed=9)
    A = sp.csr_matrix((np.ones(g.nnz, np.float32), g.colind, g.rowptr), shape=(g.M, g.M))
    op = build_aggregation_operator(A, "gcn")
    h = S.gcn_operator(g)
    np.testing.assert_array_equal(op.indptr, h.rowptr)
    np.testing.assert_array_equal(op.indices, h.colind)
    np.testing.assert_allclose(op.data, h.vals, rtol=1e-6)
    dense = A.toarray().astype(np.float64) + np.eye(g.M)
    d = dense.sum(1)
    ref = dense / np.sqrt(d)[:, None] / np.sqrt(d)[None, :]
    np.testing.assert_allclose(op.toarray(), ref, rtol=1e-6, atol=1e-9)
    desc = operator_descriptors(op)
    assert desc["M"] == g.M and desc["nnz"] == g.nnz + g.M


def test_sage_and_gin_operators():
    g = S.random_csr(50, 50, 4.0, seed=2, empty_frac=0.1)
    A = sp.csr_matrix((np.abs(g.vals), g.colind, g.rowptr), shape=(50, 50))
    gin = build_aggregation_operator(A, "gin")
    np.testing.assert_allclose(gin.toarray(), A.toarray(), rtol=1e-7)
    sage = build_aggregation_operator(A, "sage").toarray()
    rs = A.toarray().sum(1)
    nz = rs > 0
    np.testing.assert_allclose(sage[nz].sum(1), 1.0, rtol=1e-6)
    assert np.all(sage[~nz] == 0)


def test_cross_entropy_matches_torch():
    import torch
    import torch.nn.functional as F
    from ra_spmm.gnn import cross_entropy
    torch.manual_seed(0)
    logits = torch.randn(1000, 47, requires_grad=True)
    y = torch.randint(0, 47, (1000,))
    a = cross_entropy(logits, y)
    b = F.cross_entropy(logits, y)
    torch.testing.assert_close(a, b, rtol=1e-6, atol=1e-6)
    ga, = torch.autograd.grad(a, logits)
    gb, = torch.autograd.grad(b, logits)
    torch.testing.assert_close(ga, gb, rtol=1e-6, atol=1e-7)


def test_chunked_weight_grad_and_linear(monkeypatch):
    import torch
    from ra_spmm import gnn
    g = torch.randn(1000, 5, dtype=torch.float64)
    x = torch.randn(1000, 3, dtype=torch.float64)
    ref = g.t() @ x
    for rows in (7, 64, 250):  # with and without a remainder; c >= 4 chunks
        torch.testing.assert_close(gnn.weight_grad(g, x, rows), ref)
    torch.testing.assert_close(gnn.weight_grad(g[:20], x[:20], 7), g[:20].t() @ x[:20])  # < 4 chunks: one GEMM
    # Same parameters as nn.Linear(bias=False) from the same seed; gradients
    # of the chunked form equal autograd's through F.linear.
    monkeypatch.setattr(gnn, "WGRAD_ROWS", 16)
    torch.manual_seed(3)
    lin = gnn.Linear(3, 5).double()
    torch.manual_seed(3)
    ref_lin = torch.nn.Linear(3, 5, bias=False).double()
    torch.testing.assert_close(lin.weight, ref_lin.weight)
    xi = x.clone().requires_grad_(True)
    xr = x.clone().requires_grad_(True)
    out = lin(xi)
    assert out.shape == (1000, 8) and bool((out[:, 5:] == 0).all())  # width padded to a multiple of 4
    torch.testing.assert_close(out[:, :5], ref_lin(xr))
    (out[:, :5] ** 2).sum().backward()
    (ref_lin(xr) ** 2).sum().backward()
    torch.testing.assert_close(lin.weight.grad, ref_lin.weight.grad)
    torch.testing.assert_close(xi.grad, xr.grad)


def test_gcn_order_argument():
    import pytest
    from ra_spmm import gnn
    assert gnn.GCN(4, 8, 3).order == "reference"
    assert gnn.GCN(4, 8, 3, order="auto").order == "auto"
    with pytest.raises(ValueError):
        gnn.GCN(4, 8, 3, order="aggregate")


def test_gcn_operator_self_loops_and_duplicates():
    """Closed form on a matrix with an existing self-loop (kept, not doubled),
    a duplicate entry (summed), an empty row and a stored zero diagonal
    (treated as absent)."""
    A = sp.csr_matrix((np.r_[2.0, 1.0, 1.0, 1.0, 1.0, 0.0, 3.0], np.r_[0, 1, 0, 2, 2, 2, 1],
                       np.r_[0, 2, 5, 7, 7]), shape=(4, 4))  # row 1 has (1,2) twice
    dense = A.toarray()
    want = dense.copy()
    for i in range(4):
        if want[i, i] == 0:
            want[i, i] = 1.0
    d = want.sum(1)
    ref = want / np.sqrt(d)[:, None] / np.sqrt(d)[None, :]
    op = build_aggregation_operator(A, "gcn")
    np.testing.assert_allclose(op.toarray(), ref, rtol=1e-6)
    assert op.has_sorted_indices and op.dtype == np.float32
    sage = build_aggregation_operator(A, "sage").toarray()
    rs = dense.sum(1)
    np.testing.assert_allclose(sage[rs > 0], (dense / np.where(rs > 0, rs, 1)[:, None])[rs > 0], rtol=1e-6)

    # Stored zeros are dropped from the products (sparse D^-1 A keeps none):
    # the structure is exactly the nonzero pattern of the dense result.
    sage_csr = build_aggregation_operator(A, "sage")
    assert sage_csr.nnz == int(np.count_nonzero(sage)) == 5
    assert op.nnz == int(np.count_nonzero(op.toarray()))
    gin = build_aggregation_operator(A, "gin")
    assert gin.nnz == 6  # duplicates summed, the stored zero kept
