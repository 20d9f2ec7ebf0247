"""Pins of the oracle's SpMM arithmetic (CPU only).

oracle.spmm_seq_f32 restates the reference per-element fma chain
(csr/csr_direct.cu:201-228).  It is pinned here by (a) a pure-Python loop on
tiny inputs, (b) scipy's sparse product within the fp32 error bound, (c) the
closed forms B = ones (row sums) and B = unit columns (columns of A), and (d)
empty rows -> zero rows.
"""
import numpy as np
import scipy.sparse as sp

from ra_spmm import synthetic as S


def test_seq_f32_matches_python_loop(oracle):
    g = S.random_csr(7, 9, 3.0, seed=11)
    rng = np.random.default_rng(0)
    B = rng.standard_normal((9, 5)).astype(np.float32)
    got = oracle.spmm_seq_f32(g.rowptr, g.colind, g.vals, B)
    ref = oracle.spmm_python(g.rowptr, g.colind, g.vals, B)
    # fp64 product + fp64 add then one rounding equals fmaf when the sum is exact
    # in fp64, which holds here except in rare cancellations: allow 1 ulp.
    np.testing.assert_array_max_ulp(got, ref, maxulp=1)


def test_f64_matches_scipy(oracle):
    g = S.random_csr(200, 150, 6.0, seed=3, skew=1.5)
    B = np.random.default_rng(1).standard_normal((150, 33)).astype(np.float32)
    got = oracle.spmm_f64(g.rowptr, g.colind, g.vals, B)
    A = sp.csr_matrix((g.vals.astype(np.float64), g.colind, g.rowptr), shape=(200, 150))
    np.testing.assert_allclose(got, A @ B.astype(np.float64), rtol=1e-12, atol=1e-12)


def test_seq_f32_within_fp32_bound(oracle):
    g = S.random_csr(300, 300, 20.0, seed=5, skew=1.2)
    B = np.random.default_rng(2).standard_normal((300, 16)).astype(np.float32)
    c32 = oracle.spmm_seq_f32(g.rowptr, g.colind, g.vals, B)
    c64 = oracle.spmm_f64(g.rowptr, g.colind, g.vals, B)
    scale = oracle.spmm_f64(g.rowptr, g.colind, np.abs(g.vals), np.abs(B))
    deg = np.diff(g.rowptr)[:, None]
    assert np.all(np.abs(c32 - c64) <= deg * 2.0 ** -24 * scale + 1e-30)


def test_closed_forms(oracle):
    g = S.random_csr(50, 40, 5.0, seed=7, empty_frac=0.2)
    ones = np.ones((40, 3), dtype=np.float32)
    c = oracle.spmm_f64(g.rowptr, g.colind, g.vals, ones)
    rowsum = np.add.reduceat(np.append(g.vals.astype(np.float64), 0.0), g.rowptr[:-1])
    rowsum[np.diff(g.rowptr) == 0] = 0.0
    np.testing.assert_allclose(c[:, 0], rowsum, rtol=1e-12)
    E = np.eye(40, dtype=np.float32)[:, [3, 17]]
    c = oracle.spmm_seq_f32(g.rowptr, g.colind, g.vals, E)
    dense = np.zeros((50, 40), dtype=np.float32)
    for r in range(50):
        dense[r, g.colind[g.rowptr[r]:g.rowptr[r + 1]]] = g.vals[g.rowptr[r]:g.rowptr[r + 1]]
    np.testing.assert_array_equal(c, dense[:, [3, 17]])
    empty = np.diff(g.rowptr) == 0
    assert empty.any() and np.all(c[empty] == 0)


def test_quantizers(oracle):
    x = np.array([1.0, 1 + 2**-11, 1 + 3 * 2**-11, 65504, 65520, 1e-8, -2.5, 3.0e38], np.float32)
    with np.errstate(over="ignore"):
        np.testing.assert_array_equal(oracle.quantize_f16(x), x.astype(np.float16).astype(np.float32))
    # bf16 RNE: ties to even on the 16-bit boundary
    y = np.array([1 + 2**-8, 1 + 3 * 2**-8, 1 + 2**-9], np.float32)
    np.testing.assert_array_equal(oracle.quantize_bf16(y), np.array([1.0, 1 + 2**-6, 1.0], np.float32))
    # tf32 rna: ties away from zero at the 10-bit boundary
    z = np.array([1 + 2**-11, -(1 + 2**-11), 1 + 2**-12], np.float32)
    np.testing.assert_array_equal(oracle.quantize_tf32_rna(z),
                                  np.array([1 + 2**-10, -(1 + 2**-10), 1.0], np.float32))


def test_seq_f32_equals_torch_sparse_cpu_on_c1(oracle):
    """Config C1's stated bit-level reference is torch.sparse CPU SpMM.  On
    this host it equals the oracle's sequential fma chain bit for bit."""
    import torch
    g = S.CONFIGS["C1"]()
    for N in (64, 128):
        B = np.random.default_rng(N).standard_normal((g.K, N)).astype(np.float32)
        A = torch.sparse_csr_tensor(torch.from_numpy(g.rowptr).long(), torch.from_numpy(g.colind).long(),
                                    torch.from_numpy(g.vals), (g.M, g.K))
        ts = torch.sparse.mm(A, torch.from_numpy(B)).numpy()
        np.testing.assert_array_equal(oracle.spmm_seq_f32(g.rowptr, g.colind, g.vals, B), ts)
