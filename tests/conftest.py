"""Shared pytest setup: import paths, the `gpu` marker, small helpers."""
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT / "ra-spmm_amd", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct GPU (MI355X)")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O
    O.build()
    return O


def abs_bound(rowptr, colind, vals, B, oracle):
    """|A| @ |B| in fp64: the scale every fp32 summation error is measured against."""
    return oracle.spmm_f64(rowptr, colind, np.abs(vals), np.abs(B))


def assert_close_scaled(C, C64, scale, rel, what=""):
    """Elementwise |C - C64| <= rel * (|A||B|) + 1e-30 (no cancellation blow-up)."""
    err = np.abs(np.asarray(C, dtype=np.float64) - C64)
    bound = rel * scale + 1e-30
    bad = err > bound
    if bad.any():
        i = np.argwhere(bad)[0]
        raise AssertionError(
            f"{what}: {int(bad.sum())} elements beyond rel={rel}; first at {tuple(i)}: "
            f"got {C[tuple(i)]!r}, exact {C64[tuple(i)]!r}, bound {bound[tuple(i)]!r}")


def assert_fp32_route(C32, rowptr, colind, vals, B, oracle, what="fp32 route"):
    """The tile plans' FP32 route (the `_tf32` entry points) against the oracle.

    rowptr/colind/vals is the CSR a plan stores: duplicates merged, values
    rounded and scaled back (oracle.merge_duplicates, quantize_f16_scaled).
    The route drops stored zeros and runs CSR_DIRECT, one fp32 fma chain per
    element in ascending column order: bit-identical to oracle.spmm_seq_f32.
    When the row lengths are skewed (population CV >= 1.5) it runs
    ZERO_OVERHEAD_CSR: rows of <= 256 stored nonzeros stay bit-identical, longer
    rows are held to 1e-5 of |A||B|."""
    rowptr = np.asarray(rowptr, np.int64)
    colind, vals = np.asarray(colind), np.asarray(vals)
    rows = np.repeat(np.arange(rowptr.size - 1), np.diff(rowptr))
    order = np.lexsort((colind, rows))  # ascending columns within each row
    colind, vals = colind[order], vals[order]
    keep = vals != 0
    deg = np.add.reduceat(np.append(keep.astype(np.int64), 0), rowptr[:-1]) * (np.diff(rowptr) > 0)
    seq = oracle.spmm_seq_f32(rowptr.astype(np.int32), colind, vals, B)
    cv = deg.std() / deg.mean() if deg.size and deg.mean() > 0 else 0.0
    if cv < 1.5:
        np.testing.assert_array_equal(C32, seq, err_msg=what)
        return
    short = deg <= 256
    np.testing.assert_array_equal(np.asarray(C32)[short], seq[short], err_msg=what)
    assert_close_scaled(C32, oracle.spmm_f64(rowptr.astype(np.int32), colind, vals, B),
                        oracle.spmm_f64(rowptr.astype(np.int32), colind, np.abs(vals), np.abs(B)), 1e-5, what)
