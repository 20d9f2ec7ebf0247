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
