"""64-bit addressing: M*N and K*N above 2^31 elements.

A is 4,198,400 x 4,198,400 with one or two entries per row plus a few long
rows near the end, and N = 520, so C and B each hold 2.18e9 fp32 elements
(8.7 GB): any 32-bit row*N product in a kernel or a host launch wraps.
Every path runs over the whole matrix; the check reads back sampled rows
(the first, the last, random ones and the long rows) and compares them with
the oracle on the sub-matrix of those rows and the B rows they touch.

Values and B are exactly representable in fp16, so the tile routes compute
exact products; bars:
  CSR_DIRECT, baseline, fp16 guardrail   bit-identical to the oracle's fma chain
  ZERO_OVERHEAD_CSR                      rows <= 256 nnz bit-identical, all within 1e-5 of |A||B|
  tile FP16 and FP32 routes              within 1e-5 of |A||B| of the fp64 value
  bf16 plan on bf16 B (16-bit entry)     within 1e-5 of |A||Bq| of the fp64 value on bf16-rounded B
"""
import numpy as np
import pytest
import torch

from conftest import assert_close_scaled

pytestmark = pytest.mark.gpu

import ra_spmm  # noqa: E402

M = K = (1 << 22) + 4096
N = 520
LONG_ROWS = (M - 1, M - 5, M // 2)


def _matrix():
    rng = np.random.default_rng(77)
    i = np.arange(M, dtype=np.int64)
    a = i
    b = (i * 2654435761) % K
    has_b = rng.random(M) < 0.6
    cols = np.where(has_b[:, None], np.stack([a, b], 1), np.stack([a, a], 1))
    cols = np.sort(cols, axis=1)
    keep = np.ones((M, 2), bool)
    keep[:, 1] = cols[:, 1] != cols[:, 0]
    deg = keep.sum(1)
    lists = {r: np.unique(rng.integers(0, K, 3000 + 37 * j)) for j, r in enumerate(LONG_ROWS)}
    for r, c in lists.items():
        lists[r] = np.unique(np.concatenate([c, [K - 1, K - 2]]))
        deg[r] = len(lists[r])
    rowptr = np.zeros(M + 1, np.int64)
    np.cumsum(deg, out=rowptr[1:])
    colind = np.empty(rowptr[-1], np.int64)
    short = np.ones(M, bool)
    short[list(LONG_ROWS)] = False
    flat = cols[short][keep[short]]
    pos = np.repeat(rowptr[:-1][short], deg[short]) + (np.cumsum(keep[short], 1)[keep[short]] - 1)
    colind[pos] = flat
    for r, c in lists.items():
        colind[rowptr[r]:rowptr[r + 1]] = c
    # k/64 for small k: exact in fp16 and bf16
    vals = (rng.integers(-64, 65, len(colind)) / 64.0).astype(np.float32)
    vals[vals == 0] = 0.5
    return rowptr.astype(np.int32), colind.astype(np.int32), vals


@pytest.fixture(scope="module")
def big():
    if torch.cuda.get_device_properties(0).total_memory < 48 << 30:
        pytest.skip("needs a GPU with >= 48 GiB")
    rowptr, colind, vals = _matrix()
    gen = torch.Generator(device="cuda").manual_seed(5)
    B = torch.randn(K, N, device="cuda", generator=gen).half().float()
    rng = np.random.default_rng(3)
    sample = np.unique(np.concatenate([np.arange(256), np.arange(M - 256, M), rng.integers(0, M, 512),
                                       np.array(LONG_ROWS)]))
    # sub-matrix of the sampled rows over the B rows they touch
    deg = np.diff(rowptr)[sample]
    srp = np.zeros(len(sample) + 1, np.int64)
    np.cumsum(deg, out=srp[1:])
    idx = np.concatenate([np.arange(rowptr[r], rowptr[r + 1]) for r in sample])
    used, sci = np.unique(colind[idx], return_inverse=True)
    Bu = B.index_select(0, torch.from_numpy(used).cuda()).cpu().numpy()
    sub = (srp.astype(np.int32), sci.astype(np.int32), vals[idx], Bu, deg)
    dev = tuple(torch.from_numpy(x).cuda() for x in (rowptr, colind, vals))
    host = tuple(torch.from_numpy(x) for x in (rowptr, colind, vals))
    print(f"[large] M={M} K={K} N={N} nnz={len(colind)} rows checked={len(sample)}", flush=True)
    yield dict(dev=dev, host=host, B=B, sample=sample, sub=sub)


def _rows(C, sample):
    out = C.index_select(0, torch.from_numpy(sample).cuda()).cpu().numpy()
    del C
    torch.cuda.empty_cache()
    return out


def test_csr_family_64bit(oracle, big):
    rp, ci, vl = big["dev"]
    srp, sci, svl, Bu, deg = big["sub"]
    seq = oracle.spmm_seq_f32(srp, sci, svl, Bu)
    for fn in (ra_spmm.spmm_csr_direct, ra_spmm.spmm_csr_baseline, ra_spmm.spmm_cusparse_fp16):
        print(f"[large] {fn.__name__}", flush=True)
        np.testing.assert_array_equal(_rows(fn(rp, ci, vl, big["B"]), big["sample"]), seq, err_msg=fn.__name__)
    print("[large] zero_overhead", flush=True)
    z = ra_spmm.make_zero_overhead_plan(rp, M, K)
    C = _rows(ra_spmm.run_zero_overhead_plan(z, rp, ci, vl, big["B"]), big["sample"])
    np.testing.assert_array_equal(C[deg <= 256], seq[deg <= 256])
    assert_close_scaled(C, oracle.spmm_f64(srp, sci, svl, Bu), oracle.spmm_f64(srp, sci, np.abs(svl), np.abs(Bu)),
                        1e-5, "zo")


def test_bf16_tile_plan_64bit(oracle, big):
    """bf16 values and bf16 B on the 16-bit entry (values k/64 are exact in
    bf16; B is rounded to bf16, and the reference uses the same rounding)."""
    srp, sci, svl, Bu, _ = big["sub"]
    qb = oracle.quantize_bf16(Bu)
    rp, ci, vl = big["host"]
    p = ra_spmm.make_tc_direct_plan(rp, ci, vl, M, K, N, "bf16")
    print("[large] bf16 plan, bf16 B", flush=True)
    C = _rows(ra_spmm.run_tile_plan_route(p, big["B"].bfloat16(), "bf16"), big["sample"])
    assert_close_scaled(C, oracle.spmm_f64(srp, sci, svl, qb), oracle.spmm_f64(srp, sci, np.abs(svl), np.abs(qb)),
                        1e-5, "bf16")


@pytest.mark.parametrize("mk", ["make_tc_direct_plan", "make_community_tc_plan", "make_segment_hybrid_plan"])
def test_tile_routes_64bit(oracle, big, mk):
    srp, sci, svl, Bu, _ = big["sub"]
    exact = oracle.spmm_f64(srp, sci, svl, Bu)
    scale = oracle.spmm_f64(srp, sci, np.abs(svl), np.abs(Bu))
    rp, ci, vl = big["host"]
    print(f"[large] {mk} build", flush=True)
    p = getattr(ra_spmm, mk)(rp, ci, vl, M, K, N)
    for route in ("fp16", "fp32"):
        print(f"[large] {mk} route={route}", flush=True)
        C = _rows(ra_spmm.run_tile_plan_route(p, big["B"], route), big["sample"])
        assert_close_scaled(C, exact, scale, 1e-5, f"{mk} {route}")
