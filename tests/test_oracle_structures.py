"""Host plan builders of the product against the oracle restatements.

ZERO_OVERHEAD_CSR binning (csr/ra_zero_overhead.cu:331-358) and the tile
format of the three tile families (tc/ra_tc_direct.cu:654-706,
tc/ra_community_tc.cu:335-403, tc/ra_segment_hybrid.cu:470-498) are compared
array by array; the oracle tile format itself is pinned by decode == CSR and
its counting invariants; fp16/bf16 value rounding is checked against numpy.
"""
import ctypes

import numpy as np
import pytest

import torch  # noqa: F401
from ra_spmm import capi
from ra_spmm import synthetic as S


def zo_bins_capi(rowptr, M, K):
    lib = capi.load()
    info = capi.ZOInfo()
    capi.check(lib.ra_zo_bins_host(capi.ptr(rowptr), M, K, None, None, None, None, ctypes.byref(info)))
    small = np.zeros(max(1, info.num_small), np.int32)
    crow = np.zeros(max(1, info.num_chunks), np.int32)
    cst = np.zeros(max(1, info.num_chunks), np.int32)
    emp = np.zeros(max(1, info.num_empty), np.int32)
    capi.check(lib.ra_zo_bins_host(capi.ptr(rowptr), M, K, capi.ptr(small), capi.ptr(crow),
                                   capi.ptr(cst), capi.ptr(emp), ctypes.byref(info)))
    return info, small[:info.num_small], crow[:info.num_chunks], cst[:info.num_chunks], emp[:info.num_empty]


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_zo_bins_match_oracle(oracle, seed):
    g = S.random_csr(4000, 5000, 12.0, seed=seed, skew=0.9, empty_frac=0.05, max_deg=2000)
    info, small, crow, cst, emp = zo_bins_capi(g.rowptr, g.M, g.K)
    o = oracle.zo_bins(g.rowptr)
    np.testing.assert_array_equal(small, o["small_rows"])
    np.testing.assert_array_equal(crow.view(np.uint32).astype(np.int64), o["chunk_rows"])
    np.testing.assert_array_equal(cst, o["chunk_starts"])
    assert (info.num_tiny, info.num_short, info.num_medium, info.num_long, info.num_empty,
            info.max_long_chunks) == (o["num_tiny"], o["num_short"], o["num_medium"],
                                      o["num_long"], o["num_empty"], o["max_long_chunks"])
    # Brute-force invariants: every nonzero is covered exactly once.
    deg = np.diff(g.rowptr)
    covered = np.zeros(g.nnz, np.int32)
    for r in small:
        covered[g.rowptr[r]:g.rowptr[r + 1]] += 1
    for t, s in zip(crow.view(np.uint32), cst):
        row = int(t & 0x7FFFFFFF)
        covered[s:min(s + 256, g.rowptr[row + 1])] += 1
        assert bool(t & 0x80000000) == (deg[row] <= 256)
    assert np.all(covered == 1)
    assert set(emp.tolist()) == set(np.flatnonzero(deg == 0).tolist())


def tile_host(kind, g, N=64, value_dtype=capi.DTYPE_F16):
    lib = capi.load()
    h = ctypes.c_void_p()
    capi.check(lib.ra_tile_host_build(kind, capi.ptr(g.rowptr), capi.ptr(g.colind), capi.ptr(g.vals),
                                      g.M, g.K, N, value_dtype, ctypes.byref(h)))
    info = capi.TileInfo()
    capi.check(lib.ra_tile_host_get_info(h, ctypes.byref(info)))
    out = {}
    for name in ("block_offsets", "atox", "win_rows", "vals", "seg_window", "seg_bbegin",
                 "seg_bend", "seg_slot", "split_windows", "split_offsets"):
        n = ctypes.c_int64()
        capi.check(lib.ra_tile_host_export(h, name.encode(), None, ctypes.byref(n)))
        arr = np.zeros(n.value, np.uint16 if name == "vals" else np.int32)
        if n.value:
            capi.check(lib.ra_tile_host_export(h, name.encode(), capi.ptr(arr), ctypes.byref(n)))
        out[name] = arr
    lib.ra_tile_host_destroy(h)
    return info, out


def _graphs():
    yield S.random_csr(203, 180, 6.0, seed=1, skew=1.2, empty_frac=0.1)
    yield S.random_csr(64, 400, 90.0, seed=2)          # windows with > 64 blocks
    yield S.sbm(8, 40, 10.0, 0.9, seed=5)               # community structure
    yield S.random_csr(9, 9, 0.0, seed=3)               # empty matrix


@pytest.mark.parametrize("kind", [0, 1, 2])
def test_tile_format_matches_oracle(oracle, kind):
    for g in _graphs():
        info, h = tile_host(kind, g)
        o = oracle.tile_format(kind, g.rowptr, g.colind, g.vals, g.M)
        W = (g.M + 7) // 8
        assert info.active == 1 and info.num_windows == W
        np.testing.assert_array_equal(h["win_rows"], o["win_rows"])
        np.testing.assert_array_equal(h["block_offsets"], o["block_offsets"])
        real = h["atox"] >= 0
        np.testing.assert_array_equal(h["atox"][real], o["atox"][real])
        assert np.all(o["atox"][~real] == 0)  # reference pads with column 0
        assert info.num_blocks == o["block_offsets"][-1]
        assert info.num_vectors == int(real.sum())
        sc = oracle.tile_value_scale_log2(g.vals)
        assert info.value_scale_log2 == sc
        vals = h["vals"].view(np.float16).astype(np.float32).reshape(-1, 8, 8) * np.float32(2.0 ** -sc)
        np.testing.assert_array_equal(vals, oracle.quantize_f16_scaled(o["blocks"], sc))
        if kind == 2:
            for key in ("seg_bbegin", "seg_bend", "seg_slot", "split_windows", "split_offsets"):
                np.testing.assert_array_equal(h[key], o[key], err_msg=key)
            np.testing.assert_array_equal(h["seg_window"].view(np.uint32), o["seg_window"])


def test_oracle_tile_format_invariants(oracle):
    for kind in (0, 1, 2):
        for g in _graphs():
            o = oracle.tile_format(kind, g.rowptr, g.colind, g.vals, g.M)
            dense = np.zeros((g.M, g.K))
            for r in range(g.M):
                for p in range(g.rowptr[r], g.rowptr[r + 1]):
                    dense[r, g.colind[p]] += g.vals[p]
            np.testing.assert_allclose(oracle.tile_decode(o, g.M, g.K), dense, rtol=1e-6)
            bo = o["block_offsets"]
            for w in range(len(bo) - 1):
                rows = [int(r) for r in o["win_rows"][w * 8:(w + 1) * 8] if r >= 0]
                cols = set()
                for r in rows:
                    cols.update(g.colind[g.rowptr[r]:g.rowptr[r + 1]].tolist())
                assert bo[w + 1] - bo[w] == (len(cols) + 7) // 8
            if kind == 1:
                lead = [g.colind[g.rowptr[r]] if g.rowptr[r] < g.rowptr[r + 1] else 2**31 - 1
                        for r in range(g.M)]
                order = o["win_rows"][:g.M]
                keys = [(lead[r], r) for r in order]
                assert keys == sorted(keys)
            if kind == 2:
                nseg = sum(((bo[w + 1] - bo[w]) + 63) // 64 if bo[w + 1] - bo[w] > 64 else 1
                           for w in range(len(bo) - 1))
                assert len(o["seg_window"]) == nseg


def test_value_rounding_matches_numpy(oracle):
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(3000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 3000),
                        np.array([65504, 65519.99, 65520, 2**-24, 2**-25, 1.5 * 2**-25, 2**-14,
                                  2**-14 * (1 - 2**-11), -0.0, 0.0], np.float32)]).astype(np.float32)
    x = x[np.abs(x) < 1e30]
    M = len(x)
    g = S.Graph(np.arange(M + 1, dtype=np.int32), np.zeros(M, np.int32), x, M, 1)
    # bf16 plans are never scaled: the raw RNE conversion over the full range.
    _, h = tile_host(0, g, value_dtype=capi.DTYPE_BF16)
    blocks = h["vals"].reshape(-1, 8, 8)[:, :, 0].reshape(-1)[:M]
    got = (blocks.astype(np.uint32) << 16).view(np.float32)
    np.testing.assert_array_equal(got, oracle.quantize_bf16(x))
    # fp16 plans scale max|v| into [2^13, 2^14); with max|v| = 10000 the scale
    # is 2^0, so the raw RNE conversion is pinned on everything below it,
    # including the fp16 subnormal range.  (Values near the fp16 maximum are
    # unreachable through a plan by construction.)
    x0 = np.clip(x, -9000.0, 9000.0).astype(np.float32)
    x0[0] = 10000.0
    g0 = S.Graph(np.arange(M + 1, dtype=np.int32), np.zeros(M, np.int32), x0, M, 1)
    info, h = tile_host(0, g0, value_dtype=capi.DTYPE_F16)
    assert info.value_scale_log2 == 0
    blocks = h["vals"].reshape(-1, 8, 8)[:, :, 0].reshape(-1)[:M]
    np.testing.assert_array_equal(blocks.view(np.float16).astype(np.float32), oracle.quantize_f16(x0))


def test_value_scale_closed_form(oracle):
    """max|v| = 2^e maps to s = 13 - e; GCN-like tiny values keep fp16 precision."""
    for e in (-20, -5, 0, 3, 13, 14, 30):
        v = np.array([2.0 ** e, -(2.0 ** (e - 3))], np.float32)
        g = S.Graph(np.array([0, 2], np.int32), np.array([0, 1], np.int32), v, 1, 2)
        info, h = tile_host(0, g)
        assert info.value_scale_log2 == oracle.tile_value_scale_log2(v) == max(-24, min(24, 13 - e))
    tiny = np.array([3.3e-5, 1.0 / 3.0, 2.5e-6], np.float32)
    sc = oracle.tile_value_scale_log2(tiny)
    rel = np.abs(oracle.quantize_f16_scaled(tiny, sc) - tiny) / tiny
    assert np.all(rel <= 2.0 ** -11)


def test_inactive_below_n16():
    g = S.random_csr(20, 20, 3.0, seed=0)
    info, _ = tile_host(0, g, N=8)
    assert info.active == 0


@pytest.mark.parametrize("kind,limit", [(0, 512), (1, 512), (2, 64)])
def test_segments_cover_windows(kind, limit):
    """Every kind is scheduled as segments: each window's block range is cut
    into consecutive pieces of at most `limit` blocks (64 for SEGMENT_HYBRID as
    in tc/ra_segment_hybrid.cu:470-498; 512 for the other two), sole windows
    flagged in bit 31, partial slots numbered in ascending order."""
    g = S.random_csr(40, 40000, 2500.0, seed=8)
    info, h = tile_host(kind, g)
    bo = h["block_offsets"]
    segw = h["seg_window"].view(np.uint32)
    covered = {}
    for w_tag, b0, b1, slot in zip(segw, h["seg_bbegin"], h["seg_bend"], h["seg_slot"]):
        w = int(w_tag & 0x7FFFFFFF)
        assert 0 < b1 - b0 <= limit or bo[w + 1] == bo[w]
        assert bool(w_tag & 0x80000000) == (bo[w + 1] - bo[w] <= limit)
        covered.setdefault(w, []).append((int(b0), int(b1)))
    for w, pieces in covered.items():
        pieces.sort()
        assert pieces[0][0] == bo[w] and pieces[-1][1] == bo[w + 1]
        assert all(a[1] == b[0] for a, b in zip(pieces, pieces[1:]))
    assert info.num_split_windows == len(h["split_windows"]) > 0
    assert h["split_offsets"][-1] == info.num_split_segs


def test_merge_duplicates_matches_dense_accumulation(oracle):
    rng = np.random.default_rng(5)
    M, K = 40, 12
    deg = rng.integers(0, 9, M)
    rp = np.concatenate([[0], np.cumsum(deg)]).astype(np.int32)
    ci = rng.integers(0, K, rp[-1]).astype(np.int32)
    vl = rng.standard_normal(rp[-1]).astype(np.float32)
    mrp, mci, mvl = oracle.merge_duplicates(rp, ci, vl)
    dense = np.zeros((M, K), np.float64)
    np.add.at(dense, (np.repeat(np.arange(M), deg), ci), vl.astype(np.float64))
    got = np.zeros((M, K), np.float64)
    np.add.at(got, (np.repeat(np.arange(M), np.diff(mrp)), mci), mvl.astype(np.float64))
    np.testing.assert_allclose(got, dense, rtol=1e-6, atol=1e-6)
    for r in range(M):                      # distinct columns per row, first-occurrence order
        row = mci[mrp[r]:mrp[r + 1]]
        assert len(set(row.tolist())) == len(row)
        first = list(dict.fromkeys(ci[rp[r]:rp[r + 1]].tolist()))
        assert row.tolist() == first
    # fp32 accumulation in CSR order: three equal entries of 1 + 2^-24 sum exactly as float32 does
    v = np.float32(1 + 2 ** -23)
    _, _, s = oracle.merge_duplicates(np.array([0, 3]), np.array([0, 0, 0]), np.array([v, v, v], np.float32))
    assert s[0] == np.float32(np.float32(np.float32(v + v)) + v)
