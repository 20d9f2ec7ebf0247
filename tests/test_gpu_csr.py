"""GPU parity of the CSR family (CSR_DIRECT, baseline, ZERO_OVERHEAD_CSR)
against the oracle (the feature pass: test_gpu_features.py).

Bar: CSR_DIRECT, the baseline kernel and the rows of ZERO_OVERHEAD_CSR with
<= 256 nnz (the short-row bins and the sole chunks) are bit-identical to
oracle.spmm_seq_f32 (same fma chain per element).  Rows longer than 256 nnz
are split into 256-nnz chunks whose parts are summed in a fixed order: within
1e-5 of |A||B| (elementwise) of the fp64 value, and bit-identical from run to
run.
"""
import numpy as np
import pytest
import torch

from conftest import assert_close_scaled

pytestmark = pytest.mark.gpu

import ra_spmm  # noqa: E402
from ra_spmm import synthetic as S  # noqa: E402
from ra_spmm import capi  # noqa: E402


def _dev(g):
    return g.torch("cuda")


def _B(K, N, seed):
    return np.random.default_rng(seed).standard_normal((K, N)).astype(np.float32)


CASES = [
    # (M, K, avg_deg, skew, empty_frac, N)
    (257, 300, 5.0, 0.0, 0.1, 16),
    (1000, 800, 9.0, 1.3, 0.05, 32),
    (1000, 1000, 12.0, 1.1, 0.0, 47),     # ragged N: scalar packets
    (1003, 900, 11.0, 1.2, 0.02, 48),     # 12 float4 packets in 16-lane groups
    (999, 700, 7.0, 0.8, 0.05, 36),       # 9 packets
    (1001, 800, 9.0, 1.0, 0.0, 44),       # 11 packets
    (2048, 1500, 20.0, 1.2, 0.02, 64),
    (3000, 2000, 16.0, 1.05, 0.01, 128),
    (1500, 1500, 30.0, 1.5, 0.0, 256),
    (700, 900, 25.0, 1.5, 0.0, 512),
    (300, 400, 10.0, 1.0, 0.0, 1000),     # multi-tile columns
    (5, 5, 0.0, 0.0, 0.0, 64),            # all rows empty
]


@pytest.mark.parametrize("M,K,d,skew,empty,N", CASES)
def test_csr_direct_and_baseline_bit_exact(oracle, M, K, d, skew, empty, N):
    print(f"[csr] M={M} K={K} d={d} N={N}", flush=True)
    g = S.random_csr(M, K, d, seed=M + N, skew=skew, empty_frac=empty)
    B = _B(K, N, seed=N)
    ref = oracle.spmm_seq_f32(g.rowptr, g.colind, g.vals, B)
    rp, ci, vl = _dev(g)
    Bd = torch.from_numpy(B).cuda()
    for fn in (ra_spmm.spmm_csr_direct, ra_spmm.spmm_csr_baseline, ra_spmm.spmm_cusparse):
        C = fn(rp, ci, vl, Bd)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(C.cpu().numpy(), ref, err_msg=fn.__name__)


@pytest.mark.parametrize("M", [65535, 65536])
@pytest.mark.parametrize("N", [256, 512])
def test_csr_direct_xcd_slices_boundary(oracle, M, N):
    """CSR_DIRECT deals 128-column slices to the XCDs when the unsliced grid
    has fewer than 2^16 waves (one row per wave at N >= 256: M <= 65535), and
    keeps whole rows above.  Both sides of the switch are the same fma chain
    per element: bit-identical to the oracle."""
    print(f"[csr slices] M={M} N={N}", flush=True)
    g = S.random_csr(M, 20000, 4.0, seed=M + N, skew=1.1, empty_frac=0.02)
    B = _B(g.K, N, seed=N + 1)
    ref = oracle.spmm_seq_f32(g.rowptr, g.colind, g.vals, B)
    rp, ci, vl = _dev(g)
    C = ra_spmm.spmm_csr_direct(rp, ci, vl, torch.from_numpy(B).cuda())
    np.testing.assert_array_equal(C.cpu().numpy(), ref)


def test_csr_direct_unaligned_B_uses_scalar_path(oracle):
    g = S.random_csr(500, 400, 8.0, seed=9)
    B = _B(400, 65, seed=3)
    big = torch.from_numpy(B).cuda().reshape(-1)
    # A view starting 4 bytes in: not 16-byte aligned, contiguous.
    storage = torch.zeros(big.numel() + 1, device="cuda")
    storage[1:] = big
    Bu = storage[1:].view(400, 65)
    rp, ci, vl = _dev(g)
    C = ra_spmm.spmm_csr_direct(rp, ci, vl, Bu)
    np.testing.assert_array_equal(C.cpu().numpy(), oracle.spmm_seq_f32(g.rowptr, g.colind, g.vals, B))


@pytest.mark.parametrize("N", [32, 36, 44, 47, 48, 64, 128, 256, 260, 384, 512, 1000])
def test_zero_overhead_hub_rows(oracle, N):
    print(f"[zo] N={N}", flush=True)
    # Power-law rows: tiny/short/medium/long bins plus multi-chunk hubs.
    g = S.random_csr(3000, 4000, 10.0, seed=N, skew=0.9, empty_frac=0.03, max_deg=3000)
    deg = np.diff(g.rowptr)
    assert deg.max() > 256 and (deg == 0).any()
    B = _B(4000, N, seed=N + 1)
    rp, ci, vl = _dev(g)
    plan = ra_spmm.make_zero_overhead_plan(rp.cpu(), 3000, 4000)
    bins = oracle.zo_bins(g.rowptr)
    assert (plan.num_tiny, plan.num_short, plan.num_medium, plan.num_long, plan.num_empty) == (
        bins["num_tiny"], bins["num_short"], bins["num_medium"], bins["num_long"], bins["num_empty"])
    C = ra_spmm.run_zero_overhead_plan(plan, rp, ci, vl, torch.from_numpy(B).cuda()).cpu().numpy()
    seq = oracle.spmm_seq_f32(g.rowptr, g.colind, g.vals, B)
    short = deg <= 256
    np.testing.assert_array_equal(C[short], seq[short])
    c64 = oracle.spmm_f64(g.rowptr, g.colind, g.vals, B)
    scale = oracle.spmm_f64(g.rowptr, g.colind, np.abs(g.vals), np.abs(B))
    assert_close_scaled(C, c64, scale, 1e-5, "zero_overhead")
    # Deterministic: a second run is bit-identical.
    C2 = ra_spmm.run_zero_overhead_plan(plan, rp, ci, vl, torch.from_numpy(B).cuda()).cpu().numpy()
    np.testing.assert_array_equal(C, C2)


def test_router_plan_device_equals_host():
    g = S.random_csr(20_000, 20_000, 9.0, seed=4, skew=1.3)
    rp = torch.from_numpy(g.rowptr)
    for N in (16, 64, 128, 512):
        a = ra_spmm.make_router_plan(rp.cuda(), rp, rp, g.M, g.K, N)
        b = ra_spmm.make_router_plan(rp, rp, rp, g.M, g.K, N)
        assert a["feature_backend"] == "cuda_rowptr_moments"
        assert (a["chosen_path"], a["use_tf32"]) == (b["chosen_path"], b["use_tf32"])


def test_capi_csr_direct_direct_call(oracle):
    """The C ABI called directly (ctypes, no torch binding) on torch buffers."""
    lib = capi.load()
    g = S.random_csr(800, 700, 11.0, seed=21, skew=1.2)
    B = _B(700, 128, seed=5)
    rp, ci, vl = _dev(g)
    Bd = torch.from_numpy(B).cuda()
    C = torch.empty(800, 128, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    capi.check(lib.ra_spmm_csr_direct(capi.ptr(rp), capi.ptr(ci), capi.ptr(vl), capi.ptr(Bd),
                                      capi.ptr(C), 800, 700, 128, g.nnz, stream))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(C.cpu().numpy(), oracle.spmm_seq_f32(g.rowptr, g.colind, g.vals, B))


def test_c2_full_size_properties(oracle):
    """config C2 at full size: bit-exact against the oracle on a row
    sample, linearity in B and the all-ones row-sum identity on every row."""
    g = S.CONFIGS["C2"]()
    rp, ci, vl = _dev(g)
    N = 128
    rng = np.random.default_rng(12)
    B = torch.from_numpy(rng.standard_normal((g.K, N)).astype(np.float32)).cuda()
    plan = ra_spmm.make_zero_overhead_plan(rp.cpu(), g.M, g.K)
    C_zo = ra_spmm.run_zero_overhead_plan(plan, rp, ci, vl, B)
    C_cd = ra_spmm.spmm_csr_direct(rp, ci, vl, B)
    deg = np.diff(g.rowptr)
    sample = np.concatenate([np.arange(0, g.M, 997), np.argsort(deg)[-50:]])
    Bn = B.cpu().numpy()
    for rows in (sample,):
        sub_rp = np.concatenate([[0], np.cumsum(deg[rows])]).astype(np.int32)
        sub_ci = np.concatenate([g.colind[g.rowptr[r]:g.rowptr[r + 1]] for r in rows])
        sub_vl = np.concatenate([g.vals[g.rowptr[r]:g.rowptr[r + 1]] for r in rows])
        seq = oracle.spmm_seq_f32(sub_rp, sub_ci, sub_vl, Bn)
        np.testing.assert_array_equal(C_cd.cpu().numpy()[rows], seq)
        c64 = oracle.spmm_f64(sub_rp, sub_ci, sub_vl, Bn)
        scale = oracle.spmm_f64(sub_rp, sub_ci, np.abs(sub_vl), np.abs(Bn))
        assert_close_scaled(C_zo.cpu().numpy()[rows], c64, scale, 1e-5, "C2 zero_overhead")
    ones = torch.ones(g.K, 4, device="cuda")
    rs = ra_spmm.run_zero_overhead_plan(plan, rp, ci, vl, ones)[:, 0].double().cpu().numpy()
    exact = np.add.reduceat(np.append(g.vals.astype(np.float64), 0), g.rowptr[:-1])
    exact[deg == 0] = 0
    assert np.all(np.abs(rs - exact) <= 1e-5 * np.maximum(1.0, np.abs(exact)))
    # Linearity: A(2B + B') == 2AB + AB' within fp32 rounding.
    B2 = torch.randn(g.K, N, device="cuda", generator=torch.Generator("cuda").manual_seed(3))
    lhs = ra_spmm.run_zero_overhead_plan(plan, rp, ci, vl, 2 * B + B2)
    rhs = 2 * C_zo + ra_spmm.run_zero_overhead_plan(plan, rp, ci, vl, B2)
    sc = ra_spmm.run_zero_overhead_plan(plan, rp, ci, vl.abs(), (2 * B).abs() + B2.abs())
    assert torch.all((lhs - rhs).abs() <= 1e-5 * sc + 1e-30)


ZO_INFO = ("M", "K", "num_tiny", "num_short", "num_medium", "num_long", "num_empty", "num_chunks",
           "num_split_rows", "max_long_chunks", "num_split_chunks", "plan_bytes")
ZO_LISTS = ("short_rows", "chunk_rows", "chunk_starts", "chunk_slot", "split_rows", "split_off")


RANDOM_ZO = [f"random{i}" for i in range(12)]


@pytest.mark.parametrize("case", ["hubs", "all_empty", "all_long", "one_row", "mixed_large"] + RANDOM_ZO)
def test_zero_overhead_device_binning_matches_host_and_oracle(oracle, case):
    """Device binning (one scan on the GPU) == host binning, list for list, and
    both agree with the oracle's bins (csr/ra_zero_overhead.cu:331-358)."""
    print(f"[zo-build] {case}", flush=True)
    if case == "hubs":
        g = S.random_csr(3000, 4000, 10.0, seed=5, skew=0.9, empty_frac=0.03, max_deg=3000)
    elif case == "all_empty":
        g = S.random_csr(77, 10, 0.0, seed=1)
    elif case == "all_long":
        g = S.random_csr(40, 5000, 700.0, seed=2)
    elif case == "one_row":
        g = S.random_csr(1, 2000, 1000.0, seed=3)
    elif case.startswith("random"):
        # seeded degree mixes around the bin edges (4 / 16 / 64 / 256-nnz chunks)
        rng = np.random.default_rng(700 + int(case[6:]))
        M, K = int(rng.integers(1, 20000)), int(rng.integers(1, 30000))
        d = float(rng.choice([2.0, 10.0, 40.0, 300.0]))
        g = S.random_csr(M, K, min(d, K), seed=int(rng.integers(1 << 30)), skew=float(rng.choice([0.0, 1.0, 1.4])),
                         empty_frac=float(rng.choice([0.0, 0.3])), max_deg=K)
    else:
        g = S.random_csr(200000, 50000, 6.0, seed=4, skew=1.0, empty_frac=0.1, max_deg=20000)
    rp = torch.from_numpy(g.rowptr)
    host = ra_spmm.make_zero_overhead_plan(rp, g.M, g.K, build="host")
    dev = ra_spmm.make_zero_overhead_plan(rp.cuda(), g.M, g.K, build="gpu")
    for f in ZO_INFO:
        assert getattr(host, f) == getattr(dev, f), f
    lists = {n: ra_spmm.export_zero_overhead_plan(dev, n).numpy() for n in ZO_LISTS}
    for n in ZO_LISTS:
        np.testing.assert_array_equal(ra_spmm.export_zero_overhead_plan(host, n).numpy(), lists[n], err_msg=n)
    bins = oracle.zo_bins(g.rowptr)
    empty = np.flatnonzero(np.diff(g.rowptr) == 0)
    np.testing.assert_array_equal(lists["short_rows"], np.concatenate([empty, bins["small_rows"]]))
    np.testing.assert_array_equal(lists["chunk_rows"].astype(np.uint32), bins["chunk_rows"].astype(np.uint32))
    np.testing.assert_array_equal(lists["chunk_starts"], bins["chunk_starts"])
    # Split chunks own consecutive slots in chunk order.
    split = lists["chunk_slot"] >= 0
    np.testing.assert_array_equal(lists["chunk_slot"][split], np.arange(split.sum()))


def test_zero_overhead_run_device_plan_equals_host_plan():
    g = S.random_csr(3000, 4000, 10.0, seed=7, skew=0.9, empty_frac=0.03, max_deg=3000)
    rp, ci, vl = _dev(g)
    B = torch.from_numpy(_B(4000, 128, 3)).cuda()
    host = ra_spmm.make_zero_overhead_plan(rp.cpu(), g.M, g.K, build="host")
    dev = ra_spmm.make_zero_overhead_plan(rp, g.M, g.K)
    assert torch.equal(ra_spmm.run_zero_overhead_plan(host, rp, ci, vl, B),
                       ra_spmm.run_zero_overhead_plan(dev, rp, ci, vl, B))


def test_c5_full_size_routed_widths(oracle):
    """config C5 (GCN operator of a 1e6-row power-law graph) at the GCN's
    widths 256 and 48 through the routed path: rows of at most 64 nonzeros
    bit-exact against the sequential fp32 oracle, longer rows (split into
    chunks) within 1e-5 of fp64, on a row sample with the 50 longest rows."""
    g = S.CONFIGS["C5"]()
    rp, ci, vl = _dev(g)
    deg = np.diff(g.rowptr)
    rows = np.unique(np.concatenate([np.arange(0, g.M, 1999), np.argsort(deg)[-50:]]))
    sub_rp = np.concatenate([[0], np.cumsum(deg[rows])]).astype(np.int32)
    sub_ci = np.concatenate([g.colind[g.rowptr[r]:g.rowptr[r + 1]] for r in rows])
    sub_vl = np.concatenate([g.vals[g.rowptr[r]:g.rowptr[r + 1]] for r in rows])
    short = deg[rows] <= 256
    for N in (256, 48):
        print(f"[c5 full] N={N}", flush=True)
        plan_dict = ra_spmm.make_router_plan(rp, ci, vl, g.M, g.K, N)
        label = ra_spmm.route_label(plan_dict)
        assert label == "ZERO_OVERHEAD_CSR", label
        plan = ra_spmm.build_kernel_plan(label, rp.cpu(), ci.cpu(), vl.cpu(), g.M, g.K, N)
        Bn = _B(g.K, N, 50 + N)
        C = ra_spmm.run_planned_kernel(label, plan, rp, ci, vl, torch.from_numpy(Bn).cuda()).cpu().numpy()[rows]
        seq = oracle.spmm_seq_f32(sub_rp, sub_ci, sub_vl, Bn)
        np.testing.assert_array_equal(C[short], seq[short])
        assert_close_scaled(C, oracle.spmm_f64(sub_rp, sub_ci, sub_vl, Bn),
                            oracle.spmm_f64(sub_rp, sub_ci, np.abs(sub_vl), np.abs(Bn)), 1e-5, f"C5 N={N}")


def test_precision_matched_guardrail_fp16(oracle):
    """spmm_cusparse_fp16 (bindings/ra_bindings.cpp:895-907): A values and B
    rounded to fp16, one fp32 fma chain per element in CSR order: bit-identical
    to the oracle's chain on the rounded inputs.  Its warm/cold timing dicts
    carry the reference's keys."""
    g = S.random_csr(1500, 1200, 14.0, seed=21, skew=1.1, empty_frac=0.03)
    rp, ci, vl = _dev(g)
    for N in (1, 47, 64, 300):
        B = _B(g.K, N, seed=N)
        C = ra_spmm.spmm_cusparse_fp16(rp, ci, vl, torch.from_numpy(B).cuda()).cpu().numpy()
        ref = oracle.spmm_seq_f32(g.rowptr, g.colind, oracle.quantize_f16(g.vals), oracle.quantize_f16(B))
        np.testing.assert_array_equal(C, ref, err_msg=f"N={N}")
    Bd = torch.from_numpy(_B(g.K, 64, seed=1)).cuda()
    warm = ra_spmm.benchmark_cusparse_fp16(rp, ci, vl, Bd, warmup=1, iters=3)
    cold = ra_spmm.benchmark_cusparse_fp16_cold(rp, ci, vl, Bd, iters=2)
    for d in (warm, cold):
        assert d["path"] == "CUSPARSE_FP16" and d["exec_ms"] > 0 and d["external_baseline"]
        assert {"plan_ms", "exec_ms", "total_ms", "gflops", "preprocess_ms", "cusparse_algorithm"} <= set(d)
    assert cold["plan_ms"] > 0


def test_harness_helpers_run_every_deployed_kernel(oracle):
    """run_kernel / benchmark_custom_cold / correctness_gate as the real-graph
    harness uses them (ra_real_graph_eval.py:288-343, 478-495)."""
    g = S.random_csr(900, 900, 10.0, seed=4, skew=1.0)
    rp, ci, vl = _dev(g)
    B = torch.from_numpy(_B(g.K, 32, seed=2)).cuda()
    C_ref = ra_spmm.spmm_cusparse(rp, ci, vl, B)
    max_row = int(np.diff(g.rowptr).max())
    cache = {}
    for k in ra_spmm.DEPLOYED_KERNELS + ["CUSPARSE"]:
        out = ra_spmm.run_kernel(k, rp, ci, vl, B, cache, (k, 32))
        gate = ra_spmm.correctness_gate(k, float((out - C_ref).abs().max()), max_row)
        assert gate["correct"], (k, gate)
        cold = ra_spmm.benchmark_custom_cold(k, rp.cpu(), ci.cpu(), vl.cpu(), rp, ci, vl, B, 2) \
            if k != "CUSPARSE" else None
        if cold:
            assert cold["cold_exec_ms"] > 0 and (cold["preprocess_ms"] > 0) == (k != "CSR_DIRECT")
    assert len(cache) == len(ra_spmm.DEPLOYED_KERNELS) + 1
    assert ra_spmm.measure_ms(lambda: ra_spmm.spmm_csr_direct(rp, ci, vl, B), 2, 5) > 0


def test_deployed_cold_policy(oracle):
    """The cold-aware single-call policy (run_deployed_cold): uniform rows run
    CSR_DIRECT, bit-identical to the oracle; skewed rows (degree CV >= 1.5) run
    ZERO_OVERHEAD_CSR binned from the device rowptr, equal to a ZO plan built
    from the host rowptr."""
    N = 64
    uni = S.random_csr(3000, 2000, 9.0, seed=21)
    skew = S.random_csr(3000, 2000, 9.0, seed=22, skew=0.9)
    for g, want in ((uni, "CSR_DIRECT"), (skew, "ZERO_OVERHEAD_CSR")):
        rp, ci, vl = _dev(g)
        B = _B(g.K, N, seed=5)
        Bd = torch.from_numpy(B).cuda()
        C, label = ra_spmm.run_deployed_cold(rp, ci, vl, Bd)
        cv = ra_spmm.make_router_plan(rp, ci, vl, g.M, g.K, N)["feature_values"]["degree_cv"]
        assert label == want and (cv >= ra_spmm.COLD_ZO_MIN_CV) == (want == "ZERO_OVERHEAD_CSR"), (label, cv)
        if want == "CSR_DIRECT":
            np.testing.assert_array_equal(C.cpu().numpy(), oracle.spmm_seq_f32(g.rowptr, g.colind, g.vals, B))
        else:
            host = ra_spmm.make_zero_overhead_plan(rp.cpu(), g.M, g.K)
            assert torch.equal(C, ra_spmm.run_zero_overhead_plan(host, rp, ci, vl, Bd))
