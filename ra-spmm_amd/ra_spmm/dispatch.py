"""Label -> plan/run dispatch, timing drivers and one-shot helpers.

Reference: build_kernel_plan / run_planned_kernel / run_kernel /
benchmark_custom_cold, measure_ms, population_cv and the correctness gate,
ra_real_graph_eval.py:37-51, 210-343, 478-495; make_timing_breakdown / measure_cuda_exec_ms,
bench/benchmark.cpp:19-67; benchmark_cusparse[_cold], spmm_cusparse_fp16 /
benchmark_cusparse_fp16[_cold] (bindings/ra_bindings.cpp:895-960), run_router_plan,
run_router_{warm,cold}, run_oracle_{warm,cold}, bindings/ra_bindings.cpp:821-1037,
1320-1965.  Timing uses HIP events on the current stream, which is the stream
every ra_spmm launch goes to.
"""
from __future__ import annotations

import time

import torch

from . import _C
from .router import route_label

DEPLOYED_KERNELS = ["CSR_DIRECT", "ZERO_OVERHEAD_CSR", "TC_DIRECT", "COMMUNITY_TC",
                    "SEGMENT_HYBRID", "TC_DIRECT_TF32", "COMMUNITY_TC_TF32",
                    "SEGMENT_HYBRID_TF32"]
TILE_KERNELS = {"TC_DIRECT", "COMMUNITY_TC", "SEGMENT_HYBRID", "TC_DIRECT_TF32",
                "COMMUNITY_TC_TF32", "SEGMENT_HYBRID_TF32"}


def build_kernel_plan(kernel_name, rowptr_cpu, colind_cpu, vals_cpu, M, K, N):
    """ra_real_graph_eval.py:247-263."""
    if kernel_name in ("CSR_DIRECT", "CSR_BASELINE"):
        return None
    if kernel_name == "ZERO_OVERHEAD_CSR":
        return _C.make_zero_overhead_plan(rowptr_cpu, M, K)
    if kernel_name in ("TC_DIRECT", "TC_DIRECT_TF32"):
        return _C.make_tc_direct_plan(rowptr_cpu, colind_cpu, vals_cpu, M, K, N)
    if kernel_name in ("COMMUNITY_TC", "COMMUNITY_TC_TF32"):
        return _C.make_community_tc_plan(rowptr_cpu, colind_cpu, vals_cpu, M, K, N)
    if kernel_name in ("SEGMENT_HYBRID", "SEGMENT_HYBRID_TF32"):
        return _C.make_segment_hybrid_plan(rowptr_cpu, colind_cpu, vals_cpu, M, K, N)
    raise ValueError(f"Kernel has no reusable custom plan: {kernel_name}")


def run_planned_kernel(kernel_name, plan, rowptr, colind, vals, B):
    """ra_real_graph_eval.py:266-285."""
    if kernel_name == "CSR_DIRECT":
        return _C.spmm_csr_direct(rowptr, colind, vals, B)
    if kernel_name == "CSR_BASELINE":
        return _C.spmm_csr_baseline(rowptr, colind, vals, B)
    if kernel_name == "ZERO_OVERHEAD_CSR":
        return _C.run_zero_overhead_plan(plan, rowptr, colind, vals, B)
    if kernel_name == "TC_DIRECT":
        return _C.run_tc_direct_plan(plan, B)
    if kernel_name == "TC_DIRECT_TF32":
        return _C.run_tc_direct_plan_tf32(plan, B)
    if kernel_name == "COMMUNITY_TC":
        return _C.run_community_tc_plan(plan, B)
    if kernel_name == "COMMUNITY_TC_TF32":
        return _C.run_community_tc_plan_tf32(plan, B)
    if kernel_name == "SEGMENT_HYBRID":
        return _C.run_segment_hybrid_plan(plan, colind, vals, B)
    if kernel_name == "SEGMENT_HYBRID_TF32":
        return _C.run_segment_hybrid_plan_tf32(plan, colind, vals, B)
    raise ValueError(f"Unknown planned kernel: {kernel_name}")


def run_kernel(kernel_name, rowptr, colind, vals, B, plan_cache: dict, cache_key):
    """Plan once per cache_key, then run (ra_real_graph_eval.py:288-301).  The
    guardrail name uses the reusable baseline plan, which owns its C."""
    if kernel_name == "CUSPARSE":
        if cache_key not in plan_cache:
            plan_cache[cache_key] = _C.make_cusparse_plan(rowptr, colind, vals, B)
        return _C.run_cusparse_plan(plan_cache[cache_key], B)
    if cache_key not in plan_cache:
        M = int(rowptr.shape[0]) - 1
        plan_cache[cache_key] = build_kernel_plan(kernel_name, rowptr.cpu(), colind.cpu(), vals.cpu(), M,
                                                  int(B.shape[0]), int(B.shape[1]))
    return run_planned_kernel(kernel_name, plan_cache[cache_key], rowptr, colind, vals, B)


# Harness protocol and correctness gate (ra_real_graph_eval.py:37-51).
WARMUP = 50
TIMED_ITERS = 200
COLD_ITERS = 10
BASE_ATOL = 1e-3
TC_EXTRA_FACTOR = 10.0
HARD_FAIL_THRESHOLD = 1.0


def population_cv(degrees) -> float:
    """std (population) / mean of row lengths, 0 for an empty or all-zero
    vector (ra_real_graph_eval.py:235-242)."""
    d = torch.as_tensor(degrees).float()
    if d.numel() == 0:
        return 0.0
    mean = d.mean()
    if float(mean.item()) == 0.0:
        return 0.0
    return float((d.std(correction=0) / mean).item())


def correctness_gate(kernel_name: str, max_error: float, max_row_nnz: int) -> dict:
    """The harness's verdict on one kernel's max |C - C_ref|: tolerance
    1e-3 * sqrt(max row nnz), x10 for the tile paths; errors >= 1 are hard
    failures (ra_real_graph_eval.py:481-489)."""
    import math
    tol = BASE_ATOL * max(1.0, math.sqrt(max(1, int(max_row_nnz))))
    if kernel_name in TILE_KERNELS:
        tol *= TC_EXTRA_FACTOR
    return {"correct": max_error <= tol and max_error < HARD_FAIL_THRESHOLD,
            "soft_fail": tol < max_error < HARD_FAIL_THRESHOLD,
            "hard_fail": max_error >= HARD_FAIL_THRESHOLD,
            "max_error": max_error, "tolerance": tol, "error": ""}


def measure_ms(run_fn, warmup: int = WARMUP, iters: int = TIMED_ITERS) -> float:
    """Warm protocol of the harness: 50 warmup calls, one event pair over 200
    (ra_real_graph_eval.py:210-221)."""
    return measure_exec_ms(run_fn, warmup, iters)


def benchmark_custom_cold(kernel_name, rowptr_cpu, colind_cpu, vals_cpu, rowptr, colind, vals, B,
                          iters: int = COLD_ITERS) -> dict:
    """Cold protocol: plan build (host-timed, synchronised) + one event-timed
    execution, averaged over `iters`; CSR_DIRECT has no plan
    (ra_real_graph_eval.py:304-343)."""
    M = int(rowptr_cpu.numel() - 1)
    K, N = int(B.shape[0]), int(B.shape[1])
    n = max(1, iters)
    plan_total = exec_total = 0.0
    for _ in range(n):
        plan = None
        if kernel_name != "CSR_DIRECT":
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            plan = build_kernel_plan(kernel_name, rowptr_cpu, colind_cpu, vals_cpu, M, K, N)
            torch.cuda.synchronize()
            plan_total += (time.perf_counter() - t0) * 1e3
        out, ms = measure_one_ms(lambda: run_planned_kernel(kernel_name, plan, rowptr, colind, vals, B))
        exec_total += ms
        del out, plan
    pre, cold = plan_total / n, exec_total / n
    return {"preprocess_ms": pre, "cold_exec_ms": cold, "ms_cold": pre + cold}


def smallest_strict_crossover(setup_a: float, exec_a: float, setup_b: float, exec_b: float):
    """Smallest integer K >= 1 with setup_b + K*exec_b < setup_a + K*exec_a,
    None when b never wins (experiments/conversion_aware_routing.py:47-53).
    Used to state after how many SpMM calls a plan's build cost is repaid."""
    import math
    if exec_b >= exec_a:
        return None
    threshold = (setup_b - setup_a) / (exec_a - exec_b)
    return max(1, math.floor(threshold) + 1)


def make_timing_breakdown(plan_ms: float, exec_ms: float, nnz: int, N: int) -> dict:
    """bench/benchmark.cpp:29-37: GFLOP/s = 2*nnz*N / (exec_ms * 1e6)."""
    gflops = (2.0 * nnz * N) / (exec_ms * 1e6) if exec_ms > 0 else 0.0
    return {"plan_ms": plan_ms, "exec_ms": exec_ms, "total_ms": plan_ms + exec_ms,
            "gflops": gflops}


def measure_exec_ms(fn, warmup: int = 3, iters: int = 10) -> float:
    """Warmup, then one event pair around `iters` calls; mean ms per call
    (bench/benchmark.cpp:39-67)."""
    if iters <= 0:
        return 0.0
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(iters):
        fn()
    stop.record()
    stop.synchronize()
    return start.elapsed_time(stop) / iters


def measure_one_ms(fn):
    """One event-timed call; returns (output, ms) (ra_real_graph_eval.py:210-221)."""
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    out = fn()
    stop.record()
    stop.synchronize()
    return out, start.elapsed_time(stop)


def benchmark_cusparse(rowptr, colind, vals, B, warmup: int = 3, iters: int = 10) -> dict:
    """Warm guardrail timing (baseline CSR kernel), bindings/ra_bindings.cpp:838-866."""
    plan = _C.make_cusparse_plan(rowptr, colind, vals, B)
    ms = measure_exec_ms(lambda: _C.run_cusparse_plan(plan, B), warmup, max(1, iters))
    d = make_timing_breakdown(0.0, ms, int(colind.numel()), int(B.shape[1]))
    d.update(path="CUSPARSE", in_main_portfolio=False, legacy_baseline=False,
             external_baseline=True, cusparse_algorithm=plan.algorithm, preprocess_ms=0.0)
    return d


def benchmark_cusparse_cold(rowptr, colind, vals, B, iters: int = 10) -> dict:
    """Cold guardrail timing: plan construction + one execution, averaged."""
    plan_sum = exec_sum = 0.0
    name = ""
    for _ in range(max(1, iters)):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        plan = _C.make_cusparse_plan(rowptr, colind, vals, B)
        torch.cuda.synchronize()
        plan_sum += (time.perf_counter() - t0) * 1e3
        _, ms = measure_one_ms(lambda: _C.run_cusparse_plan(plan, B))
        exec_sum += ms
        name = plan.algorithm
    n = float(max(1, iters))
    d = make_timing_breakdown(plan_sum / n, exec_sum / n, int(colind.numel()), int(B.shape[1]))
    d.update(path="CUSPARSE", in_main_portfolio=True, legacy_baseline=False,
             external_baseline=False, cusparse_algorithm=name, preprocess_ms=plan_sum / n)
    return d


def spmm_cusparse_fp16(rowptr, colind, vals, B):
    """Precision-matched guardrail, one shot: A values and B rounded to fp16,
    products and sums in fp32, C fp32 (bindings/ra_bindings.cpp:895-907)."""
    return _C.spmm_csr_baseline_f16(rowptr, colind, vals.contiguous().half(), B.contiguous().half())


def benchmark_cusparse_fp16(rowptr, colind, vals, B, warmup: int = 3, iters: int = 10) -> dict:
    """Warm precision-matched guardrail timing: conversion outside the timed
    loop, as the reference's state build (bindings/ra_bindings.cpp:909-932)."""
    vh, bh = vals.contiguous().half(), B.contiguous().half()
    ms = measure_exec_ms(lambda: _C.spmm_csr_baseline_f16(rowptr, colind, vh, bh), warmup, max(1, iters))
    d = make_timing_breakdown(0.0, ms, int(colind.numel()), int(B.shape[1]))
    d.update(path="CUSPARSE_FP16", in_main_portfolio=False, legacy_baseline=False, external_baseline=True,
             cusparse_algorithm="csr_baseline_kernel_f16", preprocess_ms=0.0)
    return d


def benchmark_cusparse_fp16_cold(rowptr, colind, vals, B, iters: int = 10) -> dict:
    """Cold precision-matched guardrail timing: fp16 conversion of A values and
    B (the state build) plus one execution, averaged (bindings/ra_bindings.cpp:935-960)."""
    plan_sum = exec_sum = 0.0
    for _ in range(max(1, iters)):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        vh, bh = vals.contiguous().half(), B.contiguous().half()
        torch.cuda.synchronize()
        plan_sum += (time.perf_counter() - t0) * 1e3
        _, ms = measure_one_ms(lambda: _C.spmm_csr_baseline_f16(rowptr, colind, vh, bh))
        exec_sum += ms
    n = float(max(1, iters))
    d = make_timing_breakdown(plan_sum / n, exec_sum / n, int(colind.numel()), int(B.shape[1]))
    d.update(path="CUSPARSE_FP16", in_main_portfolio=False, legacy_baseline=False, external_baseline=True,
             cusparse_algorithm="csr_baseline_kernel_f16", preprocess_ms=plan_sum / n)
    return d


def run_router_plan(plan_dict, rowptr, colind, vals, B):
    """One-shot helper: builds the chosen plan and runs it once
    (bindings/ra_bindings.cpp:1762-1881).  Not for warm timing."""
    label = route_label(plan_dict)
    M = int(rowptr.numel()) - 1
    K, N = int(B.shape[0]), int(B.shape[1])
    if label == "CUSPARSE":
        return _C.spmm_cusparse(rowptr, colind, vals, B)
    plan = build_kernel_plan(label, rowptr.cpu(), colind.cpu(), vals.cpu(), M, K, N)
    return run_planned_kernel(label, plan, rowptr, colind, vals, B)


# Degree CV from which the cold-aware policy runs ZERO_OVERHEAD_CSR (the MI355X
# router table's zo_min_cv).
COLD_ZO_MIN_CV = 1.5


def cold_path(plan_dict) -> str:
    """Path of the cold-aware policy for a single-call or streaming caller
    (experiments/deployed_coldstart.py:1-10, gnn_bench/cold_first_step.py:61-139):
    no tile-format build.  The reference runs CSR_DIRECT.  On MI355X a
    ZERO_OVERHEAD_CSR plan is binned on the GPU from the device rowptr in
    0.3-0.7 ms, while one lane group per hub row makes CSR_DIRECT 6.6x slower
    on skewed rows (config C2: 6.6 against 1.0 ms), so rows of degree CV >= 1.5
    take ZERO_OVERHEAD_CSR."""
    cv = float(plan_dict["feature_values"]["degree_cv"])
    return "ZERO_OVERHEAD_CSR" if cv >= COLD_ZO_MIN_CV else "CSR_DIRECT"


def run_deployed_cold(rowptr, colind, vals, B, table="mi355x"):
    """One cold call under the cold-aware policy, every overhead included: the
    device feature pass and the rule tree, the policy's plan (a
    ZERO_OVERHEAD_CSR binning from the device rowptr, or none) and the
    execution.  Returns (C, label)."""
    M = int(rowptr.numel()) - 1
    K, N = int(B.shape[0]), int(B.shape[1])
    plan_dict = _C.make_router_plan(rowptr, colind, vals, M, K, N, "MAIN", table)
    label = cold_path(plan_dict)
    if label == "ZERO_OVERHEAD_CSR":
        plan = _C.make_zero_overhead_plan(rowptr, M, K)
        return _C.run_zero_overhead_plan(plan, rowptr, colind, vals, B), label
    return _C.spmm_csr_direct(rowptr, colind, vals, B), label


def _router_generic(rowptr, colind, vals, B, portfolio, warmup, iters, cold, table="mi355x"):
    M = int(rowptr.numel()) - 1
    K, N = int(B.shape[0]), int(B.shape[1])
    nnz = int(colind.numel())
    t0 = time.perf_counter()
    plan_dict = _C.make_router_plan(rowptr, colind, vals, M, K, N, portfolio, table)
    route_ms = (time.perf_counter() - t0) * 1e3
    label = route_label(plan_dict)
    if label == "CUSPARSE":
        t1 = time.perf_counter()
        p = _C.make_cusparse_plan(rowptr, colind, vals, B)
        build_ms = (time.perf_counter() - t1) * 1e3
        fn = lambda: _C.run_cusparse_plan(p, B)  # noqa: E731
    else:
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        p = build_kernel_plan(label, rowptr.cpu(), colind.cpu(), vals.cpu(), M, K, N)
        torch.cuda.synchronize()
        build_ms = (time.perf_counter() - t1) * 1e3
        fn = lambda: run_planned_kernel(label, p, rowptr, colind, vals, B)  # noqa: E731
    if cold:
        _, exec_ms = measure_one_ms(fn)
        d = make_timing_breakdown(route_ms + build_ms, exec_ms, nnz, N)
    else:
        d = make_timing_breakdown(0.0, measure_exec_ms(fn, warmup, iters), nnz, N)
    d.update(path=label, route_ms=route_ms, preprocess_ms=build_ms, router_plan=plan_dict)
    return d


def run_router_warm(rowptr, colind, vals, B, portfolio="MAIN", warmup=3, iters=10, table="mi355x"):
    return _router_generic(rowptr, colind, vals, B, portfolio, warmup, iters, False, table)


def run_router_cold(rowptr, colind, vals, B, portfolio="MAIN", warmup=3, iters=10, table="mi355x"):
    return _router_generic(rowptr, colind, vals, B, portfolio, warmup, iters, True, table)


def _oracle_generic(rowptr, colind, vals, B, warmup, iters, cold, kernels=None):
    """Time every deployed path; report the fastest (the routing oracle)."""
    M = int(rowptr.numel()) - 1
    K, N = int(B.shape[0]), int(B.shape[1])
    nnz = int(colind.numel())
    kernels = kernels or DEPLOYED_KERNELS
    results = {}
    for k in kernels:
        if k in TILE_KERNELS and N < 16:
            continue
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        p = build_kernel_plan(k, rowptr.cpu(), colind.cpu(), vals.cpu(), M, K, N)
        torch.cuda.synchronize()
        build_ms = (time.perf_counter() - t0) * 1e3
        fn = lambda: run_planned_kernel(k, p, rowptr, colind, vals, B)  # noqa: E731
        if cold:
            _, ms = measure_one_ms(fn)
            results[k] = make_timing_breakdown(build_ms, ms, nnz, N)
        else:
            results[k] = make_timing_breakdown(0.0, measure_exec_ms(fn, warmup, iters), nnz, N)
        del p
    key = "total_ms" if cold else "exec_ms"
    best = min(results, key=lambda k: results[k][key])
    d = dict(results[best])
    d.update(path=best, per_path=results)
    return d


def run_oracle_warm(rowptr, colind, vals, B, warmup=3, iters=10, portfolio="MAIN"):
    return _oracle_generic(rowptr, colind, vals, B, warmup, iters, False)


def run_oracle_cold(rowptr, colind, vals, B, warmup=3, iters=10, portfolio="MAIN"):
    return _oracle_generic(rowptr, colind, vals, B, warmup, iters, True)


def gpu_info_next() -> dict:
    """Device properties of the current GPU."""
    p = torch.cuda.get_device_properties(torch.cuda.current_device())
    return {"name": p.name, "gcn_arch": getattr(p, "gcnArchName", ""),
            "multi_processor_count": p.multi_processor_count,
            "total_memory": p.total_memory, "backend": "hip"}
