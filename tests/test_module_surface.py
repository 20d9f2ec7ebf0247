"""The `ra_spmm` module exports the reference extension's deployed names with
the same keyword arguments (bindings/ra_bindings.cpp:2318-2899), so harness and
GNN code calling them by keyword runs unchanged.  Import-only: no GPU needed."""
import inspect

import ra_spmm

REQUIRED = {
    # name: keyword arguments the reference binding declares
    "spmm_csr_direct": ["rowptr", "colind", "vals", "B"],
    "make_router_plan": ["rowptr", "colind", "vals", "M", "K", "N", "portfolio"],
    "make_zero_overhead_plan": ["rowptr_cpu", "M", "K"],
    "run_zero_overhead_plan": ["plan", "rowptr", "colind", "vals", "B"],
    "make_tc_direct_plan": ["rowptr_cpu", "colind_cpu", "vals_cpu", "M", "K", "N"],
    "run_tc_direct_plan": ["plan", "B"],
    "run_tc_direct_plan_tf32": ["plan", "B"],
    "make_community_tc_plan": ["rowptr_cpu", "colind_cpu", "vals_cpu", "M", "K", "N"],
    "run_community_tc_plan": ["plan", "B"],
    "run_community_tc_plan_tf32": ["plan", "B"],
    "make_segment_hybrid_plan": ["rowptr_cpu", "colind_cpu", "vals_cpu", "M", "K", "N"],
    "run_segment_hybrid_plan": ["plan", "colind", "vals", "B"],
    "run_segment_hybrid_plan_tf32": ["plan", "colind", "vals", "B"],
    "spmm_cusparse": ["rowptr", "colind", "vals", "B"],
    "analyze_matrix": ["rowptr", "colind", "M", "K", "N"],
    "spmm_cusparse_fp16": ["rowptr", "colind", "vals", "B"],
    "benchmark_cusparse_fp16": ["rowptr", "colind", "vals", "B", "warmup", "iters"],
    "benchmark_cusparse_fp16_cold": ["rowptr", "colind", "vals", "B", "iters"],
    # harness helpers of ra_real_graph_eval.py (the a17 call site)
    "build_kernel_plan": ["kernel_name", "rowptr_cpu", "colind_cpu", "vals_cpu", "M", "K", "N"],
    "run_planned_kernel": ["kernel_name", "plan", "rowptr", "colind", "vals", "B"],
    "run_kernel": ["kernel_name", "rowptr", "colind", "vals", "B", "plan_cache", "cache_key"],
    "benchmark_custom_cold": ["kernel_name", "rowptr_cpu", "colind_cpu", "vals_cpu", "rowptr", "colind", "vals",
                              "B", "iters"],
    "measure_ms": ["run_fn", "warmup", "iters"],
    "population_cv": ["degrees"],
}
OPTIONAL = ["make_cusparse_plan", "run_cusparse_plan", "benchmark_cusparse", "benchmark_cusparse_cold",
            "run_router_plan", "run_router_warm", "run_router_cold", "run_oracle_warm", "run_oracle_cold",
            "gpu_info_next", "route_with_rules", "simple_router"]
CLASSES = ["RAZeroOverheadPlan", "RATcDirectPlan", "RACommunityTCPlan", "RASegmentHybridPlan", "CuSparsePlan"]
PLAN_PROPS = ["valid", "M", "K", "num_tc_tiles", "plan_bytes"]


def _kwargs(fn):
    """Keyword names of a pybind11 function (from its signature line) or a Python one."""
    try:
        return list(inspect.signature(fn).parameters)
    except (TypeError, ValueError):
        first = fn.__doc__.splitlines()[0]
        inside = first[first.index("(") + 1:first.rindex(")")]
        return [a.split(":")[0].strip() for a in inside.split(",") if a.strip()]


def test_required_functions_and_keywords():
    for name, kws in REQUIRED.items():
        fn = getattr(ra_spmm, name)
        got = _kwargs(fn)
        assert got[:len(kws)] == kws, (name, got)


def test_optional_names_and_plan_classes():
    for name in OPTIONAL + CLASSES:
        assert hasattr(ra_spmm, name), name
    for cls in ("RATcDirectPlan", "RACommunityTCPlan", "RASegmentHybridPlan"):
        for prop in PLAN_PROPS:
            assert hasattr(getattr(ra_spmm, cls), prop), (cls, prop)
    for prop in ("valid", "M", "K", "plan_bytes", "num_tiny", "num_long"):
        assert hasattr(ra_spmm.RAZeroOverheadPlan, prop), prop


def test_correctness_gate_and_cv_follow_the_harness():
    """ra_real_graph_eval.py:37-51, 235-242, 481-489: tolerance 1e-3 sqrt(max row
    nnz), x10 for tile paths, hard failure at 1.0; population CV."""
    import math
    import torch
    assert (ra_spmm.WARMUP, ra_spmm.TIMED_ITERS, ra_spmm.COLD_ITERS) == (50, 200, 10)
    g = ra_spmm.correctness_gate("CSR_DIRECT", 0.0099, 100)
    assert g["correct"] and math.isclose(g["tolerance"], 0.01)
    g = ra_spmm.correctness_gate("COMMUNITY_TC_TF32", 0.05, 100)
    assert g["correct"] and math.isclose(g["tolerance"], 0.1)
    g = ra_spmm.correctness_gate("ZERO_OVERHEAD_CSR", 0.5, 0)   # max row clamps to 1: tol 1e-3
    assert g["soft_fail"] and not g["correct"] and not g["hard_fail"]
    g = ra_spmm.correctness_gate("TC_DIRECT", 1.0, 10**8)        # tol 100, but >= 1.0 is hard
    assert g["hard_fail"] and not g["correct"] and not g["soft_fail"]
    assert ra_spmm.population_cv(torch.tensor([2, 2, 2])) == 0.0
    assert ra_spmm.population_cv(torch.tensor([0, 0])) == 0.0
    assert ra_spmm.population_cv(torch.tensor([], dtype=torch.int32)) == 0.0
    assert math.isclose(ra_spmm.population_cv(torch.tensor([1, 3])), 0.5, rel_tol=1e-6)
