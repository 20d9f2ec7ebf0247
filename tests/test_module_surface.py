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
