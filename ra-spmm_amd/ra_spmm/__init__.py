"""ra_spmm — MI355X-native regime-aware SpMM (C = A @ B, A CSR, B dense).

Drop-in for the reference `ra_spmm` extension (tariqaf/RA-SpMM,
bindings/ra_bindings.cpp:2318-2899): the same plan/run functions, router dict
and plan classes, backed by hand-written HIP kernels for gfx950 through the C
ABI in include/ra_spmm.h.  There is no CPU fallback: importing fails loudly
when the HIP extension is not built.
"""
from __future__ import annotations

import torch  # noqa: F401  (loads the HIP runtime the extension binds to)

try:
    from . import _C
except ImportError as exc:  # pragma: no cover - exercised only on broken installs
    raise ImportError(
        "ra_spmm: the HIP extension is not built; run `python ra-spmm_amd/build.py` "
        f"(or __graft_entry__.build()). Original error: {exc}") from exc

from ._C import (  # noqa: F401
    CuSparsePlan, RACommunityTCPlan, analyze_matrix, RASegmentHybridPlan, RATcDirectPlan, RATilePlan,
    RAZeroOverheadPlan, compute_features, export_tile_plan, export_zero_overhead_plan, make_community_tc_plan, make_cusparse_plan,
    make_router_plan, make_segment_hybrid_plan, make_tc_direct_plan, make_zero_overhead_plan,
    route_features, run_community_tc_plan, run_community_tc_plan_tf32, run_cusparse_plan,
    run_segment_hybrid_plan, run_segment_hybrid_plan_tf32, run_tc_direct_plan,
    run_tc_direct_plan_tf32, run_tile_plan_route, run_zero_overhead_plan, spmm_csr_baseline,
    spmm_csr_baseline_f16, spmm_csr_direct, spmm_cusparse,
)
from .dispatch import (  # noqa: F401
    BASE_ATOL, COLD_ITERS, COLD_ZO_MIN_CV, DEPLOYED_KERNELS, HARD_FAIL_THRESHOLD, TC_EXTRA_FACTOR, TILE_KERNELS, TIMED_ITERS,
    WARMUP, benchmark_cusparse, benchmark_cusparse_cold, benchmark_cusparse_fp16, benchmark_cusparse_fp16_cold,
    benchmark_custom_cold, build_kernel_plan, cold_path, correctness_gate, gpu_info_next, make_timing_breakdown,
    measure_exec_ms, measure_ms, measure_one_ms, population_cv, run_kernel, run_oracle_cold, run_oracle_warm,
    run_deployed_cold, run_planned_kernel, run_router_cold, run_router_plan, run_router_warm, smallest_strict_crossover,
    spmm_cusparse_fp16,
)
from .router import (  # noqa: F401
    MI355X, REFERENCE, RouterTable, features_from_moments, features_two_pass, production_features,
    route_label,
    route_with_rules, simple_router,
)

__all__ = [n for n in dir() if not n.startswith("_")]
