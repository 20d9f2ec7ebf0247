"""Python mirror of the seven-rule router (lockstep with csrc/router.cpp).

Reference: route_with_rules / simple_router, ra_router_eval.py:37-129, and the
C++ deployed block router/router_dispatch.cpp:979-1110.

Bit-identity with the C++ router is by construction:
  * the decision reads float32 features; ``production_features`` reproduces
    both feature forms of the C++ side bit for bit (the moment form of the
    device pass, ra_features_from_moments, and the two-pass form of the host
    pass, ra_features_host);
  * every comparison is float32 value vs float32 threshold, evaluated on the
    exactly representable doubles (``_f32``), which is what the C++ float
    comparisons compute;
  * the tile gate is plan_s_per_nnz * d * M (2e-8 in the reference table)
    evaluated in doubles from the float32 d, in the C++ order.
The reference Python mirror compared float64 d and cv against float64
literals, which can disagree with its C++ twin next to a threshold; routing on
canonical float32 features removes that gap.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

__all__ = [
    "RouterTable", "REFERENCE", "MI355X", "TABLES", "production_features",
    "features_from_moments", "features_two_pass", "route_with_rules", "simple_router", "route_label",
]


def _f32(x) -> float:
    """Round to float32 and return the exactly representable double."""
    return float(np.float32(x))


@dataclass(frozen=True)
class RouterTable:
    """Threshold table; field meanings match struct RouterTable in csrc/router.cpp."""
    cv_extreme: float = 5.0
    cv_uniform: float = 0.7
    d_ultralow: float = 4.5
    n_ultralow_csr: int = 256
    cv_comm_lo: float = 0.2
    d_comm: float = 7.0
    n_comm_csr: int = 128
    cv_skewed: float = 3.0
    m_skewed_large: int = 250000
    d_dense: float = 40.0
    m_small: int = 20000
    d_small_dense: float = 25.0
    n_small_narrow: int = 96
    n_small_mid: int = 256
    d_heavy: float = 25.0
    cv_heavy: float = 1.8
    d_web: float = 9.0
    cv_web_lo: float = 1.10
    cv_web_hi: float = 1.45
    m_web: int = 250000
    cv_gate_csr: float = 1.5
    plan_s_per_nnz: float = 2e-8
    plan_budget_s: float = 20.0
    d_fp32_route: float = 5.0
    m_fp32_small: int = 25000
    d_fp32_small: float = 9.0
    fp32_route_csr: bool = False
    zo_min_cv: float = 1e30
    n_uniform_csr: int = 0
    skewed_path: str | None = None       # rule 3: None = reference split on M
    small_dense_path: str | None = None  # rule 5: None = reference split on N
    heavy_path: str = "COMMUNITY_TC"     # rule 6
    web_path: str = "COMMUNITY_TC"       # rule 7
    web_fp32: bool = True                #   rule 7 forces the FP32 route
    fp32_small_max_cv: float = 1e30      # small-graph FP32 condition only when cv <


REFERENCE = RouterTable()
# Calibrated on gfx950 (values and measurements: csrc/router.cpp, kMI355X).
MI355X = RouterTable(plan_s_per_nnz=1e-9, fp32_route_csr=True, zo_min_cv=1.5, n_uniform_csr=64,
                     skewed_path="SEGMENT_HYBRID", small_dense_path="SEGMENT_HYBRID",
                     heavy_path="SEGMENT_HYBRID", web_path="TC_DIRECT", web_fp32=False,
                     fp32_small_max_cv=0.7)
TABLES = {"reference": REFERENCE, "mi355x": MI355X}


def features_from_moments(M: int, nnz: int, sum_deg_sq: int, K: int = 1):
    """(d32, cv32) exactly as ra_features_from_moments computes them (the
    device form, router/router_features_cuda.cu:83-91)."""
    if M <= 0 or K <= 0:
        return 0.0, 0.0
    avg = float(nnz) / float(M)
    var = float(sum_deg_sq) / float(M) - avg * avg
    if var < 0.0:
        var = 0.0
    std = math.sqrt(var)
    d32 = _f32(avg)
    cv32 = _f32(std / avg) if avg > 1e-6 else 0.0
    return d32, cv32


def features_two_pass(rowptr, M: int, K: int = 1):
    """(d32, cv32) exactly as ra_features_host computes them (the host form,
    router/router_features.cpp:79-111): sum (d - avg)^2 in ascending row
    order (np.cumsum adds left to right)."""
    rp = np.asarray(rowptr.cpu() if hasattr(rowptr, "cpu") else rowptr, dtype=np.int64)
    if M <= 0 or K <= 0:
        return 0.0, 0.0
    nnz = int(rp[M] - rp[0])
    avg = nnz / M
    if nnz <= 0:
        return _f32(avg), 0.0
    delta = np.diff(rp[: M + 1]).astype(np.float64) - avg
    std = math.sqrt(float(np.cumsum(delta * delta)[-1]) / M)
    return _f32(avg), (_f32(std / avg) if avg > 1e-6 else 0.0)


def production_features(rowptr, M: int | None = None, K: int | None = None,
                        form: str = "moments"):
    """Routing features of a CSR rowptr (numpy / torch / list).

    ``form="moments"`` gives the device path's values (ra_features_device),
    ``form="two_pass"`` the host path's (ra_features_host).
    Returns dict(M, nnz, sum_deg_sq, max_deg, avg_nnz_per_row, degree_cv).
    """
    rp = np.asarray(rowptr.cpu() if hasattr(rowptr, "cpu") else rowptr, dtype=np.int64)
    if M is None:
        M = len(rp) - 1
    if K is None:
        K = max(M, 1)
    deg = np.diff(rp[: M + 1])
    nnz = int(rp[M] - rp[0]) if M > 0 else 0
    s2 = int(np.dot(deg, deg)) if M > 0 else 0
    if form == "moments":
        d32, cv32 = features_from_moments(M, nnz, s2, K)
    elif form == "two_pass":
        d32, cv32 = features_two_pass(rp, M, K)
    else:
        raise ValueError(f"unknown feature form {form!r}")
    return {"M": M, "nnz": nnz, "sum_deg_sq": s2, "max_deg": int(deg.max()) if M > 0 else 0,
            "avg_nnz_per_row": d32, "degree_cv": cv32}


def route_with_rules(avg_nnz, degree_cv, M, N, nnz=None, *, disabled_rules=(), table="mi355x"):
    """Label of the routed path ("TC_DIRECT", "COMMUNITY_TC_TF32", ...).

    ``avg_nnz`` and ``degree_cv`` are rounded to float32 first; pass the
    features from ``production_features`` for bit-identity with the C++
    router.  ``nnz`` is accepted for signature compatibility with the
    reference mirror; the tile gate uses d*M like the C++ router.
    ``disabled_rules`` skips rules (ablation, as in the reference mirror).
    """
    T = TABLES[table] if isinstance(table, str) else table
    disabled = frozenset(disabled_rules)
    d = _f32(avg_nnz)
    cv = _f32(degree_cv)
    M = int(M)
    N = int(N)
    tile_feasible = N >= 16
    est_plan_s = T.plan_s_per_nnz * d * float(M)
    tile_ok = tile_feasible and est_plan_s <= T.plan_budget_s
    choice = "TC_DIRECT" if tile_feasible else "CSR_DIRECT"
    fp32 = False

    def csr_by_skew():
        return "CSR_DIRECT" if cv < _f32(T.cv_gate_csr) else "ZERO_OVERHEAD_CSR"

    def _direct(path):
        # A rule's path from the table: a tile family goes through the tile
        # gate and the precision rule, a CSR family is taken as is.
        return pick(path) if path in ("TC_DIRECT", "COMMUNITY_TC", "SEGMENT_HYBRID") else (path, False)

    def pick(kernel, force_fp32=False):
        if tile_ok:
            want = force_fp32 or (d < _f32(T.d_fp32_route)
                                  or (M <= T.m_fp32_small and d < _f32(T.d_fp32_small)
                                      and cv < _f32(T.fp32_small_max_cv)))
            if want and T.fp32_route_csr:
                return csr_by_skew(), False
            return kernel, want
        return csr_by_skew(), False

    if 1 not in disabled and cv >= _f32(T.cv_extreme):
        choice = "ZERO_OVERHEAD_CSR"
    elif 2 not in disabled and cv < _f32(T.cv_uniform):
        if d < _f32(T.d_ultralow):
            choice, fp32 = ("CSR_DIRECT", False) if N <= T.n_ultralow_csr else pick("TC_DIRECT")
        elif cv >= _f32(T.cv_comm_lo) and d < _f32(T.d_comm):
            choice, fp32 = ("CSR_DIRECT", False) if N <= T.n_comm_csr else pick("TC_DIRECT", True)
        elif N <= T.n_uniform_csr:
            choice = "CSR_DIRECT"
        else:
            choice, fp32 = pick("TC_DIRECT")
    elif 3 not in disabled and cv >= _f32(T.cv_skewed):
        if T.skewed_path is not None:
            choice, fp32 = _direct(T.skewed_path)
        elif M >= T.m_skewed_large:
            choice, fp32 = pick("COMMUNITY_TC")
        else:
            choice, fp32 = pick("SEGMENT_HYBRID")
    elif 4 not in disabled and d >= _f32(T.d_dense):
        choice, fp32 = pick("COMMUNITY_TC")
    elif 5 not in disabled and M < T.m_small and d >= _f32(T.d_small_dense):
        if T.small_dense_path is not None:
            choice, fp32 = _direct(T.small_dense_path)
        elif N < T.n_small_narrow:
            choice = "CUSPARSE"
        elif N < T.n_small_mid:
            choice, fp32 = pick("SEGMENT_HYBRID")
        else:
            choice, fp32 = pick("COMMUNITY_TC")
    elif 6 not in disabled and d >= _f32(T.d_heavy) and cv >= _f32(T.cv_heavy):
        choice, fp32 = _direct(T.heavy_path)
    elif (7 not in disabled and d < _f32(T.d_web) and cv >= _f32(T.cv_web_lo)
          and cv <= _f32(T.cv_web_hi) and M >= T.m_web):
        choice, fp32 = (pick(T.web_path, T.web_fp32) if T.web_path in ("TC_DIRECT", "COMMUNITY_TC", "SEGMENT_HYBRID")
                        else (T.web_path, False))
    else:
        choice, fp32 = pick("TC_DIRECT")

    if choice == "CSR_DIRECT" and cv >= _f32(T.zo_min_cv):
        choice = "ZERO_OVERHEAD_CSR"
    is_tile = choice in ("TC_DIRECT", "COMMUNITY_TC", "SEGMENT_HYBRID")
    return choice + ("_TF32" if (is_tile and fp32) else "")


def simple_router(avg_nnz, degree_cv, M, N, nnz=None, table="mi355x"):
    """Rule-tree decision with all seven rules enabled (ra_router_eval.py:127-129)."""
    return route_with_rules(avg_nnz, degree_cv, M, N, nnz, table=table)


def route_label(plan: dict) -> str:
    """Executed label of a make_router_plan dict: family plus _TF32 when the
    FP32 route is selected (gnn_bench/router_vs_baselines_gcn.py:79-86)."""
    fam = str(plan["chosen_path"])
    tile = fam in ("TC_DIRECT", "COMMUNITY_TC", "SEGMENT_HYBRID")
    return fam + "_TF32" if (tile and bool(plan.get("use_tf32", False))) else fam
