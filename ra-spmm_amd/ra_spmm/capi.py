"""ctypes view of the C ABI (include/ra_spmm.h).

This is how a non-torch host (or a test) binds the library directly: plain
pointers, sizes and status codes.  Structures mirror the header exactly.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libra_spmm_hip.so"

RA_OK = 0
RA_PATH_COUNT = 15
DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2
TILE_TC_DIRECT, TILE_COMMUNITY_TC, TILE_SEGMENT_HYBRID = 0, 1, 2
ROUTE_F16, ROUTE_BF16, ROUTE_FP32 = 0, 1, 2
TABLE_REFERENCE, TABLE_MI355X = 0, 1

# Every function include/ra_spmm.h declares (checked by tests/test_capi_symbols.py).
EXPORTED = [
    "ra_abi_version", "ra_status_string", "ra_last_error", "ra_path_name", "ra_reject_name",
    "ra_features_host", "ra_features_device", "ra_features_from_moments", "ra_route_dispatch",
    "ra_analyze_matrix",
    "ra_spmm_csr_direct", "ra_spmm_csr_baseline", "ra_spmm_csr_baseline_f16", "ra_zo_bins_host", "ra_zo_plan_create",
    "ra_zo_plan_create_device", "ra_zo_plan_export", "ra_zo_plan_run", "ra_zo_plan_run_stage", "ra_zo_plan_run_noalloc", "ra_zo_plan_get_info", "ra_zo_plan_destroy", "ra_tile_host_build",
    "ra_tile_host_get_info", "ra_tile_host_export", "ra_tile_host_destroy",
    "ra_tile_plan_create", "ra_tile_plan_create_device", "ra_tile_plan_export",
    "ra_tile_plan_run", "ra_tile_plan_run_lowp",
    "ra_tile_plan_get_info", "ra_tile_plan_destroy", "ra_convert_f32",
]


class Features(ctypes.Structure):
    _fields_ = [("M", ctypes.c_int32), ("K", ctypes.c_int32), ("N", ctypes.c_int32),
                ("max_deg", ctypes.c_int32), ("nnz", ctypes.c_int64),
                ("sum_deg_sq", ctypes.c_int64), ("empty_rows", ctypes.c_int64),
                ("avg", ctypes.c_double), ("std_dev", ctypes.c_double),
                ("avg_nnz_per_row", ctypes.c_float), ("std_nnz_per_row", ctypes.c_float),
                ("degree_cv", ctypes.c_float), ("max_to_mean_ratio", ctypes.c_float)]


DIAG_FLOAT_FIELDS = (
    "avg_nnz_per_row",
    "std_nnz_per_row",
    "degree_cv",
    "max_to_mean_ratio",
    "frac_dense_rows",
    "skew_ratio",
    "long_row_fraction",
    "long_row_nnz_fraction",
    "top_1_row_nnz_fraction",
    "top_5_row_nnz_fraction",
    "tile_fill_mean",
    "tile_fill_median",
    "tile_fill_p90",
    "tile_fill_max",
    "tile_fill_variance",
    "tile_occupancy",
    "actual_nnz_coverage",
    "avg_nnz_per_tile",
    "row_window_colspan_compactness",
    "local_row_similarity_proxy",
    "reordered_locality_proxy",
    "locality_gain_proxy",
    "locality_selectivity_proxy",
    "road_likeness_proxy",
    "row_split_affinity_proxy",
    "mixedness_proxy",
    "tc_candidate_ratio",
    "tc_synergy_proxy",
    "estimated_tc_partition_ratio",
    "estimated_cuda_partition_ratio",
    "irregular_window_fraction",
    "tc_granularity_proxy",
    "redundancy_risk_proxy",
)


class DiagFeatures(ctypes.Structure):
    _fields_ = ([(k, ctypes.c_float) for k in DIAG_FLOAT_FIELDS] +
                [("tc_candidate_tiles", ctypes.c_int32), ("N", ctypes.c_int32), ("M", ctypes.c_int32),
                 ("K", ctypes.c_int32), ("nnz", ctypes.c_int64)])


class Route(ctypes.Structure):
    _fields_ = [("chosen_path", ctypes.c_int32), ("use_tf32", ctypes.c_int32),
                ("rule", ctypes.c_int32), ("tile_ok", ctypes.c_int32),
                ("estimated_risk", ctypes.c_float), ("pad_", ctypes.c_float),
                ("est_plan_s", ctypes.c_double), ("decision_reason", ctypes.c_char * 64),
                ("feasible", ctypes.c_int8 * RA_PATH_COUNT),
                ("rejection_code", ctypes.c_int8 * RA_PATH_COUNT)]


class ZOInfo(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in (
        "M", "K", "num_tiny", "num_short", "num_medium", "num_long", "num_empty", "num_small",
        "num_chunks", "num_sole_chunks", "num_split_rows", "num_split_chunks",
        "max_long_chunks", "pad_")] + [("plan_bytes", ctypes.c_int64)]


class TileInfo(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in (
        "kind", "M", "K", "active", "num_windows", "num_blocks", "num_segments",
        "num_split_windows", "num_split_segs", "max_window_blocks")] + [
        ("nnz", ctypes.c_int64), ("num_vectors", ctypes.c_int64), ("plan_bytes", ctypes.c_int64),
        ("avg_tile_density", ctypes.c_float), ("value_dtype", ctypes.c_int32),
        ("build_ms", ctypes.c_double), ("value_scale_log2", ctypes.c_int32), ("rows_per_window", ctypes.c_int32),
        ("col_parts", ctypes.c_int32), ("pad3_", ctypes.c_int32)]


_lib = None


def load():
    """Load libra_spmm_hip.so and declare signatures.  torch (if used) must be
    imported first so both share its HIP runtime."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise ImportError(f"{LIB_PATH} is missing: build with ra-spmm_amd/build.py")
    lib = ctypes.CDLL(str(LIB_PATH))
    P = ctypes.c_void_p
    I32, I64 = ctypes.c_int32, ctypes.c_int64
    sig = {
        "ra_abi_version": (ctypes.c_int, []),
        "ra_status_string": (ctypes.c_char_p, [ctypes.c_int]),
        "ra_last_error": (ctypes.c_char_p, []),
        "ra_path_name": (ctypes.c_char_p, [I32]),
        "ra_reject_name": (ctypes.c_char_p, [I32]),
        "ra_features_host": (ctypes.c_int, [P, I32, I32, I32, ctypes.POINTER(Features)]),
        "ra_analyze_matrix": (ctypes.c_int, [P, P, I32, I32, I32, ctypes.POINTER(DiagFeatures)]),
        "ra_features_device": (ctypes.c_int, [P, I32, I32, I32, P, ctypes.POINTER(Features)]),
        "ra_features_from_moments": (ctypes.c_int, [I32, I32, I32, I64, I64, I32, I64,
                                                    ctypes.POINTER(Features)]),
        "ra_route_dispatch": (ctypes.c_int, [ctypes.POINTER(Features), I32, I32,
                                             ctypes.POINTER(Route)]),
        "ra_spmm_csr_direct": (ctypes.c_int, [P, P, P, P, P, I32, I32, I32, I64, P]),
        "ra_spmm_csr_baseline": (ctypes.c_int, [P, P, P, P, P, I32, I32, I32, I64, P]),
        "ra_spmm_csr_baseline_f16": (ctypes.c_int, [P, P, P, P, P, I32, I32, I32, I64, P]),
        "ra_zo_bins_host": (ctypes.c_int, [P, I32, I32, P, P, P, P, ctypes.POINTER(ZOInfo)]),
        "ra_zo_plan_create": (ctypes.c_int, [P, I32, I32, ctypes.POINTER(P)]),
        "ra_zo_plan_create_device": (ctypes.c_int, [P, I32, I32, P, ctypes.POINTER(P)]),
        "ra_zo_plan_export": (ctypes.c_int, [P, ctypes.c_char_p, P, ctypes.POINTER(I64)]),
        "ra_zo_plan_run": (ctypes.c_int, [P, P, P, P, P, P, I32, P]),
        "ra_zo_plan_run_stage": (ctypes.c_int, [P, P, P, P, P, P, I32, I32, P]),
        "ra_zo_plan_run_noalloc": (ctypes.c_int, [P, P, P, P, P, P, I32, P]),
        "ra_zo_plan_get_info": (ctypes.c_int, [P, ctypes.POINTER(ZOInfo)]),
        "ra_zo_plan_destroy": (None, [P]),
        "ra_tile_host_build": (ctypes.c_int, [I32, P, P, P, I32, I32, I32, I32, ctypes.POINTER(P)]),
        "ra_tile_host_get_info": (ctypes.c_int, [P, ctypes.POINTER(TileInfo)]),
        "ra_tile_host_export": (ctypes.c_int, [P, ctypes.c_char_p, P, ctypes.POINTER(I64)]),
        "ra_tile_host_destroy": (None, [P]),
        "ra_tile_plan_create": (ctypes.c_int, [I32, P, P, P, I32, I32, I32, I32, ctypes.POINTER(P)]),
        "ra_tile_plan_create_device": (ctypes.c_int, [I32, P, P, P, I32, I32, I32, I32, I32, P,
                                                      ctypes.POINTER(P)]),
        "ra_tile_plan_export": (ctypes.c_int, [P, ctypes.c_char_p, P, ctypes.POINTER(I64)]),
        "ra_tile_plan_run": (ctypes.c_int, [P, P, P, I32, I32, P]),
        "ra_tile_plan_run_lowp": (ctypes.c_int, [P, P, I32, I32, P, I32, P]),
        "ra_tile_plan_get_info": (ctypes.c_int, [P, ctypes.POINTER(TileInfo)]),
        "ra_tile_plan_destroy": (None, [P]),
        "ra_convert_f32": (ctypes.c_int, [P, P, I64, I32, I32, I32, P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


class RAError(RuntimeError):
    pass


def check(status: int, what: str = "ra_spmm") -> None:
    if status != RA_OK:
        lib = load()
        raise RAError(f"{what}: {lib.ra_status_string(status).decode()}: "
                      f"{lib.ra_last_error().decode()}")


def ptr(x) -> ctypes.c_void_p:
    """Raw address of a torch tensor or numpy array (None -> NULL)."""
    if x is None:
        return ctypes.c_void_p(0)
    if hasattr(x, "data_ptr"):
        return ctypes.c_void_p(x.data_ptr())
    return ctypes.c_void_p(x.ctypes.data)
