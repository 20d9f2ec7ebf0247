"""CPU oracle for the routed SpMM hot path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this module, and only as the checker.  The product
(``ra-spmm_amd/``) never imports it.

Each function restates the reference algorithm (tariqaf/RA-SpMM) and cites the
file:line it follows.  How each one is pinned (golden rows, closed forms,
invariants, brute force) is stated in its docstring; the tests in
``tests/test_oracle_*.py`` hold the pins.
"""
from __future__ import annotations

import ctypes
import math
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
_LIB_PATH = HERE / "_build" / "liboracle.so"
_lib = None


def build(force: bool = False) -> Path:
    """Compile the C restatement (oracle/spmm_oracle.c) with oracle/Makefile."""
    if force or not _LIB_PATH.exists():
        subprocess.run(["make", "-s", "-C", str(HERE)] + (["-B"] if force else []),
                       check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        lib = ctypes.CDLL(str(_LIB_PATH))
        p = ctypes.c_void_p
        i32 = ctypes.c_int32
        lib.oracle_spmm_seq_f32.argtypes = [p, p, p, p, p, i32, i32]
        lib.oracle_spmm_f64.argtypes = [p, p, p, p, p, i32, i32]
        lib.oracle_spmm_seq_f32_rows.argtypes = [p, p, p, p, p, i32, i32, i32]
        lib.oracle_degree_moments.argtypes = [p, i32, p, p, p, p]
        _lib = lib
    return _lib


def _ptr(a: np.ndarray):
    return ctypes.c_void_p(a.ctypes.data)


def _csr_arrays(rowptr, colind, vals, B):
    rowptr = np.ascontiguousarray(rowptr, dtype=np.int32)
    colind = np.ascontiguousarray(colind, dtype=np.int32)
    vals = np.ascontiguousarray(vals, dtype=np.float32)
    B = np.ascontiguousarray(B, dtype=np.float32)
    return rowptr, colind, vals, B


# --------------------------------------------------------------------------
# SpMM arithmetic
# --------------------------------------------------------------------------
def spmm_seq_f32(rowptr, colind, vals, B) -> np.ndarray:
    """C[r,n] = fma-chain over p in CSR order, one fp32 accumulator per element.

    Follows csr/csr_direct.cu:201-228 (per-lane accumulator, `acc += av*b`
    contracted to FMA under --use_fast_math, setup.py:52).  Pinned by
    tests/test_oracle_spmm.py against the fp64 closed form, the all-ones and
    unit-column invariants and a pure-Python loop on tiny inputs.
    """
    rowptr, colind, vals, B = _csr_arrays(rowptr, colind, vals, B)
    M = rowptr.shape[0] - 1
    N = B.shape[1]
    C = np.empty((M, N), dtype=np.float32)
    _load().oracle_spmm_seq_f32(_ptr(rowptr), _ptr(colind), _ptr(vals), _ptr(B), _ptr(C), M, N)
    return C


def spmm_seq_f32_rows(rowptr, colind, vals, B, r0: int, r1: int) -> np.ndarray:
    """spmm_seq_f32 restricted to rows [r0, r1) (bounded CPU-baseline sample)."""
    rowptr, colind, vals, B = _csr_arrays(rowptr, colind, vals, B)
    N = B.shape[1]
    C = np.empty((r1 - r0, N), dtype=np.float32)
    _load().oracle_spmm_seq_f32_rows(_ptr(rowptr), _ptr(colind), _ptr(vals), _ptr(B), _ptr(C),
                                     r0, r1, N)
    return C


def spmm_f64(rowptr, colind, vals, B) -> np.ndarray:
    """Exact C = A @ B in fp64 (inputs read as fp32).  Pinned against scipy."""
    rowptr, colind, vals, B = _csr_arrays(rowptr, colind, vals, B)
    M = rowptr.shape[0] - 1
    N = B.shape[1]
    C = np.empty((M, N), dtype=np.float64)
    _load().oracle_spmm_f64(_ptr(rowptr), _ptr(colind), _ptr(vals), _ptr(B), _ptr(C), M, N)
    return C


def spmm_python(rowptr, colind, vals, B) -> np.ndarray:
    """Pure-Python loop version of spmm_seq_f32 (tiny inputs only).

    Uses math.fma semantics via an fp64 product rounded once: for fp32 a, b
    the product a*b is exact in fp64, so float32(a*b + acc) computed in fp64
    equals fmaf(a, b, acc) whenever the fp64 sum is exact, which holds for
    the magnitudes the tests use (|a|,|b| ~ 1, a few terms).
    """
    rowptr = np.asarray(rowptr)
    M = len(rowptr) - 1
    N = B.shape[1]
    C = np.zeros((M, N), dtype=np.float32)
    for r in range(M):
        for n in range(N):
            acc = np.float32(0.0)
            for p in range(int(rowptr[r]), int(rowptr[r + 1])):
                acc = np.float32(float(vals[p]) * float(B[colind[p], n]) + float(acc))
            C[r, n] = acc
    return C


# --------------------------------------------------------------------------
# Low-precision quantisers (tile paths)
# --------------------------------------------------------------------------
def quantize_f16(x) -> np.ndarray:
    """IEEE fp16 round-to-nearest-even, returned as fp32 (numpy's conversion is
    the library routine; reference host_float_to_half_bits, tc/ra_tc_direct.cu:45-69,
    and __float2half_rn in tc/ra_community_tc.cu:34-39 are both RNE)."""
    with np.errstate(over="ignore"):  # beyond 65504 rounds to inf, as RNE does
        return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def tile_value_scale_log2(vals) -> int:
    """Power-of-two exponent s the fp16 tile plans store values with (v * 2^s):
    max|v| lands in [2^13, 2^14), clamped to [-24, 24]; 0 for an all-zero
    matrix.  Pinned by tests/test_oracle_structures.py against the builder and
    by the closed form on powers of two."""
    a = np.abs(np.asarray(vals, dtype=np.float32))
    if a.size == 0 or not np.isfinite(a).all() or a.max() == 0:
        return 0
    e = int(np.floor(np.log2(np.float64(a.max()))))
    return int(min(24, max(-24, 13 - e)))


def quantize_f16_scaled(x, s: int) -> np.ndarray:
    """fp16 RNE of x * 2^s, returned as fp32 times 2^-s (exact power-of-two
    scaling: identical to quantize_f16 for normal-range values, more precise
    for values that would be fp16 subnormals)."""
    x = np.asarray(x, dtype=np.float32)
    with np.errstate(over="ignore"):
        return (np.ldexp(x, s).astype(np.float16).astype(np.float32) * np.float32(2.0 ** -s)).astype(np.float32)


def quantize_bf16(x) -> np.ndarray:
    """bf16 round-to-nearest-even (NaN kept quiet), returned as fp32."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounding = 0x7FFF + ((u >> 16) & 1)
    out = ((u + rounding) >> 16) << 16
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    out = np.where(nan, (u | 0x400000) & 0xFFFF0000, out)
    return out.astype(np.uint32).view(np.float32)


def quantize_tf32_rna(x) -> np.ndarray:
    """TF32 (10-bit mantissa) round-to-nearest, ties away from zero — the
    semantics of PTX cvt.rna.tf32.f32 used by the reference TF32 kernels
    (tc/ra_tc_direct.cu:189-261).  Returned as fp32."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    out = ((u + 0x1000) >> 13) << 13
    return out.astype(np.uint32).view(np.float32)


# --------------------------------------------------------------------------
# Routing features
# --------------------------------------------------------------------------
def degree_moments(rowptr):
    """Exact (nnz, sum deg^2, max deg, empty rows) of a CSR rowptr."""
    rowptr = np.ascontiguousarray(rowptr, dtype=np.int32)
    M = rowptr.shape[0] - 1
    nnz = ctypes.c_int64()
    s2 = ctypes.c_int64()
    mx = ctypes.c_int32()
    em = ctypes.c_int64()
    _load().oracle_degree_moments(_ptr(rowptr), M, ctypes.byref(nnz), ctypes.byref(s2),
                                  ctypes.byref(mx), ctypes.byref(em))
    return int(nnz.value), int(s2.value), int(mx.value), int(em.value)


def features_gpu_reference(rowptr, M: int, K: int = 1):
    """Features as the reference GPU pass computes them
    (router/router_features_cuda.cu:51-92): zero features when M <= 0 or K <= 0
    (:57-59); avg = S1/M, var = max(0, S2/M - avg^2), cv = float(std/avg).
    S1, S2 are exact here (integer sums), which is what the reference's fp64
    atomics give while S2 < 2^53.
    Returns (nnz, avg64, std64, avg32, std32, cv32).
    Pinned by numpy's population std (tests/test_oracle_router.py) and by
    degree sequences whose CV is known in closed form."""
    nnz, s2, _, _ = degree_moments(rowptr)
    if M <= 0 or K <= 0:
        return 0, 0.0, 0.0, 0.0, 0.0, 0.0
    avg = float(nnz) / float(M)
    var = max(0.0, float(s2) / float(M) - avg * avg)
    std = math.sqrt(var)
    cv = np.float32(std / avg) if avg > 1e-6 else np.float32(0.0)
    return nnz, avg, std, float(np.float32(avg)), float(np.float32(std)), float(cv)


def features_cpu_reference(rowptr, M: int, K: int = 1):
    """Two-pass features of compute_production_router_features
    (router/router_features.cpp:79-111): zero features when M <= 0 or K <= 0
    (:86-88); avg = nnz/M; when nnz <= 0 only avg is set (:94-96); otherwise
    sigma^2 = sum_row (d - avg)^2 / M, summed in ascending row order (the
    reference's serial loop; above 131072 rows it is an OpenMP reduction
    whose order depends on the thread count), cv = float(sigma/avg).
    np.cumsum adds strictly left to right, so the last element is the serial
    double sum.  Returns (nnz, avg32, std32, cv32).
    Pinned by numpy's population std and by degree sequences whose CV is
    known in closed form (tests/test_oracle_router.py)."""
    rowptr = np.asarray(rowptr, dtype=np.int64)
    if M <= 0 or K <= 0:
        return 0, 0.0, 0.0, 0.0
    nnz = int(rowptr[M] - rowptr[0])
    avg = nnz / M
    if nnz <= 0:
        return nnz, float(np.float32(avg)), 0.0, 0.0
    deg = np.diff(rowptr[: M + 1]).astype(np.float64)
    delta = deg - avg
    sq = float(np.cumsum(delta * delta)[-1])
    std = math.sqrt(sq / M)
    cv = float(np.float32(std / avg)) if avg > 1e-6 else 0.0
    return nnz, float(np.float32(avg)), float(np.float32(std)), cv


# --------------------------------------------------------------------------
# Router (reference thresholds)
# --------------------------------------------------------------------------
def route_python_reference(avg_nnz, degree_cv, M, N, nnz, disabled_rules=()):
    """Restatement of the reference Python mirror route_with_rules
    (ra_router_eval.py:37-124): fp64 comparisons, tile gate on nnz*2e-8 <= 20
    and N >= 16, TF32 suffix when d < 5 or (M <= 25000 and d < 9).
    Pinned by the 192 golden rows of router_quality_v8.csv and the 36 unseen
    rows (tests/test_oracle_router.py)."""
    disabled = frozenset(disabled_rules)
    d = avg_nnz
    cv = degree_cv
    tile_ok = (N >= 16) and (float(nnz) * 2e-8 <= 20.0)

    def tile(kernel):
        if not tile_ok:
            return "CSR_DIRECT" if cv < 1.5 else "ZERO_OVERHEAD_CSR"
        if d < 5.0 or (M <= 25000 and d < 9.0):
            return kernel + "_TF32"
        return kernel

    if 1 not in disabled and cv >= 5.0:
        return "ZERO_OVERHEAD_CSR"
    if 2 not in disabled and cv < 0.7:
        if d < 4.5:
            return "CSR_DIRECT" if N <= 256 else tile("TC_DIRECT")
        if cv >= 0.2 and d < 7.0:
            if N <= 128:
                return "CSR_DIRECT"
            picked = tile("TC_DIRECT")
            return picked + "_TF32" if picked == "TC_DIRECT" else picked
        return tile("TC_DIRECT")
    if 3 not in disabled and cv >= 3.0:
        return tile("COMMUNITY_TC") if M >= 250000 else tile("SEGMENT_HYBRID")
    if 4 not in disabled and d >= 40.0:
        return tile("COMMUNITY_TC")
    if 5 not in disabled and M < 20000 and d >= 25.0:
        if N < 96:
            return "CUSPARSE"
        if N < 256:
            return tile("SEGMENT_HYBRID")
        return tile("COMMUNITY_TC")
    if 6 not in disabled and d >= 25.0 and cv >= 1.8:
        return tile("COMMUNITY_TC")
    if 7 not in disabled and d < 9.0 and 1.10 <= cv <= 1.45 and M >= 250000:
        picked = tile("COMMUNITY_TC")
        return picked + "_TF32" if picked == "COMMUNITY_TC" else picked
    return tile("TC_DIRECT")


def route_cpp_reference(d32, cv32, M, N):
    """Restatement of the reference C++ deployed block
    (router/router_dispatch.cpp:979-1110) on float32 features: float
    comparisons against float literals, tile gate 2e-8*d*M <= 20 (:1011-1013),
    N >= 16 feasibility (:391-458).  Returns the label with _TF32 suffix.
    Pinned by the same golden rows (decisions agree with the Python mirror
    except on threshold-adjacent inputs, which the tests enumerate)."""
    f = lambda v: float(np.float32(v))  # noqa: E731  float literal
    d = f(d32)
    cv = f(cv32)
    tile_feasible = N >= 16
    est_plan_s = 2e-8 * d * float(M)
    tile_ok = tile_feasible and est_plan_s <= 20.0
    state = {"path": "TC_DIRECT" if tile_feasible else "CSR_DIRECT", "tf32": False}

    def pick(kernel, force_tf32=False):
        if tile_ok:
            state["path"] = kernel
            state["tf32"] = force_tf32 or (d < f(5.0) or (M <= 25000 and d < f(9.0)))
        elif cv < f(1.5):
            state["path"] = "CSR_DIRECT"
        else:
            state["path"] = "ZERO_OVERHEAD_CSR"

    if cv >= f(5.0):
        state["path"] = "ZERO_OVERHEAD_CSR"
    elif cv < f(0.7):
        if d < f(4.5):
            if N <= 256:
                state["path"] = "CSR_DIRECT"
            else:
                pick("TC_DIRECT")
        elif cv >= f(0.2) and d < f(7.0):
            if N <= 128:
                state["path"] = "CSR_DIRECT"
            else:
                pick("TC_DIRECT", True)
        else:
            pick("TC_DIRECT")
    elif cv >= f(3.0):
        pick("COMMUNITY_TC" if M >= 250000 else "SEGMENT_HYBRID")
    elif d >= f(40.0):
        pick("COMMUNITY_TC")
    elif M < 20000 and d >= f(25.0):
        if N < 96:
            state["path"] = "CUSPARSE"
        elif N < 256:
            pick("SEGMENT_HYBRID")
        else:
            pick("COMMUNITY_TC")
    elif d >= f(25.0) and cv >= f(1.8):
        pick("COMMUNITY_TC")
    elif d < f(9.0) and cv >= f(1.10) and cv <= f(1.45) and M >= 250000:
        pick("COMMUNITY_TC", True)
    else:
        pick("TC_DIRECT")
    is_tile = state["path"] in ("TC_DIRECT", "COMMUNITY_TC", "SEGMENT_HYBRID")
    return state["path"] + ("_TF32" if (is_tile and state["tf32"]) else "")


# --------------------------------------------------------------------------
# ZERO_OVERHEAD_CSR binning
# --------------------------------------------------------------------------
ZO_TINY, ZO_SHORT, ZO_MEDIUM, ZO_CHUNK = 4, 16, 64, 256
SOLE_FLAG = 0x80000000


def zo_bins(rowptr):
    """Binning of make_ra_zero_overhead_plan (csr/ra_zero_overhead.cu:331-358):
    empty / tiny (<=4) / short (<=16) / medium (<=64) / long (>64, 256-nnz chunks,
    bit 31 marks a sole chunk when the row has <= 256 nnz).  The small list is
    tiny, short, medium concatenated (:368-374).  Pinned by brute-force
    invariants in tests/test_oracle_structures.py."""
    rowptr = np.asarray(rowptr, dtype=np.int64)
    M = len(rowptr) - 1
    tiny, short, medium, chunk_rows, chunk_starts, zero_rows = [], [], [], [], [], []
    num_long = 0
    max_long = 0
    for i in range(M):
        start = int(rowptr[i])
        nnz = int(rowptr[i + 1]) - start
        if nnz == 0:
            zero_rows.append(i)
        elif nnz <= ZO_TINY:
            tiny.append(i)
        elif nnz <= ZO_SHORT:
            short.append(i)
        elif nnz <= ZO_MEDIUM:
            medium.append(i)
        else:
            num_long += 1
            max_long = max(max_long, nnz)
            if nnz <= ZO_CHUNK:
                chunk_rows.append(i | SOLE_FLAG)
                chunk_starts.append(start)
            else:
                zero_rows.append(i)
                for off in range(0, nnz, ZO_CHUNK):
                    chunk_rows.append(i)
                    chunk_starts.append(start + off)
    return {
        "small_rows": np.array(tiny + short + medium, dtype=np.int64),
        "chunk_rows": np.array(chunk_rows, dtype=np.int64),
        "chunk_starts": np.array(chunk_starts, dtype=np.int64),
        "zero_rows": np.array(zero_rows, dtype=np.int64),
        "num_tiny": len(tiny), "num_short": len(short), "num_medium": len(medium),
        "num_long": num_long,
        "num_empty": sum(1 for i in range(M) if rowptr[i + 1] == rowptr[i]),
        "max_long_chunks": (max_long + ZO_CHUNK - 1) // ZO_CHUNK,
    }


# --------------------------------------------------------------------------
# Tile format (ME-BCRS-style 8x1 vectors)
# --------------------------------------------------------------------------
WINDOW, VEC_PER_BLOCK, SEG_BLOCKS = 8, 8, 64


def community_order(rowptr, colind, M):
    """Rows stable-sorted by (first column or INT_MAX, row id)
    (tc/ra_community_tc.cu:335-347)."""
    rowptr = np.asarray(rowptr, dtype=np.int64)
    colind = np.asarray(colind, dtype=np.int64)
    INT_MAX = 2**31 - 1
    keys = [(int(colind[rowptr[r]]) if rowptr[r] < rowptr[r + 1] else INT_MAX, r)
            for r in range(M)]
    return [r for _, r in sorted(keys)]


def tile_format(kind, rowptr, colind, vals, M):
    """Restatement of the window/vector/block build shared by the three tile
    families (tc/ra_tc_direct.cu:654-706; tc/ra_community_tc.cu:335-403;
    tc/ra_segment_hybrid.cu:470-498).  kind: 0 TC_DIRECT, 1 COMMUNITY_TC,
    2 SEGMENT_HYBRID.  Entries of a window are sorted by (col, window slot);
    each distinct column opens a vector; vectors fill blocks of 8.  Values are
    kept in fp32 here; block b holds dense[b][slot][k].  Duplicate (row, col)
    entries are summed.  Pinned by decode==CSR and counting invariants
    (tests/test_oracle_structures.py)."""
    rowptr = np.asarray(rowptr, dtype=np.int64)
    colind = np.asarray(colind, dtype=np.int64)
    vals = np.asarray(vals, dtype=np.float32)
    W = (M + WINDOW - 1) // WINDOW
    if kind == 1:
        order = community_order(rowptr, colind, M)
    else:
        order = list(range(M))
    win_rows = np.full(W * WINDOW, -1, dtype=np.int64)
    win_rows[:M] = order
    block_offsets = [0]
    atox = []
    blocks = []
    for w in range(W):
        entries = {}
        for slot in range(WINDOW):
            r = int(win_rows[w * WINDOW + slot])
            if r < 0:
                continue
            for p in range(int(rowptr[r]), int(rowptr[r + 1])):
                key = (int(colind[p]), slot)
                entries[key] = entries.get(key, 0.0) + float(vals[p])
        cols = sorted({c for c, _ in entries})
        nblk = (len(cols) + VEC_PER_BLOCK - 1) // VEC_PER_BLOCK
        slot_of = {c: i for i, c in enumerate(cols)}
        wb = np.zeros((nblk, WINDOW, VEC_PER_BLOCK), dtype=np.float32)
        a = np.zeros(nblk * VEC_PER_BLOCK, dtype=np.int64)
        for c, i in slot_of.items():
            a[i] = c
        for (c, slot), v in entries.items():
            i = slot_of[c]
            wb[i // VEC_PER_BLOCK, slot, i % VEC_PER_BLOCK] = v
        atox.extend(a.tolist())
        blocks.extend(list(wb))
        block_offsets.append(block_offsets[-1] + nblk)
    out = {
        "win_rows": win_rows,
        "block_offsets": np.array(block_offsets, dtype=np.int64),
        "atox": np.array(atox, dtype=np.int64),
        "blocks": np.array(blocks, dtype=np.float32).reshape(-1, WINDOW, VEC_PER_BLOCK),
    }
    if kind == 2:
        seg_window, seg_bbegin, seg_bend, seg_slot = [], [], [], []
        split_wins, split_off = [], [0]
        slots = 0
        for w in range(W):
            b0, b1 = block_offsets[w], block_offsets[w + 1]
            if b1 - b0 <= SEG_BLOCKS:
                seg_window.append(w | SOLE_FLAG)
                seg_bbegin.append(b0)
                seg_bend.append(b1)
                seg_slot.append(-1)
            else:
                split_wins.append(w)
                for b in range(b0, b1, SEG_BLOCKS):
                    seg_window.append(w)
                    seg_bbegin.append(b)
                    seg_bend.append(min(b + SEG_BLOCKS, b1))
                    seg_slot.append(slots)
                    slots += 1
                split_off.append(slots)
        out.update({
            "seg_window": np.array(seg_window, dtype=np.int64),
            "seg_bbegin": np.array(seg_bbegin, dtype=np.int64),
            "seg_bend": np.array(seg_bend, dtype=np.int64),
            "seg_slot": np.array(seg_slot, dtype=np.int64),
            "split_windows": np.array(split_wins, dtype=np.int64),
            "split_offsets": np.array(split_off, dtype=np.int64),
        })
    return out


def tile_decode(fmt, M, K):
    """Dense M x K matrix from a tile_format() result (for decode == CSR checks)."""
    A = np.zeros((M, K), dtype=np.float64)
    bo = fmt["block_offsets"]
    for w in range(len(bo) - 1):
        for b in range(int(bo[w]), int(bo[w + 1])):
            for k in range(VEC_PER_BLOCK):
                c = int(fmt["atox"][b * VEC_PER_BLOCK + k])
                for slot in range(WINDOW):
                    v = fmt["blocks"][b, slot, k]
                    if v != 0.0:
                        r = int(fmt["win_rows"][w * WINDOW + slot])
                        A[r, c] += v
    return A


def merge_duplicates(rowptr, colind, vals):
    """CSR with repeated (row, column) entries summed in fp32, in CSR order
    (0 + v0 + v1 + ...), the first occurrence keeping its position: what a
    tile plan stores before rounding (tc/ra_tc_direct.cu:654-706 writes every
    duplicate into one fragment slot; the plan here sums them).  Pinned in
    tests/test_oracle_structures.py against a dense accumulation."""
    rowptr = np.asarray(rowptr, dtype=np.int64)
    colind = np.asarray(colind, dtype=np.int64)
    vals = np.asarray(vals, dtype=np.float32)
    M = len(rowptr) - 1
    out_rp, out_ci, out_v = [0], [], []
    for r in range(M):
        seen = {}
        for p in range(int(rowptr[r]), int(rowptr[r + 1])):
            c = int(colind[p])
            if c in seen:
                out_v[seen[c]] = np.float32(out_v[seen[c]] + vals[p])
            else:
                seen[c] = len(out_v)
                out_ci.append(c)
                out_v.append(np.float32(np.float32(0.0) + vals[p]))
        out_rp.append(len(out_ci))
    return (np.array(out_rp, dtype=np.int32), np.array(out_ci, dtype=np.int32),
            np.array(out_v, dtype=np.float32))


def spmm_tile_f64(rowptr, colind, vals, B, route: str):
    """Exact value of a tile path's output: vals quantised like the plan
    (fp16 with the plan's power-of-two scale for F16 and FP32 routes, bf16 for
    BF16), B quantised like the route
    (fp16 / bf16 / unchanged), fp64 accumulation.  The reference FP16 path
    computes the same products exactly (fp16 x fp16 is exact in fp32) and
    differs only in fp32 summation order (tc/ra_tc_direct.cu:109-179).
    Duplicate (row, column) entries are summed first (merge_duplicates)."""
    sc = tile_value_scale_log2(vals)  # from the stored entries, before merging
    rowptr, colind, vals = merge_duplicates(rowptr, colind, vals)
    if route == "f16":
        qv, qb = quantize_f16_scaled(vals, sc), quantize_f16(B)
    elif route == "bf16":
        qv, qb = quantize_bf16(vals), quantize_bf16(B)
    elif route == "fp32":
        qv, qb = quantize_f16_scaled(vals, sc), np.asarray(B, dtype=np.float32)
    elif route == "tf32_reference":
        qv, qb = quantize_f16(vals), quantize_tf32_rna(B)
    else:
        raise ValueError(route)
    return spmm_f64(rowptr, colind, qv, qb)
