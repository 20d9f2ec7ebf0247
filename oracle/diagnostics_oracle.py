"""Pure-Python restatement of the reference's diagnostic feature extractor —
TEST INFRASTRUCTURE ONLY (imported by tests/, never by the product).

Follows compute_router_features, router/router_features.cpp:113-432, step by
step: row proxies (:131-159), degree statistics (:161-196), 16x16 tile fills
through a dict of tile counts (:198-249), adjacent-row Jaccard similarity in
natural and reordered order (:251-287), 16-row window scores (:289-366) and
the composite proxies (:368-430).  float arithmetic is emulated with numpy
float32 scalars (one rounding per operation, no fused multiply-add), double
arithmetic with Python floats, so the results are comparable bit for bit.
Pinned in tests/test_diagnostics.py by closed forms on structured matrices
(identity, dense block, single row, banded) besides the comparison with the
library.  Small matrices only (pure-Python loops).
"""
import math

import numpy as np

F = np.float32
KEYS = (
    "avg_nnz_per_row", "std_nnz_per_row", "degree_cv", "max_to_mean_ratio", "frac_dense_rows",
    "skew_ratio", "long_row_fraction", "long_row_nnz_fraction", "top_1_row_nnz_fraction",
    "top_5_row_nnz_fraction", "tile_fill_mean", "tile_fill_median", "tile_fill_p90", "tile_fill_max",
    "tile_fill_variance", "tile_occupancy", "actual_nnz_coverage", "avg_nnz_per_tile",
    "row_window_colspan_compactness", "local_row_similarity_proxy", "reordered_locality_proxy",
    "locality_gain_proxy", "locality_selectivity_proxy", "road_likeness_proxy",
    "row_split_affinity_proxy", "mixedness_proxy", "tc_candidate_ratio", "tc_synergy_proxy",
    "estimated_tc_partition_ratio", "estimated_cuda_partition_ratio", "irregular_window_fraction",
    "tc_granularity_proxy", "redundancy_risk_proxy",
)


def _clamp01(x):
    return F(max(F(0.0), min(F(1.0), F(x))))


def _safe_div(n, d):
    return F(F(n) / F(d)) if abs(F(d)) > F(1e-6) else F(0.0)


def _safe_mean(vals):
    if not vals:
        return F(0.0)
    s = 0.0
    for v in vals:
        s += float(v)
    return F(s / len(vals))


def _jaccard(a, b):
    u = bin(a | b).count("1")
    return F(0.0) if u == 0 else F(F(bin(a & b).count("1")) / F(u))


def analyze_reference(rowptr, colind, M, K, N):
    """router/router_features.cpp:113-432 -> dict of the analyze_matrix keys."""
    rowptr = [int(x) for x in rowptr]
    colind = [int(x) for x in colind]
    out = {k: F(0.0) for k in KEYS}
    out["tc_candidate_tiles"] = 0
    if M <= 0 or K <= 0:
        return out
    nnz = rowptr[M]
    out["nnz"] = nnz
    if nnz <= 0:
        return out
    proxies = []
    lens = []
    sum_lens = 0.0
    max_len = 0
    for r in range(M):
        s, e = rowptr[r], rowptr[r + 1]
        ln = e - s
        lens.append(ln)
        sum_lens += ln
        max_len = max(max_len, ln)
        wsum = 0.0
        sig = 0
        for p in range(s, e):
            c = colind[p]
            wsum += float(c)
            sig |= 1 << min(63, (c * 64) // max(1, K))
        proxies.append({"len": ln, "min": colind[s] if ln > 0 else 0, "max": colind[e - 1] if ln > 0 else 0,
                        "sig": sig, "centroid": F(wsum / ln) if ln > 0 else F(0.0)})
    avg = sum_lens / M
    var = 0.0
    dense = long_rows = long_nnz = 0
    thr = max(32.0, 2.0 * avg)
    for ln in lens:
        var += (ln - avg) * (ln - avg)
        dense += ln > 2.0 * avg
        if ln >= thr:
            long_rows += 1
            long_nnz += ln
    sd = math.sqrt(var / max(1, M))
    srt = sorted(lens, reverse=True)
    top1, top5 = srt[0], sum(srt[:5])
    o = out
    o["avg_nnz_per_row"] = F(avg)
    o["std_nnz_per_row"] = F(sd)
    o["degree_cv"] = F(sd / avg) if avg > 1e-6 else F(0.0)
    o["max_to_mean_ratio"] = F(max_len / avg) if avg > 1e-6 else F(0.0)
    o["frac_dense_rows"] = F(F(dense) / F(max(1, M)))
    o["skew_ratio"] = o["max_to_mean_ratio"]
    o["long_row_fraction"] = F(F(long_rows) / F(max(1, M)))
    o["long_row_nnz_fraction"] = F(F(long_nnz) / F(max(1, nnz)))
    o["top_1_row_nnz_fraction"] = F(F(top1) / F(max(1, nnz)))
    o["top_5_row_nnz_fraction"] = F(F(top5) / F(max(1, nnz)))

    tiles = {}
    tile_rows, tile_cols = (M + 15) // 16, (K + 15) // 16
    for r in range(M):
        for p in range(rowptr[r], rowptr[r + 1]):
            key = (r // 16) * tile_cols + colind[p] // 16
            tiles[key] = tiles.get(key, 0) + 1
    fills = []
    cand_nnz = 0
    for cnt in tiles.values():
        fill = F(F(cnt) / F(256))
        fills.append(fill)
        if fill >= F(0.25):
            cand_nnz += cnt
    fills.sort()
    fm = _safe_mean(fills)
    fv = 0.0
    for x in fills:
        fv += (float(x) - float(fm)) ** 2
    fv = fv / len(fills) if fills else 0.0
    nt = len(fills)
    o["tile_fill_mean"] = fm
    o["tile_fill_median"] = fills[nt // 2]
    o["tile_fill_p90"] = fills[min(nt - 1, (nt * 9) // 10)]
    o["tile_fill_max"] = fills[-1]
    o["tile_fill_variance"] = F(fv)
    o["tile_occupancy"] = F(F(nt) / F(max(1, tile_rows * tile_cols)))
    o["actual_nnz_coverage"] = F(F(cand_nnz) / F(max(1, nnz)))
    o["avg_nnz_per_tile"] = F(F(nnz) / F(nt))
    cand = sum(1 for x in fills if x >= F(0.25))
    o["tc_candidate_tiles"] = cand
    o["tc_candidate_ratio"] = F(F(cand) / F(nt))

    sims = [_jaccard(proxies[r - 1]["sig"], proxies[r]["sig"]) for r in range(1, M)
            if proxies[r - 1]["len"] and proxies[r]["len"]]
    o["local_row_similarity_proxy"] = _safe_mean(sims)

    def sort_key(i):
        x = proxies[i]
        bucket = int(F(F(x["centroid"] * F(16.0)) / F(K)))
        span = x["max"] - x["min"] + 1 if x["len"] > 0 else K
        return (bucket, span, -x["len"])
    order = sorted(range(M), key=sort_key)  # Python's sort is stable
    rs = [_jaccard(proxies[order[i - 1]]["sig"], proxies[order[i]]["sig"]) for i in range(1, M)
          if proxies[order[i - 1]]["len"] and proxies[order[i]]["len"]]
    o["reordered_locality_proxy"] = _safe_mean(rs)

    comp, wsim, wirr = [], [], []
    tc_nnz = cuda_nnz = irregular = 0
    for base in range(0, M, 16):
        end = min(M, base + 16)
        wn = 0
        lo, hi = K, -1
        mx = 0
        ssum = F(0.0)
        sn = 0
        for r in range(base, end):
            x = proxies[r]
            wn += x["len"]
            mx = max(mx, x["len"])
            if x["len"] > 0:
                lo = min(lo, x["min"])
                hi = max(hi, x["max"])
            if r > base and proxies[r - 1]["len"] > 0 and x["len"] > 0:
                ssum = F(ssum + _jaccard(proxies[r - 1]["sig"], x["sig"]))
                sn += 1
        alen = F(F(wn) / F(max(1, end - base)))
        lthr = max(F(32.0), F(F(2.5) * alen))
        wl = sum(proxies[r]["len"] for r in range(base, end) if F(proxies[r]["len"]) >= lthr)
        span = hi - lo + 1 if hi >= lo else K
        c = F(F(wn) / F(max(1, (end - base) * max(1, span))))
        sim = F(ssum / F(sn)) if sn > 0 else F(0.0)
        aspan = max(16, ((span + 15) // 16) * 16)
        dens = F(F(wn) / F(max(16, (end - base) * aspan)))
        cn = _clamp01(F(c * F(6.0)))
        dn = _clamp01(F(dens * F(10.0)))
        un = _clamp01(F(F(1.0) - _safe_div(F(mx), F(F(F(4.0) * alen) + F(1.0)))))
        lm = _safe_div(F(wl), F(max(1, wn)))
        comp.append(c)
        wsim.append(sim)
        tcs = F(F(F(F(F(0.35) * cn) + F(F(0.30) * sim)) + F(F(0.20) * dn)) + F(F(0.15) * un))
        irr = F(F(F(F(F(0.40) * lm) + F(F(0.25) * _clamp01(F(_safe_div(F(mx), F(alen + F(1.0))) / F(6.0)))))
                    + F(F(0.20) * F(F(1.0) - cn))) + F(F(0.15) * F(F(1.0) - sim)))
        wirr.append(irr)
        if alen >= F(8.0) and tcs >= F(0.55) and irr < F(0.45):
            tc_nnz += wn
        if irr >= F(0.50) or lm >= F(0.20):
            cuda_nnz += wn
            irregular += 1
    o["row_window_colspan_compactness"] = _safe_mean(comp)
    wsm, wim = _safe_mean(wsim), _safe_mean(wirr)

    def lin(*terms):  # left-to-right float sum of products w*x
        acc = F(terms[0] * terms[1])
        for i in range(2, len(terms), 2):
            acc = F(acc + F(terms[i] * terms[i + 1]))
        return acc

    o["tc_synergy_proxy"] = lin(F(0.35), _clamp01(F(o["tile_fill_mean"] / F(0.20))), F(0.25), o["tc_candidate_ratio"],
                                F(0.20), o["reordered_locality_proxy"], F(0.20), o["row_window_colspan_compactness"])
    o["locality_gain_proxy"] = _clamp01(F(o["reordered_locality_proxy"] - o["local_row_similarity_proxy"]))
    ordered = _clamp01(F(o["local_row_similarity_proxy"] * _clamp01(F(o["row_window_colspan_compactness"] * F(2.0)))))
    o["locality_selectivity_proxy"] = _clamp01(F(o["locality_gain_proxy"] * F(F(1.0) - ordered)))
    road = F(o["local_row_similarity_proxy"] * _clamp01(F(F(1.0) - F(o["degree_cv"] / F(0.35)))))
    road = F(road * _clamp01(F(F(1.0) - F(o["avg_nnz_per_row"] / F(24.0)))))
    road = F(road * _clamp01(F(o["row_window_colspan_compactness"] / F(0.25))))
    o["road_likeness_proxy"] = _clamp01(road)
    skew = lin(F(0.45), _clamp01(F(F(o["skew_ratio"] - F(2.0)) / F(6.0))), F(0.30), o["long_row_nnz_fraction"],
               F(0.15), _clamp01(F(o["top_1_row_nnz_fraction"] / F(0.0020))),
               F(0.10), _clamp01(F(o["top_5_row_nnz_fraction"] / F(0.0100))))
    n_scale = _clamp01(F(F(F(N) - F(128.0)) / F(384.0)))
    dense_b = F(_clamp01(F(o["avg_nnz_per_row"] / F(192.0))) * F(F(0.35) + F(F(0.65) * n_scale)))
    o["row_split_affinity_proxy"] = _clamp01(max(skew, dense_b))
    o["estimated_tc_partition_ratio"] = _clamp01(F(F(tc_nnz) / F(max(1, nnz))))
    o["estimated_cuda_partition_ratio"] = _clamp01(F(F(cuda_nnz) / F(max(1, nnz))))
    o["irregular_window_fraction"] = F(F(irregular) / F(max(1, (M + 15) // 16)))
    t, c = o["estimated_tc_partition_ratio"], o["estimated_cuda_partition_ratio"]
    bal = _safe_div(F(F(2.0) * min(t, c)), F(F(t + c) + F(1e-6)))
    o["mixedness_proxy"] = _clamp01(F(bal * _clamp01(F(F(t + c) / F(0.60)))))
    o["tc_granularity_proxy"] = lin(F(0.55), _clamp01(F(o["avg_nnz_per_row"] / F(64.0))), F(0.45),
                                    _clamp01(F(F(F(1.0) - o["long_row_fraction"])
                                               + F(F(0.5) * o["locality_selectivity_proxy"]))))
    o["redundancy_risk_proxy"] = _clamp01(lin(F(0.45), o["long_row_nnz_fraction"],
                                              F(0.30), F(F(1.0) - o["row_window_colspan_compactness"]),
                                              F(0.15), F(F(1.0) - wsm), F(0.10), wim))
    return o
