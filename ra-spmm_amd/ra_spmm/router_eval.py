"""Router quality against the per-point fastest kernel (the oracle).

Reference: ra_router_eval.py:130-320 (the router-quality evaluation over a
kernel timing table).  Input here is the row list ``bench.py --sweep`` writes
(one row per graph, width and path, with the graph's float32 routing features
``d``, ``cv``, ``M``), so any threshold table can be scored offline against
one measured sweep.

Definitions, per (graph, N) point:
  * candidates: the deployed labels (``KERNELS``) whose output passed the
    harness's correctness gate, plus ``CUSPARSE``, the guardrail label, which
    on this build runs the hand-written baseline CSR kernel (``CSR_BASELINE``
    rows);
  * oracle: the fastest candidate; vendor: rocSPARSE's fastest algorithm
    (``ROCSPARSE`` rows), the yardstick every speed-up is quoted against;
  * router: the label ``route_with_rules`` picks from the point's features;
  * hit: the router's time equals the oracle's (the reference's deployed hit,
    router speed-up >= oracle speed-up); kernel hit: the same label;
  * ratio: oracle time / router time (<= 1), summarised as a geomean.
"""
from __future__ import annotations

import argparse
import json
import math
from collections import defaultdict

from .router import TABLES, route_with_rules

KERNELS = ("CSR_DIRECT", "ZERO_OVERHEAD_CSR", "TC_DIRECT", "COMMUNITY_TC", "SEGMENT_HYBRID",
           "TC_DIRECT_TF32", "COMMUNITY_TC_TF32", "SEGMENT_HYBRID_TF32")
GUARDRAIL = "CUSPARSE"

__all__ = ["KERNELS", "points_from_sweep", "rows_from_csv", "evaluate", "format_report", "main"]


def _geomean(xs):
    xs = [x for x in xs if x > 0]
    return math.exp(sum(math.log(x) for x in xs) / len(xs)) if xs else 0.0


def points_from_sweep(rows, time_key: str = "ms"):
    """Sweep rows -> {(graph, N): {"times": {label: ms}, "vendor_ms", "d", "cv", "M"}}.
    Rows failing the correctness gate are left out, as the reference drops
    incorrect kernels (ra_real_graph_eval.py:481-489)."""
    pts = defaultdict(lambda: {"times": {}})
    for r in rows:
        key = (r["config"], int(r["N"]))
        p = pts[key]
        for f in ("d", "cv", "M", "nnz"):
            if f in r:
                p[f] = r[f]
        path = r["path"]
        if path == "ROCSPARSE":
            p["vendor_ms"] = float(r["ms"])
        elif path == "CSR_BASELINE":
            p["times"][GUARDRAIL] = float(r[time_key])
        elif path in KERNELS and r.get("gate_ok", True):
            p["times"][path] = float(r[time_key])
    return dict(pts)


def rows_from_csv(graphs_csv, times_csv):
    """The row list of a sweep kept as two CSV files (graph features; times),
    the form the calibration sweep is committed in."""
    import csv

    def read(path):
        with open(path) as f:
            return list(csv.DictReader(line for line in f if not line.startswith("#")))
    graphs = {g["config"]: g for g in read(graphs_csv)}
    rows = []
    for t in read(times_csv):
        g = graphs[t["config"]]
        rows.append({"config": t["config"], "N": int(t["N"]), "path": t["path"], "ms": float(t["ms"]),
                     "gate_ok": t["gate_ok"] != "0", "M": int(g["M"]), "nnz": int(g["nnz"]),
                     "d": float(g["d"]), "cv": float(g["cv"])})
    return rows


def evaluate(points, table="mi355x", near: float = 0.05):
    """Score `table` (a name in TABLES or a RouterTable) on `points`."""
    rows = []
    for (graph, N), p in sorted(points.items()):
        times = p["times"]
        if not times or "d" not in p:
            continue
        oracle = min(times, key=times.get)
        pick = route_with_rules(p["d"], p["cv"], p["M"], N, table=table)
        if pick not in times:
            raise KeyError(f"{graph} N={N}: no time for the router's pick {pick}")
        r_ms, o_ms = times[pick], times[oracle]
        vendor = p.get("vendor_ms")
        rows.append({"graph": graph, "N": N, "d": p["d"], "cv": p["cv"], "M": p["M"],
                     "router": pick, "router_ms": r_ms, "oracle": oracle, "oracle_ms": o_ms,
                     "ratio": o_ms / r_ms, "hit": r_ms <= o_ms, "kernel_hit": pick == oracle,
                     "near_hit": r_ms <= o_ms * (1.0 + near),
                     "router_vs_vendor": (vendor / r_ms) if vendor else None,
                     "oracle_vs_vendor": (vendor / o_ms) if vendor else None})
    n = len(rows)
    summary = {
        "points": n,
        "hits": sum(r["hit"] for r in rows),
        "kernel_hits": sum(r["kernel_hit"] for r in rows),
        "near_hits": sum(r["near_hit"] for r in rows),
        "near": near,
        "router_oracle_geomean": _geomean([r["ratio"] for r in rows]),
        "worst_ratio": min((r["ratio"] for r in rows), default=0.0),
        "router_vs_vendor_geomean": _geomean([r["router_vs_vendor"] for r in rows
                                              if r["router_vs_vendor"]]),
        "oracle_vs_vendor_geomean": _geomean([r["oracle_vs_vendor"] for r in rows
                                              if r["oracle_vs_vendor"]]),
    }
    return summary, rows


def format_report(summary, rows, misses_only: bool = True) -> str:
    s = summary
    out = [f"points {s['points']}  hits {s['hits']}/{s['points']}  kernel hits "
           f"{s['kernel_hits']}/{s['points']}  within {100 * s['near']:.0f}%: "
           f"{s['near_hits']}/{s['points']}",
           f"router/oracle geomean {s['router_oracle_geomean']:.4f}  worst {s['worst_ratio']:.3f}",
           f"vs rocSPARSE: router {s['router_vs_vendor_geomean']:.3f}x  oracle "
           f"{s['oracle_vs_vendor_geomean']:.3f}x"]
    for r in rows:
        if misses_only and r["hit"]:
            continue
        out.append(f"  {r['graph']:20s} N={r['N']:4d} d={r['d']:7.2f} cv={r['cv']:6.3f} "
                   f"router {r['router']:20s} {r['router_ms']:8.3f} ms  oracle {r['oracle']:20s} "
                   f"{r['oracle_ms']:8.3f} ms  ratio {r['ratio']:.3f}")
    return "\n".join(out)


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("sweep", nargs="*", help="JSON row lists written by bench.py --sweep-out")
    ap.add_argument("--csv", nargs=2, metavar=("GRAPHS", "TIMES"), default=None,
                    help="a sweep kept as two CSV files (graph features, times)")
    ap.add_argument("--table", default="mi355x", choices=sorted(TABLES))
    ap.add_argument("--all", action="store_true", help="list every point, not only misses")
    ap.add_argument("--output", default=None, help="write the per-point rows here (JSON)")
    args = ap.parse_args(argv)
    rows = rows_from_csv(*args.csv) if args.csv else []
    for path in args.sweep:
        with open(path) as f:
            rows += json.load(f)
    summary, pts = evaluate(points_from_sweep(rows), args.table)
    print(format_report(summary, pts, misses_only=not args.all))
    if args.output:
        with open(args.output, "w") as f:
            json.dump({"summary": summary, "points": pts}, f, indent=1)
    return summary


if __name__ == "__main__":
    main()
