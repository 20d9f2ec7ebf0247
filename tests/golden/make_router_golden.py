"""Extract the reference's published routing decisions into a small fixture.

Run in the build container only (it reads /root/reference, which the GPU box
does not have).  Inputs are data files the reference ships:

  fgcs_results/revision/tf32/router_quality_v8.csv      192 (dataset, N) decisions, RTX 3090
  fgcs_results/revision/tf32/final_fair_v3.csv          per-graph avg_nnz_per_row, cv_d
  fgcs_results/revision/ada5/router_quality_ada_warm.csv the same 192 decisions on RTX 4090
  fgcs_results/revision/tf32/unseen/unseen_router_quality.csv  36 held-out decisions

Output: tests/golden/router_golden.csv with columns
  source,dataset,N,M,nnz,avg_nnz_per_row,cv_d,router_kernel
"""
import csv
import sys
from pathlib import Path

REF = Path("/root/reference/fgcs_results/revision")
OUT = Path(__file__).resolve().parent / "router_golden.csv"


def main():
    feats = {}
    with open(REF / "tf32" / "final_fair_v3.csv") as f:
        for r in csv.DictReader(f):
            feats[r["dataset"]] = (r["avg_nnz_per_row"], r["cv_d"])
    rows = []
    for source, path in (("tf32_v8", REF / "tf32" / "router_quality_v8.csv"),
                         ("ada5", REF / "ada5" / "router_quality_ada_warm.csv")):
        with open(path) as f:
            for r in csv.DictReader(f):
                d, cv = feats[r["dataset"]]
                rows.append([source, r["dataset"], r["N"], r["M"], r["nnz"], d, cv,
                             r["router_kernel"]])
    with open(REF / "tf32" / "unseen" / "unseen_router_quality.csv") as f:
        for r in csv.DictReader(f):
            rows.append(["unseen", r["dataset"], r["N"], r["M"], r["nnz"],
                         r["avg_nnz_per_row"], r["cv_d"], r["router_kernel"]])
    with open(OUT, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["source", "dataset", "N", "M", "nnz", "avg_nnz_per_row", "cv_d",
                    "router_kernel"])
        w.writerows(rows)
    print(f"wrote {len(rows)} rows to {OUT}", file=sys.stderr)


if __name__ == "__main__":
    main()
