"""The MI355X router table against its calibration sweep (27 graphs x 4
widths, every deployed path timed on one MI355X; tests/golden/router_sweep_*).

Pins the figures the table's comments and the design notes state: the hit
rate and router/oracle geomean of both tables, and the per-region winners each
MI355X knob was set from.  The sweep is measured data, so these are checks of
the calibration's arithmetic, not of GPU timing."""
from collections import Counter
from pathlib import Path

import pytest

from ra_spmm.router_eval import evaluate, points_from_sweep, rows_from_csv

GOLD = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module")
def points():
    return points_from_sweep(rows_from_csv(GOLD / "router_sweep_graphs.csv", GOLD / "router_sweep_times.csv"))


def _rule(p):
    # regions of the deployed tree (router/router_dispatch.cpp:1036-1094), thresholds of both tables
    d, cv, M = p["d"], p["cv"], p["M"]
    if cv >= 5.0:
        return 1
    if cv < 0.7:
        return 2
    if cv >= 3.0:
        return 3
    if d >= 40.0:
        return 4
    if M < 20000 and d >= 25.0:
        return 5
    if d >= 25.0 and cv >= 1.8:
        return 6
    if d < 9.0 and 1.1 <= cv <= 1.45 and M >= 250000:
        return 7
    return 8


def test_sweep_is_complete(points):
    assert len(points) == 108
    assert Counter(_rule(p) for p in points.values()) == {1: 12, 2: 24, 3: 16, 4: 12, 5: 8, 6: 8, 7: 8, 8: 20}
    for p in points.values():
        assert "CUSPARSE" in p["times"] and p.get("vendor_ms")


def test_mi355x_table_scores(points):
    mi, _ = evaluate(points, "mi355x")
    ref, _ = evaluate(points, "reference")
    assert mi["points"] == ref["points"] == 108
    assert mi["hits"] == 67 and ref["hits"] == 38
    assert round(mi["router_oracle_geomean"], 3) == 0.943
    assert round(ref["router_oracle_geomean"], 3) == 0.865
    assert mi["router_vs_vendor_geomean"] > ref["router_vs_vendor_geomean"]


def test_rule_regions_winners(points):
    """Rules 3, 5, 6: SEGMENT_HYBRID fastest on 26 of 32 points and within 19%
    elsewhere; rule 7: TC_DIRECT fastest on 5 of 8; rule 5's guardrail pick
    (the baseline kernel) 5-6.5x slower than the fastest path at N < 96."""
    sh_best = sh_points = 0
    worst = 1.0
    for p in points.values():
        t = p["times"]
        best = min(t, key=t.get)
        if _rule(p) in (3, 5, 6):
            sh_points += 1
            sh_best += best == "SEGMENT_HYBRID"
            worst = max(worst, t["SEGMENT_HYBRID"] / t[best])
    assert (sh_best, sh_points) == (26, 32) and worst < 1.19
    tc7 = [min(p["times"], key=p["times"].get) == "TC_DIRECT" for p in points.values() if _rule(p) == 7]
    assert sum(tc7) == 5 and len(tc7) == 8
    for (g, N), p in points.items():
        if _rule(p) == 5 and N < 96:
            t = p["times"]
            assert 5.0 <= t["CUSPARSE"] / min(t.values()) <= 6.5, (g, N)


def test_mi355x_table_on_held_out_graphs():
    """Ten held-out graphs (synthetic.HELDOUT: other sizes, degrees, skews,
    localities and seeds, one or more per region), never used to set a knob:
    the MI355X table keeps its advantage over the published thresholds."""
    pts = points_from_sweep(rows_from_csv(GOLD / "router_heldout_graphs.csv", GOLD / "router_heldout_times.csv"))
    assert len(pts) == 40
    mi, _ = evaluate(pts, "mi355x")
    ref, _ = evaluate(pts, "reference")
    assert (mi["hits"], mi["near_hits"]) == (17, 30) and (ref["hits"], ref["near_hits"]) == (8, 19)
    assert round(mi["router_oracle_geomean"], 3) == 0.951 and round(ref["router_oracle_geomean"], 3) == 0.846
