#!/usr/bin/env python3
"""Routed SpMM benchmark on one MI355X (driver contract: one JSON line on stdout).

Default workload = config C2: Chung-Lu power-law graph (M = 1e6, mean
degree 16, gamma 2.1, hubs), GCN-normalised fp32 values, dense B of 1e6 x 128
fp32 N(0,1) (synthetic, seeded), C = A @ B through the MI355X router.

  step      one routed SpMM over the whole matrix (plan built outside the timed
            region, inputs resident in HBM)
  value     warm GFLOP/s = 2 * nnz * N / (seconds per step)
  roofline  dominant kernel: algorithmic bytes per launch / its mean launch
            time from HIP events on the launch stream, against 8 TB/s
  cold      routing (GPU feature pass + decision) and plan build + first
            execution, each the mean of 10 repetitions
  cpu       cpu_baseline: torch.sparse CSR on all host threads (the CPU
            SpMM BASELINE names), full matrix; cpu_port: oracle/spmm_oracle.c
            sequential fma on one host core
  compare   the hand-written baseline CSR kernel and torch.sparse on the
            device (torch-ROCm's vendor sparse library) on the same inputs
  configs   every BASELINE config (C1..C5) at its own N and at N=128, each
            with its path, warm time, roofline, cold costs, comparators and
            torch.sparse CPU on a row sample; geomean speed-ups over them
  gcn       config 5's GCN training step, routed and on rocSPARSE

--config C1..C5 measures one config alone.  --sweep times every deployed path
on the chosen configs (calibration of the router table).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (ROOT / "ra-spmm_amd", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

HBM_PEAK_GBS = 8000.0
METRIC = "SpMM GFLOP/s (2*nnz*N) + % HBM roofline, warm and cold, N=128, 1 MI355X"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def bytes_alg(M, K, nnz, N, s_val=4, s_b=4, s_c=4):
    """Compulsory traffic: rowptr + (colind, vals) + B once + C once."""
    return 4 * (M + 1) + nnz * (4 + s_val) + K * N * s_b + M * N * s_c


def bytes_edgewise(M, nnz, N):
    """Reference byte model 12*nnz + 4*nnz*N + 4*M*N (ra_eval_utils.py:647-651)."""
    return 12 * nnz + 4 * nnz * N + 4 * M * N


def timed_steps(fn, steps, warmup):
    """W untimed steps, then exactly K steps bracketed by synchronize; returns
    (wall ms per step, event ms per step)."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(steps):
        fn()
    ev1.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    return wall, ev0.elapsed_time(ev1) / steps


def _cpu_csr(g, rows=None):
    """torch CPU CSR tensor of g (or of its first `rows` rows)."""
    import numpy as np
    import torch
    M = g.M if rows is None else rows
    rp = g.rowptr[: M + 1].astype(np.int64)
    e = int(rp[-1])
    return torch.sparse_csr_tensor(torch.from_numpy(rp), torch.from_numpy(g.colind[:e].astype(np.int64)),
                                   torch.from_numpy(g.vals[:e]), size=(M, g.K)), e


def torch_sparse_cpu(g, B_host, seconds, rows=None):
    """torch.sparse.mm on a CPU CSR tensor (the reference's named CPU SpMM,
    BASELINE config 1), all host threads, time-bounded repetitions."""
    import torch
    A, e = _cpu_csr(g, rows)
    torch.sparse.mm(A, B_host)  # warm (thread pool, MKL handles)
    reps, t_tot = 0, 0.0
    while t_tot < seconds and reps < 50:
        t0 = time.perf_counter()
        torch.sparse.mm(A, B_host)
        t_tot += time.perf_counter() - t0
        reps += 1
    N = int(B_host.shape[1])
    what = "full matrix" if rows is None else f"first {rows} of {g.M} rows (nnz {e}), all of B"
    return {"value": 2.0 * e * N * reps / t_tot / 1e9, "unit": "GFLOP/s",
            "cores": torch.get_num_threads(), "kind": "reference",
            "threads": torch.get_num_threads(), "affinity_cores": len(os.sched_getaffinity(0)),
            "sample": f"{what}, N={N}, {reps} repetitions in {t_tot:.2f} s: torch.sparse.mm on a CPU CSR "
                      f"tensor (fp32), the reference's named CPU SpMM, {torch.get_num_threads()} threads"}


def cpu_port(g, N, seconds=10.0):
    """oracle/spmm_oracle.c sequential fma on one host core (the CPU
    restatement of the reference's per-element chain)."""
    import numpy as np
    from oracle import oracle as O
    O.build()
    B = np.random.default_rng(7).standard_normal((g.K, N)).astype(np.float32)
    reps, t_tot = 0, 0.0
    while t_tot < seconds and reps < 20:
        t0 = time.perf_counter()
        O.spmm_seq_f32(g.rowptr, g.colind, g.vals, B)
        t_tot += time.perf_counter() - t0
        reps += 1
    return {"value": 2.0 * g.nnz * N * reps / t_tot / 1e9, "unit": "GFLOP/s", "cores": 1, "kind": "port",
            "sample": f"full matrix (M={g.M}, nnz={g.nnz}, N={N}) x {reps} repetitions, "
                      f"oracle/spmm_oracle.c sequential fma, 1 thread, {t_tot:.1f} s"}


def torch_sparse_gpu(rp, ci, vl, B, M, K, C_ref, steps):
    """torch.sparse.mm on a device CSR tensor: torch-ROCm's vendor sparse
    library SpMM (the counterpart of the reference's cuSPARSE guardrail).
    Returns its ms per call and its max error relative to |A||B| against C_ref."""
    import torch
    try:
        A = torch.sparse_csr_tensor(rp, ci, vl, size=(M, K))  # int32 indices, as the CSR arrives
        fn = lambda: torch.sparse.mm(A, B)  # noqa: E731
        C = fn()
        torch.cuda.synchronize()
        wall, ev = timed_steps(fn, steps, 2)
        import ra_spmm
        scale = ra_spmm.spmm_csr_baseline(rp, ci, vl.abs(), B.abs())
        err = float(((C - C_ref).abs() / (scale + 1e-30)).max())
        del A, C, scale
        return {"ms": wall, "event_ms": ev, "max_rel_err_vs_routed": err}
    except Exception as exc:  # reported, never hides a failure of the routed path
        return {"ms": None, "error": f"{type(exc).__name__}: {exc}"}


def rocsparse_gpu(rp, ci, vl, B, C_ref, steps):
    """rocSPARSE CSR SpMM (ra_spmm.vendor), every CSR algorithm timed on the
    same inputs; the fastest is the vendor comparator."""
    import torch
    import ra_spmm
    from ra_spmm import vendor
    out = {"algs": {}}
    scale = ra_spmm.spmm_csr_baseline(rp, ci, vl.abs(), B.abs())
    for alg in vendor.ALGS:
        try:
            C = torch.empty_like(C_ref)
            # Cold call: descriptors, buffer and preprocessing, then the first
            # compute, synchronised (the vendor library's counterpart of route +
            # plan build + first execution).  One untimed call first loads the
            # algorithm's code objects, as the routed path's cold legs do.
            v = vendor.RocsparseSpMM(rp, ci, vl, B, C, alg)
            v.run()
            v.close()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            v = vendor.RocsparseSpMM(rp, ci, vl, B, C, alg)
            v.run()
            torch.cuda.synchronize()
            cold = (time.perf_counter() - t0) * 1e3
            wall, ev = timed_steps(v.run, steps, 2)
            err = float(((C - C_ref).abs() / (scale + 1e-30)).max())
            out["algs"][alg] = {"ms": wall, "event_ms": ev, "cold_ms": cold, "max_rel_err_vs_routed": err}
            v.close()
            del C, v
        except Exception as exc:  # an algorithm rocSPARSE rejects for this shape
            out["algs"][alg] = {"ms": None, "error": f"{type(exc).__name__}: {exc}"}
    ok = {a: r for a, r in out["algs"].items() if r.get("ms") and r["max_rel_err_vs_routed"] < 1e-3}
    if ok:
        best = min(ok, key=lambda a: ok[a]["ms"])
        out.update({"ms": ok[best]["ms"], "alg": best, "cold_ms": ok[best]["cold_ms"]})
    else:
        out["ms"] = None
    del scale
    return out


def gather_ceiling(ci, B, steps):
    """The gather probe (ra_spmm.measure) over this matrix's column indices in
    CSR order, and over as many uniform random indices: ms per pass and the
    rate of requested B bytes.  A row-gathering SpMM on the matrix moves at
    least these rows; the probe does nothing else."""
    import torch
    from ra_spmm import measure
    N = int(B.shape[1])
    if N % 4 or N > 256 or (N // 4) & (N // 4 - 1):
        return None
    out = {}
    gen = torch.Generator(device=B.device).manual_seed(99)
    uni = torch.randint(0, B.shape[0], (ci.numel(),), device=B.device, dtype=torch.int32, generator=gen)
    for name, idx in (("csr_order", ci), ("uniform", uni)):
        best = None
        for span in (32, 256):  # the faster walk is the ceiling
            p = measure.GatherProbe(B, idx, span)
            _, ev = timed_steps(p.run, steps, 3)
            if best is None or ev < best["ms"]:
                best = {"ms": ev, "requested_gbs": p.bytes / (ev * 1e-3) / 1e9, "span": span}
            del p
        out[name] = best
    del uni
    return out


def tile_gather_ceiling(plan, B, steps):
    """The gather probe over a tile plan's B-row stream: every (window,
    column) vector of the plan (`atox`, padding dropped) gathers its whole
    16-bit B row once, in plan order, with nothing else to do.  The MFMA
    kernels gather exactly these rows (in column slices) plus the A values,
    so the probe is the data-movement floor of the plan's B side."""
    import torch
    import ra_spmm
    from ra_spmm import measure
    N = int(B.shape[1])
    if N % 8 or (N // 8) & (N // 8 - 1) or not 32 <= N <= 512:
        return None
    atox = ra_spmm.export_tile_plan(plan, "atox")
    idx = atox[atox >= 0].to(device=B.device, dtype=torch.int32)
    B16 = B.half().contiguous().view(torch.float32)  # [K, N/2]: one fp32 lane word holds 2 fp16
    best = None
    for span in (32, 256):
        p = measure.GatherProbe(B16, idx, span)
        _, ev = timed_steps(p.run, steps, 3)
        if best is None or ev < best["ms"]:
            best = {"ms": ev, "requested_gbs": p.bytes / (ev * 1e-3) / 1e9, "span": span,
                    "gathers": int(idx.numel())}
        del p
    del idx, B16
    return {"plan_order": best}


def gather_sweep(out_path=None):
    """Bare-gather rate against the size of the gathered working set: uniform
    random rows of an fp32 [rows, N] matrix, 2^25 gathers per pass, one
    64-lane 16-byte-per-lane load per 1 KB at N=256.  L2-resident, Infinity
    Cache-resident and HBM-sized working sets give the gather ceilings the
    kernels' instruction rates are compared with (~2.4 GHz assumed for cycles)."""
    import torch
    from ra_spmm import measure
    rows_out = []
    for rows, N in [(2048, 256), (16384, 256), (65536, 256), (1 << 20, 256), (2048, 128), (2048, 64), (2048, 32)]:
        B = torch.randn(rows, N, device="cuda")
        n = 1 << 25
        gen = torch.Generator(device="cuda").manual_seed(rows + N)
        idx = torch.randint(0, rows, (n,), device="cuda", dtype=torch.int32, generator=gen)
        best = None
        for span in (32, 256):
            p = measure.GatherProbe(B, idx, span)
            _, ev = timed_steps(p.run, 10, 3)
            best = ev if best is None else min(best, ev)
            del p
        instr = n * N * 4 / 1024.0  # 64 lanes x 16 B
        rec = {"rows": rows, "N": N, "working_set_MB": rows * N * 4 / 1e6, "ms": best,
               "requested_TBps": n * N * 4 / (best * 1e-3) / 1e12,
               "cu_cycles_per_1KB_instr": 256 * best * 1e-3 * 2.4e9 / instr}
        rows_out.append(rec)
        log(f"[gather-sweep] {json.dumps(rec)}")
        del B, idx
    if out_path:
        Path(out_path).parent.mkdir(parents=True, exist_ok=True)
        Path(out_path).write_text(json.dumps(rows_out, indent=1))
    return rows_out


def kernel_time_ms(label, plan, rp, ci, vl, B, steps):
    """Mean launch time of the dominant kernel of `label`, HIP events on the
    current stream (the stream every ra_spmm launch uses)."""
    import torch
    import ra_spmm
    if label == "ZERO_OVERHEAD_CSR":
        C = torch.empty(rp.numel() - 1, B.shape[1], device=B.device)
        fn = lambda: ra_spmm._C.run_zero_overhead_plan_stage(plan, rp, ci, vl, B, C, 1)  # noqa: E731
        name = "zo_fused_kernel"
    elif label == "CSR_DIRECT":
        fn = lambda: ra_spmm.spmm_csr_direct(rp, ci, vl, B)  # noqa: E731
        name = "csr_rows_kernel"
    elif not label.endswith("_TF32") and B.shape[1] % 8 == 0:
        # The MFMA launches alone: the same plan on B already in 16-bit, so
        # the per-call conversion pass is left out (its bytes are not the
        # kernel's).  Column partitions make this one launch per range.
        Bh = B.half()  # build_kernel_plan stores fp16 values
        fn = lambda: ra_spmm.run_tile_plan_route(plan, Bh, "fp16")  # noqa: E731
        name = "tile_mfma_tall_kernel" if plan.rows_per_window in (16, 32) else "tile_mfma_kernel"
        m32 = os.environ.get("RA_TILE_MFMA32", "")
        if plan.rows_per_window == 32 and m32 != "0" and (B.shape[1] >= 512 or (m32 == "1" and B.shape[1] > 128)):
            name = "tile_mfma_tall32_kernel"  # the library's choice for 32-row windows at this width
    else:
        fn = lambda: ra_spmm.run_planned_kernel(label, plan, rp, ci, vl, B)  # noqa: E731
        name = "tile path (total)"
    _, ev = timed_steps(fn, steps, 5)
    return ev, name


def copy_probe(nbytes=1 << 30):
    """One device-to-device copy of a known size: the reference point that
    scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes."""
    import torch
    src = torch.ones(nbytes // 4, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    log(f"[bench] copy probe: {nbytes} bytes read + {nbytes} bytes written")
    del src, dst


def gather_probe(rows=1 << 20, width=128):
    """One gather of known size: every row of a [rows, width] fp32 matrix read
    once, in a random order (index_select over a permutation), and written
    once.  Scales rocprofv3 FETCH_SIZE for 512-byte random row gathers, the
    access pattern of the CSR kernels, as copy_probe does for streaming."""
    import torch
    src = torch.ones(rows, width, device="cuda")
    perm = torch.randperm(rows, device="cuda")
    torch.cuda.synchronize()
    out = torch.index_select(src, 0, perm)
    torch.cuda.synchronize()
    log(f"[bench] gather probe: {rows * width * 4} bytes gathered + {rows * 8} index bytes read, "
        f"{rows * width * 4} bytes written")
    del src, perm, out


def hbm_copy_gbs(nbytes=2 << 30, reps=10):
    """Device-to-device copy rate (bytes read + written per second, GB/s): the
    HBM bandwidth a streaming kernel reaches on this GPU, beside the 8 TB/s
    published peak the roofline is priced against."""
    import torch
    src = torch.ones(nbytes // 4, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    del src, dst
    return 2.0 * nbytes / (ms * 1e-3) / 1e9


def bench_config(cfg, N, steps, warmup, table, do_cpu, cold_reps=10, force_path=None, g=None,
                 cpu_seconds=10.0, cpu_rows=None, port=True):
    import numpy as np
    import torch
    import ra_spmm
    from ra_spmm import synthetic as S

    t0 = time.perf_counter()
    if g is None:
        S.use_device_sort("cuda")
        g = S.CONFIGS[cfg]()
    log(f"[bench] {cfg}: {g.name} M={g.M} nnz={g.nnz} generated in {time.perf_counter() - t0:.1f} s")
    rp, ci, vl = g.torch("cuda")
    gen = torch.Generator(device="cuda").manual_seed(1234)
    B = torch.randn(g.K, N, device="cuda", generator=gen)
    torch.cuda.synchronize()

    # Cold part (i): routing = GPU feature pass + rule tree.  One untimed call
    # first: it allocates the feature pass's per-device moment buffers once
    # per process, which no later routing call pays.
    ra_spmm.make_router_plan(rp, ci, vl, g.M, g.K, N, "MAIN", table)
    route_ms = []
    for _ in range(cold_reps):
        torch.cuda.synchronize()
        t = time.perf_counter()
        plan_dict = ra_spmm.make_router_plan(rp, ci, vl, g.M, g.K, N, "MAIN", table)
        route_ms.append((time.perf_counter() - t) * 1e3)
    label = force_path or ra_spmm.route_label(plan_dict)
    log(f"[bench] routed to {label} ({plan_dict['decision_reason']}), "
        f"d={plan_dict['feature_values']['avg_nnz_per_row']:.3f} "
        f"cv={plan_dict['feature_values']['degree_cv']:.3f}")

    # Cold part (ii): plan build + first execution.
    rp_cpu, ci_cpu, vl_cpu = rp.cpu(), ci.cpu(), vl.cpu()
    # As ra_real_graph_eval.py:322-335: each repetition builds, runs once and
    # drops its plan after the timed execution, so no build pays for freeing
    # the previous plan.  One untimed build + run first loads the build and
    # run kernels' code objects (loaded on first launch, once per process;
    # the first device binning takes ~3.5 ms, later ones ~0.3 ms).
    warm_plan = ra_spmm.build_kernel_plan(label, rp_cpu, ci_cpu, vl_cpu, g.M, g.K, N)
    ra_spmm.run_planned_kernel(label, warm_plan, rp, ci, vl, B)
    del warm_plan
    torch.cuda.synchronize()
    build_ms, first_ms = [], []
    for _ in range(cold_reps):
        torch.cuda.synchronize()
        t = time.perf_counter()
        plan = ra_spmm.build_kernel_plan(label, rp_cpu, ci_cpu, vl_cpu, g.M, g.K, N)
        torch.cuda.synchronize()
        build_ms.append((time.perf_counter() - t) * 1e3)
        out, ms = ra_spmm.measure_one_ms(lambda: ra_spmm.run_planned_kernel(label, plan, rp, ci, vl, B))
        first_ms.append(ms)
        del out, plan
        torch.cuda.synchronize()
    plan = ra_spmm.build_kernel_plan(label, rp_cpu, ci_cpu, vl_cpu, g.M, g.K, N)

    run = lambda: ra_spmm.run_planned_kernel(label, plan, rp, ci, vl, B)  # noqa: E731
    wall_ms, ev_ms = timed_steps(run, steps, warmup)
    C = run()
    flops = 2.0 * g.nnz * N
    gflops = flops / (wall_ms * 1e-3) / 1e9
    k_ms, k_name = kernel_time_ms(label, plan, rp, ci, vl, B, steps)
    ceiling = gather_ceiling(ci, B, max(5, steps // 4)) if k_name in ("zo_fused_kernel", "csr_rows_kernel") else None
    if k_name.startswith("tile_mfma"):
        ceiling = tile_gather_ceiling(plan, B, max(5, steps // 4))
    # the MFMA kernels read 16-bit B and stored values
    b_alg = bytes_alg(g.M, g.K, g.nnz, N, *((2, 2) if k_name.startswith("tile_mfma") else (4, 4)))

    # Comparators on the same inputs.
    base_wall, base_ev = timed_steps(lambda: ra_spmm.spmm_csr_baseline(rp, ci, vl, B), max(5, steps // 4), 2)
    cd_wall, cd_ev = timed_steps(lambda: ra_spmm.spmm_csr_direct(rp, ci, vl, B), max(5, steps // 4), 2)
    vendor = torch_sparse_gpu(rp, ci, vl, B, g.M, g.K, C, max(3, steps // 8))
    roc = rocsparse_gpu(rp, ci, vl, B, C, max(5, steps // 4))
    C_base = ra_spmm.spmm_csr_baseline(rp, ci, vl, B)
    scale = ra_spmm.spmm_csr_baseline(rp, ci, vl.abs(), B.abs())
    max_rel = float(((C - C_base).abs() / (scale + 1e-30)).max())

    res = {
        "config": cfg, "graph": g.name, "M": g.M, "K": g.K, "nnz": g.nnz, "N": N, "path": label,
        "decision_reason": plan_dict["decision_reason"],
        "avg_nnz_per_row": plan_dict["feature_values"]["avg_nnz_per_row"],
        "degree_cv": plan_dict["feature_values"]["degree_cv"],
        "ms_per_step": wall_ms, "event_ms_per_step": ev_ms, "gflops": gflops,
        "kernel": k_name, "kernel_ms": k_ms, "bytes_alg": b_alg,
        "bytes_edgewise": bytes_edgewise(g.M, g.nnz, N),
        "cold_route_ms": sum(route_ms) / len(route_ms),
        "cold_build_ms": sum(build_ms) / len(build_ms),
        "cold_first_exec_ms": sum(first_ms) / len(first_ms),
        "baseline_ms": base_wall, "baseline_gflops": flops / (base_wall * 1e-3) / 1e9,
        "csr_direct_ms": cd_wall, "csr_direct_gflops": flops / (cd_wall * 1e-3) / 1e9,
        "speedup_vs_baseline": base_wall / wall_ms,
        "max_rel_err_vs_baseline": max_rel,
        "torch_sparse_gpu": vendor,
        "speedup_vs_torch_sparse_gpu": (vendor["ms"] / wall_ms) if vendor.get("ms") else None,
        "gather_ceiling": ceiling,
        "rocsparse": roc,
        "speedup_vs_rocsparse": (roc["ms"] / wall_ms) if roc.get("ms") else None,
    }
    # The cold-aware deployed first call (the reference's deployed cold start,
    # experiments/deployed_coldstart.py): device feature pass + route, then a
    # path without a tile-format build, every overhead in, device CSR.
    ra_spmm.run_deployed_cold(rp, ci, vl, B, table)  # untimed: code objects
    dts = []
    for _ in range(cold_reps):
        torch.cuda.synchronize()
        t = time.perf_counter()
        out_d, dlab = ra_spmm.run_deployed_cold(rp, ci, vl, B, table)
        torch.cuda.synchronize()
        dts.append((time.perf_counter() - t) * 1e3)
        del out_d
    res["deployed_cold"] = {"path": dlab, "ms": sum(dts) / len(dts),
                            "speedup_vs_rocsparse": (roc["cold_ms"] / (sum(dts) / len(dts)))
                            if roc.get("cold_ms") else None}
    cold_total = res["cold_route_ms"] + res["cold_build_ms"] + res["cold_first_exec_ms"]
    res["cold_total_ms"] = cold_total
    res["cold_speedup_vs_rocsparse"] = (roc["cold_ms"] / cold_total) if roc.get("cold_ms") else None
    if label in ra_spmm.TILE_KERNELS and not label.endswith("_TF32") and N % 8 == 0:
        # Native 16-bit B (the fp16-B configs C3 and C4): the same plan run on
        # B already in fp16, with no per-call conversion pass; bytes_alg then
        # counts 2-byte B and stored values (s_B = s_val = 2).
        B16 = B.half()
        run16 = lambda: ra_spmm.run_tile_plan_route(plan, B16, "fp16")  # noqa: E731
        w16, e16 = timed_steps(run16, steps, warmup)
        b16 = bytes_alg(g.M, g.K, g.nnz, N, s_val=2, s_b=2)
        res["native_fp16_B"] = {
            "ms_per_step": w16, "event_ms_per_step": e16, "gflops": flops / (w16 * 1e-3) / 1e9,
            "bytes_alg": b16, "roofline_frac": b16 / (e16 * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "identical_to_fp32_B_call": bool(torch.equal(run16(), C)),
        }
        log(f"[bench] native fp16 B: {w16:.4f} ms/step, {res['native_fp16_B']['gflops']:.1f} GFLOP/s, "
            f"identical to the fp32-B call: {res['native_fp16_B']['identical_to_fp32_B_call']}")
        del B16
    if do_cpu:
        Bh = B.cpu()
        del B, C, C_base, scale
        torch.cuda.empty_cache()
        res["cpu_torch_sparse"] = torch_sparse_cpu(g, Bh, cpu_seconds, cpu_rows)
        if port:
            res["cpu_port"] = cpu_port(g, N)
    return res


# Per-config blocks of the default run: each config at its own width and at 128.
CONFIG_BLOCK_N = {"C1": (64, 128), "C2": (128,), "C3": (256, 128), "C4": (512, 128), "C5": (256, 128)}


def cpu_sample_rows(g, N, flops=4e9):
    """Rows of the CPU leg's sample: the first rows whose SpMM is ~`flops`
    (about 0.05-0.15 s per torch.sparse CPU call), or the whole matrix."""
    import numpy as np
    want = flops / (2.0 * N)
    if g.nnz <= want:
        return None
    return max(1, int(np.searchsorted(g.rowptr, want)))


def block_of(res):
    """The per-config summary the default JSON line carries."""
    frac = res["bytes_alg"] / (res["kernel_ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS
    ts = res.get("torch_sparse_gpu") or {}
    cpu = res.get("cpu_torch_sparse") or {}
    b = {
        "path": res["path"], "ms": round(res["ms_per_step"], 5), "gflops": round(res["gflops"], 2),
        # kernel_ms and bytes_alg are per SpMM call: every launch of the kernel
        # in one call (one per column partition of a tile plan)
        "roofline": {"kernel": res["kernel"], "kernel_ms": round(res["kernel_ms"], 5),
                     "bytes_alg": res["bytes_alg"], "frac": round(frac, 4), "per": "call"},
        "cold": {"route_ms": round(res["cold_route_ms"], 4), "build_ms": round(res["cold_build_ms"], 3),
                 "first_exec_ms": round(res["cold_first_exec_ms"], 4),
                 "rocsparse_cold_ms": round(res["rocsparse"]["cold_ms"], 4) if res["rocsparse"].get("cold_ms") else None,
                 "speedup_vs_rocsparse": round(res["cold_speedup_vs_rocsparse"], 3)
                 if res.get("cold_speedup_vs_rocsparse") else None,
                 "deployed_path": res["deployed_cold"]["path"],
                 "deployed_ms": round(res["deployed_cold"]["ms"], 4),
                 "deployed_speedup_vs_rocsparse": round(res["deployed_cold"]["speedup_vs_rocsparse"], 3)
                 if res["deployed_cold"].get("speedup_vs_rocsparse") else None},
        "baseline_kernel_ms": round(res["baseline_ms"], 5),
        "speedup_vs_baseline_kernel": round(res["speedup_vs_baseline"], 3),
        "rocsparse_ms": round(res["rocsparse"]["ms"], 5) if res["rocsparse"].get("ms") else None,
        "rocsparse_alg": res["rocsparse"].get("alg"),
        "speedup_vs_rocsparse": round(res["speedup_vs_rocsparse"], 3) if res.get("speedup_vs_rocsparse") else None,
        "torch_sparse_gpu_ms": round(ts["ms"], 5) if ts.get("ms") else None,
        "speedup_vs_torch_sparse_gpu": round(res["speedup_vs_torch_sparse_gpu"], 3)
        if res.get("speedup_vs_torch_sparse_gpu") else None,
        "max_rel_err_vs_baseline_kernel": res["max_rel_err_vs_baseline"],
        "cpu_torch_sparse_gflops": round(cpu["value"], 2) if cpu else None,
        "cpu_sample": cpu.get("sample"),
    }
    if ts.get("error"):
        b["torch_sparse_gpu_error"] = ts["error"]
    if res.get("gather_ceiling"):
        gc = next(iter(res["gather_ceiling"].values()))  # csr_order, or a tile plan's plan_order
        b["roofline"]["gather_probe_ms"] = round(gc["ms"], 5)
        b["roofline"]["frac_of_gather_probe"] = round(gc["ms"] / res["kernel_ms"], 4)
    if "native_fp16_B" in res:
        n16 = res["native_fp16_B"]
        b["native_fp16_B"] = {"ms": round(n16["ms_per_step"], 5), "gflops": round(n16["gflops"], 2),
                              "roofline_frac": round(n16["roofline_frac"], 4)}
    return b


def config_blocks(cfgs, table, steps, warmup, headline=None):
    """Every config of BASELINE at its own N and at N=128: routed path, warm
    time, roofline of the dominant kernel, cold costs, the baseline kernel and
    torch.sparse on the GPU as comparators, torch.sparse CPU on a row sample."""
    import math
    import torch
    from ra_spmm import synthetic as S
    S.use_device_sort("cuda")
    blocks = {}
    for cfg in cfgs:
        t0 = time.perf_counter()
        g = S.CONFIGS[cfg]()
        log(f"[bench] {cfg}: {g.name} M={g.M} nnz={g.nnz} generated in {time.perf_counter() - t0:.1f} s")
        for N in CONFIG_BLOCK_N[cfg]:
            if headline is not None and headline["config"] == cfg and headline["N"] == N:
                res = headline
            else:
                res = bench_config(cfg, N, steps, warmup, table, True, cold_reps=3, g=g,
                                   cpu_seconds=1.0, cpu_rows=cpu_sample_rows(g, N), port=False)
            blocks[f"{cfg}_N{N}"] = block_of(res)
            log(f"[bench] {cfg} N={N}: {json.dumps(blocks[f'{cfg}_N{N}'])}")
            torch.cuda.empty_cache()
        del g
        torch.cuda.empty_cache()

    def geomean(key):
        v = [b[key] for b in blocks.values() if b.get(key)]
        return round(math.exp(sum(math.log(x) for x in v) / len(v)), 3) if v else None
    def cold_geomean(key):
        v = [b["cold"][key] for b in blocks.values() if b["cold"].get(key)]
        return round(math.exp(sum(math.log(x) for x in v) / len(v)), 3) if v else None
    summary = {"geomean_speedup_vs_rocsparse": geomean("speedup_vs_rocsparse"),
               # first calls: the routed path with its plan build from host CSR
               # (the reference harness's cold protocol), and the cold-aware
               # deployed policy on device CSR
               "geomean_cold_speedup_vs_rocsparse": cold_geomean("speedup_vs_rocsparse"),
               "geomean_deployed_cold_speedup_vs_rocsparse": cold_geomean("deployed_speedup_vs_rocsparse"),
               "geomean_speedup_vs_baseline_kernel": geomean("speedup_vs_baseline_kernel"),
               "geomean_speedup_vs_torch_sparse_gpu": geomean("speedup_vs_torch_sparse_gpu"),
               "points": len(blocks)}
    return blocks, summary


def profile_traffic(kernel: str, cfg: str, N: int):
    """HBM bytes per launch of `kernel` on (cfg, N) from the committed rocprofv3
    summary profiles/<kernel>_<cfg>_N<N>.md (FETCH_SIZE + WRITE_SIZE, each
    scaled by a 1 GiB copy probe), or None when no summary exists."""
    path = ROOT / "profiles" / f"{kernel}_{cfg}_N{N}.md"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":", 1)[1])
    return None


def bench_gcn(steps, warmup, table, backends=("router", "router_cold", "rocsparse", "cusparse", "zero_overhead",
                                              "csr_direct"), order_auto=True, model="gcn"):
    """config C5: 2-layer GNN training step (128 -> 256 -> 47) on the
    synthetic power-law graph, forward A X and backward A^T G routed per
    (transpose, N).  model "gcn" (the config) runs on C5's GCN operator;
    "sage" and "gin" (gnn_bench/router_vs_baselines_{sage,gin}.py) on the same
    graph's mean and raw-sum operators.  Reports step time per backend and
    the routed paths."""
    import numpy as np
    import scipy.sparse as sp
    import torch
    from ra_spmm import gnn
    from ra_spmm import synthetic as S
    S.use_device_sort("cuda")
    if model == "gcn":
        g = S.CONFIGS["C5"]()
        op = sp.csr_matrix((g.vals, g.colind, g.rowptr), shape=(g.M, g.M))
    else:
        base = S.chung_lu(1_000_000, 25.0, 2.3, 50_000, seed=5)  # C5's graph before normalisation
        adj = sp.csr_matrix((np.ones(base.nnz, np.float32), base.colind, base.rowptr), shape=(base.M, base.M))
        op = gnn.build_aggregation_operator(adj, model)
        g = S.Graph(op.indptr.astype(np.int32), op.indices.astype(np.int32), op.data.astype(np.float32),
                    op.shape[0], op.shape[1], f"{model}_{base.name}")
        order_auto = False
    cls = gnn.MODELS[model]
    torch.manual_seed(0)
    X = torch.randn(g.M, 128, device="cuda")
    y = torch.randint(0, 47, (g.M,), device="cuda")
    widths = {"gcn": (256, 47), "sage": (128, 256), "graphsage": (128, 256), "gin": (128, 256)}[model]
    # forward SpMMs at both widths, backward A^T SpMMs where the operand takes a
    # gradient (every GCN layer; SAGE and GIN: not X)
    n_bwd = widths if model == "gcn" else widths[1:]
    out = {"model": model, "graph": g.name, "M": g.M, "nnz": g.nnz, "in": 128, "hidden": 256, "classes": 47,
           "spmm_flops_per_step": 2.0 * g.nnz * (sum(widths) + sum(n_bwd))}
    # Load the dense (GEMM, softmax, Adam) kernels once, so that the first
    # backend's cold step measures routing and plan builds, not library start-up.
    warm = gnn.GCN(128, 256, 47).cuda()
    wopt = torch.optim.Adam(warm.parameters(), lr=1e-2)
    for _ in range(2):
        wopt.zero_grad(set_to_none=True)
        gnn.cross_entropy(warm.lin2(torch.relu(warm.lin1(X)))[:, :47], y).backward()
        wopt.step()
    widths_val = (256, 47) if model == "gcn" else (128, 256)
    torch.cuda.synchronize()
    del warm, wopt
    for backend in backends:
        # Every backend is validated on this operator before it is timed, as
        # the reference does (gnn_bench/router_vs_baselines_gcn.py:413-446,
        # 566-567): each (transpose, N) SpMM of the step, N = 256 and 47,
        # against the baseline kernel with the harness's gate.
        val = gnn.validate_backend(op, "cuda", backend, widths_val, seed=0, table=table)
        torch.cuda.empty_cache()
        log(f"[gcn] {backend:14s} validation: correct={val['correct']} max_error={val['max_error']:.3e} "
            f"tolerance={val['tolerance']:.3e}")
        torch.manual_seed(1)
        graph = gnn.GraphBackend(op, "cuda", table)
        net = cls(128, 256, 47).cuda()
        opt = torch.optim.Adam(net.parameters(), lr=1e-2)
        cold = gnn.train_step(net, graph, backend, X, y, opt)
        for _ in range(warmup):
            gnn.train_step(net, graph, backend, X, y, opt)
        ts = [gnn.train_step(net, graph, backend, X, y, opt) for _ in range(steps)]
        ms = 1e3 * sum(ts) / len(ts)
        rec = {"step_ms": ms, "cold_first_step_ms": cold * 1e3,
               "validation": {k: val[k] for k in ("correct", "max_error", "tolerance")}}
        if backend == "router":
            rec["paths"] = {f"{'bwd' if t else 'fwd'}_N{n}": lab
                            for (b, t, n), (lab, _) in graph.exec_cache.items()}
        out[backend] = rec
        log(f"[gcn] {backend:14s} step {ms:8.3f} ms  cold first step {cold * 1e3:9.1f} ms "
            f"{rec.get('paths', '')}")
        del graph, net, opt
        torch.cuda.empty_cache()
    if "router" in backends and order_auto:
        # The same model with order="auto": layer 1 aggregates before its
        # linear map (SpMM at N=128, no backward SpMM).  Reported beside the
        # reference-order step, never in its place.
        torch.manual_seed(1)
        graph = gnn.GraphBackend(op, "cuda", table)
        net = gnn.GCN(128, 256, 47, order="auto").cuda()
        opt = torch.optim.Adam(net.parameters(), lr=1e-2)
        cold = gnn.train_step(net, graph, "router", X, y, opt)
        for _ in range(warmup):
            gnn.train_step(net, graph, "router", X, y, opt)
        ts = [gnn.train_step(net, graph, "router", X, y, opt) for _ in range(steps)]
        ms = 1e3 * sum(ts) / len(ts)
        out["router_order_auto"] = {"step_ms": ms, "cold_first_step_ms": cold * 1e3,
                                    "spmm_flops_per_step": 2.0 * g.nnz * (128 + 47 + 47)}
        log(f"[gcn] router order=auto step {ms:8.3f} ms  cold first step {cold * 1e3:9.1f} ms")
        del graph, net, opt
        torch.cuda.empty_cache()
    return out


def route_probe(cfgs=("C1", "C2"), N=128, reps=200, table="mi355x"):
    """Cold routing cost, broken down: make_router_plan on device tensors (GPU
    feature pass + rule tree + plan dict) and on host tensors, the feature
    pass alone, and the rule tree + dict alone (route_features).  Wall-clock
    means over `reps` calls, each call synchronised first as a cold caller is."""
    import torch
    import ra_spmm
    from ra_spmm import synthetic as S
    S.use_device_sort("cuda")
    out = {}
    for cfg in cfgs:
        g = S.CONFIGS[cfg]()
        rp, ci, vl = g.torch("cuda")
        hrp, hci, hvl = rp.cpu(), ci.cpu(), vl.cpu()
        f = ra_spmm.compute_features(rp, g.M, g.K, N)

        def mean_us(fn):
            fn()
            ts = []
            for _ in range(reps):
                torch.cuda.synchronize()
                t = time.perf_counter()
                fn()
                ts.append(time.perf_counter() - t)
            ts.sort()
            return {"mean_us": round(1e6 * sum(ts) / len(ts), 2), "median_us": round(1e6 * ts[len(ts) // 2], 2)}
        rec = {
            "make_router_plan_device": mean_us(lambda: ra_spmm.make_router_plan(rp, ci, vl, g.M, g.K, N, "MAIN", table)),
            "make_router_plan_host": mean_us(lambda: ra_spmm.make_router_plan(hrp, hci, hvl, g.M, g.K, N, "MAIN", table)),
            "features_device": mean_us(lambda: ra_spmm.compute_features(rp, g.M, g.K, N)),
            "features_host": mean_us(lambda: ra_spmm.compute_features(hrp, g.M, g.K, N)),
            "route_and_dict": mean_us(lambda: ra_spmm.route_features(g.M, g.K, N, f["nnz"], f["sum_deg_sq"],
                                                                     f["max_deg"], f["empty_rows"], "MAIN", table)),
        }
        out[f"{cfg}_N{N}"] = rec
        log(f"[route] {cfg} M={g.M}: {json.dumps(rec)}")
        del rp, ci, vl
    return out


def bf16x3_probe(cfgs=("C2", "C5"), Ns=(128, 256), steps=20, kind="COMMUNITY_TC"):
    """A stated-tolerance route for fp32 data on the MFMA kernels, measured
    before it is built: A = Ahi + Alo and B = Bhi + Blo with bf16 halves, and
    C ~ Ahi Bhi + Ahi Blo + Alo Bhi (the Alo Blo term, ~2^-16 relative, is
    dropped).  Here it is composed from three bf16 calls of the tile kernel
    plus two adds (an upper bound on a fused kernel's time). The fused
    kernel's gathers, a hi and a lo half of every B row, are the bytes of one
    16-bit call at 2N, which is timed as its estimate.  Error: elementwise
    |C - C64| / (|A||B|) against a float64 torch.sparse product on the GPU."""
    import torch
    import ra_spmm
    from ra_spmm import synthetic as S
    S.use_device_sort("cuda")
    make = {"COMMUNITY_TC": ra_spmm.make_community_tc_plan, "TC_DIRECT": ra_spmm.make_tc_direct_plan,
            "SEGMENT_HYBRID": ra_spmm.make_segment_hybrid_plan}[kind]
    out = {}
    for cfg in cfgs:
        g = S.CONFIGS[cfg]()
        rp, ci, vl = g.torch("cuda")
        vhi = vl.to(torch.bfloat16).float()
        vlo = (vl - vhi).to(torch.bfloat16).float()
        p_hi = make(rp, ci, vl, g.M, g.K, max(Ns), "bf16")
        p_lo = make(rp, ci, vlo, g.M, g.K, max(Ns), "bf16")
        A64 = torch.sparse_csr_tensor(rp.long(), ci.long(), vl.double(), size=(g.M, g.K))
        Aabs = torch.sparse_csr_tensor(rp.long(), ci.long(), vl.double().abs(), size=(g.M, g.K))
        zo = ra_spmm.make_zero_overhead_plan(rp.cpu(), g.M, g.K)
        for N in Ns:
            B = torch.randn(g.K, N, device="cuda", generator=torch.Generator(device="cuda").manual_seed(N))
            Bhi = B.to(torch.bfloat16)
            Blo = (B - Bhi.float()).to(torch.bfloat16)
            run = ra_spmm.run_tile_plan_route

            def three():
                return run(p_hi, Bhi, "bf16") + run(p_hi, Blo, "bf16") + run(p_lo, Bhi, "bf16")
            B2 = torch.cat([Bhi, Blo], dim=1).contiguous()
            t3, _ = timed_steps(three, steps, 3)
            t1, _ = timed_steps(lambda: run(p_hi, Bhi, "bf16"), steps, 3)
            t2n, _ = timed_steps(lambda: run(p_hi, B2, "bf16"), steps, 3)
            tzo, _ = timed_steps(lambda: ra_spmm.run_zero_overhead_plan(zo, rp, ci, vl, B), steps, 3)
            C = three().double()
            C64 = torch.sparse.mm(A64, B.double())
            scale = torch.sparse.mm(Aabs, B.double().abs())
            err3 = float(((C - C64).abs() / (scale + 1e-300)).max())
            C1 = run(p_hi, Bhi, "bf16").double()
            err1 = float(((C1 - C64).abs() / (scale + 1e-300)).max())
            rec = {"kind": kind, "bf16x3_three_calls_ms": round(t3, 4), "bf16x3_fused_estimate_ms": round(t2n, 4),
                   "bf16_one_call_ms": round(t1, 4), "zero_overhead_fp32_ms": round(tzo, 4),
                   "bf16x3_max_rel_err": err3, "bf16_max_rel_err": err1}
            out[f"{cfg}_N{N}"] = rec
            log(f"[bf16x3] {cfg} N={N}: {json.dumps(rec)}")
            del B, Bhi, Blo, B2, C, C64, scale, C1
            torch.cuda.empty_cache()
        del p_hi, p_lo, A64, Aabs, zo, rp, ci, vl, vhi, vlo
        torch.cuda.empty_cache()
    return out


def order_study(cfg="C4", heights=(8, 16, 32), g=None):
    """Host-side study (no GPU): B rows gathered by a tile plan (= vectors =
    distinct columns per window, summed over windows) under candidate row
    orders and window heights.  nnz / vectors is the nonzeros each gathered
    B row serves; the MFMA tile kernels are bound by the gathers."""
    import numpy as np
    from ra_spmm import synthetic as S
    if g is None:
        g = S.CONFIGS[cfg]()
    rp = g.rowptr.astype(np.int64)
    ci = g.colind.astype(np.int64)
    M = g.M
    deg = np.diff(rp)
    rows_of = np.repeat(np.arange(M), deg)
    ident = np.arange(M)
    lead = np.where(deg > 0, ci[np.minimum(rp[:-1], max(int(rp[-1]) - 1, 0))], np.iinfo(np.int64).max)
    indeg = np.bincount(ci, minlength=g.K)
    by_pop = np.lexsort((-indeg[ci], rows_of))  # within each row, most popular column first
    top = np.where(deg > 0, ci[by_pop[np.minimum(rp[:-1], max(int(rp[-1]) - 1, 0))]], -1)
    rng = np.random.default_rng(0)
    a, b = int(rng.integers(1, 2 ** 31 - 1)), int(rng.integers(0, 2 ** 31 - 1))
    mh = np.full(M, np.iinfo(np.int64).max)
    np.minimum.at(mh, rows_of, (a * ci + b) % 2147483647)
    # The diagnostic reorder of router/router_features.cpp:271-285: 16 buckets
    # of the mean column, then column span ascending, then length descending.
    csum = np.zeros(M)
    np.add.at(csum, rows_of, ci.astype(np.float64))
    bucket = np.where(deg > 0, (csum / np.maximum(deg, 1) * 16.0 / g.K).astype(np.int64), 0)
    lo = np.where(deg > 0, ci[np.minimum(rp[:-1], max(int(rp[-1]) - 1, 0))], 0)
    hi = np.where(deg > 0, ci[np.maximum(rp[1:] - 1, 0)], 0)
    span = np.where(deg > 0, hi - lo + 1, g.K)
    orders = {
        "identity (TC_DIRECT)": ident,
        "centroid bucket, span, length (diagnostic reorder)": np.lexsort((ident, -deg, span, bucket)),
        "leading column (COMMUNITY_TC)": np.lexsort((ident, lead)),
        "most popular column": np.lexsort((ident, top)),
        "minhash of the column set": np.lexsort((ident, mh)),
        "row length, descending": np.lexsort((ident, -deg)),
        "row length desc., then most popular column": np.lexsort((top, -deg)),
    }
    out = {"config": cfg, "nnz": g.nnz, "rows": {}}
    for name, order in orders.items():
        pos = np.empty(M, np.int64)
        pos[order] = np.arange(M)
        for H in heights:
            v = int(np.unique((pos[rows_of] // H) * g.K + ci).size)
            out["rows"][f"{name} | H={H}"] = {"gathered_rows": v, "nnz_per_gathered_row": round(g.nnz / v, 4)}
            log(f"[order] {name:45s} H={H:2d} gathered B rows {v:11d}  nnz per row {g.nnz / v:.3f}")
    return out


def sweep(configs, Ns, steps, out_path):
    """Every deployed path on each config (calibration of the MI355X table)."""
    import torch
    import ra_spmm
    from ra_spmm import synthetic as S
    from ra_spmm.router import production_features
    rows = []
    for cfg in configs:
        S.use_device_sort("cuda")
        g = S.CONFIGS[cfg]() if cfg in S.CONFIGS else S.REGIMES[cfg]() if cfg in S.REGIMES else S.HELDOUT[cfg]()
        feat = production_features(g.rowptr)
        rp, ci, vl = g.torch("cuda")
        host = (rp.cpu(), ci.cpu(), vl.cpu())  # plan builders take host CSR, as in the reference
        gdesc = {"M": g.M, "nnz": g.nnz, "d": feat["avg_nnz_per_row"], "cv": feat["degree_cv"],
                 "max_deg": feat["max_deg"]}
        log(f"[sweep] {cfg}: M={g.M} nnz={g.nnz} d={gdesc['d']:.3f} cv={gdesc['cv']:.4f}")
        for N in Ns:
            B = torch.randn(g.K, N, device="cuda")
            base = ra_spmm.spmm_csr_baseline(rp, ci, vl, B)
            scale = ra_spmm.spmm_csr_baseline(rp, ci, vl.abs(), B.abs())
            routed = ra_spmm.route_label(ra_spmm.make_router_plan(rp, ci, vl, g.M, g.K, N, "MAIN", "mi355x"))
            roc = rocsparse_gpu(rp, ci, vl, B, base, max(5, steps // 2))
            if roc.get("ms"):
                rows.append({"config": cfg, "N": N, "path": "ROCSPARSE", "ms": roc["ms"],
                             "gflops": 2.0 * g.nnz * N / (roc["ms"] * 1e-3) / 1e9, "alg": roc["alg"],
                             "routed": False, **gdesc})
                log(f"[sweep] {cfg} N={N:4d} {'ROCSPARSE':22s} {roc['ms']:9.3f} ms ({roc['alg']})")
            for label in ["CSR_BASELINE"] + ra_spmm.DEPLOYED_KERNELS:
                if label in ra_spmm.TILE_KERNELS and N < 16:
                    continue
                t = time.perf_counter()
                plan = ra_spmm.build_kernel_plan(label, *host, g.M, g.K, N)
                torch.cuda.synchronize()
                build = (time.perf_counter() - t) * 1e3
                fn = lambda: ra_spmm.run_planned_kernel(label, plan, rp, ci, vl, B)  # noqa: E731
                wall, ev = timed_steps(fn, steps, 3)
                out = fn()
                err = float(((out - base).abs() / (scale + 1e-30)).max())
                # The harness's gate (absolute, 1e-3 sqrt(max row nnz), x10 for the
                # tile paths): the elementwise relative error of a 16-bit path is
                # 1 wherever a B entry rounds to zero in a one-term row.
                gate = ra_spmm.correctness_gate(label, float((out - base).abs().max()),
                                                gdesc["max_deg"])
                del out
                row = {"config": cfg, "N": N, "path": label, "ms": wall, "event_ms": ev,
                       "gflops": 2.0 * g.nnz * N / (wall * 1e-3) / 1e9, "build_ms": build,
                       "max_rel_err_vs_baseline": err, "max_abs_err": gate["max_error"],
                       "gate_ok": gate["correct"], "routed": label == routed, **gdesc}
                rows.append(row)
                log(f"[sweep] {cfg} N={N:4d} {label:22s} {wall:9.3f} ms {row['gflops']:9.1f} GF/s "
                    f"build {build:8.1f} ms err {err:.2e} abs {gate['max_error']:.2e} "
                    f"{'ok' if gate['correct'] else 'GATE-FAIL'}")
                if label in ("TC_DIRECT", "COMMUNITY_TC", "SEGMENT_HYBRID") and cfg in ("C3", "C4") \
                        and N % 8 == 0:
                    # fp16-B configs: the native 16-bit-B entry, no conversion pass
                    B16 = B.half()
                    f16 = lambda: ra_spmm.run_tile_plan_route(plan, B16, "fp16")  # noqa: E731
                    w16, e16 = timed_steps(f16, steps, 3)
                    err16 = float(((f16() - base).abs() / (scale + 1e-30)).max())
                    rows.append({"config": cfg, "N": N, "path": label + "+B16", "ms": w16, "event_ms": e16,
                                 "gflops": 2.0 * g.nnz * N / (w16 * 1e-3) / 1e9, "build_ms": build,
                                 "max_rel_err_vs_baseline": err16, "routed": False, **gdesc})
                    log(f"[sweep] {cfg} N={N:4d} {label + '+B16':22s} {w16:9.3f} ms "
                        f"{rows[-1]['gflops']:9.1f} GF/s err {err16:.2e}")
                    del B16
                del plan
            del B
        del rp, ci, vl, host
        torch.cuda.empty_cache()
        if out_path:  # after every graph, so a cut-off run keeps what it measured
            Path(out_path).parent.mkdir(parents=True, exist_ok=True)
            Path(out_path).write_text(json.dumps(rows, indent=1))
    if out_path:
        Path(out_path).parent.mkdir(parents=True, exist_ok=True)
        Path(out_path).write_text(json.dumps(rows, indent=1))
    return rows


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--config", default=None, choices=["C1", "C2", "C3", "C4", "C5"],
                    help="measure this config alone (default: C2 as the headline, plus every config's block)")
    ap.add_argument("--configs", default=None,
                    help="comma-separated configs for the per-config blocks "
                         "(default: C1,C2,C3,C4,C5 when --config is not given)")
    ap.add_argument("--no-configs", action="store_true", help="headline line only, no per-config blocks")
    ap.add_argument("--no-gcn", action="store_true", help="leave the C5 GCN step out of the default run")
    ap.add_argument("--gather-sweep", action="store_true",
                    help="bare-gather rate against working-set size (details on stderr / --details)")
    ap.add_argument("--gather-probe", action="store_true",
                    help="run a random-row gather of known size first (PMC scale for gathers)")
    ap.add_argument("--N", type=int, default=128)
    ap.add_argument("--table", default="mi355x", choices=["mi355x", "reference"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--traffic", type=float, default=None,
                    help="HBM bytes per launch of the dominant kernel from rocprofv3 --pmc")
    ap.add_argument("--sweep", default=None, help="comma-separated configs (C1..C5, regime names, 'regimes' for the router "
                         "calibration suite, 'heldout' for its held-out graphs) to sweep all paths on")
    ap.add_argument("--sweep-N", default="64,128,256")
    ap.add_argument("--sweep-out", default=None, help="write the sweep rows here as JSON")
    ap.add_argument("--details", default=None, help="write the full result dict here")
    ap.add_argument("--path", default=None, help="force a kernel path instead of the router's pick")
    ap.add_argument("--order-study", default=None, choices=["C1", "C2", "C3", "C4", "C5"],
                    help="host-only: B rows a tile plan gathers under candidate row orders and heights")
    ap.add_argument("--bf16x3-probe", action="store_true",
                    help="time and error of a bf16x3 split route for fp32 data on C2 and C5")
    ap.add_argument("--route-probe", action="store_true",
                    help="cold routing cost (make_router_plan) broken down on C1 and C2")
    ap.add_argument("--copy-probe", action="store_true", help="run a 1 GiB copy first (PMC scale)")
    ap.add_argument("--gcn", action="store_true", help="config 5 GCN training step (details on stderr)")
    ap.add_argument("--gnn-model", default="gcn", choices=["gcn", "sage", "gin"],
                    help="model of --gcn: the config's GCN, or GraphSAGE / GIN on the same graph")
    ap.add_argument("--gcn-backends", default="router,router_cold,rocsparse,cusparse,zero_overhead,csr_direct",
                    help="comma-separated GraphBackend backends timed by --gcn")
    args = ap.parse_args(argv)

    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              f"(the SpMM shards by row blocks, see the sharding notes; run with --gpus 1)",
              file=sys.stderr)
        return 2
    if args.order_study:  # host only
        print(json.dumps({"order_study": order_study(args.order_study)}), flush=True)
        return 0
    import torch
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 3
    import ra_spmm
    if args.gcn:
        res = bench_gcn(max(5, args.steps // 20), max(2, args.warmup // 10), args.table,
                        tuple(args.gcn_backends.split(",")), model=args.gnn_model)
        if args.details:
            Path(args.details).parent.mkdir(parents=True, exist_ok=True)
            Path(args.details).write_text(json.dumps(res, indent=1))
        return 0
    if args.gather_sweep:
        gather_sweep(args.details)
        return 0
    if args.bf16x3_probe:
        print(json.dumps({"bf16x3_probe": bf16x3_probe()}), flush=True)
        return 0
    if args.route_probe:
        print(json.dumps({"route_probe": route_probe(table=args.table)}), flush=True)
        return 0
    if args.sweep:
        names = []
        for n in args.sweep.split(","):
            if n in ("regimes", "heldout"):  # the router calibration suite / its held-out graphs
                from ra_spmm import synthetic as S
                names += list(S.REGIMES if n == "regimes" else S.HELDOUT)
            else:
                names.append(n)
        sweep(names, [int(n) for n in args.sweep_N.split(",")], max(10, args.steps // 4),
              args.sweep_out)
        return 0

    if args.copy_probe:
        copy_probe()
    if args.gather_probe:
        gather_probe()
    cfg = args.config or "C2"
    res = bench_config(cfg, args.N, args.steps, args.warmup, args.table, not args.no_cpu,
                       force_path=args.path)
    blocks = summary = None
    cfgs = args.configs.split(",") if args.configs else ([] if args.config else list(CONFIG_BLOCK_N))
    if cfgs and not args.no_configs and not args.path:
        blocks, summary = config_blocks(cfgs, args.table, max(10, min(args.steps, 50)),
                                        max(2, min(args.warmup, 5)), headline=res)
    gcn = None
    if not args.config and not args.no_configs and not args.no_gcn:
        # Config 5's GCN training step, routed and on rocSPARSE (bench --gcn has every backend).
        g5 = bench_gcn(10, 3, args.table, ("router", "rocsparse"), order_auto=False)
        gcn = {"model": "2-layer GCN 128 -> 256 -> 47, 4 routed SpMMs per step", "graph": g5["graph"],
               "nnz": g5["nnz"], "router_step_ms": round(g5["router"]["step_ms"], 3),
               "router_cold_first_step_ms": round(g5["router"]["cold_first_step_ms"], 2),
               "router_paths": g5["router"]["paths"],
               "rocsparse_step_ms": round(g5["rocsparse"]["step_ms"], 3),
               "speedup_vs_rocsparse": round(g5["rocsparse"]["step_ms"] / g5["router"]["step_ms"], 3),
               # each backend checked at full size before it was timed
               "router_validation": g5["router"]["validation"],
               "rocsparse_validation": g5["rocsparse"]["validation"]}
    achieved = res["bytes_alg"] / (res["kernel_ms"] * 1e-3) / 1e9
    copy_gbs = hbm_copy_gbs()
    traffic = args.traffic if args.traffic is not None else profile_traffic(res["kernel"], cfg, res["N"])
    l2_miss_gbs = traffic / (res["kernel_ms"] * 1e-3) / 1e9 if traffic else None
    gather_ms = next(iter(res["gather_ceiling"].values()))["ms"] if res.get("gather_ceiling") else None
    line = {
        "metric": METRIC, "value": round(res["gflops"], 3), "unit": "GFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(res["ms_per_step"], 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded generator, ra_spmm.synthetic)",
        "config": {"workload": f"{cfg} {res['graph']} M={res['M']} nnz={res['nnz']} "
                               f"N={res['N']} fp32, routed ({res['path']})",
                   "N": res["N"], "router_table": args.table},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     # the north star's bar for the CSR regimes, and the fraction a
                     # kernel running at the gather probe's time would reach: the
                     # gap between frac and target_frac is not closed
                     "target_frac": 0.6,
                     "gather_ceiling_ms": round(gather_ms, 5) if gather_ms else None,
                     "frac_at_gather_ceiling": round(res["bytes_alg"] / (gather_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
                     if gather_ms else None,
                     # bytes per launch of the named kernel (the path is one launch
                     # of it per SpMM call)
                     "traffic": traffic, "traffic_unit": "bytes per launch", "kernel": res["kernel"],
                     "kernel_ms": round(res["kernel_ms"], 5), "bytes_alg": res["bytes_alg"],
                     # rocprofv3 FETCH_SIZE + WRITE_SIZE per launch counts the L2's
                     # requests to the fabric, which the 256 MB Infinity Cache (MALL)
                     # serves in part: it is L2-miss traffic, not HBM bytes.  Its rate
                     # is set beside the HBM peak only for scale.
                     "l2_miss_traffic_gbs": round(l2_miss_gbs, 1) if traffic else None,
                     "l2_miss_traffic_over_hbm_peak": round(l2_miss_gbs / HBM_PEAK_GBS, 4)
                     if traffic else None,
                     "measured_copy_gbs": round(copy_gbs, 1),
                     # the same B rows gathered in the same order by a kernel that
                     # does nothing else: the data-movement ceiling on this matrix
                     "gather_probe": res.get("gather_ceiling"),
                     "frac_of_gather_probe": round(next(iter(res["gather_ceiling"].values()))["ms"] / res["kernel_ms"], 4)
                     if res.get("gather_ceiling") else None},
        "cpu_baseline": res.get("cpu_torch_sparse"),
        "cold": {"route_ms": round(res["cold_route_ms"], 4), "build_ms": round(res["cold_build_ms"], 3),
                 "first_exec_ms": round(res["cold_first_exec_ms"], 4),
                 # SpMM calls after which routing + plan build is repaid against
                 # CSR_DIRECT, which needs no plan.
                 "crossover_calls_vs_csr_direct": ra_spmm.smallest_strict_crossover(
                     0.0, res["csr_direct_ms"], res["cold_route_ms"] + res["cold_build_ms"],
                     res["ms_per_step"]),
                 # first call, cold, against rocSPARSE's cold first call (descriptors,
                 # buffer, preprocessing, first compute)
                 "total_ms": round(res["cold_total_ms"], 4),
                 "rocsparse_cold_ms": round(res["rocsparse"]["cold_ms"], 4) if res["rocsparse"].get("cold_ms") else None,
                 "speedup_vs_rocsparse": round(res["cold_speedup_vs_rocsparse"], 3)
                 if res.get("cold_speedup_vs_rocsparse") else None,
                 "deployed_path": res["deployed_cold"]["path"],
                 "deployed_ms": round(res["deployed_cold"]["ms"], 4),
                 "deployed_speedup_vs_rocsparse": round(res["deployed_cold"]["speedup_vs_rocsparse"], 3)
                 if res["deployed_cold"].get("speedup_vs_rocsparse") else None},
        "path": res["path"],
        "baseline_csr_gflops": round(res["baseline_gflops"], 3),
        "csr_direct_gflops": round(res["csr_direct_gflops"], 3),
        "speedup_vs_baseline_kernel": round(res["speedup_vs_baseline"], 4),
        "rocsparse": res.get("rocsparse"),
        "speedup_vs_rocsparse": round(res["speedup_vs_rocsparse"], 4) if res.get("speedup_vs_rocsparse") else None,
        "torch_sparse_gpu": res.get("torch_sparse_gpu"),
        "speedup_vs_torch_sparse_gpu": round(res["speedup_vs_torch_sparse_gpu"], 4)
        if res.get("speedup_vs_torch_sparse_gpu") else None,
        "edgewise_gbs": round(res["bytes_edgewise"] / (res["ms_per_step"] * 1e-3) / 1e9, 1),
        "max_rel_err_vs_baseline": res["max_rel_err_vs_baseline"],
        "cpu_port": res.get("cpu_port"),
    }
    if blocks is not None:
        line["configs"] = blocks
        line["configs_summary"] = summary
    if gcn is not None:
        line["gcn_step_C5"] = gcn
    if "native_fp16_B" in res:
        line["native_fp16_B"] = res["native_fp16_B"]
    if args.details:
        Path(args.details).parent.mkdir(parents=True, exist_ok=True)
        Path(args.details).write_text(json.dumps(res, indent=1))
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
