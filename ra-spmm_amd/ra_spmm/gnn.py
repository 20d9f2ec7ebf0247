"""GNN call site of the routed SpMM: graph backend, autograd SpMM and GCN.

Reference: gnn_bench/router_vs_baselines_gcn.py — build_aggregation_operator
(:89-126), GraphBackend (:162-410), validate_backend (:413-445),
SparseMMFunction (:451-461), GCNBench (:464-476), measure_step (:482-498);
SAGEBench gnn_bench/router_vs_baselines_sage.py:48-67; GINBench
gnn_bench/router_vs_baselines_gin.py:47-73;
cold first-step policy gnn_bench/cold_first_step.py:61-139 (route, then run
a path without a tile-format build).

A GraphBackend owns the CSR of A and of A^T on the device, one router plan
per (transpose, N) and one executor (path label + plan) per
(backend, transpose, N).  Backends:
  "router"        MI355X router (default table), plan built on first use
  "router_cold"   first call per (transpose, N): feature pass + route, then
                  the cold-aware policy's path (dispatch.cold_path: CSR_DIRECT,
                  or ZERO_OVERHEAD_CSR binned on the GPU for skewed rows; no
                  tile-format build); later calls as "router"
  "cusparse"      the guardrail name, served by the baseline CSR kernel
  "csr_direct", "zero_overhead", "tc_direct", "tc_direct_tf32",
  "community_tc", "segment_hybrid"   fixed paths
  "torch"         torch.sparse CSR on the device (external comparison only)
  "rocsparse"     rocSPARSE's fastest CSR SpMM algorithm per (transpose, N),
                  the vendor-library comparison (ra_spmm.vendor)
"""
from __future__ import annotations

import math
import time
from typing import Dict, Tuple

import numpy as np
import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _C
from .dispatch import BASE_ATOL, TC_EXTRA_FACTOR, TILE_KERNELS, build_kernel_plan, cold_path, run_planned_kernel
from .router import route_label


_FIXED = {"csr_direct": "CSR_DIRECT", "zero_overhead": "ZERO_OVERHEAD_CSR",
          "tc_direct": "TC_DIRECT", "tc_direct_tf32": "TC_DIRECT_TF32",
          "community_tc": "COMMUNITY_TC", "segment_hybrid": "SEGMENT_HYBRID"}


_AGGREGATIONS = ("gcn", "sage", "graphsage", "gin")


def build_aggregation_operator(csr, model: str):
    """Aggregation matrix of a GNN layer as scipy CSR (fp32, sorted columns).

    gcn           W[i, j] = a~_ij / sqrt(deg~_i * deg~_j), where a~ is A with a
                  unit self-loop on every row whose diagonal entry is zero or
                  absent, and deg~ its row sums (rows of zero degree stay 0)
    sage          W[i, j] = a_ij / deg_i (row mean; empty rows stay zero)
    gin           W = A
    The gcn and sage operators store no zero entries (the reference forms
    them as sparse products, which drop zeros); gin keeps A's structure.
    Duplicate entries of A are summed first.  The matrix is built once, so
    every backend and the correctness reference consume the same operator
    (gnn_bench/router_vs_baselines_gcn.py:89-126)."""
    import scipy.sparse as sp
    kind = model.lower()
    if kind not in _AGGREGATIONS:
        raise ValueError(f"no aggregation operator for model {model!r} "
                         f"(expected one of {', '.join(_AGGREGATIONS)})")
    adj = sp.csr_matrix(csr, dtype=np.float64, copy=True)
    adj.sum_duplicates()
    n = adj.shape[0]

    def row_of_entry(m):
        return np.repeat(np.arange(m.shape[0]), np.diff(m.indptr))

    def reciprocal(x, power):
        r = np.zeros_like(x)
        live = x > 0
        r[live] = x[live] ** -power
        return r

    if kind == "gcn":
        missing_loop = (adj.diagonal() == 0).astype(np.float64)
        tilde = (adj + sp.diags(missing_loop, format="csr")).tocsr()
        tilde.eliminate_zeros()
        tilde.sort_indices()
        norm = reciprocal(np.asarray(tilde.sum(axis=1)).ravel(), 0.5)
        tilde.data = tilde.data * (norm[row_of_entry(tilde)] * norm[tilde.indices])
        tilde.eliminate_zeros()  # the product D A D stores no zero entries
        weights = tilde
    elif kind == "gin":
        weights = adj
    else:
        inv_deg = reciprocal(np.asarray(adj.sum(axis=1)).ravel(), 1.0)
        weights = adj.copy()
        weights.data = weights.data * inv_deg[row_of_entry(weights)]
        weights.eliminate_zeros()  # the product D^-1 A stores no zero entries
    out = sp.csr_matrix(weights, dtype=np.float32)
    out.sort_indices()
    return out


def operator_descriptors(csr) -> Dict[str, float]:
    """M, nnz, d_bar, population CV of row lengths."""
    deg = np.diff(csr.indptr).astype(np.float64)
    M = int(csr.shape[0])
    mean = deg.mean() if M else 0.0
    return {"M": M, "nnz": int(csr.indptr[-1]), "d_bar": float(mean),
            "cv_d": float(deg.std() / mean) if mean > 0 else 0.0}


def _tensors(csr, device):
    return {
        "rowptr_cpu": torch.from_numpy(csr.indptr.astype(np.int32)),
        "colind_cpu": torch.from_numpy(csr.indices.astype(np.int32)),
        "vals_cpu": torch.from_numpy(csr.data.astype(np.float32)),
        "rowptr": torch.from_numpy(csr.indptr.astype(np.int32)).to(device),
        "colind": torch.from_numpy(csr.indices.astype(np.int32)).to(device),
        "vals": torch.from_numpy(csr.data.astype(np.float32)).to(device),
    }


class GraphBackend:
    def __init__(self, csr, device, table: str = "mi355x"):
        self.device = torch.device(device)
        self.table = table
        self.csr = csr.tocsr()
        self.csr_t = self.csr.transpose().tocsr()
        self.forward = _tensors(self.csr, self.device)
        self.backward = _tensors(self.csr_t, self.device)
        self.plan_cache: Dict[Tuple[bool, int], dict] = {}
        self.exec_cache: Dict[Tuple[str, bool, int], tuple] = {}
        self._torch_sparse: Dict[bool, torch.Tensor] = {}
        self._cold_seen: set = set()
        self._cold_zo: Dict[bool, object] = {}  # ZERO_OVERHEAD_CSR plans of cold first calls

    def _tensors(self, transpose: bool):
        return self.backward if transpose else self.forward

    def get_router_plan(self, transpose: bool, ncols: int) -> dict:
        key = (transpose, int(ncols))
        if key not in self.plan_cache:
            t = self._tensors(transpose)
            M = int(t["rowptr"].numel()) - 1
            # Device rowptr: the feature pass runs on the GPU.
            self.plan_cache[key] = _C.make_router_plan(t["rowptr"], t["colind"], t["vals"], M, M,
                                                       int(ncols), "MAIN", self.table)
        return self.plan_cache[key]

    def routed_label(self, transpose: bool, ncols: int) -> str:
        return route_label(self.get_router_plan(transpose, ncols))

    def _get_executor(self, backend: str, transpose: bool, ncols: int):
        key = (backend, transpose, int(ncols))
        if key in self.exec_cache:
            return self.exec_cache[key]
        t = self._tensors(transpose)
        M = int(t["rowptr"].numel()) - 1
        if backend == "cusparse":
            tmpl = torch.empty((M, int(ncols)), device=self.device, dtype=torch.float32)
            ex = ("CUSPARSE", _C.make_cusparse_plan(t["rowptr"], t["colind"], t["vals"], tmpl))
        elif backend == "torch":
            ex = ("torch", None)
        elif backend == "rocsparse":
            from . import vendor
            B0 = torch.zeros((M, int(ncols)), device=self.device)
            plan, alg = vendor.fastest(t["rowptr"], t["colind"], t["vals"], B0)
            ex = ("rocsparse", plan)
        else:
            if backend in ("router", "router_cold"):
                label = self.routed_label(transpose, ncols)
            elif backend in _FIXED:
                label = _FIXED[backend]
            else:
                raise ValueError(f"Unknown backend {backend}")
            if label in TILE_KERNELS and int(ncols) < 16:
                label = "CSR_DIRECT"
            if label == "CUSPARSE":
                tmpl = torch.empty((M, int(ncols)), device=self.device, dtype=torch.float32)
                ex = (label, _C.make_cusparse_plan(t["rowptr"], t["colind"], t["vals"], tmpl))
            else:
                # Tile plans (N only gates N >= 16) and ZERO_OVERHEAD_CSR plans
                # (a partial buffer that grows to the widest N) do not depend
                # on N: share one plan per (family, transpose) across widths
                # and precisions.
                plan = self._cold_zo.get(transpose) if label == "ZERO_OVERHEAD_CSR" else None
                if plan is None and (label in TILE_KERNELS or label == "ZERO_OVERHEAD_CSR"):
                    fam = label.replace("_TF32", "")
                    for (b, tr, n), (lab, p) in self.exec_cache.items():
                        if tr == transpose and lab.replace("_TF32", "") == fam and p is not None:
                            plan = p
                            break
                if plan is None:
                    plan = build_kernel_plan(label, t["rowptr_cpu"], t["colind_cpu"],
                                             t["vals_cpu"], M, M, max(int(ncols), 16))
                ex = (label, plan)
        self.exec_cache[key] = ex
        return ex

    def run(self, B: torch.Tensor, backend: str, transpose: bool = False) -> torch.Tensor:
        t = self._tensors(transpose)
        ncols = int(B.shape[1])
        if backend == "router_cold" and (transpose, ncols) not in self._cold_seen:
            # Cold first call: feature pass + route, then the cold-aware
            # policy's path, which builds no tile format.
            self._cold_seen.add((transpose, ncols))
            label, plan = cold_path(self.get_router_plan(transpose, ncols)), None
            if label == "ZERO_OVERHEAD_CSR":
                plan = self._cold_zo.get(transpose)
                if plan is None:  # binned on the GPU from the device rowptr
                    M = int(t["rowptr"].numel()) - 1
                    plan = self._cold_zo[transpose] = _C.make_zero_overhead_plan(t["rowptr"], M, M)
        else:
            label, plan = self._get_executor(backend, transpose, ncols)
        if label == "CUSPARSE":
            return _C.run_cusparse_plan(plan, B).clone()
        if label == "rocsparse":
            C = torch.empty((int(t["rowptr"].numel()) - 1, ncols), device=B.device)
            plan.rebind(B.contiguous(), C)
            return plan.run()
        if label == "torch":
            if transpose not in self._torch_sparse:
                M = int(t["rowptr"].numel()) - 1
                self._torch_sparse[transpose] = torch.sparse_csr_tensor(
                    t["rowptr"].long(), t["colind"].long(), t["vals"], size=(M, M))
            return torch.sparse.mm(self._torch_sparse[transpose], B)
        N = B.shape[1]
        if N % 4 and B.dtype == torch.float32 and label in ("CSR_DIRECT", "ZERO_OVERHEAD_CSR"):
            # Widths that are not a multiple of 4 (47 classes) gather with
            # 4-byte loads; a zero-padded copy lets the kernels use 16-byte
            # loads (C5 N=47: 1.08 ms, N=48: 0.83 ms).  The padding columns
            # of C are zero and dropped.
            Bp = B.new_zeros((B.shape[0], (N + 3) // 4 * 4))
            Bp[:, :N] = B
            return run_planned_kernel(label, plan, t["rowptr"], t["colind"], t["vals"], Bp)[:, :N]
        return run_planned_kernel(label, plan, t["rowptr"], t["colind"], t["vals"], B)


def validate_backend(csr, device, backend: str, ncols_values, seed: int, table="mi355x"):
    """Every (transpose, N) SpMM of a fresh backend against the baseline kernel
    with the reference's gate (ra_real_graph_eval.py:41-51)."""
    graph = GraphBackend(csr, device, table)
    max_err = max_tol = 0.0
    for transpose in (False, True):
        t = graph._tensors(transpose)
        deg = t["rowptr_cpu"][1:] - t["rowptr_cpu"][:-1]
        max_row = max(1, int(deg.max().item())) if deg.numel() else 1
        for ncols in sorted(set(int(v) for v in ncols_values)):
            gen = torch.Generator(device=device).manual_seed(
                (int(seed) * 8191 + ncols) * 2 + int(transpose))
            B = torch.randn((csr.shape[0], ncols), device=device, generator=gen)
            out = graph.run(B, backend, transpose)
            ref = _C.spmm_cusparse(t["rowptr"], t["colind"], t["vals"], B)
            err = float((out.float() - ref).abs().max().item())
            path = graph._get_executor(backend, transpose, ncols)[0]
            tol = BASE_ATOL * max(1.0, math.sqrt(max_row))
            if path in TILE_KERNELS:
                tol *= TC_EXTRA_FACTOR
            max_err, max_tol = max(max_err, err), max(max_tol, tol)
            if err > tol or err >= 1.0:
                return {"correct": False, "soft_fail": tol < err < 1.0, "hard_fail": err >= 1.0,
                        "max_error": err, "tolerance": tol, "path": path}
    return {"correct": True, "soft_fail": False, "hard_fail": False, "max_error": max_err,
            "tolerance": max_tol}


class SparseMMFunction(torch.autograd.Function):
    """Y = A @ B; dL/dB = A^T @ dL/dY (gnn_bench/router_vs_baselines_gcn.py:451-461)."""

    @staticmethod
    def forward(ctx, B, graph: GraphBackend, backend: str):
        ctx.graph = graph
        ctx.backend = backend
        return graph.run(B.contiguous(), backend, transpose=False)

    @staticmethod
    def backward(ctx, grad_output):
        return ctx.graph.run(grad_output.contiguous(), ctx.backend, transpose=True), None, None


# Rows per chunk of the weight-gradient reduction (below).
WGRAD_ROWS = 8192


def weight_grad(g: torch.Tensor, x: torch.Tensor, rows: int = 0) -> torch.Tensor:
    """g^T x, the weight gradient of y = x W^T, for tall g [M, out], x [M, in].

    A single GEMM reduces over all M rows with only out*in/1024 output tiles:
    on MI355X hipBLASLt runs [1e6 x 256]^T [1e6 x 128] in 1.82 ms and
    [1e6 x 47]^T [1e6 x 256] in 1.95 ms.  Cutting M into chunks of `rows` rows
    gives one batched GEMM with a tile grid per chunk, then a sum over the
    chunks: 0.59 and 0.33 ms, and a shorter fp32 summation chain per element."""
    rows = rows or WGRAD_ROWS
    M = g.shape[0]
    c = M // rows
    if c < 4:
        return g.t() @ x
    m = c * rows
    out = torch.bmm(g[:m].view(c, rows, g.shape[1]).transpose(1, 2), x[:m].view(c, rows, x.shape[1])).sum(0)
    if m < M:
        out = out + g[m:].t() @ x[m:]
    return out


class _LinearFn(torch.autograd.Function):
    """y = x W^T with the chunked weight gradient."""

    @staticmethod
    def forward(ctx, x, weight):
        ctx.save_for_backward(x, weight)
        return F.linear(x, weight)

    @staticmethod
    def backward(ctx, grad):
        x, weight = ctx.saved_tensors
        grad = grad.contiguous()
        gx = grad @ weight if ctx.needs_input_grad[0] else None
        gw = weight_grad(grad, x.contiguous()) if ctx.needs_input_grad[1] else None
        return gx, gw


class Linear(nn.Linear):
    """nn.Linear without bias (same parameters and initialisation) whose weight
    gradient is reduced in row chunks (weight_grad).

    An output width that is not a multiple of 4 (47 classes) is computed with
    the weight zero-padded to the next multiple of 4, and the padded output is
    returned: the extra columns are exactly zero.  On MI355X the padded GEMMs
    are faster ([1e6 x 256] x [256 x 47]: 0.56 ms, x 48: 0.31 ms; backward
    0.46 -> 0.38 ms), and the CSR SpMM that follows gathers 16-byte packets
    without a padded copy.  Callers slice [:, :out_features]."""

    def __init__(self, in_features: int, out_features: int):
        super().__init__(in_features, out_features, bias=False)

    def forward(self, x):
        pad = -self.out_features % 4
        w = F.pad(self.weight, (0, 0, 0, pad)) if pad else self.weight
        return _LinearFn.apply(x, w)


class GCN(nn.Module):
    """2-layer GCN: A relu(A X W1) W2 (gnn_bench/router_vs_baselines_gcn.py:464-476).
    The linear layers are bias-free nn.Linear, as in the reference, with the
    chunked weight-gradient reduction.

    order="reference" (default) transforms before aggregating in both layers,
    as the reference does: A (X W1), then A (H W2).  order="auto" aggregates
    first where a layer widens (in_features < out_features), the rule DGL's
    GraphConv uses: (A X) W1 is the same product with the SpMM at the input
    width (128 instead of 256 for config 5), and since X needs no gradient
    the layer's backward A^T SpMM disappears.  The results agree to fp32
    rounding; the reference's SpMM count per step is kept only by the
    default."""

    def __init__(self, in_dim: int, hidden_dim: int, out_dim: int, order: str = "reference"):
        super().__init__()
        if order not in ("reference", "auto"):
            raise ValueError(f"order must be 'reference' or 'auto', got {order!r}")
        self.order = order
        self.lin1 = Linear(in_dim, hidden_dim)
        self.lin2 = Linear(hidden_dim, out_dim)

    def _layer(self, lin, x, graph, backend):
        if self.order == "auto" and lin.in_features < lin.out_features:
            return lin(SparseMMFunction.apply(x, graph, backend))
        return SparseMMFunction.apply(lin(x), graph, backend)

    def forward(self, X, graph: GraphBackend, backend: str):
        h = F.relu(self._layer(self.lin1, X, graph, backend))
        return self._layer(self.lin2, h, graph, backend)[:, :self.lin2.out_features]


GCNBench = GCN


class SAGE(nn.Module):
    """2-layer GraphSAGE with the mean aggregator, full batch
    (gnn_bench/router_vs_baselines_sage.py:48-67): per layer
    h' = W [h, A h], with A = D^-1 A_raw (build_aggregation_operator(..., "sage"),
    no self-loops: the self term is the concatenated h).  Two routed SpMMs per
    forward, at the input and the hidden width; the first needs no backward
    SpMM (X takes no gradient).  Bias-free linear maps as in the reference,
    with the chunked weight gradient of ``Linear``."""

    def __init__(self, in_dim: int, hidden_dim: int, out_dim: int):
        super().__init__()
        self.lin1 = Linear(2 * in_dim, hidden_dim)
        self.lin2 = Linear(2 * hidden_dim, out_dim)

    def forward(self, X, graph: GraphBackend, backend: str):
        h = F.relu(self.lin1(torch.cat([X, SparseMMFunction.apply(X, graph, backend)], dim=1)))
        h = h[:, :self.lin1.out_features]
        out = self.lin2(torch.cat([h, SparseMMFunction.apply(h, graph, backend)], dim=1))
        return out[:, :self.lin2.out_features]


class GIN(nn.Module):
    """2-layer GIN (gnn_bench/router_vs_baselines_gin.py:47-73): per layer
    h' = MLP((1 + eps) h + A h) with A the raw adjacency
    (build_aggregation_operator(..., "gin")), a learnable eps per layer
    (initialised to 0) and 2-layer bias-free MLPs (in -> hidden -> hidden,
    hidden -> hidden -> out), ReLU between the layers."""

    def __init__(self, in_dim: int, hidden_dim: int, out_dim: int):
        super().__init__()
        self.eps1 = nn.Parameter(torch.zeros(1))
        self.eps2 = nn.Parameter(torch.zeros(1))
        self.mlp1 = nn.ModuleList([Linear(in_dim, hidden_dim), Linear(hidden_dim, hidden_dim)])
        self.mlp2 = nn.ModuleList([Linear(hidden_dim, hidden_dim), Linear(hidden_dim, out_dim)])

    @staticmethod
    def _mlp(layers, h):
        a, b = layers
        h = F.relu(a(h)[:, :a.out_features])
        return b(h)[:, :b.out_features]

    def forward(self, X, graph: GraphBackend, backend: str):
        h = (1.0 + self.eps1) * X + SparseMMFunction.apply(X, graph, backend)
        h = F.relu(self._mlp(self.mlp1, h))
        h = (1.0 + self.eps2) * h + SparseMMFunction.apply(h.contiguous(), graph, backend)
        return self._mlp(self.mlp2, h)


SAGEBench = SAGE
GINBench = GIN
MODELS = {"gcn": GCN, "sage": SAGE, "graphsage": SAGE, "gin": GIN}


def cross_entropy(logits: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    """Mean cross-entropy, the value of F.cross_entropy(logits, y)
    (gnn_bench/router_vs_baselines_gcn.py:494), as log_softmax + gather + mean:
    the fused nll_loss reduction kernel takes 1.8 ms forward and 1.5 ms backward
    on 1e6 x 47 logits on MI355X, the gather form a few tens of microseconds."""
    logp = F.log_softmax(logits, dim=1)
    return -logp.gather(1, y.view(-1, 1)).mean()


def train_step(model, graph, backend, X, y, optimizer) -> float:
    """One forward + backward + optimizer step; seconds (synchronised)."""
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    optimizer.zero_grad(set_to_none=True)
    loss = cross_entropy(model(X, graph, backend), y)
    loss.backward()
    optimizer.step()
    torch.cuda.synchronize()
    return time.perf_counter() - t0


measure_step = train_step
