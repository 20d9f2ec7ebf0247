"""GNN call site on the GPU: GraphBackend per (transpose, N) routing, the
autograd SpMM (backward through A^T) and a 2-layer GCN step, against the
baseline kernel and a dense fp32 torch reference."""
import numpy as np
import pytest
import scipy.sparse as sp
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu

from ra_spmm import synthetic as S  # noqa: E402
from ra_spmm import gnn  # noqa: E402
import ra_spmm  # noqa: E402


def _operator(M=4000, seed=3):
    g = S.chung_lu(M, 12.0, 2.3, 600, seed=seed)
    A = sp.csr_matrix((np.ones(g.nnz, np.float32), g.colind, g.rowptr), shape=(M, M))
    return gnn.build_aggregation_operator(A, "gcn")


@pytest.mark.parametrize("backend", ["router", "router_cold", "cusparse", "rocsparse", "csr_direct",
                                     "zero_overhead", "tc_direct", "tc_direct_tf32",
                                     "segment_hybrid"])
def test_validate_backend(backend):
    op = _operator()
    res = gnn.validate_backend(op, "cuda", backend, (16, 47, 64, 256), seed=1)
    assert res["correct"], res


def test_gcn_step_matches_dense_reference():
    op = _operator(3000, seed=5)
    M = op.shape[0]
    torch.manual_seed(0)
    X = torch.randn(M, 32, device="cuda")
    y = torch.randint(0, 7, (M,), device="cuda")
    dense = torch.from_numpy(op.toarray()).cuda()
    results = {}
    for backend in ("cusparse", "rocsparse", "router", "zero_overhead", "csr_direct", "segment_hybrid"):
        torch.manual_seed(1)
        model = gnn.GCN(32, 64, 7).cuda()
        graph = gnn.GraphBackend(op, "cuda")
        out = model(X, graph, backend)
        loss = F.cross_entropy(out, y)
        loss.backward()
        fp16 = any(lab in gnn.TILE_KERNELS and not lab.endswith("_TF32")
                   for lab, _ in graph.exec_cache.values())
        results[backend] = (out.detach(), [p.grad.detach().clone() for p in model.parameters()], fp16)
    torch.manual_seed(1)
    ref_model = gnn.GCN(32, 64, 7).cuda()
    h = F.relu(dense @ F.linear(X, ref_model.lin1.weight))
    ref_out = dense @ F.linear(h, ref_model.lin2.weight)
    F.cross_entropy(ref_out, y).backward()
    ref_grads = [p.grad for p in ref_model.parameters()]
    for backend, (out, grads, fp16) in results.items():
        # fp32 paths: accumulation-order differences only; fp16 tile paths round
        # A and the dense operand to fp16 (2^-11 relative each).
        rtol, atol = (2e-2, 2e-3) if fp16 else (2e-4, 2e-5)
        torch.testing.assert_close(out, ref_out, rtol=rtol, atol=atol, msg=backend)
        for g_, r_ in zip(grads, ref_grads):
            torch.testing.assert_close(g_, r_, rtol=10 * rtol, atol=atol, msg=backend)


def test_gcn_order_auto_matches_dense_reference():
    """order="auto": layer 1 (32 -> 64) aggregates first, (A X) W1, and runs
    no backward SpMM for it; same outputs and gradients as the dense model."""
    op = _operator(3000, seed=5)
    M = op.shape[0]
    torch.manual_seed(0)
    X = torch.randn(M, 32, device="cuda")
    y = torch.randint(0, 7, (M,), device="cuda")
    dense = torch.from_numpy(op.toarray()).cuda()
    torch.manual_seed(1)
    model = gnn.GCN(32, 64, 7, order="auto").cuda()
    graph = gnn.GraphBackend(op, "cuda")
    out = model(X, graph, "zero_overhead")
    F.cross_entropy(out, y).backward()
    # forward at widths 32 (layer 1, aggregated first) and 8 (layer 2, padded
    # 7), backward only for layer 2
    assert sorted((t, n) for (_, t, n) in graph.exec_cache) == [(False, 8), (False, 32), (True, 8)]
    torch.manual_seed(1)
    ref_model = gnn.GCN(32, 64, 7).cuda()
    h = F.relu(dense @ F.linear(X, ref_model.lin1.weight))
    ref_out = dense @ F.linear(h, ref_model.lin2.weight)
    F.cross_entropy(ref_out, y).backward()
    torch.testing.assert_close(out, ref_out, rtol=2e-4, atol=2e-5)
    for p, r in zip(model.parameters(), ref_model.parameters()):
        torch.testing.assert_close(p.grad, r.grad, rtol=2e-3, atol=2e-5)


def test_router_plans_per_transpose_and_width():
    op = _operator(5000, seed=7)
    graph = gnn.GraphBackend(op, "cuda")
    labels = {(t, n): graph.routed_label(t, n) for t in (False, True) for n in (47, 256)}
    assert len(graph.plan_cache) == 4
    for (t, n), lab in labels.items():
        assert lab in ("CSR_DIRECT", "ZERO_OVERHEAD_CSR", "CUSPARSE", "TC_DIRECT", "COMMUNITY_TC",
                       "SEGMENT_HYBRID", "TC_DIRECT_TF32", "COMMUNITY_TC_TF32",
                       "SEGMENT_HYBRID_TF32")
    model = gnn.GCN(16, 256, 47).cuda()
    opt = torch.optim.Adam(model.parameters(), lr=1e-2)
    X = torch.randn(op.shape[0], 16, device="cuda")
    y = torch.randint(0, 47, (op.shape[0],), device="cuda")
    for _ in range(3):
        dt = gnn.train_step(model, graph, "router", X, y, opt)
        assert dt > 0


def test_zero_overhead_plan_shared_across_widths():
    """One ZERO_OVERHEAD_CSR plan per transpose serves every width (its
    partial buffer grows to the widest); results stay exact against dense."""
    op = _operator(4000, seed=9)
    graph = gnn.GraphBackend(op, "cuda")
    dense = torch.from_numpy(op.toarray()).cuda()
    for n in (48, 256, 16, 256):
        for t in (False, True):
            B = torch.randn(op.shape[0], n, device="cuda")
            out = graph.run(B, "zero_overhead", transpose=t)
            ref = (dense.t() if t else dense) @ B
            torch.testing.assert_close(out, ref, rtol=1e-4, atol=1e-5)
    for t in (False, True):
        plans = {id(p) for (b, tr, n), (lab, p) in graph.exec_cache.items() if tr == t}
        assert len(plans) == 1


def test_padded_narrow_width_is_exact(oracle):
    """Widths not divisible by 4 run on a zero-padded copy in the CSR family.
    CSR_DIRECT keeps its fma chain per element: bit-identical to the unpadded
    call.  ZERO_OVERHEAD_CSR's split rows (> 256 nnz) divide a chunk over lane
    groups whose count depends on the width, so only rows <= 256 nnz are
    bit-identical; the rest stay within 1e-5 of |A||B|."""
    g = S.random_csr(3000, 3000, 12.0, seed=11, skew=1.0)
    import scipy.sparse as sp
    op = sp.csr_matrix((g.vals, g.colind, g.rowptr), shape=(g.M, g.K))
    graph = gnn.GraphBackend(op, "cuda")
    B = torch.randn(g.K, 47, device="cuda")
    t = graph._tensors(False)
    for backend, fn in (("csr_direct", ra_spmm.spmm_csr_direct),):
        out = graph.run(B, backend)
        ref = fn(t["rowptr"], t["colind"], t["vals"], B)
        assert out.shape == ref.shape and torch.equal(out, ref)
    p = ra_spmm.make_zero_overhead_plan(t["rowptr"], g.M, g.K)
    got = graph.run(B, "zero_overhead").cpu().numpy()
    ref = ra_spmm.run_zero_overhead_plan(p, t["rowptr"], t["colind"], t["vals"], B).cpu().numpy()
    short = np.diff(g.rowptr) <= 256
    np.testing.assert_array_equal(got[short], ref[short])
    scale = oracle.spmm_f64(g.rowptr, g.colind, np.abs(g.vals), np.abs(B.cpu().numpy()))
    assert np.all(np.abs(got - ref) <= 1e-5 * scale + 1e-30)


def test_chunked_weight_grad_on_device():
    """The GCN's weight gradient over 300k rows (36 chunks + a remainder) against
    fp64: the chunked sum is held to 1e-5 of sum |g||x|."""
    torch.manual_seed(5)
    for out_f, in_f in ((256, 128), (47, 256)):
        g = torch.randn(300_001, out_f, device="cuda")
        x = torch.randn(300_001, in_f, device="cuda")
        got = gnn.weight_grad(g, x).double()
        ref = g.double().t() @ x.double()
        scale = g.double().abs().t() @ x.double().abs()
        assert float(((got - ref).abs() / scale).max()) < 1e-5


def test_gcn_full_size_c5_step():
    """One full-size config C5 training step (1e6-row power-law GCN operator,
    128 -> 256 -> 47) through the router backend against the csr_direct
    backend (one fp32 fma chain per element, the arithmetic
    oracle.spmm_seq_f32 pins).  Logits: elementwise, within the propagated
    bound of 1e-5 |A||B| per SpMM plus the GEMM rounding of the perturbed
    hidden layer (256 * 2^-24 |H||W2|, twice).  Weight gradients (reductions
    over all 1e6 rows): max |difference| <= 1e-5 max |gradient|."""
    S.use_device_sort("cuda")
    try:
        g = S.CONFIGS["C5"]()
    finally:
        S.use_device_sort(None)
    M = g.M
    op = sp.csr_matrix((g.vals, g.colind, g.rowptr), shape=(M, M))
    torch.manual_seed(0)
    X = torch.randn(M, 128, device="cuda")
    y = torch.randint(0, 47, (M,), device="cuda")
    res = {}
    for backend in ("router", "csr_direct"):
        print(f"[c5 gcn step] {backend}", flush=True)
        torch.manual_seed(1)
        model = gnn.GCN(128, 256, 47).cuda()
        graph = gnn.GraphBackend(op, "cuda")
        out = model(X, graph, backend)
        gnn.cross_entropy(out, y).backward()
        labels = {k: lab for k, (lab, _) in graph.exec_cache.items()}
        res[backend] = (out.detach(), [p.grad.detach().clone() for p in model.parameters()], labels)
        del graph, model
        torch.cuda.empty_cache()
    # the router routes all four SpMMs (forward and backward, N = 256 and 47)
    assert len(res["router"][2]) == 4 and set(res["router"][2].values()) == {"ZERO_OVERHEAD_CSR"}
    out_r, grads_r, _ = res["router"]
    out_c, grads_c, _ = res["csr_direct"]
    rp, ci, vl = g.torch("cuda")
    va = vl.abs()

    def spmm(vals, B):
        return ra_spmm.spmm_csr_direct(rp, ci, vals, B.contiguous())

    torch.manual_seed(1)
    ref = gnn.GCN(128, 256, 47).cuda()
    W1, W2 = ref.lin1.weight.detach(), ref.lin2.weight.detach()
    with torch.no_grad():
        XW1 = X @ W1.t()
        H = F.relu(spmm(vl, XW1))
        s1 = spmm(va, XW1.abs())
        HW2a = H.abs() @ W2.abs().t()
        bound = (1e-5 * spmm(va, (H @ W2.t()).abs()) + spmm(va, (1e-5 * s1) @ W2.abs().t())
                 + 2.0 * 256 * 2.0 ** -24 * spmm(va, HW2a))
        err = (out_r - out_c).abs()
        bad = err > bound + 1e-30
        assert not bool(bad.any()), (int(bad.sum()), float(err.max()))
    for name, gr, gc in zip(("lin1", "lin2"), grads_r, grads_c):
        diff = float((gr - gc).abs().max())
        assert diff <= 1e-5 * float(gc.abs().max()), (name, diff, float(gc.abs().max()))


def _adjacency(M=3000, seed=5):
    g = S.chung_lu(M, 12.0, 2.3, 600, seed=seed)
    return sp.csr_matrix((np.ones(g.nnz, np.float32), g.colind, g.rowptr), shape=(M, M))


def _dense_sage(X, A, model):
    W1, W2 = model.lin1.weight, model.lin2.weight
    h = F.relu(torch.cat([X, A @ X], dim=1) @ W1.t())
    return torch.cat([h, A @ h], dim=1) @ W2.t()


def _dense_gin(X, A, model):
    Wa1, Wb1 = model.mlp1[0].weight, model.mlp1[1].weight
    Wa2, Wb2 = model.mlp2[0].weight, model.mlp2[1].weight
    h = (1.0 + model.eps1) * X + A @ X
    h = F.relu(F.relu(h @ Wa1.t()) @ Wb1.t())
    h = (1.0 + model.eps2) * h + A @ h
    return F.relu(h @ Wa2.t()) @ Wb2.t()


@pytest.mark.parametrize("kind", ["sage", "gin"])
def test_sage_and_gin_steps_match_dense_reference(kind):
    """GraphSAGE (mean aggregator, gnn_bench/router_vs_baselines_sage.py:48-67)
    and GIN (gnn_bench/router_vs_baselines_gin.py:47-73) on their own
    aggregation operators: logits and every gradient (weights and GIN's eps)
    against a dense fp32 autograd model with the same parameters, for the
    router and fixed backends."""
    op = gnn.build_aggregation_operator(_adjacency(), kind)
    M = op.shape[0]
    torch.manual_seed(0)
    X = torch.randn(M, 32, device="cuda")
    y = torch.randint(0, 7, (M,), device="cuda")
    dense = torch.from_numpy(op.toarray()).cuda()
    cls = gnn.MODELS[kind]
    torch.manual_seed(1)
    ref = cls(32, 64, 7).cuda()
    ref_out = (_dense_sage if kind == "sage" else _dense_gin)(X, dense, ref)
    F.cross_entropy(ref_out, y).backward()
    ref_grads = [p.grad for p in ref.parameters()]
    for backend in ("router", "csr_direct", "zero_overhead", "cusparse", "segment_hybrid"):
        torch.manual_seed(1)
        model = cls(32, 64, 7).cuda()
        graph = gnn.GraphBackend(op, "cuda")
        out = model(X, graph, backend)
        assert out.shape == (M, 7)
        F.cross_entropy(out, y).backward()
        fp16 = any(lab in gnn.TILE_KERNELS and not lab.endswith("_TF32")
                   for lab, _ in graph.exec_cache.values())
        rtol, atol = (2e-2, 2e-3) if fp16 else (2e-4, 2e-5)
        torch.testing.assert_close(out, ref_out, rtol=rtol, atol=atol, msg=f"{kind} {backend}")
        for (name, p), r in zip(model.named_parameters(), ref_grads):
            torch.testing.assert_close(p.grad, r, rtol=10 * rtol, atol=10 * atol, msg=f"{kind} {backend} {name}")
