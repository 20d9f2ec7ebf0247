"""Seeded synthetic graphs for the five benchmark configurations.

All generators return a ``Graph`` (int32 rowptr/colind, float32 vals, M, K) in
sorted, duplicate-free CSR.  numpy only; deterministic for a given seed.

  C1  er(10_000, 8)                              ER, GCN-normalised values
  C2  chung_lu(1_000_000, 16, 2.1, 50_000)       power law, hubs, GCN-normalised
  C3  sbm(1024, 500, 32, 0.9)                    communities, shuffled then
                                                 locality-reordered, fp16 values
  C4  lognormal_social(250_000, 500, 1.0, ...)   log-normal degrees, fp16 values
  C5  gcn_operator(chung_lu(1_000_000, 25, 2.3)) D^-1/2 (A+I) D^-1/2
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass
class Graph:
    rowptr: np.ndarray  # int32 [M+1]
    colind: np.ndarray  # int32 [nnz]
    vals: np.ndarray    # float32 [nnz]
    M: int
    K: int
    name: str = ""

    @property
    def nnz(self) -> int:
        return int(self.rowptr[-1])

    def degrees(self) -> np.ndarray:
        return np.diff(self.rowptr.astype(np.int64))

    def torch(self, device="cuda"):
        import torch
        return (torch.from_numpy(self.rowptr).to(device), torch.from_numpy(self.colind).to(device),
                torch.from_numpy(self.vals).to(device))

    def scipy(self):
        import scipy.sparse as sp
        return sp.csr_matrix((self.vals, self.colind, self.rowptr), shape=(self.M, self.K))


_SORT_DEVICE = None


def use_device_sort(device) -> None:
    """Sort the generators' edge keys on `device` (a torch device such as
    "cuda", or None for numpy on the host).  The sorted unique keys, and so
    every generated graph, are the same either way; the device sort takes the
    minute-long host sort of config C4 (1.25e8 keys) down to under a second."""
    global _SORT_DEVICE
    _SORT_DEVICE = device


def _unique_sorted(keys: np.ndarray) -> np.ndarray:
    if _SORT_DEVICE is None:
        return np.unique(keys)
    import torch
    t = torch.from_numpy(np.ascontiguousarray(keys, dtype=np.int64)).to(_SORT_DEVICE)
    out = torch.unique(t, sorted=True).cpu().numpy()
    del t
    return out


def _csr_from_keys(keys: np.ndarray, M: int, K: int) -> tuple[np.ndarray, np.ndarray]:
    """Sorted unique int64 keys row*K+col -> (rowptr, colind)."""
    keys = _unique_sorted(keys)
    rows = keys // K
    cols = (keys - rows * K).astype(np.int32)
    rowptr = np.zeros(M + 1, dtype=np.int64)
    np.cumsum(np.bincount(rows, minlength=M), out=rowptr[1:])
    return rowptr.astype(np.int32), cols


def _symmetric(u: np.ndarray, v: np.ndarray, M: int) -> tuple[np.ndarray, np.ndarray]:
    keep = u != v
    u, v = u[keep].astype(np.int64), v[keep].astype(np.int64)
    keys = np.concatenate([u * M + v, v * M + u])
    return _csr_from_keys(keys, M, M)


def gcn_norm_values(rowptr: np.ndarray, colind: np.ndarray) -> np.ndarray:
    """1/sqrt(d_i d_j) with d = row length (fp32); rows/cols of degree 0 get 0."""
    cnt = np.diff(rowptr.astype(np.int64))
    deg = cnt.astype(np.float64)
    dis = np.zeros_like(deg)
    nz = deg > 0
    dis[nz] = 1.0 / np.sqrt(deg[nz])
    return (np.repeat(dis, cnt) * dis[colind]).astype(np.float32)


def er(M: int = 10_000, avg_deg: float = 8.0, seed: int = 1) -> Graph:
    """Undirected Erdos-Renyi with mean degree ~avg_deg, GCN-normalised values."""
    rng = np.random.default_rng(seed)
    m = int(M * avg_deg / 2)
    u = rng.integers(0, M, size=m)
    v = rng.integers(0, M, size=m)
    rowptr, colind = _symmetric(u, v, M)
    return Graph(rowptr, colind, gcn_norm_values(rowptr, colind), M, M, f"er_{M}_{avg_deg}")


def _power_law_weights(M: int, avg_deg: float, gamma: float, max_deg: float) -> np.ndarray:
    w = np.arange(1, M + 1, dtype=np.float64) ** (-1.0 / (gamma - 1.0))
    for _ in range(20):  # scale to the target mean with the hub cap applied
        w *= avg_deg / w.mean()
        w = np.minimum(w, max_deg)
    return w


def _weighted_endpoints(rng, w: np.ndarray, m: int) -> np.ndarray:
    """m i.i.d. node draws with P(i) = w_i / sum(w): multinomial counts, then a
    random order (same distribution as independent draws, without the
    random-access inverse-CDF search)."""
    counts = rng.multinomial(m, w / w.sum())
    ends = np.repeat(np.arange(len(w), dtype=np.int64), counts)
    rng.shuffle(ends)
    return ends


def chung_lu(M: int = 1_000_000, avg_deg: float = 16.0, gamma: float = 2.1,
             max_deg: float = 50_000, seed: int = 2) -> Graph:
    """Undirected Chung-Lu graph: endpoints drawn proportional to power-law
    weights w_i ~ i^(-1/(gamma-1)) capped at max_deg; GCN-normalised values.
    Node ids are randomly permuted so hubs are spread over the id space.  Edge
    draws are topped up once so the mean degree after de-duplication is
    within ~1% of avg_deg."""
    rng = np.random.default_rng(seed)
    w = _power_law_weights(M, avg_deg, gamma, max_deg)
    perm = rng.permutation(M)
    target = int(M * avg_deg)
    m = target // 2
    u = _weighted_endpoints(rng, w, m)
    v = _weighted_endpoints(rng, w, m)
    rowptr, colind = _symmetric(perm[u], perm[v], M)
    short = target - int(rowptr[-1])
    if short > 0.01 * target:
        extra = int(short / 2 * target / max(1, int(rowptr[-1])))
        u = np.concatenate([u, _weighted_endpoints(rng, w, extra)])
        v = np.concatenate([v, _weighted_endpoints(rng, w, extra)])
        rowptr, colind = _symmetric(perm[u], perm[v], M)
    return Graph(rowptr, colind, gcn_norm_values(rowptr, colind), M, M,
                 f"chung_lu_{M}_{avg_deg}_{gamma}")


def sbm(communities: int = 1024, size: int = 500, avg_deg: float = 32.0, intra: float = 0.9,
        seed: int = 3) -> Graph:
    """Stochastic block model; labels shuffled, then locality-reordered
    (communities contiguous, random order of communities and of nodes within
    each).  Values: GCN normalisation rounded to fp16 (fp16-representable fp32)."""
    rng = np.random.default_rng(seed)
    M = communities * size
    m = int(M * avg_deg / 2)
    m_in = int(m * intra)
    c = rng.integers(0, communities, size=m_in)
    u_in = c * size + rng.integers(0, size, size=m_in)
    v_in = c * size + rng.integers(0, size, size=m_in)
    u_out = rng.integers(0, M, size=m - m_in)
    v_out = rng.integers(0, M, size=m - m_in)
    u = np.concatenate([u_in, u_out])
    v = np.concatenate([v_in, v_out])
    # Shuffle, then locality-reorder: the composition is a community-preserving
    # relabelling (random community order, random order inside each).
    corder = rng.permutation(communities)
    inner = np.argsort(rng.random((communities, size)), axis=1)
    new_id = np.empty(M, dtype=np.int64)
    for pos, cc in enumerate(corder):
        new_id[cc * size + inner[cc]] = pos * size + np.arange(size)
    rowptr, colind = _symmetric(new_id[u], new_id[v], M)
    vals = gcn_norm_values(rowptr, colind).astype(np.float16).astype(np.float32)
    return Graph(rowptr, colind, vals, M, M, f"sbm_{communities}x{size}")


def lognormal_social(M: int = 250_000, avg_deg: float = 500.0, sigma: float = 1.0,
                     min_deg: int = 1, max_deg: int = 20_000, seed: int = 4) -> Graph:
    """Directed graph with log-normal out-degrees (mean avg_deg, clipped) and
    destinations drawn proportional to the same degree weights (social-style
    popularity).  Values: GCN normalisation rounded to fp16."""
    rng = np.random.default_rng(seed)
    mu = np.log(avg_deg) - sigma * sigma / 2.0
    deg = np.clip(np.rint(rng.lognormal(mu, sigma, size=M)), min_deg, max_deg).astype(np.int64)
    total = int(deg.sum())
    rows = np.repeat(np.arange(M, dtype=np.int64), deg)
    cols = _weighted_endpoints(rng, deg.astype(np.float64), total)
    rowptr, colind = _csr_from_keys(rows * M + cols, M, M)
    del rows, cols
    vals = gcn_norm_values(rowptr, colind).astype(np.float16).astype(np.float32)
    return Graph(rowptr, colind, vals, M, M, f"lognormal_{M}_{avg_deg}")


def gcn_operator(g: Graph) -> Graph:
    """A_hat = D~^-1/2 (A + I) D~^-1/2 with D~ = rowsum(A + I); the diagonal is
    added only where absent (gnn_bench/router_vs_baselines_gcn.py:89-126).
    Binary adjacency is assumed (the structure of g, values ignored)."""
    M = g.M
    deg = np.diff(g.rowptr.astype(np.int64))
    rows = np.repeat(np.arange(M, dtype=np.int64), deg)
    keys = np.concatenate([rows * M + g.colind.astype(np.int64),
                           np.arange(M, dtype=np.int64) * (M + 1)])
    rowptr, colind = _csr_from_keys(keys, M, M)
    d = np.diff(rowptr.astype(np.int64)).astype(np.float64)
    dis = 1.0 / np.sqrt(d)
    r = np.repeat(np.arange(M), np.diff(rowptr.astype(np.int64)))
    vals = (dis[r] * dis[colind]).astype(np.float32)
    return Graph(rowptr, colind, vals, M, M, "gcn_" + g.name)


def transpose(g: Graph) -> Graph:
    """CSR of A^T (sorted, values carried)."""
    deg = np.diff(g.rowptr.astype(np.int64))
    rows = np.repeat(np.arange(g.M, dtype=np.int64), deg)
    order = np.lexsort((rows, g.colind))
    t_rows = g.colind[order].astype(np.int64)
    rowptr = np.zeros(g.K + 1, dtype=np.int64)
    np.cumsum(np.bincount(t_rows, minlength=g.K), out=rowptr[1:])
    return Graph(rowptr.astype(np.int32), rows[order].astype(np.int32), g.vals[order], g.K, g.M,
                 g.name + "_T")


def random_csr(M: int, K: int, avg_deg: float, seed: int = 0, skew: float = 0.0,
               max_deg: int | None = None, empty_frac: float = 0.0) -> Graph:
    """Small test matrices: row lengths Poisson(avg_deg) (skew > 0 mixes in a
    power-law tail), columns uniform without duplicates, values N(0,1)."""
    rng = np.random.default_rng(seed)
    deg = rng.poisson(avg_deg, size=M).astype(np.int64)
    if skew > 0:
        tail = (rng.pareto(skew, size=M) * avg_deg).astype(np.int64)
        pick = rng.random(M) < 0.05
        deg = np.where(pick, deg + tail, deg)
    if empty_frac > 0:
        deg[rng.random(M) < empty_frac] = 0
    deg = np.minimum(deg, K if max_deg is None else min(K, max_deg))
    rowptr = np.zeros(M + 1, dtype=np.int64)
    np.cumsum(deg, out=rowptr[1:])
    cols = np.empty(int(rowptr[-1]), dtype=np.int32)
    for r in range(M):
        d = int(deg[r])
        if d:
            cols[rowptr[r]:rowptr[r + 1]] = np.sort(rng.choice(K, size=d, replace=False))
    vals = rng.standard_normal(int(rowptr[-1])).astype(np.float32)
    return Graph(rowptr.astype(np.int32), cols, vals, M, K, f"random_{M}x{K}")


def degree_sequence(rng, M: int, avg_deg: float, cv: float, max_deg: int) -> np.ndarray:
    """Row lengths with mean ~avg_deg and population CV ~cv, clipped to
    [1, max_deg].  cv < 0.7: gamma-Poisson mixture (CV^2 = 1/k + 1/avg);
    otherwise log-normal with sigma^2 = ln(1 + cv^2), rescaled after clipping."""
    if cv * cv <= 1.0 / avg_deg:
        deg = rng.poisson(avg_deg, size=M)
    elif cv < 0.7:
        k = 1.0 / (cv * cv - 1.0 / avg_deg)
        deg = rng.poisson(rng.gamma(k, avg_deg / k, size=M))
    else:
        sigma = float(np.sqrt(np.log1p(cv * cv)))
        z = rng.standard_normal(M)
        scale = avg_deg
        for _ in range(30):  # mean after clipping and rounding -> avg_deg
            raw = np.exp(sigma * z - sigma * sigma / 2.0) * scale
            deg = np.clip(np.rint(raw), 1, max_deg)
            scale *= avg_deg / max(deg.mean(), 1e-9)
    return np.clip(deg, 1, max_deg).astype(np.int64)


def regime_graph(M: int, avg_deg: float, cv: float, locality: float = 0.0, window: int = 256,
                 popular: bool = False, seed: int = 0, max_deg: int | None = None,
                 name: str = "") -> Graph:
    """Directed graph of a routing regime: row lengths from degree_sequence;
    a fraction `locality` of each row's columns lies within +-window of the
    row (banded, as road and web graphs), the rest uniform over the columns,
    or drawn proportional to the row lengths when `popular` (social-style
    hubs among the columns).  Duplicates are dropped, so the realised degree
    features are measured, not assumed.  GCN-normalised fp32 values."""
    rng = np.random.default_rng(seed)
    K = M
    deg = degree_sequence(rng, M, avg_deg, cv, max_deg or min(K, 50_000))
    rows = np.repeat(np.arange(M, dtype=np.int64), deg)
    total = rows.size
    near = rng.random(total) < locality
    cols = np.empty(total, dtype=np.int64)
    n_near = int(near.sum())
    cols[near] = np.clip(rows[near] + rng.integers(-window, window + 1, size=n_near), 0, K - 1)
    far = ~near
    if popular:
        cols[far] = _weighted_endpoints(rng, deg.astype(np.float64), total - n_near)
    else:
        cols[far] = rng.integers(0, K, size=total - n_near)
    rowptr, colind = _csr_from_keys(rows * K + cols, M, K)
    del rows, cols
    return Graph(rowptr, colind, gcn_norm_values(rowptr, colind), M, K,
                 name or f"regime_{M}_{avg_deg}_{cv}")


# Calibration suite of the router on gfx950: one or more graphs per region of
# the seven-rule tree (router/router_dispatch.cpp:1036-1094) that the five
# benchmark configurations leave empty.  Keys name the rule and branch the
# graph is built to land in; the realised (d, cv, M) decide.
REGIMES = {
    "R1_extreme": lambda: chung_lu(200_000, 8.0, 2.0, 20_000, seed=11),
    "R2_ultralow_road": lambda: regime_graph(1_000_000, 3.0, 0.3, 0.95, 64, seed=12, name="R2_ultralow_road"),
    "R2_community_lowd": lambda: regime_graph(200_000, 6.0, 0.4, 0.8, 512, seed=13, name="R2_community_lowd"),
    "R2_uniform": lambda: er(500_000, 16.0, seed=14),
    "R3_medium": lambda: regime_graph(100_000, 12.0, 4.0, seed=15, name="R3_medium"),
    "R3_medium_pop": lambda: regime_graph(150_000, 20.0, 3.5, popular=True, seed=16, name="R3_medium_pop"),
    "R3_large": lambda: regime_graph(500_000, 12.0, 4.0, seed=17, name="R3_large"),
    "R4_dense": lambda: regime_graph(50_000, 80.0, 1.0, popular=True, seed=18, name="R4_dense"),
    "R5_small_dense": lambda: regime_graph(15_000, 30.0, 0.9, seed=19, name="R5_small_dense"),
    "R5_small_skew": lambda: regime_graph(8_000, 32.0, 1.4, 0.3, 256, popular=True, seed=20,
                                          name="R5_small_skew"),
    "R6_heavy": lambda: regime_graph(200_000, 30.0, 2.2, popular=True, seed=21, name="R6_heavy"),
    "R7_web": lambda: regime_graph(300_000, 6.0, 1.3, 0.7, 256, seed=22, name="R7_web"),
    "R8_mid": lambda: regime_graph(300_000, 12.0, 1.2, 0.3, 1024, seed=23, name="R8_mid"),
    "R8_lowd": lambda: regime_graph(500_000, 4.0, 1.0, seed=24, name="R8_lowd"),
    "R8_small": lambda: regime_graph(20_000, 8.0, 1.0, seed=25, name="R8_small"),
    "R2_uniform_banded": lambda: regime_graph(300_000, 10.0, 0.3, 0.9, 256, seed=26, name="R2_uniform_banded"),
    "R3_large_local": lambda: regime_graph(400_000, 10.0, 4.2, 0.5, 512, seed=27, name="R3_large_local"),
    "R4_dense_wide": lambda: regime_graph(100_000, 60.0, 0.8, seed=28, name="R4_dense_wide"),
    "R6_heavy_local": lambda: regime_graph(300_000, 28.0, 2.5, 0.5, 512, popular=True, seed=29,
                                           name="R6_heavy_local"),
    "R7_web_popular": lambda: regime_graph(500_000, 8.0, 1.2, 0.8, 128, popular=True, seed=30,
                                           name="R7_web_popular"),
    "R8_mid_uniform": lambda: regime_graph(200_000, 20.0, 1.0, seed=31, name="R8_mid_uniform"),
    "R8_lowd_banded": lambda: regime_graph(400_000, 4.5, 0.9, 0.8, 64, seed=32, name="R8_lowd_banded"),
}


# Held-out graphs for the router calibration: the same generators with other
# sizes, degrees, skews, localities and seeds, never used to set a knob; they
# check that the MI355X table carries beyond the suite it was set on
# (the reference's unseen-graph validation, experiments/unseen_validation.py).
HELDOUT = {
    "H1_extreme_small": lambda: chung_lu(60_000, 10.0, 2.05, 8_000, seed=41),
    "H2_uniform_mid": lambda: er(250_000, 24.0, seed=42),
    "H2_lowd_banded": lambda: regime_graph(700_000, 3.5, 0.45, 0.9, 128, seed=43, name="H2_lowd_banded"),
    "H3_skewed_pop": lambda: regime_graph(350_000, 15.0, 3.6, popular=True, seed=44, name="H3_skewed_pop"),
    "H4_dense_skew": lambda: regime_graph(80_000, 120.0, 1.6, 0.3, 512, popular=True, seed=45,
                                          name="H4_dense_skew"),
    "H5_small_dense": lambda: regime_graph(12_000, 32.0, 0.8, 0.5, 256, seed=46, name="H5_small_dense"),
    "H6_heavy": lambda: regime_graph(150_000, 35.0, 2.6, 0.2, 256, popular=True, seed=47, name="H6_heavy"),
    "H7_web": lambda: regime_graph(400_000, 7.0, 1.25, 0.6, 512, seed=48, name="H7_web"),
    "H8_mid_local": lambda: regime_graph(250_000, 16.0, 1.5, 0.6, 2048, seed=49, name="H8_mid_local"),
    "H8_small_skew": lambda: regime_graph(15_000, 6.0, 1.8, seed=50, name="H8_small_skew"),
}


CONFIGS = {
    "C1": lambda: er(10_000, 8.0, seed=1),
    "C2": lambda: chung_lu(1_000_000, 16.0, 2.1, 50_000, seed=2),
    "C3": lambda: sbm(1024, 500, 32.0, 0.9, seed=3),
    "C4": lambda: lognormal_social(250_000, 500.0, 1.0, 1, 20_000, seed=4),
    "C5": lambda: gcn_operator(chung_lu(1_000_000, 25.0, 2.3, 50_000, seed=5)),
}
CONFIG_N = {"C1": 64, "C2": 128, "C3": 256, "C4": 512, "C5": 256}
CONFIG_DTYPE = {"C1": "f32", "C2": "f32", "C3": "f16", "C4": "f16", "C5": "f32"}
