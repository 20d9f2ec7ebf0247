"""Pure-Python restatement of the reference's graph loaders — TEST
INFRASTRUCTURE ONLY (imported by tests/, never by the product).

Follows ra_real_graph_eval.py:83-178 step by step (line loop, list-based CSR
build, per-row sorted(set(...)) de-duplication, the three .npz layouts), for
small files.  Pinned in tests/test_loaders.py by hand-computed CSRs of small
files (comments, duplicates, self loops, one-indexed ids, symmetrize, M_hint).
Negative ids are outside what it restates (the reference wraps them into the
last row through Python list indexing); the product raises on them.
"""
from collections import Counter

import numpy as np


def load_edge_list_reference(path, directed, symmetrize, one_indexed, M_hint=0):
    """ra_real_graph_eval.py:83-143 -> (rowptr, colind, vals, n) as lists."""
    edges = []
    max_node = 0
    with open(path) as f:
        for line in f:
            line = line.strip()
            if not line or line.startswith("#") or line.startswith("%"):
                continue
            parts = line.split()
            if len(parts) < 2:
                continue
            try:
                a, b = int(parts[0]), int(parts[1])
            except ValueError:
                continue
            if one_indexed:
                a, b = a - 1, b - 1
            edges.append((a, b))
            max_node = max(max_node, a, b)
            if symmetrize and a != b:
                edges.append((b, a))
    n = max(max_node + 1, M_hint)
    rows = [[] for _ in range(n)]
    for a, b in edges:
        if a < n:
            rows[a].append(min(b, n - 1))
    rowptr, colind = [0], []
    for r in rows:
        seg = sorted(set(r))
        colind.extend(seg)
        rowptr.append(len(colind))
    return rowptr, colind, [1.0] * len(colind), n


def load_npz_edge_index_reference(edge_index):
    """ra_real_graph_eval.py:163-173 (edge_index layout) -> (rowptr, colind)."""
    src, dst = np.asarray(edge_index[0]), np.asarray(edge_index[1])
    n = int(max(src.max(), dst.max())) + 1
    counts = Counter(src.tolist())
    rowptr = [0]
    for i in range(n):
        rowptr.append(rowptr[-1] + counts.get(i, 0))
    order = np.lexsort((dst, src))
    return rowptr, dst[order].tolist()
