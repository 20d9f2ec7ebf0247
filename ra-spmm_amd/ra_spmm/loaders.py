"""On-disk graph loaders of the real-graph harness.

Same entry points, formats and results as ra_real_graph_eval.py:83-204:

* ``load_edge_list(path, directed, symmetrize, one_indexed, M_hint)`` — text,
  two integer columns ``src dst`` per line; lines that are empty, start with
  ``#`` or ``%``, have fewer than two fields or whose first two fields are not
  integers are skipped; ``one_indexed`` subtracts 1; ``symmetrize`` adds
  ``(dst, src)`` for every non-loop edge; rows are sorted and de-duplicated;
  all values 1.0; ``M = K = max(max id + 1, M_hint)``.
* ``load_npz(path)`` — ``rowptr/colind[/vals]``, scipy ``indptr/indices[/data]``
  or ``edge_index`` (rows sorted by (src, dst), duplicates kept); ``K = M``.
* ``load_dataset(entry)`` — one ``paper_datasets.json`` entry (``format``
  "edge" or "npz"); ``None`` when the file is absent.

The reference parses line by line in Python; here one compiled regular
expression per 64 MB piece picks the edge lines and numpy builds the CSR.

Differences, on purpose:
  * negative node ids (e.g. a 0 in a file read with ``one_indexed``) raise
    ``ValueError``; the reference indexed Python lists with them (wrapping to
    the last row);
  * ``.npz`` files are opened with ``allow_pickle=False``: object arrays are
    refused instead of unpickled.
"""
from __future__ import annotations

import json
import os
import re
from typing import Dict, Optional

import numpy as np
import torch

__all__ = ["load_edge_list", "load_npz", "load_dataset", "load_manifest", "csr_from_edges"]

# A line is an edge when its first two whitespace-separated fields are
# integers (optional sign, decimal digits), as int(parts[0]), int(parts[1])
# accept them; comment lines ('#', '%') and short lines never match.
_WS = rb"[ \t\r\f\v]"
_EDGE_RE = re.compile(rb"^" + _WS + rb"*([+-]?[0-9]+)" + _WS + rb"+([+-]?[0-9]+)(?:" + _WS + rb"[^\n]*)?$",
                      re.MULTILINE)
_CHUNK = 64 << 20


def _read_edge_columns(path: str):
    """(src, dst) int64 arrays of the lines ra_real_graph_eval.py:88-101 accepts.
    The file is scanned in ~64 MB pieces cut at line ends."""
    src, dst = [], []
    with open(path, "rb") as f:
        tail = b""
        while True:
            block = f.read(_CHUNK)
            data = tail + block
            if not block:
                tail = b""
            else:
                cut = data.rfind(b"\n")
                if cut < 0:
                    tail = data
                    continue
                data, tail = data[:cut + 1], data[cut + 1:]
            pairs = _EDGE_RE.findall(data)
            if pairs:
                a = np.array(pairs, dtype="S").astype(np.int64)
                src.append(a[:, 0])
                dst.append(a[:, 1])
            if not block:
                break
    if not src:
        return np.zeros(0, np.int64), np.zeros(0, np.int64)
    return np.concatenate(src), np.concatenate(dst)


def csr_from_edges(src, dst, n: int, dedupe: bool = True):
    """CSR (int32 rowptr, int32 colind) of an edge list, rows sorted by column;
    duplicates removed when ``dedupe`` (ra_real_graph_eval.py:127-136)."""
    src = np.asarray(src, np.int64)
    dst = np.asarray(dst, np.int64)
    key = src * np.int64(n) + dst
    key = np.unique(key) if dedupe else np.sort(key, kind="stable")
    rows = key // n
    cols = key - rows * n
    counts = np.bincount(rows, minlength=n) if n > 0 else np.zeros(0, np.int64)
    rowptr = np.zeros(n + 1, np.int64)
    np.cumsum(counts, out=rowptr[1:])
    if rowptr[-1] > np.iinfo(np.int32).max:
        raise ValueError("graph has more than 2^31-1 edges; the int32 CSR cannot hold it")
    return rowptr.astype(np.int32), cols.astype(np.int32)


def load_edge_list(path: str, directed: bool = False, symmetrize: bool = False,
                   one_indexed: bool = False, M_hint: int = 0) -> Dict:
    """ra_real_graph_eval.py:83-143.  ``directed`` is accepted and unused, as in
    the reference."""
    del directed
    src, dst = _read_edge_columns(path)
    if one_indexed:
        src = src - 1
        dst = dst - 1
    if src.size and (src.min() < 0 or dst.min() < 0):
        raise ValueError(f"{path}: negative node id (check one_indexed)")
    max_node = int(max(src.max(), dst.max())) if src.size else 0
    if symmetrize:
        loop = src == dst
        src, dst = np.concatenate([src, dst[~loop]]), np.concatenate([dst, src[~loop]])
    n = max(max_node + 1, int(M_hint))
    rowptr, colind = csr_from_edges(src, dst, n, dedupe=True)
    return {
        "rowptr": torch.from_numpy(rowptr),
        "colind": torch.from_numpy(colind),
        "vals": torch.ones(colind.shape[0], dtype=torch.float32),
        "M": n, "K": n,
    }


def load_npz(path: str) -> Dict:
    """ra_real_graph_eval.py:146-178."""
    with np.load(path, allow_pickle=False) as data:
        keys = set(data.files)
        if "rowptr" in keys:
            rowptr = data["rowptr"].astype(np.int32)
            colind = data["colind"].astype(np.int32)
            vals = (data["vals"].astype(np.float32) if "vals" in keys
                    else np.ones(len(colind), np.float32))
        elif "indptr" in keys and "indices" in keys:
            rowptr = data["indptr"].astype(np.int32)
            colind = data["indices"].astype(np.int32)
            d = data["data"] if "data" in keys else None
            vals = (d.astype(np.float32) if d is not None and d.ndim > 0 and len(d) > 0
                    else np.ones(len(colind), np.float32))
        elif "edge_index" in keys:
            ei = data["edge_index"]
            src, dst = ei[0].astype(np.int64), ei[1].astype(np.int64)
            n = int(max(src.max(), dst.max())) + 1
            rowptr, colind = csr_from_edges(src, dst, n, dedupe=False)
            vals = np.ones(len(colind), np.float32)
        else:
            raise ValueError(f"Unknown NPZ format: {sorted(keys)}")
    M = int(rowptr.shape[0] - 1)
    return {"rowptr": torch.from_numpy(np.ascontiguousarray(rowptr)),
            "colind": torch.from_numpy(np.ascontiguousarray(colind)),
            "vals": torch.from_numpy(np.ascontiguousarray(vals)), "M": M, "K": M}


def load_manifest(path: str) -> list:
    """Entries of a ``paper_datasets.json``-style manifest, each with its
    ``path`` resolved against the manifest's directory when relative."""
    with open(path) as f:
        doc = json.load(f)
    base = os.path.dirname(os.path.abspath(path))
    out = []
    for e in doc.get("datasets", []):
        e = dict(e)
        if not os.path.isabs(e["path"]):
            e["_base_dir"] = base
        out.append(e)
    return out


def load_dataset(entry: dict, base_dir: Optional[str] = None) -> Optional[Dict]:
    """ra_real_graph_eval.py:181-204: the path as given, else relative to
    ``base_dir`` (default: the manifest's directory recorded by
    ``load_manifest``); ``None`` when the file does not exist."""
    path = entry["path"]
    if not os.path.exists(path):
        base = base_dir or entry.get("_base_dir")
        if base:
            path = os.path.join(base, entry["path"])
    if not os.path.exists(path):
        return None
    fmt = entry.get("format", "edge")
    if fmt == "edge":
        return load_edge_list(path, directed=entry.get("directed", False),
                              symmetrize=entry.get("symmetrize", False),
                              one_indexed=entry.get("one_indexed", False),
                              M_hint=entry.get("M", 0))
    if fmt == "npz":
        return load_npz(path)
    return None
