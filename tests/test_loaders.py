"""On-disk loaders (ra_real_graph_eval.py:83-204) against hand-computed CSRs
and against the pure-Python restatement in oracle/loaders_oracle.py."""
import json
import os

import numpy as np
import pytest
import scipy.sparse as sp

from ra_spmm import loaders as L

from oracle import loaders_oracle as LO


def _write(tmp_path, name, text):
    p = tmp_path / name
    p.write_text(text)
    return str(p)


def _csr(d):
    return d["rowptr"].numpy().tolist(), d["colind"].numpy().tolist(), d["vals"].numpy().tolist(), d["M"]


def test_hand_computed_edge_list(tmp_path):
    text = """# comment line
% matrix-market style comment
0 2
0 1 7.5
0\t1
2 2

3 0 extra fields here
x 1
1 y
4
1.5 2
  1   3
"""
    p = _write(tmp_path, "g.txt", text)
    # Accepted edges: (0,2) (0,1) (0,1) (2,2) (3,0) (1,3); max id 3 -> n = 4.
    rp, ci, vl, n = _csr(L.load_edge_list(p))
    assert n == 4
    assert rp == [0, 2, 3, 4, 5]
    assert ci == [1, 2, 3, 2, 0]
    assert vl == [1.0] * 5
    # symmetrize adds reverses of non-loop edges, then de-duplicates.
    rp, ci, _, n = _csr(L.load_edge_list(p, symmetrize=True))
    assert rp == [0, 3, 5, 7, 9]
    assert ci == [1, 2, 3, 0, 3, 0, 2, 0, 1]
    # M_hint pads empty rows.
    rp, ci, _, n = _csr(L.load_edge_list(p, M_hint=6))
    assert n == 6 and rp == [0, 2, 3, 4, 5, 5, 5]


def test_one_indexed_and_negative_ids(tmp_path):
    p = _write(tmp_path, "g1.txt", "1 2\n2 3\n3 1\n")
    rp, ci, _, n = _csr(L.load_edge_list(p, one_indexed=True))
    assert n == 3 and rp == [0, 1, 2, 3] and ci == [1, 2, 0]
    q = _write(tmp_path, "g0.txt", "0 1\n")
    with pytest.raises(ValueError, match="negative"):
        L.load_edge_list(q, one_indexed=True)


@pytest.mark.parametrize("seed", range(6))
def test_edge_list_matches_reference_restatement(tmp_path, seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(5, 60))
    lines = []
    for _ in range(int(rng.integers(0, 400))):
        r = rng.random()
        a, b = rng.integers(0, n, 2)
        if r < 0.05:
            lines.append("# " + " ".join(["w"] * int(rng.integers(0, 5))))
        elif r < 0.08:
            lines.append("")
        elif r < 0.10:
            lines.append(f"{a}")
        elif r < 0.12:
            lines.append(f"{a}.0 {b}")
        elif r < 0.20:
            lines.append(f"{a}\t{b}\t{rng.random():.3f}")
        elif r < 0.25:
            lines.append(f"  {a} {a}")
        else:
            lines.append(f"{a} {b}")
    p = _write(tmp_path, f"r{seed}.txt", "\n".join(lines) + "\n")
    for sym in (False, True):
        for hint in (0, n + 3):
            got = _csr(L.load_edge_list(p, symmetrize=sym, M_hint=hint))
            ref = LO.load_edge_list_reference(p, False, sym, False, hint)
            assert got == tuple(ref)


def test_npz_layouts(tmp_path):
    rng = np.random.default_rng(1)
    A = sp.random(30, 30, density=0.1, random_state=2, format="csr", dtype=np.float32)
    # scipy save_npz layout (indptr / indices / data + format, shape)
    sp.save_npz(tmp_path / "s.npz", A)
    d = L.load_npz(str(tmp_path / "s.npz"))
    assert d["M"] == d["K"] == 30
    np.testing.assert_array_equal(d["rowptr"].numpy(), A.indptr)
    np.testing.assert_array_equal(d["colind"].numpy(), A.indices)
    np.testing.assert_array_equal(d["vals"].numpy(), A.data)
    # custom rowptr / colind (no vals -> ones)
    np.savez(tmp_path / "c.npz", rowptr=A.indptr, colind=A.indices)
    d = L.load_npz(str(tmp_path / "c.npz"))
    np.testing.assert_array_equal(d["vals"].numpy(), np.ones(A.nnz, np.float32))
    # edge_index: rows sorted by (src, dst), duplicates kept
    ei = rng.integers(0, 25, (2, 200))
    np.savez(tmp_path / "e.npz", edge_index=ei)
    d = L.load_npz(str(tmp_path / "e.npz"))
    rp, ci = LO.load_npz_edge_index_reference(ei)
    assert d["rowptr"].numpy().tolist() == rp and d["colind"].numpy().tolist() == ci
    assert d["M"] == int(ei.max()) + 1
    np.savez(tmp_path / "bad.npz", foo=np.zeros(3))
    with pytest.raises(ValueError, match="Unknown NPZ"):
        L.load_npz(str(tmp_path / "bad.npz"))
    np.savez(tmp_path / "obj.npz", rowptr=np.array([0, 1], dtype=object), colind=np.array([0]))
    with pytest.raises(ValueError):
        L.load_npz(str(tmp_path / "obj.npz"))


def test_manifest_and_dataset(tmp_path):
    os.makedirs(tmp_path / "datasets")
    (tmp_path / "datasets" / "tiny.txt").write_text("0 1\n1 2\n")
    man = {"datasets": [
        {"name": "tiny", "path": "datasets/tiny.txt", "format": "edge", "symmetrize": True, "M": 4},
        {"name": "absent", "path": "datasets/none.txt", "format": "edge"},
    ]}
    (tmp_path / "m.json").write_text(json.dumps(man))
    entries = L.load_manifest(str(tmp_path / "m.json"))
    d = L.load_dataset(entries[0])
    assert d["M"] == 4 and d["rowptr"].numpy().tolist() == [0, 1, 3, 4, 4]
    assert L.load_dataset(entries[1]) is None
