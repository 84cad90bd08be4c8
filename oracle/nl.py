"""TEST INFRASTRUCTURE ONLY: Python side of the C brute-force radius graph oracle.

:func:`neighbor_list` follows build_neighbor_list's brute force
(src/xnn/common/data/neighborlist.py:462-506) with the image repeats of
``_n_repeats`` (neighborlist.py:74-104); the arithmetic lives in ``oracle/neighbor.c``.
"""
from __future__ import annotations

import ctypes
import math
import os
from typing import Optional, Tuple

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_lib = None


def _load():
    global _lib
    if _lib is None:
        path = os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            from .build import build
            build()
        lib = ctypes.CDLL(path)
        vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        for t, ct in (("f32", ctypes.c_float), ("f64", ctypes.c_double)):
            c = getattr(lib, f"oracle_nl_count_{t}")
            c.argtypes = [vp, i64, vp, vp, vp, vp, ct, i32, ctypes.c_double, vp, vp]
            c.restype = i64
            f = getattr(lib, f"oracle_nl_fill_{t}")
            f.argtypes = [vp, i64, vp, vp, vp, vp, ct, i32, vp, i64, vp, vp]
            f.restype = None
        _lib = lib
    return _lib


def n_repeats(cell: np.ndarray, cutoff: float, pbc) -> list:
    """Images per axis from the interplanar spacing 1/|reciprocal row| (neighborlist.py:96-104)."""
    recip = np.linalg.inv(cell).T
    spacing = 1.0 / np.linalg.norm(recip, axis=1)
    return [int(math.ceil(cutoff / spacing[i])) if pbc[i] else 0 for i in range(3)]


def neighbor_list(pos: np.ndarray, cutoff: float, cell: Optional[np.ndarray] = None,
                  pbc=None, self_interaction: bool = False, dtype=np.float32,
                  margin: float = 1e-4) -> Tuple[np.ndarray, np.ndarray, int]:
    """``(edge_index (2, E), cell_shifts (E, 3), near)`` in the reference's order.

    ``near`` counts candidate pairs whose distance is within ``margin`` of the cutoff
    (margin-checked inputs have none)."""
    lib = _load()
    t = "f32" if np.dtype(dtype) == np.float32 else "f64"
    ct = ctypes.c_float if t == "f32" else ctypes.c_double
    pos = np.ascontiguousarray(pos, dtype=dtype)
    n = pos.shape[0]
    periodic = cell is not None and pbc is not None and bool(np.any(pbc))
    if periodic:
        cell_t = np.ascontiguousarray(np.asarray(cell, dtype=np.float64).reshape(3, 3), dtype=dtype)
        inv_t = np.ascontiguousarray(np.linalg.inv(np.asarray(cell, np.float64).reshape(3, 3)),
                                     dtype=dtype)
        pbc_i = np.ascontiguousarray(np.asarray(pbc, dtype=bool).astype(np.int32))
        reps = np.array(n_repeats(np.asarray(cell, np.float64).reshape(3, 3), cutoff, pbc_i),
                        dtype=np.int32)
        cp, ip = cell_t.ctypes.data, inv_t.ctypes.data
    else:
        pbc_i = np.zeros(3, np.int32)
        reps = np.zeros(3, np.int32)
        cp = ip = None
    ns = int(np.prod(2 * reps + 1))
    counts = np.zeros(ns * max(n, 1), dtype=np.int64)
    near = np.zeros(1, dtype=np.int64)
    total = getattr(lib, f"oracle_nl_count_{t}")(
        pos.ctypes.data, n, cp, ip, pbc_i.ctypes.data, reps.ctypes.data, ct(cutoff),
        int(self_interaction), float(margin), counts.ctypes.data, near.ctypes.data)
    offsets = np.zeros_like(counts)
    offsets[1:] = np.cumsum(counts)[:-1]
    edge_index = np.zeros((2, total), dtype=np.int64)
    shifts = np.zeros((total, 3), dtype=np.int64)
    getattr(lib, f"oracle_nl_fill_{t}")(
        pos.ctypes.data, n, cp, ip, pbc_i.ctypes.data, reps.ctypes.data, ct(cutoff),
        int(self_interaction), offsets.ctypes.data, total, edge_index.ctypes.data,
        shifts.ctypes.data)
    return edge_index, shifts, int(near[0])


def canonical(edge_index: np.ndarray, shifts: np.ndarray) -> np.ndarray:
    """Edges as rows ``(dst, src, sx, sy, sz)`` in lexicographic order (for set equality)."""
    rows = np.concatenate([edge_index[1][:, None], edge_index[0][:, None], shifts], axis=1)
    order = np.lexsort(rows.T[::-1])
    return rows[order]


def nearest_edges(dist: np.ndarray, dst: np.ndarray, num_nodes: int, k: int):
    """The kept edge ids of max_neighbors, by brute force: for every receiver in turn, its
    edges sorted by (length, id), the first k (neighborlist.py:509-552, the case where some
    receiver has more than k edges). A NaN length sorts after every number, as the
    reference's stable ``torch.sort`` places it."""
    out = []
    for i in range(num_nodes):
        mine = [e for e in range(len(dst)) if dst[e] == i]
        mine.sort(key=lambda e: (math.isnan(float(dist[e])),
                                 0.0 if math.isnan(float(dist[e])) else float(dist[e]), e))
        out.extend(mine[:k])
    return np.asarray(out, dtype=np.int64)
