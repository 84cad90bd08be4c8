"""TEST INFRASTRUCTURE ONLY: CPU restatement of the large-regime EEQ operator and charges.

Checker of ``xnn_amd.eeq`` (the GPU large regime). It restates the operator of the
reference's ``EEQSystem`` (src/xnn/common/models/eeq.py:170-397: Ewald split at
``alpha = erfc^-1(eps) / r_c``, the screened kernel ``[erf(gamma r) - erf(alpha r)] / r``
over every image within ``r_c``, the reciprocal sum over ``exp(-G^2 / 4 alpha^2) >= eps``,
the diagonal ``J + sqrt(2/pi) / a - 2 alpha / sqrt(pi)``) and the constrained solve of
``eeq_charges_large`` (eeq.py:664), brute force in float64 NumPy: every image of every
pair, the full reciprocal set (G and -G both), a dense solve of the bordered system.
Small systems only (O(N^2 images)).
"""
from __future__ import annotations

import math
from typing import Optional

import numpy as np

EPS = 1e-10


def erfc_inverse(eps: float) -> float:
    lo, hi = 0.0, 10.0
    for _ in range(200):                      # bisection: independent of the product's Newton
        mid = 0.5 * (lo + hi)
        if math.erfc(mid) > eps:
            lo = mid
        else:
            hi = mid
    return 0.5 * (lo + hi)


def ewald_matrix(pos: np.ndarray, cell: Optional[np.ndarray], rad: np.ndarray, cutoff: float,
                 eps: float = EPS) -> np.ndarray:
    """The off-diagonal operator R + A_rec (N, N) in bohr units (cell rows; None: molecule)
    plus, for a cell, the ``-2 alpha / sqrt(pi)`` self term on the diagonal."""
    from scipy.special import erf
    n = len(pos)
    gam = 1.0 / np.sqrt(rad[:, None] ** 2 + rad[None, :] ** 2)
    A = np.zeros((n, n))
    if cell is None:
        d = pos[None, :, :] - pos[:, None, :]
        r = np.sqrt((d * d).sum(-1))
        off = ~np.eye(n, dtype=bool) & (r <= cutoff)
        A[off] = erf(gam[off] * r[off]) / r[off]
        return A
    alpha = erfc_inverse(eps) / cutoff
    inv = np.linalg.inv(cell)
    spacing = 1.0 / np.linalg.norm(inv, axis=0)
    reps = [int(math.ceil(cutoff / s)) + 1 for s in spacing]
    for a in range(-reps[0], reps[0] + 1):
        for b in range(-reps[1], reps[1] + 1):
            for c in range(-reps[2], reps[2] + 1):
                t = a * cell[0] + b * cell[1] + c * cell[2]
                d = pos[None, :, :] + t - pos[:, None, :]
                r = np.sqrt((d * d).sum(-1))
                use = (r <= cutoff) & (r > 1e-10)
                A[use] += (erf(gam[use] * r[use]) - erf(alpha * r[use])) / r[use]
    vol = abs(np.linalg.det(cell))
    recip = 2.0 * math.pi * inv.T
    g_max = 2.0 * alpha * math.sqrt(-math.log(eps))
    span = [int(g_max * np.linalg.norm(cell[k]) / (2 * math.pi)) + 1 for k in range(3)]
    for a in range(-span[0], span[0] + 1):
        for b in range(-span[1], span[1] + 1):
            for c in range(-span[2], span[2] + 1):
                if a == b == c == 0:
                    continue
                g = a * recip[0] + b * recip[1] + c * recip[2]
                g2 = float(g @ g)
                if g2 > g_max * g_max:
                    continue
                w = 4 * math.pi / vol * math.exp(-g2 / (4 * alpha * alpha)) / g2
                ph = pos @ g
                A += w * np.cos(ph[:, None] - ph[None, :])
    A[np.diag_indices(n)] -= 2.0 * alpha / math.sqrt(math.pi)
    return A


def charges(pos: np.ndarray, cell: Optional[np.ndarray], rad: np.ndarray, diag: np.ndarray,
            x: np.ndarray, total: float, cutoff: float, eps: float = EPS) -> np.ndarray:
    """``[[A, 1], [1^T, 0]] [q; mu] = [x; Q]`` with ``A = ewald_matrix + diag(J + sqrt(2/pi)/a)``
    (``diag`` given without the Ewald self term), dense solve."""
    n = len(pos)
    A = ewald_matrix(pos, cell, rad, cutoff, eps) + np.diag(diag)
    M = np.zeros((n + 1, n + 1))
    M[:n, :n] = A
    M[:n, n] = M[n, :n] = 1.0
    rhs = np.concatenate([x, [total]])
    return np.linalg.solve(M, rhs)[:n]


def _full_reciprocal_set(cell: np.ndarray, alpha: float, eps: float):
    """Every G != 0 (G and -G both) with exp(-G^2 / 4 alpha^2) >= eps and its weight
    4 pi / V exp(-G^2 / 4 alpha^2) / G^2, as in ewald_matrix."""
    vol = abs(np.linalg.det(cell))
    recip = 2.0 * math.pi * np.linalg.inv(cell).T
    g_max = 2.0 * alpha * math.sqrt(-math.log(eps))
    span = [int(g_max * np.linalg.norm(cell[k]) / (2 * math.pi)) + 1 for k in range(3)]
    m = np.stack(np.meshgrid(*[np.arange(-s, s + 1) for s in span], indexing="ij"), -1).reshape(-1, 3)
    g = m @ recip
    g2 = (g * g).sum(1)
    keep = (g2 <= g_max * g_max) & (g2 > 0)
    g, g2 = g[keep], g2[keep]
    return g, 4 * math.pi / vol * np.exp(-g2 / (4 * alpha * alpha)) / g2


def operator_rows(pos: np.ndarray, cell: np.ndarray, rad: np.ndarray, diag: np.ndarray,
                  q: np.ndarray, rows, cutoff: float, eps: float = EPS) -> np.ndarray:
    """``(A q)[rows]`` for the periodic operator of :func:`charges` (ewald_matrix plus
    diag(J + sqrt(2/pi)/a)) without forming A, for systems too large for it: the real-space
    part over every image of every pair of the sampled rows, the reciprocal part from the
    structure factors of q on the full set, sum_G w_G [cos(G r_i) C_G + sin(G r_i) S_G]
    with C_G, S_G = sum_j q_j cos, sin(G r_j). O(N_G N + len(rows) N images)."""
    from scipy.special import erf
    alpha = erfc_inverse(eps) / cutoff
    inv = np.linalg.inv(cell)
    spacing = 1.0 / np.linalg.norm(inv, axis=0)
    reps = [int(math.ceil(cutoff / s)) + 1 for s in spacing]
    shifts = np.stack(np.meshgrid(*[np.arange(-r, r + 1) for r in reps], indexing="ij"),
                      -1).reshape(-1, 3) @ cell
    g, w = _full_reciprocal_set(cell, alpha, eps)
    cs = np.zeros(len(g))
    sn = np.zeros(len(g))
    for k0 in range(0, len(g), 256):
        ph = pos @ g[k0:k0 + 256].T
        cs[k0:k0 + 256] = q @ np.cos(ph)
        sn[k0:k0 + 256] = q @ np.sin(ph)
    out = []
    for i in rows:
        gam = 1.0 / np.sqrt(rad[i] ** 2 + rad ** 2)
        acc = 0.0
        for t in shifts:
            d = pos + t - pos[i]
            r = np.sqrt((d * d).sum(1))
            use = (r <= cutoff) & (r > 1e-10)
            acc += float(((erf(gam[use] * r[use]) - erf(alpha * r[use])) / r[use]) @ q[use])
        ph = g @ pos[i]
        acc += float(w @ (np.cos(ph) * cs + np.sin(ph) * sn))
        acc += (diag[i] - 2.0 * alpha / math.sqrt(math.pi)) * q[i]
        out.append(acc)
    return np.array(out)
