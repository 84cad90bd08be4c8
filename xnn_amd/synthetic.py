"""Seeded synthetic inputs of the benchmark configurations (no datasets offline).

``water_box`` (the measured configuration), ``argon_fcc``, ``ragged_molecules``,
``random_molecules`` and ``organic_box`` follow the generators stated with the
configurations: rigid waters with random orientations on a jittered grid, a noisy
fcc crystal, random-walk molecules, rejection-sampled clusters and a random
organic-like periodic box. All return numpy arrays (positions in Angstrom).
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import List, Optional

import numpy as np


@dataclass
class Structure:
    pos: np.ndarray                 # (N, 3) float64
    numbers: np.ndarray             # (N,) int64
    cell: Optional[np.ndarray]      # (3, 3) or None
    pbc: Optional[np.ndarray]       # (3,) bool or None

    def as_dict(self) -> dict:
        d = {"pos": self.pos, "atomic_numbers": self.numbers}
        if self.cell is not None:
            d["cell"] = self.cell
            d["pbc"] = self.pbc
        return d


def _rotation(rng: np.random.Generator) -> np.ndarray:
    """Uniform random rotation: QR of a Gaussian matrix with det +1."""
    q, r = np.linalg.qr(rng.normal(size=(3, 3)))
    q = q * np.sign(np.diag(r))
    if np.linalg.det(q) < 0:
        q[:, 0] = -q[:, 0]
    return q


def water_box(n_molecules: int = 3000, box: float = 44.8, grid: int = 15, seed: int = 0,
              wrap: bool = True) -> Structure:
    """Rigid H2O (O-H 0.96 A, H-O-H 104.5 deg), random orientations, O on a jittered
    grid of ``grid^3`` sites (``n_molecules`` of them chosen by a seeded permutation,
    jitter N(0, 0.1 A)), cubic periodic cell. 3000 molecules in 44.8 A is 1.0 g/cm^3."""
    rng = np.random.default_rng(seed)
    spacing = box / grid
    sites = np.stack(np.meshgrid(*[np.arange(grid)] * 3, indexing="ij"), -1).reshape(-1, 3)
    chosen = sites[rng.permutation(len(sites))[:n_molecules]]
    oxygen = (chosen + 0.5) * spacing + rng.normal(0.0, 0.1, size=(n_molecules, 3))
    half = math.radians(104.5) / 2.0
    local = 0.96 * np.array([[math.sin(half), math.cos(half), 0.0],
                             [-math.sin(half), math.cos(half), 0.0]])
    pos = np.empty((3 * n_molecules, 3))
    for m in range(n_molecules):
        rot = _rotation(rng)
        pos[3 * m] = oxygen[m]
        pos[3 * m + 1:3 * m + 3] = oxygen[m] + local @ rot.T
    if wrap:
        pos = np.mod(pos, box)
    numbers = np.tile(np.array([8, 1, 1]), n_molecules)
    return Structure(pos, numbers, np.eye(3) * box, np.array([True, True, True]))


def argon_fcc(n_cells: int = 10, a: float = 5.26, sigma: float = 0.1, seed: int = 0) -> Structure:
    """fcc argon, ``n_cells^3`` conventional cells of edge ``a``, i.i.d. N(0, sigma) noise."""
    rng = np.random.default_rng(seed)
    basis = np.array([[0, 0, 0], [0.5, 0.5, 0], [0.5, 0, 0.5], [0, 0.5, 0.5]])
    cells = np.stack(np.meshgrid(*[np.arange(n_cells)] * 3, indexing="ij"), -1).reshape(-1, 1, 3)
    pos = ((cells + basis[None]) * a).reshape(-1, 3)
    pos = pos + rng.normal(0.0, sigma, size=pos.shape)
    numbers = np.full(len(pos), 18)
    return Structure(pos, numbers, np.eye(3) * (a * n_cells), np.array([True, True, True]))


def _far_enough(pos: np.ndarray, p: np.ndarray, dmin: float) -> bool:
    return len(pos) == 0 or float(np.min(np.linalg.norm(pos - p, axis=1))) >= dmin


def random_molecules(n_molecules: int = 32, counts=((6, 9), (8, 4), (1, 8)), box: float = 6.0,
                     dmin: float = 0.9, seed: int = 0) -> List[Structure]:
    """Molecules of fixed composition (default 9 C, 4 O, 8 H), positions uniform in a
    ``box`` cube, rejection-sampled to a minimum pair distance ``dmin``; no cell."""
    rng = np.random.default_rng(seed)
    numbers = np.concatenate([np.full(n, z) for z, n in counts]).astype(np.int64)
    out = []
    for _ in range(n_molecules):
        pos = np.zeros((0, 3))
        while len(pos) < len(numbers):
            p = rng.uniform(0.0, box, size=3)
            if _far_enough(pos, p, dmin):
                pos = np.vstack([pos, p])
        out.append(Structure(pos, numbers.copy(), None, None))
    return out


def ragged_molecules(n_molecules: int = 1024, n_min: int = 10, n_max: int = 60,
                     dmin: float = 0.9, seed: int = 0) -> List[Structure]:
    """Random-walk molecules: atom counts uniform in [n_min, n_max], elements
    {H: .5, C: .3, N: .1, O: .1}, steps of a random direction times U(1.1, 1.5) A from
    the previous atom, a step rejected when it lands within ``dmin`` of any atom."""
    rng = np.random.default_rng(seed)
    elements = np.array([1, 6, 7, 8])
    probs = np.array([0.5, 0.3, 0.1, 0.1])
    out = []
    for _ in range(n_molecules):
        n = int(rng.integers(n_min, n_max + 1))
        numbers = rng.choice(elements, size=n, p=probs).astype(np.int64)
        pos = np.zeros((1, 3))
        while len(pos) < n:
            d = rng.normal(size=3)
            d /= np.linalg.norm(d)
            p = pos[-1] + d * rng.uniform(1.1, 1.5)
            if _far_enough(pos, p, dmin):
                pos = np.vstack([pos, p])
        out.append(Structure(pos, numbers, None, None))
    return out


def organic_box(n_atoms: int = 5000, box: float = 36.8, dmin: float = 0.9,
                seed: int = 0) -> Structure:
    """Uniform positions in a cubic periodic cell rejected below ``dmin`` (minimum
    image), elements {H: .45, C: .35, N: .1, O: .1}."""
    rng = np.random.default_rng(seed)
    nb = max(1, int(box // dmin))
    width = box / nb
    bins: dict = {}
    pos = np.empty((n_atoms, 3))
    k = 0
    while k < n_atoms:
        p = rng.uniform(0.0, box, size=3)
        b = tuple((p // width).astype(int) % nb)
        ok = True
        for dx in (-1, 0, 1):
            for dy in (-1, 0, 1):
                for dz in (-1, 0, 1):
                    key = ((b[0] + dx) % nb, (b[1] + dy) % nb, (b[2] + dz) % nb)
                    for q in bins.get(key, ()):
                        d = p - pos[q]
                        d -= box * np.round(d / box)
                        if d @ d < dmin * dmin:
                            ok = False
                            break
                    if not ok:
                        break
                if not ok:
                    break
            if not ok:
                break
        if ok:
            pos[k] = p
            bins.setdefault(b, []).append(k)
            k += 1
    numbers = rng.choice(np.array([1, 6, 7, 8]), size=n_atoms,
                         p=np.array([0.45, 0.35, 0.1, 0.1])).astype(np.int64)
    return Structure(pos, numbers, np.eye(3) * box, np.array([True, True, True]))
