"""Pins the oracle's energy derivatives: forces against central finite differences,
stress against a finite symmetric strain (the reference's own checks,
tests/common/test_d4.py:202-226), translation invariance and the force sum."""
import numpy as np
import pytest
import torch

import oracle.reference as R
from xnn_amd import synthetic

F64 = torch.float64


def _setup(seed=0):
    from oracle.nl import neighbor_list
    s = synthetic.water_box(n_molecules=27, box=9.3, grid=3, seed=seed)
    ei, sh, _ = neighbor_list(s.pos, 4.0, s.cell, s.pbc, dtype=np.float64)
    gen = torch.Generator().manual_seed(seed)
    model = dict(W=torch.randn(8, 4, generator=gen, dtype=F64),
                 U=torch.randn(4, 16, generator=gen, dtype=F64),
                 atom_ref=torch.randn(9, generator=gen, dtype=F64), l_max=3, n_rbf=8, cutoff=4.0,
                 radial="bessel", envelope="polynomial")
    g = dict(pos=torch.tensor(s.pos), numbers=torch.tensor(s.numbers),
             edge_index=torch.tensor(ei), cell_shifts=torch.tensor(sh),
             cell=torch.tensor(s.cell), batch=torch.zeros(len(s.pos), dtype=torch.long),
             n_graphs=1, model=model)
    return g


def _energy(g, pos=None, cell=None):
    out = R.energy_forces_stress(pos if pos is not None else g["pos"], g["numbers"],
                                 g["edge_index"], g["cell_shifts"],
                                 cell if cell is not None else g["cell"], g["batch"], 1,
                                 g["model"], stress=False)
    return float(out["energy"][0])


def test_forces_match_finite_differences():
    g = _setup()
    out = R.energy_forces_stress(**g)
    h = 1e-5
    for i, a in [(0, 0), (7, 2), (40, 1)]:
        pp, pm = g["pos"].clone(), g["pos"].clone()
        pp[i, a] += h
        pm[i, a] -= h
        fd = -(_energy(g, pp) - _energy(g, pm)) / (2 * h)
        assert abs(float(out["forces"][i, a]) - fd) < 1e-6 * max(1.0, abs(fd))


def test_stress_matches_finite_strain():
    g = _setup(1)
    out = R.energy_forces_stress(**g)
    vol = float(torch.linalg.det(g["cell"]).abs())
    h = 1e-5
    for a, b in [(0, 0), (1, 2), (2, 2)]:
        eps = torch.zeros(3, 3, dtype=F64)
        eps[a, b] = eps[b, a] = h
        ep = _energy(g, g["pos"] @ (torch.eye(3, dtype=F64) + eps), g["cell"] @ (torch.eye(3, dtype=F64) + eps))
        em = _energy(g, g["pos"] @ (torch.eye(3, dtype=F64) - eps), g["cell"] @ (torch.eye(3, dtype=F64) - eps))
        fd = (ep - em) / (2 * h) / vol / (1 if a == b else 2)
        assert abs(float(out["stress"][0, a, b]) - fd) < 1e-6 * max(1.0, abs(fd))


def test_translation_invariance_and_zero_net_force():
    g = _setup(2)
    out = R.energy_forces_stress(**g)
    e2 = _energy(g, g["pos"] + torch.tensor([0.3, -1.1, 2.0], dtype=F64))
    assert abs(float(out["energy"][0]) - e2) < 1e-10
    assert float(out["forces"].sum(0).abs().max()) < 1e-10
