"""TEST INFRASTRUCTURE ONLY: CPU restatement of the reference's D3 two-body dispersion.

Used by ``tests/`` as the checker of the HIP D3 kernels and by
``tests/golden/make_dispersion_tables.py`` to derive the per-element tables. Float64
PyTorch on the CPU; gradients from autograd.

Reference (molssi-ai/xnn, src/xnn/common/models/):
  d3.py:464-478      constants (k1 = 16, k3 = 4), cutoffs, PBE0 parameter sets
  d3.py:194-219      reference_tables ("2024" set: the stored tables as they are)
  d3.py:617-628      derived tables: 4/3-scaled covalent radii (bohr), r4r2, rvdw (bohr)
  d3.py:632-649      coordination_numbers (exponential count), reference_weights
  d3.py:651-674      species vectors / pair C6 = sum_ab W_ia W_jb C6ref[a, b, Z_i, Z_j]
  d3.py:678-722      pair_radius, two_body_energy (bj / zero / mzero / op damping)
  dispersion.py:70-121 gaussian_reference_weights (one Gaussian per reference, exact-zero
                       norm fallback)
Golden values: tests/common/test_d3.py:112-119 (simple-dftd3 1.6.0, PBE0, water).
"""
from __future__ import annotations

import math
from typing import Dict, Sequence

import numpy as np
import torch

from oracle.d4 import BOHR, pair_images, edge_vectors_au, switching

KCN, WF = 16.0, 4.0
PBE0_D3BJ = {"s6": 1.0, "s8": 1.2177, "a1": 0.4145, "a2": 4.8593, "rs6": 1.287, "rs8": 1.0,
             "alp": 14.0, "bet": 0.0}
PBE0_D3ZERO = {"s6": 1.0, "s8": 0.928, "a1": 0.4145, "a2": 4.8593, "rs6": 1.287, "rs8": 1.0,
               "alp": 14.0, "bet": 0.0}


def derive_tables(raw: Dict[str, np.ndarray], elements: Sequence[int]) -> Dict[str, np.ndarray]:
    """Compact per-element tables for ``elements`` (the "2024" reference set): ``z``,
    ``rcov`` (4/3-scaled covalent radii, bohr), ``r4r2`` = sqrt(0.5 <r4>/<r2> sqrt(Z)),
    ``rvdw`` (pair cutoff radii, bohr, (S, S)), ``nref`` (S,), ``refcn`` (7, S) and
    ``c6ref`` (7, 7, S, S) indexed [ref_i, ref_j, species_i, species_j]."""
    z = np.asarray(list(elements), dtype=np.int64)
    zz = np.arange(raw["r4r2_raw"].shape[0], dtype=np.float64)
    return {
        "z": z,
        "rcov": (4.0 / 3.0 * raw["covalent_radius_aa"] / BOHR)[z],
        "r4r2": np.sqrt(0.5 * raw["r4r2_raw"] * np.sqrt(zz))[z],
        "rvdw": (raw["rvdw_aa"] / BOHR)[np.ix_(z, z)],
        "nref": raw["nref"][z].astype(np.int64),
        "refcn": raw["refcn"][:, z],
        "c6ref": raw["c6"][:, :, z][:, :, :, z],
    }


def species_of(tables, numbers) -> torch.Tensor:
    lut = {int(v): k for k, v in enumerate(tables["z"])}
    return torch.as_tensor([lut[int(x)] for x in numbers], dtype=torch.long)


def coordination_numbers(s, dst, src, r_au, tables, cutoff_cn_au, n_atoms):
    """CN_i = sum_j 1 / (1 + exp(-k1 (rc / r - 1))) within the CN cutoff (d3.py:632-642)."""
    rcov = torch.as_tensor(tables["rcov"])
    rc = rcov[s[dst]] + rcov[s[src]]
    count = 1.0 / (1.0 + torch.exp(-KCN * (rc / r_au - 1.0)))
    count = torch.where(r_au <= cutoff_cn_au, count, torch.zeros_like(count))
    return torch.zeros(n_atoms, dtype=r_au.dtype).index_add(0, torch.as_tensor(dst), count)


def weights(s, cn, tables):
    """One Gaussian exp(-4 (CN - CN_ref)^2) per reference, normalized; the largest-CN
    reference(s) when the norm is exactly zero (dispersion.py:70-121 with ngw None)."""
    refcn = torch.as_tensor(tables["refcn"])[:, s].t()
    valid = torch.arange(refcn.shape[1])[None, :] < torch.as_tensor(tables["nref"])[s][:, None]
    gw = torch.where(valid, torch.exp(-WF * (cn[:, None] - refcn) ** 2), torch.zeros_like(refcn))
    norm = gw.sum(1)
    ok = norm > 0.0
    w = gw / torch.where(ok, norm, torch.ones_like(norm))[:, None]
    top = torch.where(valid, refcn, torch.full_like(refcn, -math.inf)).max(1).values
    fb = (valid & ((refcn - top[:, None]).abs() < 1e-12)).to(cn.dtype)
    return torch.where(ok[:, None], w, fb)


def pair_c6(s, w, i, j, tables):
    """C6_ij = sum_ab W_i[a] W_j[b] C6ref[a, b, Z_i, Z_j] (d3.py:651-674)."""
    c6ref = torch.as_tensor(tables["c6ref"])               # (7, 7, S, S)
    block = c6ref[:, :, s[i], s[j]].permute(2, 0, 1)        # (E, 7, 7)
    return torch.einsum("ea,eab,eb->e", w[i], block, w[j])


def two_body(s, dst, src, r_au, c6, tables, prm, damping, cutoff_pair_au, width_au, n_atoms):
    """Per-atom two-body energy for the damping variants (d3.py:678-722)."""
    r4r2 = torch.as_tensor(tables["r4r2"])
    zi, zj = s[dst], s[src]
    rr = 3.0 * r4r2[zi] * r4r2[zj]
    if damping in ("bj", "op"):
        r0 = prm["a1"] * torch.sqrt(rr) + prm["a2"]
    else:
        r0 = torch.as_tensor(tables["rvdw"])[zi, zj]
    r = r_au
    r2 = r * r
    r6, r8 = r2 ** 3, r2 ** 4
    alp, bet = prm["alp"], prm["bet"]
    if damping == "bj":
        t6, t8 = 1.0 / (r6 + r0 ** 6), 1.0 / (r8 + r0 ** 8)
    elif damping == "zero":
        t6 = 1.0 / (1.0 + 6.0 * (prm["rs6"] * r0 / r) ** alp) / r6
        t8 = 1.0 / (1.0 + 6.0 * (prm["rs8"] * r0 / r) ** (alp + 2.0)) / r8
    elif damping == "mzero":
        t6 = 1.0 / (1.0 + 6.0 * (r / (prm["rs6"] * r0) + bet * r0) ** (-alp)) / r6
        t8 = 1.0 / (1.0 + 6.0 * (r / (prm["rs8"] * r0) + bet * r0) ** (-(alp + 2.0))) / r8
    else:
        rb, ab = r ** bet, r0 ** bet
        t6 = rb / (rb * r6 + ab * r0 ** 6)
        t8 = rb / (rb * r8 + ab * r0 ** 8)
    sw = switching(r, cutoff_pair_au, width_au)
    e = -0.5 * c6 * sw * (prm["s6"] * t6 + prm["s8"] * rr * t8)
    e = torch.where(r <= cutoff_pair_au, e, torch.zeros_like(e))
    return torch.zeros(n_atoms, dtype=r.dtype).index_add(0, torch.as_tensor(dst), e)


def d3(pos_aa: np.ndarray, numbers, tables, damping: str = "bj", prm=None,
       cell: np.ndarray = None, cutoffs_au=(60.0, 40.0), width_au: float = 0.0) -> dict:
    """Two-body D3 energy (hartree), CN, weights and pair list of one structure."""
    prm = prm or (PBE0_D3BJ if damping in ("bj", "op") else PBE0_D3ZERO)
    cut_pair, cut_cn = cutoffs_au
    s = species_of(tables, numbers)
    pos = torch.as_tensor(pos_aa, dtype=torch.float64)
    ct = None if cell is None else torch.as_tensor(cell, dtype=torch.float64)
    dst, src, sh = pair_images(pos_aa, cell, max(cutoffs_au) * BOHR)
    v = edge_vectors_au(pos, ct, dst, src, sh)
    r = torch.linalg.norm(v, dim=-1)
    n = pos.shape[0]
    cn = coordination_numbers(s, dst, src, r, tables, cut_cn, n)
    w = weights(s, cn, tables)
    c6 = pair_c6(s, w, torch.as_tensor(dst), torch.as_tensor(src), tables)
    e2 = two_body(s, dst, src, r, c6, tables, prm, damping, cut_pair, width_au, n)
    return {"cn": cn, "weights": w, "e2": e2, "energy": e2.sum()}
