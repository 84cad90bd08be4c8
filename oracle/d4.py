"""TEST INFRASTRUCTURE ONLY: CPU restatement of the reference's D4 dispersion model.

Used by ``tests/`` as the checker of the HIP D4 kernels and of the host-side D4 module,
and by ``tests/golden/make_dispersion_tables.py`` to derive the per-element tables.
Everything is float64 PyTorch on the CPU; forces and virials come from autograd.

Reference (molssi-ai/xnn, src/xnn/common/models/):
  d4.py:114-151      model constants, PBE0-D4 parameters, Casimir-Polder grid
  d4.py:481-500      charge-scaled reference polarizabilities (setup)
  d4.py:552-591      coordination_numbers (erf count x EN factor; capped EEQ CN)
  d4.py:593-606      molecular EEQ matrix; d4.py:682-723 eeq_charges
  d4.py:984-1042     reference_weights, gaussian_weights, charge_scaling, alpha(i w)
  d4.py:1044-1071    pair_c6, two_body_energy, pair_damping
  dispersion.py:42-121  switching_function, gaussian_reference_weights
  dispersion.py:124-222 three-body ATM energy: atm_molecule (the direct triple loop that
                        pins the golden water total) and atm_edges (per-atom energies over
                        an edge list with lattice images, every corner visited)
Golden values: tests/common/test_d4.py:110-126 (dftd4 4.2.0, PBE0-D4, water).
"""
from __future__ import annotations

import math
from typing import Dict, Optional, Sequence

import numpy as np
import torch
from torch import Tensor

BOHR = 0.5291772109044924        # Angstrom per bohr (dispersion.py:37)
HARTREE = 27.21138624593551      # eV per hartree
KCN, K4, K5, K6 = 7.5, 4.10451, 19.08857, 2.0 * 11.28174 ** 2
EEQ_CN_MAX, EEQ_CN_REG = 8.0, 1.0e-14
PBE0_D4 = {"s6": 1.0, "s8": 1.20065498, "a1": 0.40085597, "a2": 5.02928789, "s9": 1.0,
           "alp": 16.0}
GA, GC, WF = 3.0, 2.0, 6.0
FREQ = [0.000001, 0.05, 0.1, 0.2, 0.3, 0.4, 0.5, 0.6, 0.7, 0.8, 0.9, 1.0,
        1.2, 1.4, 1.6, 1.8, 2.0, 2.5, 3.0, 4.0, 5.0, 7.5, 10.0]


def cp_weights() -> np.ndarray:
    """Trapezoid weights of the 23-point imaginary-frequency grid (d4.py:147-150)."""
    f = FREQ
    n = len(f)
    return np.array([0.5 * ((f[k] - f[k - 1] if k > 0 else 0.0) + (f[k + 1] - f[k] if k < n - 1 else 0.0))
                     for k in range(n)])


# --------------------------------------------------------------------------- tables
def derive_tables(raw: Dict[str, np.ndarray], ga: float = GA, gc: float = GC) -> Dict[str, np.ndarray]:
    """Per-element tables (index = atomic number) from the reference's raw arrays
    (d4.py:444-500): covalent radii scaled by 4/3 in bohr, the C8/C6 factor
    sqrt(0.5 <r4>/<r2> sqrt(Z)), and the atom-in-molecule reference polarizabilities
    alpha_ref(i w) = ascale (alphaiw - hcount * sscale secaiw zeta_X), clamped at 0."""
    out = {}
    out["rcov"] = 4.0 / 3.0 * raw["covalent_radius_aa"] / BOHR
    out["en"] = raw["pauling_en"].astype(np.float64)
    out["zeff"] = raw["zeff"].astype(np.float64)
    out["hardness"] = raw["hardness"].astype(np.float64)
    zz = np.arange(raw["r4r2_raw"].shape[0], dtype=np.float64)
    out["r4r2"] = np.sqrt(0.5 * raw["r4r2_raw"] * np.sqrt(zz))
    for k in ("eeq_chi", "eeq_eta", "eeq_kcnchi", "eeq_rad"):
        out[k] = np.nan_to_num(raw[k], nan=0.0)
    out["nref"] = raw["nref"].astype(np.int64)
    out["ngw"] = raw["ngw"].astype(np.int64)
    out["refcn"] = raw["refcn"].astype(np.float64)
    out["refq"] = raw["refq"].astype(np.float64)
    refsys = raw["refsys"]
    present = refsys > 0
    sec = np.where(present, refsys, 0)
    zeff_x = raw["zeff"][sec]
    hard_x = raw["hardness"][sec] * gc
    qmod = raw["refh"] + zeff_x
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        zeta = np.exp(ga * (1.0 - np.exp(hard_x * (1.0 - zeff_x / qmod))))
    zeta = np.where(qmod < 0.0, np.exp(ga), zeta)
    aiw_x = raw["sscale"][sec] * raw["secaiw"][:, sec] * zeta          # (23, 7, 119)
    alpha = raw["ascale"] * (raw["alphaiw"] - raw["hcount"] * aiw_x)
    out["refalpha"] = np.where(present, np.maximum(alpha, 0.0), 0.0)
    return out


def subset_tables(tables: Dict[str, np.ndarray], elements: Sequence[int]) -> Dict[str, np.ndarray]:
    """The same tables with every element outside ``elements`` zeroed (nref = 0)."""
    keep = np.zeros(tables["rcov"].shape[0], dtype=bool)
    keep[list(elements)] = True
    out = {}
    for k, v in tables.items():
        if v.shape[-1] == keep.shape[0]:
            out[k] = np.where(keep, v, np.zeros_like(v))
        else:
            out[k] = v
    return out


def _t(tables, key, dtype=torch.float64):
    return torch.as_tensor(tables[key], dtype=dtype)


# --------------------------------------------------------------------------- geometry
def pair_images(pos: np.ndarray, cell: Optional[np.ndarray], cutoff: float,
                receivers: Optional[np.ndarray] = None):
    """Every ordered pair (dst i, src j) and lattice translation T with
    0 < |pos_i - pos_j + T| <= cutoff (Angstrom, float64, brute force over the image
    range that covers the cutoff): arrays dst, src, shift (E, 3) int. ``receivers``
    restricts dst to those atom indices (a sample of a large system)."""
    n = pos.shape[0]
    rows = np.arange(n) if receivers is None else np.asarray(receivers, dtype=np.int64)
    if cell is None:
        rng = [np.zeros((1, 3), dtype=np.int64)]
        shifts = rng[0]
    else:
        inv = np.linalg.inv(cell)
        spacing = 1.0 / np.linalg.norm(inv.T, axis=1)
        reps = [int(math.ceil(cutoff / s)) for s in spacing]
        grids = np.meshgrid(*[np.arange(-r, r + 1) for r in reps], indexing="ij")
        shifts = np.stack([g.ravel() for g in grids], axis=1).astype(np.int64)
    dst, src, sh = [], [], []
    for s in shifts:
        t = s @ cell if cell is not None else np.zeros(3)
        d = pos[rows, None, :] - pos[None, :, :] + t
        r = np.sqrt((d * d).sum(-1))
        ok = (r <= cutoff) & (r > 0)
        ii, jj = np.nonzero(ok)
        dst.append(rows[ii])
        src.append(jj)
        sh.append(np.repeat(s[None, :], len(ii), axis=0))
    return (np.concatenate(dst), np.concatenate(src), np.concatenate(sh).reshape(-1, 3))


def edge_vectors_au(pos: Tensor, cell: Optional[Tensor], dst, src, shift) -> Tensor:
    """``(pos[dst] - pos[src] + shift @ cell) / bohr`` (d4.py:1201-1207)."""
    v = pos[dst] - pos[src]
    if cell is not None:
        v = v + torch.as_tensor(shift, dtype=pos.dtype) @ cell
    return v / BOHR


# --------------------------------------------------------------------------- D4 pieces
def erf_count(r: Tensor, rc: Tensor) -> Tensor:
    """``(1 + erf(-k0 (r - rc) / rc)) / 2`` (d4.py:168-170)."""
    return 0.5 * (1.0 + torch.erf(-KCN * (r - rc) / rc))


def coordination_numbers(z, dst, src, r_au, tables, cutoff_cn_au, cutoff_eeq_cn_au, n_atoms):
    """D4 CN (EN-weighted, r <= cutoff_cn) and capped EEQ CN (r <= cutoff_eeq_cn),
    summed to dst (d4.py:552-591)."""
    rcov, en = _t(tables, "rcov"), _t(tables, "en")
    zi, zj = z[dst], z[src]
    rc = rcov[zi] + rcov[zj]
    count = erf_count(r_au, rc)
    enf = K4 * torch.exp(-((en[zi] - en[zj]).abs() + K5) ** 2 / K6)
    cn = torch.zeros(n_atoms, dtype=r_au.dtype).index_add(
        0, torch.as_tensor(dst), torch.where(r_au <= cutoff_cn_au, enf * count, torch.zeros_like(count)))
    raw = torch.zeros(n_atoms, dtype=r_au.dtype).index_add(
        0, torch.as_tensor(dst), torch.where(r_au <= cutoff_eeq_cn_au, count, torch.zeros_like(count)))
    cn_eeq = math.log(1.0 + math.exp(EEQ_CN_MAX)) - torch.log(1.0 + torch.exp(EEQ_CN_MAX - raw))
    return cn, cn_eeq, raw


def eeq_charges_molecular(z, pos_au, cn_eeq, total_charge, tables):
    """EEQ charges of an isolated structure: [A 1; 1^T 0] [q; mu] = [x; Q] with
    A_ij = erf(gamma_ij r_ij) / r_ij, A_ii = eta + sqrt(2/pi)/rad,
    x = -chi + kcn cn / sqrt(cn + reg) (d4.py:593-606, 682-723)."""
    n = pos_au.shape[0]
    rad = _t(tables, "eeq_rad")[z]
    gamma = 1.0 / torch.sqrt(rad[:, None] ** 2 + rad[None, :] ** 2)
    d = pos_au[None, :, :] - pos_au[:, None, :]
    r = torch.sqrt((d * d).sum(-1) + torch.eye(n, dtype=pos_au.dtype))
    eye = torch.eye(n, dtype=torch.bool)
    A = torch.where(eye, torch.zeros_like(r), torch.erf(gamma * r) / r)
    A = A + torch.diag(_t(tables, "eeq_eta")[z] + math.sqrt(2.0 / math.pi) / rad)
    x = -_t(tables, "eeq_chi")[z] + _t(tables, "eeq_kcnchi")[z] * cn_eeq / torch.sqrt(cn_eeq + EEQ_CN_REG)
    M = torch.zeros((n + 1, n + 1), dtype=pos_au.dtype)
    M[:n, :n] = A
    M[:n, n] = 1.0
    M[n, :n] = 1.0
    rhs = torch.cat([x, torch.as_tensor([float(total_charge)], dtype=pos_au.dtype)])
    return torch.linalg.solve(M, rhs)[:n]


def gaussian_weights(z, cn, tables, wf: float = WF):
    """Normalized Gaussian weights of the reference CNs with ngw Gaussians per
    reference; fallback to the largest-CN reference(s) when all underflow
    (dispersion.py:70-121, d4.py:1004-1012)."""
    refcn = _t(tables, "refcn")[:, z].t()
    ngw = torch.as_tensor(tables["ngw"])[:, z].t()
    nref = torch.as_tensor(tables["nref"])[z]
    valid = torch.arange(refcn.shape[1])[None, :] < nref[:, None]
    d2 = (cn[:, None] - refcn) ** 2
    nmax = int(ngw.max()) if ngw.numel() else 1
    gw = torch.zeros_like(d2)
    for j in range(1, nmax + 1):
        gw = gw + torch.where(ngw >= j, torch.exp(-wf * j * d2), torch.zeros_like(d2))
    gw = torch.where(valid, gw, torch.zeros_like(gw))
    norm = gw.sum(1)
    eps = 1.4916681462400413e-154
    ok = norm > eps
    w = gw / torch.where(ok, norm, torch.ones_like(norm))[:, None]
    maxcn = torch.where(valid, refcn, torch.full_like(refcn, -math.inf)).max(1).values
    fb = (valid & ((refcn - maxcn[:, None]).abs() < 1e-12)).to(cn.dtype)
    return torch.where(ok[:, None], w, fb)


def charge_scaling(z, q, tables, ga: float = GA, gc: float = GC):
    """zeta(q) per reference slot (d4.py:1014-1023)."""
    zi = _t(tables, "zeff")[z][:, None]
    gi = (_t(tables, "hardness")[z] * gc)[:, None]
    qmod = q[:, None] + zi
    qref = _t(tables, "refq")[:, z].t() + zi
    neg = qmod < 0.0
    safe = torch.where(neg, torch.ones_like(qmod), qmod)
    scaled = torch.exp(ga * (1.0 - torch.exp(gi * (1.0 - qref / safe))))
    return torch.where(neg, torch.full_like(qmod, math.exp(ga)), scaled)


def dynamic_polarizabilities(z, cn, q, tables):
    """alpha_A(i w) = sum_ref W_ref zeta_ref alpha_ref(i w), (N, 23) (d4.py:1036-1042)."""
    w = gaussian_weights(z, cn, tables) * charge_scaling(z, q, tables)
    ref = _t(tables, "refalpha")[:, :, z]                 # (23, 7, N)
    return torch.einsum("nr,krn->nk", w, ref)


def c6_pairs(alpha_i, alpha_j):
    """(3/pi) sum_w cp_w alpha_i(w) alpha_j(w) (d4.py:1044-1046)."""
    cp = torch.as_tensor(cp_weights(), dtype=alpha_i.dtype)
    return (3.0 / math.pi) * (alpha_i * alpha_j * cp).sum(-1)


def switching(r, cutoff, width):
    """Quintic window (dispersion.py:42-67): 1 below cutoff - width, 0 above cutoff."""
    if width <= 0.0:
        return torch.ones_like(r)
    w = min(width, cutoff)
    x = torch.clamp((cutoff - r) / w, 0.0, 1.0)
    return x ** 3 * (10.0 + x * (6.0 * x - 15.0))


def two_body(z, dst, src, r_au, alpha, tables, prm, cutoff_pair_au, width_au, n_atoms):
    """-1/2 C6 sw (s6/(r^6+R0^6) + s8 rr/(r^8+R0^8)) to dst per directed edge within
    the pair cutoff (d4.py:1048-1071)."""
    r4r2 = _t(tables, "r4r2")
    keep = r_au <= cutoff_pair_au
    dst_t = torch.as_tensor(dst)
    zi, zj = z[dst], z[src]
    c6 = c6_pairs(alpha[dst], alpha[src])
    rr = 3.0 * r4r2[zi] * r4r2[zj]
    r0 = prm["a1"] * torch.sqrt(rr) + prm["a2"]
    r2 = r_au * r_au
    t6 = 1.0 / (r2 ** 3 + r0 ** 6)
    t8 = 1.0 / (r2 ** 4 + r0 ** 8)
    sw = switching(r_au, cutoff_pair_au, width_au)
    e = -0.5 * c6 * sw * (prm["s6"] * t6 + prm["s8"] * rr * t8)
    e = torch.where(keep, e, torch.zeros_like(e))
    return torch.zeros(n_atoms, dtype=r_au.dtype).index_add(0, dst_t, e)


def atm_molecule(z, pos_au, alpha_neutral, tables, prm, cutoff_au):
    """ATM three-body energy of a small molecule by the direct triple loop (sharp
    cutoff), the formula of dispersion.py:188-222 summed over distinct triples."""
    n = pos_au.shape[0]
    r4r2 = _t(tables, "r4r2")
    c6 = c6_pairs(alpha_neutral[:, None, :], alpha_neutral[None, :, :])
    e = torch.zeros((), dtype=pos_au.dtype)
    alp3 = prm["alp"] / 3.0
    for a in range(n):
        for b in range(a + 1, n):
            for c in range(b + 1, n):
                rab = pos_au[b] - pos_au[a]
                rbc = pos_au[c] - pos_au[b]
                rca = pos_au[a] - pos_au[c]
                r2ab, r2bc, r2ca = (rab * rab).sum(), (rbc * rbc).sum(), (rca * rca).sum()
                if max(float(r2ab), float(r2bc), float(r2ca)) > cutoff_au ** 2:
                    continue
                r0 = 1.0
                for (p, s) in ((a, b), (b, c), (c, a)):
                    r0 = r0 * (prm["a1"] * torch.sqrt(3.0 * r4r2[z[p]] * r4r2[z[s]]) + prm["a2"])
                c9 = prm["s9"] * torch.sqrt((c6[a, b] * c6[b, c] * c6[c, a]).abs())
                prod2 = r2ab * r2bc * r2ca
                prod1 = torch.sqrt(prod2)
                prod3 = prod2 * prod1
                prod5 = prod3 * prod2
                damp = 1.0 / (1.0 + 6.0 * (r0 / prod1) ** alp3)
                ang = (0.375 * (r2ab + r2bc - r2ca) * (r2ab - r2bc + r2ca) * (-r2ab + r2bc + r2ca)
                       / prod5 + 1.0 / prod3)
                e = e + c9 * ang * damp
    return e


def atm_edges(edge_index, edge_vec, feat_a, feat_b, species, r0_table, s9: float, alp3: float,
              cutoff: float, width: float, n_atoms: int) -> Tensor:
    """Per-atom ATM energies (hartree) from directed edges ``[src, dst]`` within the
    three-body cutoff and their vectors (bohr), the formula of dispersion.py:183-222 with
    the bookkeeping of dispersion.py:124-181: every pair of edges sharing a center is a
    triangle visit, and a third of the triangle energy goes to that center. Pair C6 are
    ``<feat_a[x], feat_b[y]>`` (dispersion_fast/atm.py:512-535 interface); the damping
    radius is the product of the three ``r0_table[species, species]`` pair factors.
    Differentiable (autograd) in ``edge_vec``, ``feat_a`` and ``feat_b``."""
    src, dst = edge_index[0], edge_index[1]
    order = torch.argsort(dst, stable=True)
    energy = edge_vec.new_zeros(n_atoms)
    counts = torch.bincount(dst, minlength=n_atoms).tolist()
    start = 0
    parts = []
    for c in range(n_atoms):
        m = counts[c]
        ids = order[start:start + m]
        start += m
        if m < 2:
            continue
        ia, ib = torch.triu_indices(m, m, offset=1)
        a, b = ids[ia], ids[ib]
        parts.append((a, b, torch.full_like(a, c)))
    if not parts:
        return energy
    a = torch.cat([p[0] for p in parts])
    b = torch.cat([p[1] for p in parts])
    c = torch.cat([p[2] for p in parts])
    j, k = src[a], src[b]
    va, vb = edge_vec[a], edge_vec[b]
    x, y = (va * va).sum(-1), (vb * vb).sum(-1)
    d = va - vb
    w = (d * d).sum(-1)
    keep = (w <= cutoff * cutoff) & (w > 2.220446049250313e-16)
    w = torch.where(keep, w, torch.ones_like(w))
    c6a = (feat_a[c] * feat_b[j]).sum(-1)
    c6b = (feat_a[c] * feat_b[k]).sum(-1)
    c6jk = (feat_a[j] * feat_b[k]).sum(-1)
    c9 = s9 * torch.sqrt((c6a * c6b * c6jk).abs())
    sc, sj, sk = species[c], species[j], species[k]
    r0 = r0_table[sc, sj] * r0_table[sc, sk] * r0_table[sj, sk]
    prod2 = x * y * w
    prod1 = torch.sqrt(prod2)
    prod3 = prod2 * prod1
    prod5 = prod3 * prod2
    damp = 1.0 / (1.0 + 6.0 * (r0 / prod1) ** alp3)
    ang = 0.375 * (x + w - y) * (x - w + y) * (-x + w + y) / prod5 + 1.0 / prod3
    sw = switching(torch.sqrt(x), cutoff, width) * switching(torch.sqrt(y), cutoff, width) \
        * switching(torch.sqrt(w), cutoff, width)
    e = torch.where(keep, c9 * ang * damp * sw / 3.0, torch.zeros_like(x))
    return energy.index_add(0, c, e)


def bj_radius_factors(z, tables, a1: float, a2: float):
    """Species table of the BJ pair radii ``a1 sqrt(3 Q_A Q_B) + a2`` over the unique
    elements of ``z`` (d4.py:970-978), and each atom's species index."""
    uniq, species = torch.unique(torch.as_tensor(z), return_inverse=True)
    q = _t(tables, "r4r2")[uniq]
    return a1 * torch.sqrt(3.0 * q[:, None] * q[None, :]) + a2, species


def d4_molecule(pos_aa: np.ndarray, numbers, tables, prm=PBE0_D4, total_charge: float = 0.0,
                cutoffs_au=(60.0, 40.0, 30.0, 25.0), with_atm: bool = True) -> dict:
    """Energy (hartree) and properties of one molecule, all pairs (no cell)."""
    cut_pair, cut_tri, cut_cn, cut_eeq = cutoffs_au
    z = torch.as_tensor(np.asarray(numbers), dtype=torch.long)
    pos = torch.as_tensor(pos_aa, dtype=torch.float64)
    dst, src, sh = pair_images(pos_aa, None, max(cutoffs_au) * BOHR)
    v = edge_vectors_au(pos, None, dst, src, sh)
    r = torch.linalg.norm(v, dim=-1)
    n = pos.shape[0]
    cn, cn_eeq, _ = coordination_numbers(z, dst, src, r, tables, cut_cn, cut_eeq, n)
    q = eeq_charges_molecular(z, pos / BOHR, cn_eeq, total_charge, tables)
    alpha = dynamic_polarizabilities(z, cn, q, tables)
    e2 = two_body(z, dst, src, r, alpha, tables, prm, cut_pair, 0.0, n)
    out = {"cn": cn, "q": q, "alpha": alpha, "e2": e2, "energy_2body": e2.sum()}
    if with_atm and prm.get("s9", 0.0) != 0.0:
        alpha0 = dynamic_polarizabilities(z, cn, torch.zeros_like(q), tables)
        out["energy_3body"] = atm_molecule(z, pos / BOHR, alpha0, tables, prm, cut_tri)
    else:
        out["energy_3body"] = torch.zeros((), dtype=torch.float64)
    out["energy"] = out["energy_2body"] + out["energy_3body"]
    return out
