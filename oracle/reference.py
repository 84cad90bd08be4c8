"""TEST INFRASTRUCTURE ONLY: CPU restatement of the reference's per-edge path.

Every function follows the reference (molssi-ai/xnn) at the cited lines, in PyTorch on
the CPU (float64 unless asked otherwise), and is used by the tests as the checker and
by ``bench.py`` as the timed CPU baseline. Forces and stress come from autograd, as in
ForceStressOutput (src/xnn/common/models/outputs.py:166-239).

Spherical harmonics: the reference evaluates e3nn 0.4.4 ``SphericalHarmonics(normalize
=True, normalization="component")`` (gnn/featurizers/spherical.py:91-93; e3nn is pinned
at uv.lock:756-757 and absent offline). Its published convention: real harmonics with
``sum_m Y_lm^2 = 2l+1`` and the y axis as polar axis (equiformer_v2.py:35). Here they are
formed from the reference's own orthonormal real harmonics
(gnn/featurizers/spherical_bessel.py:348-407, z polar, no Condon-Shortley phase, from
the associated-Legendre recurrences) with the axes relabelled ``(x_s, y_s, z_s) = (z, x,
y)`` and the factor ``sqrt(4 pi)``; a different algorithm from the kernels' closed-form
polynomials.
"""
from __future__ import annotations

import math
from typing import List, Optional

import torch
from torch import Tensor


# --------------------------------------------------------------------------- geometry
def edge_vectors(pos: Tensor, edge_index: Tensor, cell_shifts: Tensor,
                 cell: Optional[Tensor], batch: Optional[Tensor] = None,
                 geometry_dtype: Optional[torch.dtype] = None) -> Tensor:
    """``pos[dst] - pos[src] + shift @ cell`` (atomic_data.py:371-418).

    With ``geometry_dtype`` (float32), the vector's value is formed in that dtype in the
    reference's order -- the difference, then the image offset -- as a float32 geometry
    does (atomic_data.py:406-410), while its derivative stays the exact linear map in
    the working dtype; the rest of the evaluation then runs in the working dtype."""
    src, dst = edge_index[0], edge_index[1]

    def form(p, c):
        v = p.index_select(0, dst) - p.index_select(0, src)
        if c is not None:
            c = c.reshape(-1, 3, 3)
            if c.shape[0] == 1:
                v = v + cell_shifts.to(v.dtype) @ c[0]
            else:
                per_edge = c.index_select(0, batch.index_select(0, src))
                v = v + torch.einsum("ei,eij->ej", cell_shifts.to(v.dtype), per_edge)
        return v

    vec = form(pos, cell)
    if geometry_dtype is None or geometry_dtype == pos.dtype:
        return vec
    with torch.no_grad():
        rounded = form(pos.detach().to(geometry_dtype),
                       None if cell is None else cell.detach().to(geometry_dtype)).to(pos.dtype)
    return vec + (rounded - vec.detach())


# --------------------------------------------------------------------------- radial
def bessel(r: Tensor, n_rbf: int, cutoff: float, prefactor: Optional[float] = None,
           freqs: Optional[Tensor] = None) -> Tensor:
    """``prefactor * sin(n pi r / rc) / r`` with r clamped at 1e-8 (radial.py:221-268)."""
    if freqs is None:
        freqs = math.pi * torch.arange(1, n_rbf + 1, dtype=r.dtype)
    norm = math.sqrt(2.0 / cutoff) if prefactor is None else prefactor
    rr = r.clamp(min=1e-8)[..., None]
    return norm * torch.sin(freqs * rr / cutoff) / rr


def gaussian(r: Tensor, n_rbf: int, cutoff: float, start: float = 0.0) -> Tensor:
    """``exp(-gamma (r - mu_k)^2)``, centers on [start, rc], gamma = 0.5 / spacing^2
    (radial.py:49-75)."""
    centers = torch.linspace(start, cutoff, n_rbf, dtype=r.dtype)
    width = float(centers[1] - centers[0]) if n_rbf > 1 else 1.0
    gamma = 0.5 / width ** 2
    return torch.exp(-gamma * (r[..., None] - centers) ** 2)


def polynomial_envelope(r: Tensor, cutoff: float, p: int = 6) -> Tensor:
    """cutoff.py:119-125."""
    x = r / cutoff
    tail = ((-(p * (p + 1) / 2)) * x + p * (p + 2)) * x - (p + 1) * (p + 2) / 2
    return (1.0 + tail * x ** p) * (r < cutoff)


def cosine_envelope(r: Tensor, cutoff: float) -> Tensor:
    """cutoff.py:40-41."""
    return 0.5 * (torch.cos(math.pi * r / cutoff) + 1.0) * (r < cutoff)


# --------------------------------------------------------------------------- harmonics
def real_sh_zpolar(l_max: int, x: Tensor, y: Tensor, z: Tensor) -> Tensor:
    """Orthonormal real SH of unit vectors, z polar, no Condon-Shortley phase, column
    ``l^2 + l + m`` -- the algorithm of spherical_bessel.py:348-407 (associated Legendre
    recurrences for P_l^m / sin^m, cos/sin m phi from powers of x + i y)."""
    cos_m: List[Tensor] = [torch.ones_like(z)]
    sin_m: List[Tensor] = [torch.zeros_like(z)]
    for m in range(l_max):
        cos_m.append(cos_m[m] * x - sin_m[m] * y)
        sin_m.append(sin_m[m] * x + cos_m[m] * y)
    q = [[torch.zeros_like(z) for _ in range(l + 1)] for l in range(l_max + 1)]
    dfact = 1.0
    for m in range(l_max + 1):
        if m > 0:
            dfact *= 2 * m - 1
        q[m][m] = torch.full_like(z, dfact)
        if m + 1 <= l_max:
            q[m + 1][m] = (2 * m + 1) * z * q[m][m]
        for l in range(m + 2, l_max + 1):
            q[l][m] = ((2 * l - 1) * z * q[l - 1][m] - (l + m - 1) * q[l - 2][m]) / (l - m)
    out = []
    for l in range(l_max + 1):
        for m in range(-l, l + 1):
            a = abs(m)
            ratio = 1.0
            for k in range(l - a + 1, l + a + 1):
                ratio /= k
            norm = math.sqrt((2 * l + 1) / (4.0 * math.pi) * ratio)
            if m == 0:
                out.append(norm * q[l][0])
            elif m > 0:
                out.append(math.sqrt(2.0) * norm * q[l][a] * cos_m[a])
            else:
                out.append(math.sqrt(2.0) * norm * q[l][a] * sin_m[a])
    return torch.stack(out, dim=-1)


def e3nn_sh(l_max: int, vec: Tensor) -> Tensor:
    """e3nn component-normalized SH of ``vec / |vec|`` (y polar), ``(E, (l_max+1)^2)``."""
    u = vec / torch.linalg.norm(vec, dim=-1, keepdim=True).clamp(min=1e-12)
    return math.sqrt(4.0 * math.pi) * real_sh_zpolar(l_max, u[..., 2], u[..., 0], u[..., 1])


# --------------------------------------------------------------------------- the sh_edge model
def radial_features(length: Tensor, n_rbf: int, cutoff: float, radial: str = "bessel",
                    envelope: str = "polynomial", p: int = 6) -> Tensor:
    """rbf(|r|) * envelope(|r|) (spherical.py:135-138)."""
    rb = bessel(length, n_rbf, cutoff) if radial == "bessel" else gaussian(length, n_rbf, cutoff)
    env = polynomial_envelope(length, cutoff, p) if envelope == "polynomial" else \
        cosine_envelope(length, cutoff)
    return rb * env[:, None]


def scatter_sum(src: Tensor, index: Tensor, dim_size: int) -> Tensor:
    """CPU ``index_add`` (ops.py:403-448)."""
    out = torch.zeros([dim_size] + list(src.shape[1:]), dtype=src.dtype)
    return out.index_add_(0, index, src)


def structure_sum(src: Tensor, index: Tensor, dim_size: int) -> Tensor:
    """float64 totals (ops.py:531-557)."""
    if dim_size == 1:
        return src.to(torch.float64).sum(0, keepdim=True)
    return torch.zeros(dim_size, dtype=torch.float64).index_add(0, index, src.to(torch.float64))


def sh_edge_node_energy(vec: Tensor, edge_index: Tensor, n_nodes: int, numbers: Tensor,
                        W: Tensor, U: Tensor, atom_ref: Tensor, *, l_max: int, n_rbf: int,
                        cutoff: float, radial: str, envelope: str, p: int = 6,
                        sh_sign: int = 1, edge_chunk: int = 1 << 15) -> Tensor:
    """Per-atom energy of the measured model: ``A_i = sum_{dst=i} (u_e W) (x) Y(sign r_e)``
    (the uvu product of conv.py:137-143 with materialized messages, scattered with
    ``index_add``), ``E_i = <U, A_i> + atom_ref[Z_i]``. Edges in chunks of ``edge_chunk``
    so the (E, C, L) messages never exist whole."""
    length = torch.linalg.norm(vec, dim=-1)
    u = radial_features(length, n_rbf, cutoff, radial, envelope, p)
    sh = e3nn_sh(l_max, vec if sh_sign == 1 else -vec)
    phi = u @ W
    C, L = W.shape[1], sh.shape[1]
    A = torch.zeros((n_nodes, C * L), dtype=vec.dtype)
    for e0 in range(0, vec.shape[0], edge_chunk):
        e1 = min(vec.shape[0], e0 + edge_chunk)
        msg = (phi[e0:e1, :, None] * sh[e0:e1, None, :]).reshape(e1 - e0, C * L)
        A = A.index_add(0, edge_index[1, e0:e1], msg)
    return A @ U.reshape(-1) + atom_ref[numbers]


def energy_forces_stress(pos: Tensor, numbers: Tensor, edge_index: Tensor, cell_shifts: Tensor,
                         cell: Optional[Tensor], batch: Tensor, n_graphs: int, model: dict,
                         stress: bool = True, geometry_dtype: Optional[torch.dtype] = None):
    """Energy (B,) float64, forces (N, 3) and stress (B, 3, 3) by autograd through the
    symmetric strain (outputs.py:166-239), for the sh_edge model parameters in ``model``;
    ``geometry_dtype`` as in :func:`edge_vectors`."""
    strain = torch.zeros((n_graphs, 3, 3), dtype=pos.dtype, requires_grad=True)
    sym = 0.5 * (strain + strain.transpose(-1, -2))
    pos = pos.detach().clone().requires_grad_(True)
    p2 = pos + (pos[:, :, None] * sym.index_select(0, batch)).sum(1)
    c2 = None
    if cell is not None:
        c2 = cell.reshape(-1, 3, 3) + (cell.reshape(-1, 3, 3)[:, :, :, None] * sym[:, None]).sum(2)
    vec = edge_vectors(p2, edge_index, cell_shifts, c2, batch, geometry_dtype)
    node_e = sh_edge_node_energy(vec, edge_index, pos.shape[0], numbers, **model)
    energy = structure_sum(node_e, batch, n_graphs)
    inputs = [pos, strain] if (stress and cell is not None) else [pos]
    grads = torch.autograd.grad(energy.sum(), inputs)
    out = {"energy": energy.detach(), "node_energy": node_e.detach(), "forces": -grads[0]}
    if stress and cell is not None:
        vol = torch.linalg.det(cell.reshape(-1, 3, 3)).abs()
        out["stress"] = grads[1] / vol[:, None, None]
    return out
