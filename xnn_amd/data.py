"""Atomic graphs and neighbor lists, the xnn data contract on MI355X.

* :class:`AtomicGraph` -- the one data object (common/data/atomic_data.py:28-261):
  positions, atomic numbers, ``edge_index = [src, dst]``, integer ``cell_shifts``,
  ``batch``/``n_atoms``, optional ``cell``/``pbc``; :meth:`AtomicGraph.edge_vectors`
  gives ``pos[dst] - pos[src] + cell_shift @ cell`` (atomic_data.py:371-418).
* :func:`build_neighbor_list` -- the radius graph (common/data/neighborlist.py:411-506):
  on a GPU the HIP cell list, with the reference's edge set and conventions
  (``dst`` = receiver, negated and unwrapped shifts); edges come grouped by receiver.
* :func:`structure_to_graph` / :func:`collate` (common/data/dataset.py:21-175, 371-577).

GPU tensors always take the HIP kernels (and raise when the library is missing).
CPU tensors take the reference formulation in PyTorch, as the reference does on a CPU.
"""
from __future__ import annotations

import ctypes
import itertools
import math
import weakref
from dataclasses import dataclass, fields
from typing import Optional, Sequence

import numpy as np
import torch
from torch import Tensor

from . import _lib


@dataclass
class AtomicGraph:
    """Graph of one or a batch of atomic systems (atomic_data.py:28-261).

    ``edge_index`` is ``(2, E)`` ``[src, dst]``: the energy of ``dst`` depends on
    ``src``. ``cell`` is ``(B, 3, 3)`` (rows are lattice vectors) or ``None`` for
    molecules; a molecule in a mixed batch has a zero cell.
    """

    pos: Tensor
    atomic_numbers: Tensor
    edge_index: Tensor
    cell_shifts: Tensor
    batch: Tensor
    n_atoms: Tensor
    cell: Optional[Tensor] = None
    pbc: Optional[Tensor] = None
    # labels and per-structure metadata (atomic_data.py:194-223): carried, never read by
    # the hot path; masks are bool (B,) and say which structures carry a label
    energy: Optional[Tensor] = None                  # (B,)
    forces: Optional[Tensor] = None                  # (N, 3)
    stress: Optional[Tensor] = None                  # (B, 3, 3)
    energy_mask: Optional[Tensor] = None
    forces_mask: Optional[Tensor] = None
    stress_mask: Optional[Tensor] = None
    dipole: Optional[Tensor] = None                  # (B, 3)
    polarizability: Optional[Tensor] = None          # (B, 3, 3)
    dipole_mask: Optional[Tensor] = None
    polarizability_mask: Optional[Tensor] = None
    charges: Optional[Tensor] = None                 # (N,)
    charges_mask: Optional[Tensor] = None
    fragment_charges: Optional[Tensor] = None        # (N,)
    fragment_charges_mask: Optional[Tensor] = None
    external_potential: Optional[Tensor] = None      # (N,)
    total_charge: Optional[Tensor] = None            # (B,) read by D4 / D3 EEQ
    spin_multiplicity: Optional[Tensor] = None       # (B,)
    weight: Optional[Tensor] = None                  # (B,)
    head: Optional[Tensor] = None                    # (B,)
    properties: Optional[Tensor] = None              # (B,) or (B, k)
    properties_mask: Optional[Tensor] = None
    state: Optional[Tensor] = None                   # (B,) labels or (B, d)
    site_species: Optional[Tensor] = None            # (N, K)
    site_occupancy: Optional[Tensor] = None          # (N, K)
    energy_weight: Optional[Tensor] = None           # (B,)
    force_weight: Optional[Tensor] = None            # (B,)
    stress_weight: Optional[Tensor] = None           # (B,)
    atom_force_weight: Optional[Tensor] = None       # (N,)
    compute_dtype: Optional[torch.dtype] = None
    # (B, 3, 3) zeros set by ForceStressOutput: the strain whose gradient the edge-vector
    # backward forms directly (sym of sum_e r_e (x) dE/dr_e), in place of deforming pos and cell
    strain_probe: Optional[Tensor] = None

    @property
    def model_dtype(self) -> torch.dtype:
        return self.compute_dtype if self.compute_dtype is not None else self.pos.dtype

    @property
    def num_graphs(self) -> int:
        return int(self.n_atoms.shape[0])

    @property
    def num_nodes(self) -> int:
        return int(self.pos.shape[0])

    @property
    def num_edges(self) -> int:
        return int(self.edge_index.shape[1])

    def to(self, device) -> "AtomicGraph":
        kwargs = {}
        for f in fields(self):
            v = getattr(self, f.name)
            kwargs[f.name] = v.to(device) if isinstance(v, Tensor) else v
        return AtomicGraph(**kwargs)

    #: per-atom optional fields (the rest of the optional tensors are per structure)
    _PER_ATOM = ("forces", "charges", "fragment_charges", "external_potential", "site_species",
                 "site_occupancy", "atom_force_weight")
    _STRUCTURE = ("pos", "atomic_numbers", "edge_index", "cell_shifts", "batch", "n_atoms",
                  "compute_dtype", "strain_probe")

    def subset(self, keep: Tensor) -> "AtomicGraph":
        """The structures flagged in the bool ``keep`` (B,) as a batch of their own, in
        their original order, with atoms and edges renumbered and every optional field
        restricted the same way (atomic_data.py:284-340). Positions are gathered, so
        derivatives on the subset reach the full graph."""
        keep = keep.to(device=self.batch.device, dtype=torch.bool)
        atom_keep = keep.index_select(0, self.batch)
        edge_keep = atom_keep.index_select(0, self.edge_index[0])
        new_atom = torch.cumsum(atom_keep.to(torch.int64), 0) - 1
        new_structure = torch.cumsum(keep.to(torch.int64), 0) - 1
        kw = dict(pos=self.pos[atom_keep], atomic_numbers=self.atomic_numbers[atom_keep],
                  edge_index=new_atom[self.edge_index[:, edge_keep]],
                  cell_shifts=self.cell_shifts[edge_keep],
                  batch=new_structure[self.batch[atom_keep]], n_atoms=self.n_atoms[keep],
                  compute_dtype=self.compute_dtype)
        for f in fields(self):
            if f.name in self._STRUCTURE:
                continue
            v = getattr(self, f.name)
            if v is not None:
                mask = atom_keep if f.name in self._PER_ATOM else keep
                v = v[mask.to(v.device)]
            kw[f.name] = v
        return AtomicGraph(**kw)

    def plan(self):
        """The cached :class:`~xnn_amd.plan.EdgePlan` of this graph (GPU only)."""
        from .plan import plan_for
        return plan_for(self)

    def edge_vectors(self) -> Tensor:
        """``pos[dst] - pos[src] + cell_shift @ cell`` per edge, in :attr:`model_dtype`,
        differentiable with respect to ``pos`` and ``cell`` (atomic_data.py:371-418)."""
        if self.pos.is_cuda:
            from .ops import edge_vectors
            return edge_vectors(self.pos, self.cell, self.plan(), self.model_dtype,
                                strain_probe=self.strain_probe)
        if self.strain_probe is not None:
            raise RuntimeError("strain_probe is a GPU path; deform pos and cell on the CPU")
        src, dst = self.edge_index[0], self.edge_index[1]
        vec = self.pos.index_select(0, dst) - self.pos.index_select(0, src)
        if self.cell is not None:
            if self.cell.shape[0] == 1:
                vec = vec + self.cell_shifts.to(vec.dtype) @ self.cell[0].to(vec.dtype)
            else:
                cell_per_edge = self.cell.index_select(0, self.batch.index_select(0, src))
                vec = vec + torch.einsum("ei,eij->ej", self.cell_shifts.to(vec.dtype),
                                         cell_per_edge.to(vec.dtype))
        return vec.to(self.model_dtype)


# --------------------------------------------------------------------------- neighbor lists
def _n_repeats(cell: Tensor, cutoff: float, pbc: Tensor) -> list[int]:
    """Image repeats per axis from the interplanar spacing (neighborlist.py:74-104)."""
    recip = torch.linalg.inv(cell).T
    spacing = 1.0 / torch.linalg.norm(recip, dim=1)
    return [int(math.ceil(cutoff / float(spacing[i]))) if bool(pbc[i]) else 0 for i in range(3)]


def _brute_force_cpu(pos: Tensor, cutoff: float, cell: Optional[Tensor], pbc: Optional[Tensor],
                     self_interaction: bool) -> tuple[Tensor, Tensor]:
    """The reference's brute force (neighborlist.py:462-506), chunked by receivers so
    that no (S, N, N, 3) tensor is formed; same edges, order (s, i, j)."""
    dtype, n = pos.dtype, pos.shape[0]
    offsets = None
    if cell is None or pbc is None or not bool(pbc.any()):
        shifts = torch.zeros((1, 3), dtype=dtype)
        shift_idx = torch.zeros((1, 3), dtype=torch.long)
    else:
        frac = pos @ torch.linalg.inv(cell)
        offsets = torch.floor(frac).to(torch.long)
        offsets[:, ~pbc.to(torch.bool)] = 0
        pos = pos - offsets.to(dtype) @ cell
        reps = _n_repeats(cell, cutoff, pbc)
        combos = list(itertools.product(*[range(-r, r + 1) for r in reps]))
        shift_idx = torch.tensor(combos, dtype=torch.long)
        shifts = shift_idx.to(dtype) @ cell
    zero_shift = (shift_idx == 0).all(dim=1)
    parts = []
    chunk = max(1, (1 << 24) // max(1, n * shifts.shape[0]))
    for i0 in range(0, n, chunk):
        i1 = min(n, i0 + chunk)
        rij = (pos[None, None, :, :] - pos[None, i0:i1, None, :]) + shifts[:, None, None, :]
        within = torch.linalg.norm(rij, dim=-1) < cutoff
        if not self_interaction:
            eye = torch.zeros((i1 - i0, n), dtype=torch.bool)
            eye[torch.arange(i1 - i0), torch.arange(i0, i1)] = True
            within = within & ~(eye[None] & zero_shift[:, None, None])
        s, i, j = torch.nonzero(within, as_tuple=True)
        parts.append((s, i + i0, j))
    s = torch.cat([p[0] for p in parts])
    i = torch.cat([p[1] for p in parts])
    j = torch.cat([p[2] for p in parts])
    order = torch.argsort(s * n + i, stable=True)          # the nonzero order (s, i, j)
    s, i, j = s[order], i[order], j[order]
    edge_index = torch.stack([j, i], dim=0)
    cell_shifts = -shift_idx[s]
    if offsets is not None:
        cell_shifts = cell_shifts + offsets[j] - offsets[i]
    return edge_index, cell_shifts


def _check_finite(lo_hi: list) -> None:
    if not all(math.isfinite(v) for v in lo_hi):
        raise ValueError("the positions are not finite (an unstable simulation?)")


def _spacings(c: Sequence[float]) -> list[float]:
    """Interplanar spacings of a cell given as its 9 row-major entries (rows a, b, c): the
    volume over the area spanned by the other two rows, |det| / |a_j x a_k|."""
    a, b, c3 = c[0:3], c[3:6], c[6:9]

    def cross(u, v):
        return (u[1] * v[2] - u[2] * v[1], u[2] * v[0] - u[0] * v[2], u[0] * v[1] - u[1] * v[0])

    bc, ca, ab = cross(b, c3), cross(c3, a), cross(a, b)
    vol = abs(a[0] * bc[0] + a[1] * bc[1] + a[2] * bc[2])
    return [vol / math.sqrt(x[0] * x[0] + x[1] * x[1] + x[2] * x[2]) for x in (bc, ca, ab)]


def _supercell_reps(cell, cutoff: float, pbc) -> list[int]:
    """Replicas per axis that bring every periodic interplanar spacing to at least a third
    of the cutoff (the cell list reaches at most three cells along an axis). ``cell``: a
    tensor or the 9 row-major entries; ``pbc``: a tensor or 3 flags."""
    entries = cell.reshape(-1).tolist() if isinstance(cell, Tensor) else list(cell)
    spacing = _spacings([float(v) for v in entries])
    flags = pbc.reshape(-1).tolist() if isinstance(pbc, Tensor) else list(pbc)
    return [max(1, int(math.ceil(cutoff / (3.0 * spacing[a]) * (1.0 + 1e-9))))
            if bool(flags[a]) else 1 for a in range(3)]


def _supercell_graph(pos: Tensor, cutoff: float, cell: Tensor, pbc: Tensor,
                     self_interaction: bool, reps: list[int]) -> tuple[Tensor, Tensor]:
    """The radius graph of a cell narrower than a third of the cutoff: list the edges of
    the ``reps`` supercell whose receivers are the primitive atoms (replica 0, the first
    rows of the receiver-grouped list) and map each sender replica ``m`` back to its atom
    and shift: ``pos_sup[i + m n] = pos[i] + o_m @ cell`` and ``cell_sup = diag(reps) cell``
    give ``shift = S_sup * reps - o_m`` for the same edge vector."""
    dev = pos.device
    n = pos.shape[0]
    c = cell.reshape(3, 3).to(device=dev, dtype=pos.dtype)
    offs = torch.tensor(list(itertools.product(*[range(r) for r in reps])), dtype=torch.long,
                        device=dev)
    pos_sup = (pos[None, :, :] + (offs.to(pos.dtype) @ c)[:, None, :]).reshape(-1, 3)
    R = torch.tensor(reps, dtype=torch.long, device=dev)
    cell_sup = c * R.to(pos.dtype)[:, None]
    ei, sh = _radius_graph_cuda(pos_sup, cutoff, cell_sup, pbc, self_interaction)
    keep = (ei[1] < n).nonzero()[:, 0]
    src_sup = ei[0][keep]
    edge_index = torch.stack([src_sup % n, ei[1][keep]])
    return edge_index, sh[keep] * R - offs[src_sup // n]


#: grid plans of fully periodic cells, one per (device, atoms, dtype, cutoff, self-edges):
#: (weak reference to the cell tensor, its version, plan, device cell, workspace). A plan
#: owns its workspace: builds with one key must not run concurrently on different streams.
_PERIODIC_PLANS: dict = {}


def _radius_graph_cuda(pos: Tensor, cutoff: float, cell: Optional[Tensor], pbc: Optional[Tensor],
                       self_interaction: bool) -> tuple[Tensor, Tensor]:
    """The HIP cell list. The host reads the device twice at most: the atoms' bounds and the
    cell (to plan the grid), then the edge count (to size the outputs). A fully periodic
    cell's grid depends on the cell alone (positions are wrapped into it), so for the same,
    unchanged cell tensor the plan is reused and the outputs are sized from the last list
    of that plan with some room: the count pass, the fill (which reads the count on the
    device) and one read of the count and the non-finite flag run back to back, and only a
    list that outgrew the room is filled again."""
    lib = _lib.load()
    dev = pos.device
    pos = pos.contiguous()
    n = pos.shape[0]
    molecular = cell is None or pbc is None or not bool(pbc.any())
    if n == 0:
        return (torch.zeros((2, 0), dtype=torch.long, device=dev),
                torch.zeros((0, 3), dtype=torch.long, device=dev))
    pbc_list = [0, 0, 0] if molecular else [int(bool(b)) for b in pbc.reshape(-1).tolist()]
    key = (str(dev), n, pos.dtype, float(cutoff), bool(self_interaction))
    hit = None
    if not molecular and all(pbc_list) and isinstance(cell, Tensor):
        hit = _PERIODIC_PLANS.get(key)
        if hit is not None and not (hit[0]() is cell and hit[1] == cell._version):
            hit = None
    if hit is not None:
        _, _, plan, cell_dev, ws, last = hit
    else:
        last = None
        cell_dev = (None if molecular
                    else cell.reshape(3, 3).detach().to(device=dev, dtype=pos.dtype).contiguous())
        # the atoms' bounds (fractional for a cell) and the cell itself in one launch and
        # one read
        bounds = torch.empty(15, dtype=torch.float64, device=dev)
        _lib.call("xnn_radius_graph_bounds", _lib.dtype_code(pos.dtype), _lib.ptr(pos), n,
                  _lib.ptr(cell_dev), _lib.ptr(bounds), _lib.stream(dev))
        vals = bounds.tolist()
        lo_hi = vals[:6]
        _check_finite(lo_hi)
        if molecular:
            cell_host = None
        else:
            reps = _supercell_reps(vals[6:], cutoff, pbc_list)
            if max(reps) > 1:
                return _supercell_graph(pos, cutoff, cell, pbc, self_interaction, reps)
            cell_host = (_lib.dbl * 9)(*vals[6:])
        plan = _lib.GridPlan()
        _lib.check("xnn_radius_graph_plan",
                   lib.xnn_radius_graph_plan(n, cell_host, (ctypes.c_int32 * 3)(*pbc_list),
                                             float(cutoff), (_lib.dbl * 3)(*lo_hi[:3]),
                                             (_lib.dbl * 3)(*lo_hi[3:]), ctypes.byref(plan)))
        ws = torch.empty(max(1, int(plan.workspace_bytes)), dtype=torch.uint8, device=dev)
        if not molecular and all(pbc_list) and isinstance(cell, Tensor):
            last = [-1]
            _PERIODIC_PLANS[key] = (weakref.ref(cell), cell._version, plan, cell_dev, ws, last)
    row_ptr = torch.empty(n + 1, dtype=torch.int32, device=dev)
    status = torch.empty(2, dtype=torch.int32, device=dev)
    geom = _lib.dtype_code(pos.dtype)
    s = _lib.stream(dev)
    si = int(bool(self_interaction))

    _lib.call("xnn_radius_graph_count", geom, _lib.ptr(pos), n, _lib.ptr(cell_dev), float(cutoff),
              si, ctypes.byref(plan), _lib.ptr(ws), _lib.ptr(row_ptr), s)
    cap = -1
    if last is not None and last[0] >= 0:
        # room for the last list of this plan plus 5 % (atoms drift between MD steps)
        cap = last[0] + last[0] // 20 + 64
        ei_buf = torch.empty(2 * cap, dtype=torch.long, device=dev)
        sh_buf = torch.empty(3 * cap, dtype=torch.long, device=dev)
        _lib.call("xnn_radius_graph_fill_capacity", geom, _lib.ptr(pos), n, _lib.ptr(cell_dev),
                  float(cutoff), si, ctypes.byref(plan), _lib.ptr(ws), _lib.ptr(row_ptr), cap,
                  _lib.ptr(ei_buf), _lib.ptr(sh_buf), _lib.ptr(status), s)
    else:
        _lib.call("xnn_radius_graph_status", geom, n, ctypes.byref(plan), _lib.ptr(ws),
                  _lib.ptr(row_ptr), _lib.ptr(status), s)
    n_edges, nonfinite = status.tolist()
    if nonfinite:
        raise ValueError("the positions are not finite (an unstable simulation?)")
    if last is not None:
        last[0] = n_edges
    if 0 <= n_edges <= cap:
        return ei_buf[:2 * n_edges].view(2, n_edges), sh_buf[:3 * n_edges].view(n_edges, 3)
    edge_index = torch.empty((2, n_edges), dtype=torch.long, device=dev)
    cell_shifts = torch.empty((n_edges, 3), dtype=torch.long, device=dev)
    _lib.call("xnn_radius_graph_fill", geom, _lib.ptr(pos), n, _lib.ptr(cell_dev), float(cutoff),
              si, ctypes.byref(plan), _lib.ptr(ws), _lib.ptr(row_ptr), n_edges, None, None, None,
              _lib.ptr(edge_index), _lib.ptr(cell_shifts), None, s)
    return edge_index, cell_shifts


class NeighborListPlan:
    """The HIP cell list of :func:`build_neighbor_list` planned once, for positions that
    move inside a fixed cell (or, on non-periodic axes, inside the range of ``pos`` widened
    by ``margin``, default the cutoff; atoms beyond it are still found, in the boundary
    bins). ``plan(pos, capacity)`` then makes no host reads: it writes the edges into
    buffers of ``capacity`` entries and returns their number on the device, so it can run
    behind a step or inside a captured HIP graph (the reference's capacity mode,
    grid_pairs.py:414-499). The plan owns its workspace: calls on one plan must not
    overlap."""

    def __init__(self, pos: Tensor, cutoff: float, cell: Optional[Tensor] = None,
                 pbc: Optional[Tensor] = None, self_interaction: bool = False,
                 margin: Optional[float] = None):
        if not pos.is_cuda:
            raise RuntimeError("NeighborListPlan runs on the GPU")
        dev = pos.device
        n = int(pos.shape[0])
        self.n, self.cutoff, self.dtype = n, float(cutoff), pos.dtype
        self.self_interaction = bool(self_interaction)
        margin = self.cutoff if margin is None else float(margin)
        molecular = cell is None or pbc is None or not bool(pbc.any())
        if not molecular and max(_supercell_reps(cell, cutoff, pbc)) > 1:
            raise ValueError("capacity mode needs periodic interplanar spacings of at least a "
                             "third of the cutoff")
        pbc_list = [0, 0, 0] if molecular else [int(bool(b)) for b in pbc.reshape(-1).tolist()]
        pbc_host = (ctypes.c_int32 * 3)(*pbc_list)
        p64 = pos.detach().double()
        if molecular:
            lo_hi = torch.stack([p64.amin(0) - margin, p64.amax(0) + margin]).flatten().tolist()
            cell_host, self.cell_dev = None, None
        else:
            cell64 = cell.reshape(3, 3).detach().double().cpu()
            inv = torch.linalg.inv(cell64)
            spacing = 1.0 / torch.linalg.norm(inv.T, dim=1)
            frac = p64 @ inv.to(dev)
            widen = (margin / spacing).to(dev)
            lo_hi = torch.stack([frac.amin(0) - widen, frac.amax(0) + widen]).flatten().tolist()
            cell_host = (_lib.dbl * 9)(*cell64.flatten().tolist())
            self.cell_dev = cell.reshape(3, 3).detach().to(device=dev, dtype=pos.dtype).contiguous()
        if n > 0:
            _check_finite(lo_hi)
        self.grid = _lib.GridPlan()
        if n > 0:
            _lib.check("xnn_radius_graph_plan",
                       _lib.load().xnn_radius_graph_plan(n, cell_host, pbc_host, self.cutoff,
                                                         (_lib.dbl * 3)(*lo_hi[:3]),
                                                         (_lib.dbl * 3)(*lo_hi[3:]),
                                                         ctypes.byref(self.grid)))
        self.ws = torch.empty(max(1, int(self.grid.workspace_bytes)), dtype=torch.uint8, device=dev)
        self.row_ptr = torch.zeros(n + 1, dtype=torch.int32, device=dev)

    def __call__(self, pos: Tensor, capacity: int) -> tuple[Tensor, Tensor, Tensor]:
        """``(edge_index (2, capacity), cell_shifts (capacity, 3), n_edges (1,))``: the
        edges of :func:`build_neighbor_list` (grouped by receiver) in the first
        ``n_edges`` entries, the rest repeating the first edge; ``n_edges`` above
        ``capacity`` means the list did not fit (the entries hold its first
        ``capacity`` edges)."""
        if pos.shape[0] != self.n or pos.dtype != self.dtype or not pos.is_cuda:
            raise ValueError(f"the plan is for {self.n} atoms in {self.dtype} on a GPU")
        dev = pos.device
        cap = int(capacity)
        if cap < 1:
            raise ValueError("capacity must be positive")
        pos = pos.detach().contiguous()
        edge_index = torch.zeros((2, cap), dtype=torch.long, device=dev)
        cell_shifts = torch.zeros((cap, 3), dtype=torch.long, device=dev)
        if self.n == 0:
            return edge_index, cell_shifts, torch.zeros(1, dtype=torch.long, device=dev)
        geom = _lib.dtype_code(pos.dtype)
        s = _lib.stream(dev)
        si = int(self.self_interaction)
        _lib.call("xnn_radius_graph_count", geom, _lib.ptr(pos), self.n, _lib.ptr(self.cell_dev),
                  self.cutoff, si, ctypes.byref(self.grid), _lib.ptr(self.ws),
                  _lib.ptr(self.row_ptr), s)
        _lib.call("xnn_radius_graph_fill", geom, _lib.ptr(pos), self.n, _lib.ptr(self.cell_dev),
                  self.cutoff, si, ctypes.byref(self.grid), _lib.ptr(self.ws),
                  _lib.ptr(self.row_ptr), cap, None, None, None, _lib.ptr(edge_index),
                  _lib.ptr(cell_shifts), None, s)
        n_edges = self.row_ptr[self.n:].to(torch.long)
        pad = torch.arange(cap, device=dev) >= n_edges
        edge_index = torch.where(pad[None, :], edge_index[:, :1], edge_index)
        cell_shifts = torch.where(pad[:, None], cell_shifts[:1], cell_shifts)
        return edge_index, cell_shifts, n_edges


def build_neighbor_list(pos: Tensor, cutoff: float, cell: Optional[Tensor] = None,
                        pbc: Optional[Tensor] = None, self_interaction: bool = False,
                        capacity: Optional[int] = None) -> tuple:
    """Radius graph of one structure: ``(edge_index (2, E) [src, dst], cell_shifts (E, 3))``.

    Same edge set and conventions as the reference (neighborlist.py:411-506): pairs with
    ``dist < cutoff`` in the positions' dtype, ``dst`` = receiver, shifts negated and
    re-expressed for unwrapped positions, self-edges only with ``self_interaction``.
    On a GPU the edges come grouped by receiver (the order the kernels walk). With
    ``capacity`` (GPU): fixed-size buffers and the edge count on the device, see
    :class:`NeighborListPlan` (keep the plan to repeat the call without host reads).
    """
    if capacity is not None:
        return NeighborListPlan(pos, cutoff, cell, pbc, self_interaction)(pos, capacity)
    if pos.is_cuda:
        return _radius_graph_cuda(pos, cutoff, cell, pbc, self_interaction)
    return _brute_force_cpu(pos, cutoff, cell, pbc, self_interaction)


def half_list(pos: Tensor, cutoff: float, cell: Optional[Tensor] = None,
              pbc: Optional[Tensor] = None) -> Optional[tuple]:
    """Every pair within ``cutoff`` once, as ``((i, j), shift)`` with the displacement
    ``pos[j] - pos[i] + shift @ cell``, an atom's own periodic images included once
    (neighborlist.py:217-241, there vesin's half list). Here it is the full list's
    edges ``src < dst`` plus, of an atom's two opposite images, the one whose shift is
    lexicographically positive; never ``None``."""
    edge_index, shifts = build_neighbor_list(pos, cutoff, cell, pbc)
    a, b = edge_index[0], edge_index[1]
    # of the two images (s, -s) of a self-pair: the first nonzero component positive
    sign = torch.where(shifts[:, 0] != 0, shifts[:, 0],
                       torch.where(shifts[:, 1] != 0, shifts[:, 1], shifts[:, 2]))
    keep = ((a < b) | ((a == b) & (sign > 0))).nonzero()[:, 0]
    return (a[keep], b[keep]), shifts[keep]


def unique_pairs(pos: Tensor, cutoff: float, cell: Optional[Tensor] = None,
                 pbc: Optional[Tensor] = None, half: Optional[tuple] = None
                 ) -> tuple[Tensor, Tensor, Tensor]:
    """Every pair within ``cutoff`` once, as ``(i, k, shift)`` with ``i < k``, sorted by
    ``i`` (stable): the edges ``src < dst`` of :func:`build_neighbor_list`, with the
    displacement ``pos[k] - pos[i] + shift @ cell``; an atom's own images are not pairs
    (neighborlist.py:335-387). ``half``: a :func:`half_list` of these positions (each pair
    once in either order), oriented smaller index first (the reversed displacement takes
    the negated shift)."""
    if half is None:
        # the full list holds every pair in both orders: take the order src < dst
        edge_index, shift = build_neighbor_list(pos, cutoff, cell, pbc)
        first, second = edge_index[0], edge_index[1]
        take = first < second
    else:
        # each pair once, in either order: every pair but an atom's own images
        (first, second), shift = half
        take = first != second
    # orient smaller index first; the reversed displacement negates the shift
    flipped = first > second
    i, k = torch.minimum(first, second), torch.maximum(first, second)
    shift = torch.where(flipped[:, None], -shift, shift)
    rows = take.nonzero().squeeze(1)
    rows = rows.index_select(0, torch.argsort(i.index_select(0, rows).to(torch.int32), stable=True))
    return i.index_select(0, rows), k.index_select(0, rows), shift.index_select(0, rows)


def batched_neighbor_list(pos: Tensor, n_atoms: Tensor, cutoff: float,
                          self_interaction: bool = False) -> tuple[Tensor, Tensor]:
    """Radius graph of a batch of molecules (no cell) in one pass on the GPU:
    the edges every structure's own :func:`build_neighbor_list` gives, offset by its
    first atom, grouped by receiver (what :func:`collate` of the single graphs holds,
    up to the edge order)."""
    if not pos.is_cuda:
        raise RuntimeError("batched_neighbor_list runs on the GPU")
    dev = pos.device
    pos = pos.contiguous()
    n = pos.shape[0]
    n_atoms = n_atoms.to(device=dev, dtype=torch.long)
    if n == 0:
        return (torch.zeros((2, 0), dtype=torch.long, device=dev),
                torch.zeros((0, 3), dtype=torch.long, device=dev))
    node_ptr = torch.zeros(n_atoms.shape[0] + 1, dtype=torch.long, device=dev)
    node_ptr[1:] = torch.cumsum(n_atoms, 0)
    batch32 = torch.repeat_interleave(torch.arange(n_atoms.shape[0], device=dev, dtype=torch.int32),
                                      n_atoms)
    lo_hi = torch.stack([pos.detach().amin(0), pos.detach().amax(0)]).double().flatten().tolist()
    _check_finite(lo_hi)
    if int(n_atoms.max()) > 1024:
        raise ValueError("batched_neighbor_list takes molecules of at most 1024 atoms; list "
                         "larger structures one by one with build_neighbor_list")
    geom = _lib.dtype_code(pos.dtype)
    s = _lib.stream(dev)
    row_ptr = torch.empty(n + 1, dtype=torch.int32, device=dev)
    _lib.call("xnn_radius_graph_molecules_count", geom, _lib.ptr(pos), n, _lib.ptr(node_ptr),
              _lib.ptr(batch32), n_atoms.shape[0], float(cutoff), int(bool(self_interaction)),
              _lib.ptr(row_ptr), s)
    ws = torch.empty(int(_lib.load().xnn_scan_workspace_bytes(n)), dtype=torch.uint8, device=dev)
    _lib.call("xnn_scan_counts", _lib.ptr(row_ptr), n, _lib.ptr(ws), s)
    n_edges = int(row_ptr[-1])
    edge_index = torch.empty((2, n_edges), dtype=torch.long, device=dev)
    cell_shifts = torch.empty((n_edges, 3), dtype=torch.long, device=dev)
    src = torch.empty(n_edges, dtype=torch.int32, device=dev)
    dst = torch.empty(n_edges, dtype=torch.int32, device=dev)
    shift = torch.empty(n_edges, dtype=torch.int32, device=dev)
    _lib.call("xnn_radius_graph_molecules_fill", geom, _lib.ptr(pos), n, _lib.ptr(node_ptr),
              _lib.ptr(batch32), n_atoms.shape[0], float(cutoff), int(bool(self_interaction)),
              _lib.ptr(row_ptr), n_edges, _lib.ptr(src), _lib.ptr(dst), _lib.ptr(shift),
              _lib.ptr(edge_index), _lib.ptr(cell_shifts), s)
    return edge_index, cell_shifts


# --------------------------------------------------------------------------- graphs
def nearest_edges(dist, dst: Tensor, num_nodes: int, k: int):
    """The edges to the ``k`` nearest neighbors of every receiver (neighborlist.py:509-552).

    ``dist``: edge lengths (E,) or a function returning them, called only when edges are
    dropped. Returns ``(keep, per_atom)``: ``keep`` the kept edge ids grouped by receiver
    and ordered by (length, edge id) within each, or ``None`` to keep every edge where it
    is; ``per_atom`` the kept count of every atom when it is the same for all. One host
    synchronization (plus one for the kept count on the GPU). On a GPU the ranks come from
    ``xnn_nearest_edges_count`` / ``_fill`` over the receiver CSR.
    """
    if dst.numel() == 0:
        return None, None
    counts = torch.bincount(dst, minlength=num_nodes)
    grouped = (dst[1:] >= dst[:-1]).all() if dst.numel() > 1 else torch.ones((), dtype=torch.bool,
                                                                              device=dst.device)
    lo, hi, grouped = torch.stack([counts.min(), counts.max(), grouped.long()]).tolist()
    if hi <= k:
        if lo < hi:
            return None, None
        return (None if grouped else torch.sort(dst, stable=True).indices), hi
    if callable(dist):
        dist = dist()
    dist = dist.detach()
    per_atom = k if lo >= k else None
    if dst.is_cuda:
        from .functional import csr_of
        _, ptr, perm = csr_of(dst, num_nodes)
        dev = dst.device
        kept_ptr = torch.empty(num_nodes + 1, dtype=torch.int32, device=dev)
        _lib.call("xnn_nearest_edges_count", _lib.ptr(ptr), num_nodes, int(k), _lib.ptr(kept_ptr),
                  _lib.stream(dev))
        need = int(_lib.load().xnn_scan_workspace_bytes(num_nodes))
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
        _lib.call("xnn_scan_counts", _lib.ptr(kept_ptr), num_nodes, _lib.ptr(ws), _lib.stream(dev))
        total = int(counts.clamp(max=k).sum())
        keep = torch.empty(total, dtype=torch.int64, device=dev)
        d = dist.contiguous() if dist.dtype in (torch.float32, torch.float64) else \
            dist.double().contiguous()
        _lib.call("xnn_nearest_edges_fill", _lib.dtype_code(d.dtype), _lib.ptr(d), int(d.numel()),
                  _lib.ptr(ptr), _lib.ptr(perm), num_nodes, int(k), _lib.ptr(kept_ptr),
                  _lib.ptr(keep), _lib.stream(dev))
        return keep, per_atom
    # CPU: order the edges by (receiver, length, id), then keep the first k of each row
    by_len = torch.sort(dist, stable=True).indices
    order = by_len.index_select(0, torch.sort(dst.index_select(0, by_len), stable=True).indices)
    start = torch.cumsum(counts, 0) - counts
    rank = torch.arange(order.numel()) - start.index_select(0, dst.index_select(0, order))
    return order[rank < k], per_atom


def _nearest_in_edges(pos: Tensor, cell: Optional[Tensor], edge_index: Tensor,
                      shifts: Tensor, k: int) -> tuple[Tensor, Tensor]:
    """The edges of :func:`nearest_edges` (each receiver's ``k`` nearest senders), the
    lengths taken in float64 from the positions, shifts and cell whatever their dtype."""
    f64 = torch.float64
    src, dst = edge_index[0], edge_index[1]
    disp = pos.to(f64).index_select(0, dst) - pos.to(f64).index_select(0, src)
    if cell is not None:
        disp = disp + shifts.to(f64) @ cell.to(f64)
    kept, _ = nearest_edges(torch.linalg.vector_norm(disp, dim=1), dst, pos.shape[0], k)
    if kept is None:
        return edge_index, shifts
    return edge_index.index_select(1, kept), shifts.index_select(0, kept)


def structure_to_graph(s: dict, cutoff: float, device=None,
                       max_neighbors: Optional[int] = None) -> AtomicGraph:
    """One structure (dict of arrays) to a graph (dataset.py:21-175): ``pos``,
    ``atomic_numbers`` and optional ``cell``/``pbc`` (a cell without pbc is periodic on
    every axis), ``energy``, ``forces``, ``stress``, ``total_charge``. With
    ``max_neighbors`` every atom keeps its nearest in-edges only (lengths in float64, so
    that the choice does not depend on the run's dtype; dataset.py:112-120)."""
    def t(x, dtype=torch.get_default_dtype()):
        out = x if isinstance(x, Tensor) else torch.as_tensor(np.asarray(x), dtype=dtype)
        return out if device is None else out.to(device)

    pos = t(s["pos"])
    z = t(s["atomic_numbers"], dtype=torch.long)
    cell = t(s["cell"]).reshape(3, 3) if s.get("cell") is not None else None
    pbc = (torch.as_tensor(s["pbc"], dtype=torch.bool) if s.get("pbc") is not None
           else (torch.ones(3, dtype=torch.bool) if cell is not None else None))
    edge_index, cell_shifts = build_neighbor_list(pos, cutoff, cell, pbc)
    if max_neighbors is not None and edge_index.numel():
        edge_index, cell_shifts = _nearest_in_edges(pos, cell, edge_index, cell_shifts,
                                                    int(max_neighbors))
    n = pos.shape[0]
    dev = pos.device
    charge = s.get("total_charge", s.get("charge"))
    return AtomicGraph(
        pos=pos, atomic_numbers=z, edge_index=edge_index, cell_shifts=cell_shifts,
        batch=torch.zeros(n, dtype=torch.long, device=dev),
        n_atoms=torch.tensor([n], dtype=torch.long, device=dev),
        cell=cell[None] if cell is not None else None,
        pbc=pbc.to(dev)[None] if pbc is not None else None,
        energy=(torch.as_tensor(s["energy"], dtype=torch.float64).reshape(1).to(dev)
                if s.get("energy") is not None else None),
        forces=t(s["forces"]) if s.get("forces") is not None else None,
        stress=t(s["stress"]).reshape(1, 3, 3) if s.get("stress") is not None else None,
        total_charge=(t([charge]).reshape(1) if charge is not None else None),
    )


def collate(graphs: Sequence[AtomicGraph]) -> AtomicGraph:
    """Concatenate graphs into one batch (dataset.py:371-577): edge indices offset by
    the running atom count, a ``batch`` vector, zero cells for molecules when any
    structure has a cell."""
    dtype, device = graphs[0].pos.dtype, graphs[0].pos.device
    # where each graph's atoms and structures start in the batch
    node_start = np.cumsum([0] + [g.num_nodes for g in graphs])[:-1].tolist()
    graph_start = np.cumsum([0] + [g.num_graphs for g in graphs])[:-1].tolist()
    periodic = any(g.cell is not None for g in graphs)
    charged = any(g.total_charge is not None for g in graphs)

    def cell_and_pbc(g: AtomicGraph) -> tuple[Tensor, Tensor]:
        # a molecule in a periodic batch: a zero cell, periodic along no axis
        if g.cell is None:
            return (torch.zeros((g.num_graphs, 3, 3), dtype=dtype, device=device),
                    torch.zeros((g.num_graphs, 3), dtype=torch.bool, device=device))
        pbc = (torch.ones((g.num_graphs, 3), dtype=torch.bool, device=device)
               if g.pbc is None else g.pbc.to(device))
        return g.cell, pbc

    cells = [cell_and_pbc(g) for g in graphs] if periodic else None
    return AtomicGraph(
        pos=torch.cat([g.pos for g in graphs], 0),
        atomic_numbers=torch.cat([g.atomic_numbers for g in graphs], 0),
        edge_index=torch.cat([g.edge_index + o for g, o in zip(graphs, node_start)], 1),
        cell_shifts=torch.cat([g.cell_shifts for g in graphs], 0),
        batch=torch.cat([g.batch + o for g, o in zip(graphs, graph_start)], 0),
        n_atoms=torch.cat([g.n_atoms for g in graphs], 0),
        cell=torch.cat([c for c, _ in cells], 0) if periodic else None,
        pbc=torch.cat([p for _, p in cells], 0) if periodic else None,
        total_charge=torch.cat([g.total_charge if g.total_charge is not None
                                else torch.zeros(g.num_graphs, dtype=dtype, device=device)
                                for g in graphs], 0) if charged else None)
