"""Deployment entry points (common/deploy/lammps.py, common/deploy/torchscript.py:883-921).

:class:`LAMMPSWrapper` keeps the reference's pair-style tensor ABI -- ``forward(pos,
edge_index, cell_shifts, atomic_numbers, cell)`` returning ``total_energy`` (1,),
``node_energy`` (N,) and ``forces`` (N, 3), plus ``virial`` (3, 3), which the reference's
pair styles form themselves -- for any registered model (``forward(AtomicGraph) ->
{"node_energy", "energy"}``), optionally wrapped in D4 / D3 dispersion corrections, as the
reference splits a model into its core and its dispersion head (lammps.py:70-79) and adds
the head's per-atom energies (lammps.py:128-134).

For the measured edge potential (:class:`~xnn_amd.models.ShEdgePotential`) the core runs
as one C-ABI call, ``xnn_sh_pair_energy_forces``, which a C++ pair style can make directly
without Python or libtorch; this class is its Python face, for tests and for Python MD
drivers. Other cores run through :class:`~xnn_amd.outputs.ForceStressOutput` on the HIP
ops. The dispersion heads need no edge list (their HIP kernels sum every pair image
within their own cutoffs from the positions and the cell), so the pair style supplies the
core's list only.
"""
from __future__ import annotations

import ctypes
from typing import Dict, List, Optional, Tuple

import torch
from torch import Tensor, nn

from . import _lib
from .featurizers import radial_spec
from .ops import linear_message_supported


def build_neighbor_list_ts(pos: Tensor, cutoff: float, cell: Tensor,
                           pbc: Tensor) -> Tuple[Tensor, Tensor]:
    """The deployment form of the neighbor list (torchscript.py:124-212): the same arguments
    as the exported artifact's, ``cell`` (3, 3) all zeros and / or no periodic flag for a
    molecule, ``pbc`` (3,); returns ``(edge_index [src, dst], cell_shifts)`` with the same
    conventions. On the GPU it is the HIP cell list (:func:`~xnn_amd.data.
    build_neighbor_list`), O(N x neighbors) instead of the exported artifact's brute force
    over (images, N, N), so it serves large cells too; it is a Python function, not a
    TorchScript one (the HIP path is reached through the C ABI in a C++ engine)."""
    from .data import build_neighbor_list
    cell = cell.reshape(3, 3)
    pbc = pbc.reshape(3).to(torch.bool)
    periodic = bool(pbc.any()) and bool(torch.linalg.norm(cell.to(torch.float64), dim=1).sum() > 1e-8)
    if not periodic:
        return build_neighbor_list(pos, cutoff)
    return build_neighbor_list(pos, cutoff, cell.to(pos.dtype), pbc.cpu())


def split_dispersion(model: nn.Module) -> Tuple[Optional[nn.Module], List[nn.Module]]:
    """``(core, terms)``: the innermost model (``None`` for a standalone dispersion model)
    and the dispersion terms of every :class:`~xnn_amd.dispersion.DispersionCorrection`
    wrapped around it, outermost first (torchscript.py:561-615 for the D4 / D3 heads)."""
    from .dispersion import DispersionCorrection
    terms: List[nn.Module] = []
    core: Optional[nn.Module] = model
    while isinstance(core, DispersionCorrection):
        terms.append(core.term)
        core = core.model
    return core, terms


def _sh_pair_supported(core: nn.Module) -> bool:
    from .models import ShEdgePotential
    return (isinstance(core, ShEdgePotential)
            and linear_message_supported(core.W.shape[0], core.W.shape[1], core.l_max)
            and not getattr(core.edge_feat, "radial_trainable", False))


class LAMMPSWrapper(nn.Module):
    """Pair-style bridge for a registered model and its dispersion heads (lammps.py:23-145).

    ``cutoff`` is the neighbor-list radius the pair style supplies (the core's own by
    default). Edges at or beyond the core's cutoff are dropped before the core sees them
    (lammps.py:117-120), so a model whose envelope does not vanish there (``"none"``)
    is evaluated on its own cutoff's edges only. ``total_charge`` is the system's net charge
    for the D4 charges. Positions and cell in float32 or float64.
    """

    def __init__(self, model: nn.Module, cutoff: Optional[float] = None,
                 total_charge: float = 0.0):
        super().__init__()
        core, terms = split_dispersion(model)
        self.model = core
        self.terms = nn.ModuleList(terms)
        self.total_charge = float(total_charge)
        self.core_cutoff = float(getattr(core, "cutoff", 0.0)) if core is not None else 0.0
        self.cutoff = float(self.core_cutoff if cutoff is None else cutoff)
        if core is not None and self.cutoff < self.core_cutoff:
            raise ValueError(f"the neighbor list ({self.cutoff}) must reach the model's "
                             f"cutoff ({self.core_cutoff})")
        self.fused_core = core is not None and _sh_pair_supported(core)
        self._ws: Optional[Tensor] = None

    # ------------------------------------------------------------------ the fused core
    def _model_struct(self, device: torch.device):
        m = self.model
        spec = radial_spec(m.edge_feat)
        table = spec["table"].to(device=device, dtype=torch.float32).contiguous()
        W = m.W.detach().to(device=device, dtype=torch.float32).contiguous()
        U = m.U.detach().to(device=device, dtype=torch.float32).contiguous()
        ref = m.atom_ref.detach().to(device=device, dtype=torch.float32).contiguous()
        prm = _lib.FeaturizeParams(int(W.shape[0]), _lib.BASIS[spec["basis"]],
                                   _lib.ENVELOPE[spec["envelope"]], int(spec["poly_p"]),
                                   int(m.l_max), int(m.sh_sign), float(spec["cutoff"]),
                                   float(spec["prefactor"]), float(spec["gamma"]))
        keep = (table, W, U, ref, prm)
        st = _lib.ShPairModel(ctypes.pointer(prm), table.data_ptr(), int(W.shape[1]), W.data_ptr(),
                              U.data_ptr(), ref.data_ptr(), int(ref.numel()))
        return st, keep

    def _fused_core(self, pos, ei, sh, z, cl):
        dev, dtype = pos.device, pos.dtype
        n, e = int(pos.shape[0]), int(ei.shape[1])
        need = int(_lib.load().xnn_sh_pair_workspace_bytes(n, e))
        if self._ws is None or self._ws.numel() < need or self._ws.device != dev:
            self._ws = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
        node_energy = torch.empty(n, dtype=torch.float32, device=dev)
        forces = torch.empty((n, 3), dtype=dtype, device=dev)
        virial = torch.empty((3, 3), dtype=torch.float64, device=dev)
        energy = ctypes.c_double(0.0)
        st, keep = self._model_struct(dev)
        _lib.call("xnn_sh_pair_energy_forces", ctypes.byref(st), _lib.dtype_code(dtype),
                  _lib.ptr(pos), n, _lib.ptr(z), _lib.ptr(ei), _lib.ptr(sh), e, _lib.ptr(cl),
                  ctypes.byref(energy), _lib.ptr(node_energy), _lib.ptr(forces), _lib.ptr(virial),
                  _lib.ptr(self._ws), int(self._ws.numel()), _lib.stream(dev))
        del keep
        return node_energy.to(torch.float64), forces, virial

    # ------------------------------------------------------------------ any potential
    def _graph(self, pos, ei, sh, z, cl):
        from .data import AtomicGraph
        n, dev = pos.shape[0], pos.device
        return AtomicGraph(
            pos=pos, atomic_numbers=z, edge_index=ei,
            cell_shifts=sh if sh is not None else torch.zeros((ei.shape[1], 3), dtype=torch.long,
                                                              device=dev),
            batch=torch.zeros(n, dtype=torch.long, device=dev),
            n_atoms=torch.tensor([n], dtype=torch.long, device=dev),
            cell=None if cl is None else cl[None],
            pbc=None if cl is None else torch.ones((1, 3), dtype=torch.bool, device=dev),
            total_charge=torch.full((1,), self.total_charge, dtype=pos.dtype, device=dev))

    def _evaluate(self, potential: nn.Module, pos, ei, sh, z, cl):
        """Per-atom energies (float64), forces and the virial -sym(sum_e r_e (x) dE/dr_e)
        of ``potential`` through :class:`~xnn_amd.outputs.ForceStressOutput`: from the
        stress (``-V sigma``) for a cell, from ``sym(sum_i r_i (x) F_i)`` for a molecule."""
        from .functional import cell_volume
        from .outputs import ForceStressOutput
        g = self._graph(pos, ei, sh, z, cl)
        out = ForceStressOutput(potential, compute_stress=cl is not None).eval()(g)
        forces = out["forces"].detach().to(pos.dtype)
        if cl is not None:
            vol = cell_volume(cl[None].to(torch.float64))[0]
            virial = -vol * out["stress"].detach()[0].to(torch.float64)
        else:
            rf = pos.to(torch.float64).T @ forces.to(torch.float64)
            virial = 0.5 * (rf + rf.T)
        return out["node_energy"].detach().to(torch.float64), forces, virial

    def forward(self, pos: Tensor, edge_index: Tensor, cell_shifts: Tensor,
                atomic_numbers: Tensor, cell: Tensor) -> Dict[str, Tensor]:
        """Energy, per-atom energies, forces and virial from the pair style's tensors; the
        cell is all zeros for a molecule (periodicity is read from it, as
        torchscript.py:917-921 does)."""
        if not pos.is_cuda:
            raise RuntimeError("the pair-style entry point runs on the GPU only")
        dev = pos.device
        dtype = pos.dtype if pos.dtype in (torch.float32, torch.float64) else torch.float64
        pos = pos.detach().to(dtype).contiguous()
        n = int(pos.shape[0])
        periodic = bool(torch.linalg.norm(cell.detach().to(torch.float64), dim=1).sum() > 1e-8)
        cl = cell.detach().to(device=dev, dtype=dtype).reshape(3, 3).contiguous() if periodic else None
        ei = edge_index.to(device=dev, dtype=torch.int64).contiguous()
        sh = cell_shifts.to(device=dev, dtype=torch.int64).contiguous() if periodic else None
        z = atomic_numbers.to(device=dev, dtype=torch.int64).contiguous()
        node_energy = torch.zeros(n, dtype=torch.float64, device=dev)
        forces = torch.zeros((n, 3), dtype=dtype, device=dev)
        virial = torch.zeros((3, 3), dtype=torch.float64, device=dev)
        if self.model is not None:
            if self.cutoff > self.core_cutoff:
                # the core sees the edges within its own cutoff only (strict, as the list's)
                vec = pos.index_select(0, ei[1]) - pos.index_select(0, ei[0])
                if cl is not None:
                    vec = vec + sh.to(dtype) @ cl
                keep = (torch.linalg.vector_norm(vec, dim=1) < self.core_cutoff).nonzero().squeeze(1)
                ei = ei.index_select(1, keep).contiguous()
                sh = sh.index_select(0, keep).contiguous() if sh is not None else None
            if self.fused_core:
                parts = self._fused_core(pos, ei, sh, z, cl)
            else:
                parts = self._evaluate(self.model, pos, ei, sh, z, cl)
            node_energy += parts[0]
            forces += parts[1]
            virial += parts[2]
        if len(self.terms):
            from .dispersion import DispersionCorrection
            empty = torch.zeros((2, 0), dtype=torch.int64, device=dev)
            no_shift = torch.zeros((0, 3), dtype=torch.int64, device=dev)
            for term in self.terms:
                e_i, f, w = self._evaluate(DispersionCorrection(term), pos, empty,
                                           no_shift if cl is not None else None, z, cl)
                node_energy += e_i
                forces += f
                virial += w
        total = node_energy.sum().reshape(1)
        return {"total_energy": total, "node_energy": node_energy, "forces": forces,
                "virial": virial}
