"""Deployment entry points (common/deploy/lammps.py, common/deploy/torchscript.py:883-921).

:class:`LAMMPSWrapper` keeps the reference's pair-style tensor ABI -- ``forward(pos,
edge_index, cell_shifts, atomic_numbers, cell)`` returning ``total_energy`` (1,),
``node_energy`` (N,) and ``forces`` (N, 3) (plus ``virial`` (3, 3), which the reference's
pair styles form themselves) -- for the measured edge potential
(:class:`~xnn_amd.models.ShEdgePotential`). Each call is one C-ABI call,
``xnn_sh_pair_energy_forces``, which a C++ pair style can make directly without Python or
libtorch; this class is its Python face, for tests and for Python MD drivers.
"""
from __future__ import annotations

import ctypes
from typing import Dict, Optional

import torch
from torch import Tensor, nn

from . import _lib
from .featurizers import radial_spec
from .ops import linear_message_supported


class LAMMPSWrapper(nn.Module):
    """Pair-style bridge for :class:`~xnn_amd.models.ShEdgePotential` (lammps.py:23-145).

    ``cutoff`` is the neighbor-list radius the pair style must supply (the model's own by
    default); edges beyond the model's cutoff contribute nothing (its envelope is zero
    there). Float32 model arithmetic; positions and cell in float32 or float64.
    """

    def __init__(self, model, cutoff: Optional[float] = None):
        super().__init__()
        self.model = model
        self.cutoff = float(model.cutoff if cutoff is None else cutoff)
        feat = model.edge_feat
        if not linear_message_supported(model.W.shape[0], model.W.shape[1], model.l_max):
            raise ValueError("the pair-style kernels take this model's fused-kernel shapes only "
                             "(see ops.linear_message_supported)")
        if getattr(feat, "radial_trainable", False):
            raise ValueError("trainable radial frequencies are not on the pair-style path")
        self._ws: Optional[Tensor] = None

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
        n, e = int(pos.shape[0]), int(edge_index.shape[1])
        periodic = bool(torch.linalg.norm(cell.detach().to(torch.float64), dim=1).sum() > 1e-8)
        cl = cell.detach().to(device=dev, dtype=dtype).reshape(3, 3).contiguous() if periodic else None
        ei = edge_index.to(device=dev, dtype=torch.int64).contiguous()
        sh = cell_shifts.to(device=dev, dtype=torch.int64).contiguous() if periodic else None
        z = atomic_numbers.to(device=dev, dtype=torch.int64).contiguous()
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
        return {"total_energy": torch.tensor([energy.value], dtype=torch.float64, device=dev),
                "node_energy": node_energy, "forces": forces, "virial": virial}
