"""Conservative forces and stress by differentiation (common/models/outputs.py:96-239).

``forces = -dE/dpos``; ``stress = (1/V) dE/d(strain)`` with the symmetric-strain trick:
positions and cell are displaced by ``sym(eps)`` at ``eps = 0`` so that autograd
carries the virial back to ``eps``. On a GPU the backward of the edge vectors is the
HIP CSR force reduction, so no float atomics touch the forces; for a model whose energy
depends on positions only through the edge vectors, that same reduction also forms
``dE/d(eps) = sym(sum_e r_e (x) dE/dr_e)`` (the identity behind the trick), so nothing
deforms positions or cell in the forward.
"""
from __future__ import annotations

import itertools
from typing import Optional

import torch
from torch import Tensor, nn

from .functional import cell_volume


class ForceStressOutput(nn.Module):
    """Wrap a model to add ``forces`` (N, 3) and, for periodic structures, ``stress``
    (B, 3, 3) (outputs.py:25-224)."""

    def __init__(self, model: nn.Module, compute_forces: bool = True, compute_stress: bool = False):
        super().__init__()
        self.model = model
        self.compute_forces = compute_forces
        self.compute_stress = compute_stress
        self.cutoff = getattr(model, "cutoff", None)

    def _model_dtype(self) -> Optional[torch.dtype]:
        """The floating dtype the wrapped model computes in: its parameters' when it has a
        floating parameter, else its buffers', else ``None`` (outputs.py:73-94). The search
        stops at the first floating tensor, normally the first parameter."""
        tensors = itertools.chain(self.model.parameters(), self.model.buffers())
        first = next((t for t in tensors if t.is_floating_point()), None)
        return None if first is None else first.dtype

    def _direct_evaluation(self, data, plan) -> bool:
        """True in evaluation mode when the model offers to form forces and the strain
        derivative in its own forward (``forms_forces(data)``), so that no autograd pass
        is needed; never with a plan or when forces are not wanted."""
        offer = getattr(self.model, "forms_forces", None)
        if self.training or not self.compute_forces or plan is not None or not callable(offer):
            return False
        return bool(offer(data))

    @staticmethod
    def _zero_strain(data) -> Tensor:
        # a fresh leaf per call: a leaf kept across calls would keep the gradient
        # accumulator of the call that first used it, bound to that call's stream; a later
        # call under stream capture would then synchronize the capturing stream with that
        # other stream (autograd's producer/consumer stream sync), which breaks the capture
        return torch.zeros((data.num_graphs, 3, 3), dtype=data.pos.dtype,
                           device=data.pos.device, requires_grad=True)

    def forward(self, data, plan=None) -> dict:
        create_graph = self.training
        if self._direct_evaluation(data, plan):
            # the model returns forces and its virial itself (outputs.py:136-143)
            out = self.model.forward_direct(data)
            virial = out.pop("virial")
            if self.compute_stress and data.cell is not None:
                out["stress"] = _stress(virial, data)
            return out
        # a float64 geometry for a float32 model: the model computes in its own dtype
        # through edge_vectors(), the derivatives are taken at the float64 leaves
        # (outputs.py:146-151)
        if data.compute_dtype is None:
            dtype = self._model_dtype()
            if dtype is not None and dtype != data.pos.dtype:
                data.compute_dtype = dtype
        strain: Optional[Tensor] = None
        # A model whose energy depends on positions and cell only through the edge vectors
        # (``edge_virial``) gets the strain derivative from the edge-vector backward itself,
        # sym(sum_e r_e (x) dE/dr_e), the same derivative as deforming pos and cell by the
        # strain; the training step (create_graph) and the CPU keep the deformation.
        probe = (self.compute_stress and data.cell is not None and not create_graph
                 and data.pos.is_cuda and bool(getattr(self.model, "edge_virial", False)))
        if probe:
            # the probe's value is never read (zero by contract): no fill launch
            strain = torch.empty((data.num_graphs, 3, 3), dtype=data.pos.dtype,
                                 device=data.pos.device, requires_grad=True)
            data.strain_probe = strain
        elif self.compute_stress and data.cell is not None and data.pos.is_cuda and not create_graph:
            # one HIP kernel each way instead of the broadcast products (differentiable once)
            from .ops import strain_apply_op
            strain = self._zero_strain(data)
            batch32, node_ptr = _layout(data)
            data.pos, cell = strain_apply_op(data.pos.contiguous(),
                                             data.cell.reshape(-1, 3, 3).to(data.pos.dtype).contiguous(),
                                             strain, batch32, node_ptr)
            data.cell = cell.to(data.cell.dtype)
        elif self.compute_stress and data.cell is not None:
            strain = torch.zeros((data.num_graphs, 3, 3), dtype=data.pos.dtype,
                                 device=data.pos.device, requires_grad=True)
            sym = 0.5 * (strain + strain.transpose(-1, -2))
            if data.num_graphs == 1:
                data.pos = data.pos + (data.pos[:, :, None] * sym[0]).sum(1)
            else:
                data.pos = data.pos + (data.pos[:, :, None] * sym.index_select(0, data.batch)).sum(1)
            data.cell = data.cell + (data.cell[:, :, :, None] * sym[:, None]).sum(2)
        if self.compute_forces and not data.pos.requires_grad:
            # a fresh leaf per call; the caller's tensor is left untouched. Turning the
            # caller's positions into a leaf would keep one gradient accumulator across
            # calls, bound to the stream of the call that made it, and autograd would sync a
            # later call's stream with that one -- which breaks HIP graph capture (a host
            # crash in capture_end) when the later call is captured.
            data.pos = data.pos.detach().requires_grad_(True)
        # the double-backward of a training step needs the differentiable formulation
        if hasattr(self.model, "double_backward"):
            self.model.double_backward = bool(create_graph)
        # forces and stress alone need no parameter gradients (the training step's
        # create_graph=True keeps them)
        had_param_grads = getattr(self.model, "param_grads", None)
        if had_param_grads is not None:
            self.model.param_grads = bool(create_graph)
        # a model whose total is not the sum of its returned node energies (a dispersion
        # correction) is differentiated through its per-structure energies only: its
        # per-atom energies need no gradient outside a training step
        had_node_grads = getattr(self.model, "node_energy_grads", None)
        if had_node_grads is not None and not getattr(self.model, "energy_is_node_sum", False):
            self.model.node_energy_grads = bool(create_graph)
        # one structure whose energy is the sum of its node energies: the model leaves the
        # total to this wrapper, which forms it with the stress in one kernel after the
        # backward (the backward starts from the node energies anyway)
        defer = (probe and self.compute_forces and plan is None and data.num_graphs == 1
                 and bool(getattr(self.model, "energy_is_node_sum", False))
                 and hasattr(self.model, "defer_energy_sum")
                 and data.num_nodes <= _energy_stress_max_nodes())
        if defer:
            self.model.defer_energy_sum = True
        try:
            out = self.model(data) if plan is None else self.model(data, plan)
        finally:
            if had_param_grads is not None:
                self.model.param_grads = had_param_grads
            if had_node_grads is not None:
                self.model.node_energy_grads = had_node_grads
            if defer:
                self.model.defer_energy_sum = False
            if probe:
                data.strain_probe = None
        if "energy" not in out:
            # a property model predicts no energy: no forces or stress (outputs.py:187-189)
            return out
        energy = out["energy"]
        if energy is None:
            return self._deferred_energy_stress(out, data, strain)
        # a model that predicts its forces directly returns them itself (outputs.py:191-194)
        # forces the model predicts itself are returned as they are (outputs.py:191-194);
        # an added energy term would then have no forces of its own, so that is refused
        direct = "forces" in out
        if direct and "energy_sr" in out:
            raise ValueError("forces predicted by the model itself leave no gradient for the "
                             "added energy terms (dispersion, long-range): use a conservative "
                             "model with them")
        inputs, need = [], []
        if self.compute_forces and not direct:
            inputs.append(data.pos)
            need.append("pos")
        if strain is not None:
            inputs.append(strain)
            need.append("strain")
        g = {k: None for k in need}
        if inputs and energy.requires_grad:
            # the backward is seeded with -1: it returns d(-E), so the forces need no extra
            # negation (negation is exact, the result is bitwise -dE/dpos). A model whose
            # energy is exactly the structure sum of its node energies is differentiated
            # from the node energies (dE/dE_i = 1), skipping the sum's backward.
            target = energy
            seed = None
            node_energy = out.get("node_energy")
            if (not create_graph and bool(getattr(self.model, "energy_is_node_sum", False))
                    and node_energy is not None and node_energy.requires_grad):
                target = node_energy
                seed = _minus_one(node_energy).expand(node_energy.shape)
            else:
                seed = torch.full_like(energy, -1.0)
            grads = torch.autograd.grad([target], inputs, grad_outputs=[seed],
                                        create_graph=create_graph, retain_graph=create_graph,
                                        allow_unused=True)
            g = dict(zip(need, grads))
        if self.compute_forces and not direct:
            out["forces"] = g["pos"] if g.get("pos") is not None else torch.zeros_like(data.pos)
        if strain is not None:
            out["stress"] = (_stress(g["strain"], data, scale=-1.0, differentiable=create_graph)
                             if g.get("strain") is not None else torch.zeros_like(strain))
        return out


    def _deferred_energy_stress(self, out: dict, data, strain: Tensor) -> dict:
        """Forces and strain derivative from the node energies (seed -1), then the energy
        total and the stress in one kernel (one structure, no training graph)."""
        from .ops import energy_stress_finish
        node_energy = out["node_energy"]
        seed = _minus_one(node_energy).expand(node_energy.shape)
        g_pos, g_strain = torch.autograd.grad([node_energy], [data.pos, strain],
                                              grad_outputs=[seed], allow_unused=True)
        out["forces"] = g_pos if g_pos is not None else torch.zeros_like(data.pos)
        if g_strain is None:
            g_strain = torch.zeros_like(strain)
        out["energy"], out["stress"] = energy_stress_finish(node_energy, g_strain, data.cell,
                                                            data.pbc, scale=-1.0)
        return out


_ES_MAX = []


def _energy_stress_max_nodes() -> int:
    if not _ES_MAX:
        from . import _lib
        _ES_MAX.append(int(_lib.load().xnn_energy_stress_max_nodes()))
    return _ES_MAX[0]


_MINUS_ONE = {}


def _minus_one(like: Tensor) -> Tensor:
    """A (1,) tensor of -1 on ``like``'s device and dtype, made once outside graph capture
    (a captured step then reads it instead of launching a fill)."""
    key = (like.device, like.dtype)
    t = _MINUS_ONE.get(key)
    if t is None:
        t = torch.full((1,), -1.0, dtype=like.dtype, device=like.device)
        if not (like.is_cuda and torch.cuda.is_current_stream_capturing()):
            _MINUS_ONE[key] = t
    return t


def _layout(data):
    """int32 structure index per atom and int64 structure offsets (B+1): from the edge
    plan when the graph has one (cached), else from n_atoms."""
    if data.num_edges > 0:
        plan = data.plan()
        return plan.batch32, plan.node_ptr
    node_ptr = torch.zeros(data.num_graphs + 1, dtype=torch.int64, device=data.pos.device)
    node_ptr[1:] = torch.cumsum(data.n_atoms.to(data.pos.device), 0)
    return data.batch.to(torch.int32).contiguous(), node_ptr


def _stress(strain_gradient: Tensor, data, scale: float = 1.0,
            differentiable: bool = False) -> Tensor:
    """``scale * strain_gradient / V`` per structure, zero for molecules of a batch
    (outputs.py:227-239); ``scale = -1`` when the gradient is that of ``-E``. On a GPU
    outside training this is one HIP kernel."""
    if strain_gradient.is_cuda and data.cell.is_cuda and not differentiable:
        from .ops import stress_finish
        return stress_finish(strain_gradient, data.cell, data.pbc, scale)
    volume = cell_volume(data.cell)
    periodic = volume > 1e-8
    if data.pbc is not None:
        periodic = periodic & data.pbc.any(-1).to(periodic.device)
    safe = torch.where(periodic, volume, torch.ones_like(volume))
    return torch.where(periodic[:, None, None], (scale * strain_gradient) / safe[:, None, None],
                       torch.zeros_like(strain_gradient))
