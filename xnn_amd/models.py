"""The model contract and registry (common/models/base.py:24-180, registry.py:23-111),
and :class:`ShEdgePotential`, the edge -> atom model the hot path is measured on.

Every model maps an :class:`~xnn_amd.data.AtomicGraph` to
``{"node_energy": (N,), "energy": (B,) float64}``; forces and stress come from
:class:`~xnn_amd.outputs.ForceStressOutput`.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Callable, Dict, Optional, Sequence, Type

import torch
from torch import Tensor, nn

from .fast import MI355X_POLICY, UseFast, fast_modules, resolve_use_fast, select
from .featurizers import SphericalHarmonicEdgeEmbedding
from .functional import scatter_sum, structure_sum

_MODELS: Dict[str, Type] = {}


def register_model(name: str) -> Callable[[Type], Type]:
    """Class decorator registering a model under ``name`` (case-insensitive; registry.py:23-71)."""
    def deco(cls: Type) -> Type:
        key = name.lower()
        if key in _MODELS and _MODELS[key] is not cls:
            raise KeyError(f"model '{name}' already registered")
        _MODELS[key] = cls
        return cls
    return deco


def get_model_class(name: str) -> Type:
    try:
        return _MODELS[name.lower()]
    except KeyError:
        raise KeyError(f"unknown model {name!r}; registered: {sorted(_MODELS)}") from None


@dataclass
class ModelConfig:
    """``name`` selects the registered class; ``params`` go to its constructor
    (the shape of config/schema.py ModelConfig for this path)."""
    name: str
    params: dict = field(default_factory=dict)


def build_model(cfg: ModelConfig) -> nn.Module:
    """Instantiate a registered model from its config (registry.py:74-111)."""
    return get_model_class(cfg.name).from_config(cfg)


class InteratomicPotential(nn.Module):
    """Base class: ``forward(AtomicGraph) -> {"node_energy", "energy"}`` (base.py:24-180)."""

    head_modules = ()
    # True when the energy depends on positions and cell only through
    # data.edge_vectors(): ForceStressOutput then takes the strain derivative from the
    # edge-vector backward instead of deforming positions and cell
    edge_virial = False
    # True when ``energy`` is exactly the structure sum of ``node_energy`` (ForceStressOutput
    # then differentiates the node energies directly)
    energy_is_node_sum = False
    # set by ForceStressOutput for one structure on a GPU: ``energy`` comes back as None
    # and the wrapper forms the total together with the stress after the backward
    defer_energy_sum = False

    def forward(self, data) -> dict:
        raise NotImplementedError

    @classmethod
    def from_config(cls, cfg: ModelConfig) -> "InteratomicPotential":
        return cls(**cfg.params)

    def aggregate_energy(self, node_energy: Tensor, data) -> Tensor:
        """Per-structure energies in float64 (base.py:161-180); on a GPU over the
        plan's structure ranges (no host synchronization, so it can be graph-captured).
        None when the caller asked to form the total itself (``defer_energy_sum``)."""
        if self.defer_energy_sum and node_energy.is_cuda:
            return None
        if node_energy.is_cuda:
            from .ops import structure_sum_op
            plan = data.plan()
            return structure_sum_op(node_energy, plan.node_ptr, plan.batch32)
        return structure_sum(node_energy, data.batch, data.num_graphs)


@register_model("sh_edge")
class ShEdgePotential(InteratomicPotential):
    """One equivariant edge -> atom interaction, the measured hot path.

    Per edge ``e = (src -> dst)`` with vector ``r_e``: radial features
    ``u_e = rbf(|r_e|) * envelope(|r_e|)`` (K), channel weights ``phi_e = u_e W`` (C,
    a PyTorch linear), and the message ``phi_e (x) Y(r_e)`` summed onto the receiver:
    ``A_i = sum_{dst(e)=i} phi_e (x) Y(r_e)``, ``(N, C, (l_max+1)^2)``. This is the uvu
    tensor product of scalar weights with the edge harmonics followed by
    ``scatter_sum`` (gnn/fast/conv.py:137-143). The readout is
    ``E_i = sum_{c,lm} U[c, lm] A_i[c, lm] + atom_ref[Z_i]`` and ``E = sum_i E_i`` in
    float64. On a GPU the featurizer and the fused message sum are HIP kernels (the
    message never exists in memory); with ``fused_linear`` (the default, for the channel
    counts the fused kernels take) the radial linear layer is applied inside the message
    kernels too, per atom (``A_i = W^T sum_e u_e (x) Y_e``, the same sum reassociated), so
    ``phi`` is never formed, and with ``fused_radial`` (the default) forces and stress
    evaluate the radial basis inside those kernels as well (one kernel each way; parameter
    gradients take the two-kernel path). The (N, C, L) rows A are written to memory and
    read out by their own op, whose backward hands the message backward a general
    (N, C, L) cotangent, as a model whose rows feed PyTorch layers needs. With
    ``fused_readout`` the message kernels apply the readout themselves instead (no rows in
    memory), and ``one_pass`` then takes energies and forces from one backward launch.
    ``use_fast=False`` or a CPU evaluates the same function with the PyTorch formulation.
    """

    edge_virial = True
    # forces and stress with energies and gradients from one backward launch (the readout
    # path; node energies as CSR sums of the edges' shares, exact gradients for any seed)
    one_pass = False
    # energy = structure_sum(node_energy), nothing added at the structure level
    energy_is_node_sum = True

    def __init__(self, species: Sequence[int] = (1, 6, 7, 8), n_rbf: int = 8, l_max: int = 3,
                 channels: int = 128, cutoff: float = 5.0, radial_type: str = "bessel",
                 envelope: str = "polynomial", p: int = 6, sh_sign: int = 1,
                 use_fast: UseFast = "auto", seed: Optional[int] = 0, fused_linear: bool = True,
                 fused_radial: bool = True, fused_readout: bool = False):
        super().__init__()
        self.cutoff = float(cutoff)
        self.l_max = int(l_max)
        self.channels = int(channels)
        self.sh_sign = int(sh_sign)
        self.fused_linear = bool(fused_linear)
        self.fused_radial = bool(fused_radial)
        self.fused_readout = bool(fused_readout)
        self.use_fast = resolve_use_fast(use_fast)
        self.double_backward = False
        # False while ForceStressOutput evaluates forces only (no parameter gradients)
        self.param_grads = True
        self.edge_feat = SphericalHarmonicEdgeEmbedding(
            l_max=l_max, n_rbf=n_rbf, cutoff=cutoff, p=p, radial_type=radial_type,
            envelope=envelope)
        gen = torch.Generator().manual_seed(seed) if seed is not None else None
        L = (l_max + 1) ** 2
        self.W = nn.Parameter(torch.randn(n_rbf, channels, generator=gen) / n_rbf ** 0.5)
        self.U = nn.Parameter(torch.randn(channels, L, generator=gen) / (channels * L) ** 0.5)
        z_max = max(species) + 1
        self.register_buffer("species", torch.tensor(list(species), dtype=torch.long))
        self.atom_ref = nn.Parameter(0.1 * torch.randn(z_max, generator=gen))

    def messages(self, data, vec: Tensor) -> Tensor:
        """``A (N, C, L)`` from edge vectors (HIP fused sum or PyTorch scatter)."""
        feat = self.edge_feat
        if feat.fast_active:
            from .ops import linear_message_supported, sh_linear_message_sum, sh_message_sum
            W = self.W.to(vec.dtype)
            if not self.param_grads:
                W = W.detach()
            if self.fused_linear and linear_message_supported(W.shape[0], W.shape[1], self.l_max):
                if self.fused_radial and not W.requires_grad and not feat.radial_trainable:
                    # forces and stress only: radial basis, linear layer and message in one
                    # kernel each way (neither u nor phi is stored)
                    return feat.radial_message_sum(vec, W, data.plan(), self.sh_sign)
                # the radial linear layer runs inside the message kernels: phi = u W is
                # formed per edge tile in registers, never stored
                u = feat.radial(vec)
                return sh_linear_message_sum(vec, u, W, data.plan(), self.l_max, self.sh_sign)
            u = feat.radial(vec)
            return sh_message_sum(vec, u @ W, data.plan(), self.l_max, self.sh_sign)
        _, sh, u = feat.embed(vec, sh_sign=self.sh_sign)
        phi = u @ self.W.to(u.dtype)
        msg = (phi[:, :, None] * sh[:, None, :]).reshape(vec.shape[0], -1)
        if msg.is_cuda:
            from .ops import segment_sum_op
            plan = data.plan()
            out = segment_sum_op(msg.contiguous(), plan.dst, plan.ptr_dst, plan.perm_dst)
        else:
            out = scatter_sum(msg, data.edge_index[1], data.num_nodes)
        return out.reshape(data.num_nodes, self.channels, -1)

    def forward(self, data) -> dict:
        dtype = data.model_dtype
        select(fast_modules(self), self.use_fast, MI355X_POLICY, data.pos.device, dtype,
               data.num_edges, double_backward=self.double_backward)
        vec = data.edge_vectors()
        feat = self.edge_feat
        if (feat.fast_active and self.fused_radial and self.fused_readout and not self.param_grads
                and not feat.radial_trainable and vec.dtype == torch.float32):
            from .ops import linear_message_supported
            if linear_message_supported(self.W.shape[0], self.W.shape[1], self.l_max):
                # forces and stress only: radial basis, linear layer, message and readout in
                # one kernel each way (neither u, phi nor the (N, C, L) rows are stored)
                node_energy = feat.radial_message_energy(
                    vec, self.W.detach().float(), self.U.detach().float(), data.atomic_numbers,
                    self.atom_ref.detach(), data.plan(), self.sh_sign, one_pass=self.one_pass)
                return {"node_energy": node_energy,
                        "energy": self.aggregate_energy(node_energy, data)}
        A = self.messages(data, vec)
        # readout E_i = <U, A_i> + atom_ref[Z_i]: on the fast path one HIP launch each
        # way (the rows streamed once, the reference energy gathered in the same pass)
        if self.edge_feat.fast_active:
            from .ops import node_readout_op
            U, ref = self.U.reshape(-1), self.atom_ref
            if not self.param_grads:
                # a custom op's backward cannot see which inputs the current backward
                # asks for: detached parameters keep it to the rows' gradient
                U, ref = U.detach(), ref.detach()
            node_energy = node_readout_op(A.reshape(A.shape[0], -1), U, data.atomic_numbers,
                                          ref)
        else:
            node_energy = torch.addmv(self.atom_ref.to(A.dtype)[data.atomic_numbers],
                                      A.reshape(A.shape[0], -1), self.U.to(A.dtype).reshape(-1))
        return {"node_energy": node_energy, "energy": self.aggregate_energy(node_energy, data)}
