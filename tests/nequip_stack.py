"""A NequIP-like three-layer stack for the GPU tests (the layer of gnn/models/nequip.py:296-540
without the self-connection): per layer an equivariant linear, the uvu convolution of the
sender features with the edge harmonics under per-edge weights from the radial network,
an equivariant linear to the gate's inputs, and the gate; a scalar readout.

The convolution, the radial network and the edge featurizer are the package's (HIP on
the GPU); the linears, the gate and the readout are plain PyTorch, as a model's own layers
are. :func:`reference_energy_forces` evaluates the same parameters in float64 on the CPU
through the oracles (``oracle/reference.py`` edge vectors, harmonics and radial basis,
``oracle/radial.py`` network, ``oracle/tp.py`` convolution), forces by autograd.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F
from torch import nn

import oracle.radial as OR
import oracle.reference as R
import oracle.tp as OT
from xnn_amd import irreps as I
from xnn_amd.conv import ConvTensorProduct
from xnn_amd.fast import MI355X_POLICY, fast_modules, select
from xnn_amd.featurizers import SphericalHarmonicEdgeEmbedding
from xnn_amd.models import InteratomicPotential, register_model
from xnn_amd.radial import RadialNet


class EquivariantLinear(nn.Module):
    """Channel mixing between irreps: output block (mul_out, ir) = sum over the input
    blocks of the same irrep of x_block W / sqrt(fan_in), fan_in the input multiplicity of
    that irrep (e3nn's ``Linear`` with its path normalization, no biases)."""

    def __init__(self, irreps_in, irreps_out, gen: torch.Generator):
        super().__init__()
        self.irreps_in, self.irreps_out = I.Irreps(irreps_in), I.Irreps(irreps_out)
        self.paths = []
        self.weights = nn.ParameterList()
        for io, mo in enumerate(self.irreps_out):
            ins = [ii for ii, mi in enumerate(self.irreps_in) if mi.ir == mo.ir]
            fan = sum(self.irreps_in[ii].mul for ii in ins)
            for ii in ins:
                self.paths.append((ii, io, len(self.weights), fan))
                self.weights.append(nn.Parameter(
                    torch.randn(self.irreps_in[ii].mul, mo.mul, generator=gen)))

    def forward(self, x):
        n = x.shape[0]
        s_in, s_out = self.irreps_in.slices(), self.irreps_out.slices()
        blocks = [x.new_zeros(n, mo.mul, mo.ir.dim) for mo in self.irreps_out]
        for ii, io, wi, fan in self.paths:
            mi = self.irreps_in[ii]
            xb = x[:, s_in[ii]].reshape(n, mi.mul, mi.ir.dim)
            blocks[io] = blocks[io] + torch.einsum("nui,uw->nwi", xb, self.weights[wi]) / math.sqrt(fan)
        return torch.cat([b.reshape(n, -1) for b in blocks], dim=1)


def gate(x, C: int):
    """``32x0e (scalars) + 64x0e (gates) + 32x1o + 32x2e`` -> ``32x0e + 32x1o + 32x2e``:
    SiLU on the scalars, each gated channel times SiLU of its gate."""
    n = x.shape[0]
    scalars, gates = x[:, :C], F.silu(x[:, C:3 * C])
    v1 = x[:, 3 * C:6 * C].reshape(n, C, 3) * gates[:, :C, None]
    v2 = x[:, 6 * C:11 * C].reshape(n, C, 5) * gates[:, C:, None]
    return torch.cat([F.silu(scalars), v1.reshape(n, -1), v2.reshape(n, -1)], dim=1)


class StackLayer(nn.Module):
    def __init__(self, irreps_in, sh, C: int, n_rbf: int, gen):
        super().__init__()
        hidden_in = I.Irreps(f"{C}x0e+{2 * C}x0e+{C}x1o+{C}x2e")
        self.irreps_in = I.Irreps(irreps_in)
        self.lin1 = EquivariantLinear(self.irreps_in, self.irreps_in, gen)
        self.mid, ins = I.tp_out_irreps_with_instructions(self.irreps_in, sh, hidden_in,
                                                          sort_instructions=False)
        self.paths = [(a, b, c) for a, b, c, _, _ in ins]
        self.tp = ConvTensorProduct(self.irreps_in, sh, self.mid, ins, shared_weights=False,
                                    internal_weights=False)
        # the output variance keeps the messages of order one through three layers
        self.fc = RadialNet([n_rbf, 64, 64, self.tp.weight_numel], F.silu, variance_out=16.0)
        with torch.no_grad():
            for layer in self.fc:
                layer.weight.copy_(torch.randn(layer.weight.shape, generator=gen))
        self.lin2 = EquivariantLinear(self.mid, hidden_in, gen)


@register_model("nequip_stack_test")
class NequIPStack(InteratomicPotential):
    """The stack as a registered model: ``AtomicGraph -> {node_energy, energy}``."""

    edge_virial = True
    energy_is_node_sum = True

    def __init__(self, species=(1, 6, 8), channels: int = 32, l_max: int = 2, n_layers: int = 3,
                 cutoff: float = 5.0, n_rbf: int = 8, avg_neighbors: float = 12.0, seed: int = 0):
        super().__init__()
        gen = torch.Generator().manual_seed(seed)
        self.C, self.l_max, self.cutoff = channels, l_max, float(cutoff)
        self.divisor = math.sqrt(avg_neighbors)
        self.register_buffer("species", torch.tensor(list(species)))
        self.edge_feat = SphericalHarmonicEdgeEmbedding(l_max=l_max, n_rbf=n_rbf, cutoff=cutoff)
        self.sh = I.spherical_harmonics_irreps(l_max)
        self.embedding = nn.Parameter(torch.randn(len(species), channels, generator=gen))
        hidden = I.Irreps(f"{channels}x0e+{channels}x1o+{channels}x2e")
        self.layers = nn.ModuleList(
            [StackLayer(I.Irreps(f"{channels}x0e") if t == 0 else hidden, self.sh, channels,
                        n_rbf, gen) for t in range(n_layers)])
        self.readout = nn.Parameter(torch.randn(channels, generator=gen))
        self.atom_ref = nn.Parameter(0.1 * torch.randn(int(max(species)) + 1, generator=gen))

    def one_hot(self, z):
        return (z[:, None] == self.species[None, :].to(z.device)).to(self.embedding.dtype)

    def forward(self, data):
        select(fast_modules(self), "auto", MI355X_POLICY, data.pos.device, data.model_dtype,
               data.num_edges)
        vec = data.edge_vectors()
        # NequIP's harmonics are of r_j - r_i, the edge vector reversed (nequip.py:721-722)
        _, sh, radial = self.edge_feat.embed(vec, sh_sign=-1)
        ei, n = data.edge_index, data.num_nodes
        x = self.one_hot(data.atomic_numbers) @ self.embedding
        for t, layer in enumerate(self.layers):
            w = layer.fc(radial)
            m = layer.tp.conv(layer.lin1(x), sh, w, ei, n, self.divisor)
            # the residual update where the irreps are kept (nequip.py "resnet")
            x = gate(layer.lin2(m), self.C) + (x if t > 0 else 0.0)
        node_energy = x[:, :self.C] @ self.readout + self.atom_ref[data.atomic_numbers]
        return {"node_energy": node_energy, "energy": self.aggregate_energy(node_energy, data)}


def reference_energy_forces(model: NequIPStack, data):
    """Per-structure energies and forces of ``model`` in float64 on the CPU through the
    oracles, with the model's parameters (the radial network's normalization constant is
    the module's own estimate)."""
    import copy
    m = copy.deepcopy(model).cpu().double()
    pos = data.pos.detach().cpu().double().requires_grad_(True)
    ei, batch = data.edge_index.cpu(), data.batch.cpu()
    vec = R.edge_vectors(pos, ei, data.cell_shifts.cpu(), None, batch, data.pos.dtype)
    length = torch.linalg.norm(vec, dim=-1)
    rbf = m.edge_feat.rbf
    sh = R.e3nn_sh(m.l_max, -vec)
    radial = R.radial_features(length, rbf.freqs.numel(), m.cutoff, "bessel", "polynomial")
    x = m.one_hot(data.atomic_numbers.cpu()) @ m.embedding
    for t, layer in enumerate(m.layers):
        cst = layer.fc.layer0.act.cst
        w = OR.fully_connected_torch(radial, [l.weight for l in layer.fc], cst,
                                     variance_out=layer.fc[-1].var_out)
        mm = OT.uvu_conv_torch(layer.lin1(x), sh, w, ei[0], ei[1], x.shape[0],
                               repr(layer.irreps_in), repr(m.sh), repr(layer.mid), layer.paths,
                               m.divisor)
        x = gate(layer.lin2(mm), m.C) + (x if t > 0 else 0.0)
    z = data.atomic_numbers.cpu()
    node = x[:, :m.C] @ m.readout + m.atom_ref[z]
    energy = R.structure_sum(node, batch, data.num_graphs)
    (g,) = torch.autograd.grad(energy.sum(), (pos,))
    return energy.detach(), node.detach(), -g
