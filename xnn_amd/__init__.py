"""xnn_amd: the per-edge hot path of molssi-ai/xnn, MI355X-native.

Positions/cell/pbc -> HIP cell-list radius graph -> fused edge featurizer
(Bessel/Gaussian x cosine/polynomial envelope, real SH l <= 3) -> deterministic
CSR edge -> atom sums -> forces and virial by a CSR reduction, behind the
reference's module and function interfaces; the radial network's hidden layers on one
matrix-core kernel and the equivariant convolution's message step on one kernel each way.
"""
from . import _lib
from .data import (AtomicGraph, NeighborListPlan, batched_neighbor_list, build_neighbor_list, collate,
                   half_list, structure_to_graph, unique_pairs)
from .fast import (AutoPolicy, FastPathModule, FastPathPrecisionWarning, MI355X_POLICY, select,
                   set_use_fast)
from .featurizers import (BesselRBF, CosineCutoff, GaussianRBF, PolynomialCutoff,
                          SphericalHarmonicEdgeEmbedding, spherical_harmonics)
from .functional import cell_volume, gather_rows, scatter_sum, structure_sum
from .models import (InteratomicPotential, ModelConfig, ShEdgePotential, build_model,
                     get_model_class, register_model)
from .outputs import ForceStressOutput
from .radial import FullyConnectedNet, RadialNet, set_recompute_radial
from .conv import ConvTensorProduct
from .irreps import Irrep, Irreps, tp_out_irreps_with_instructions, wigner_3j

__all__ = [
    "AtomicGraph", "NeighborListPlan", "build_neighbor_list", "batched_neighbor_list", "structure_to_graph", "collate",
    "half_list", "unique_pairs",
    "AutoPolicy", "FastPathModule", "FastPathPrecisionWarning", "MI355X_POLICY", "select",
    "set_use_fast",
    "BesselRBF", "GaussianRBF", "CosineCutoff", "PolynomialCutoff",
    "SphericalHarmonicEdgeEmbedding", "spherical_harmonics",
    "scatter_sum", "gather_rows", "structure_sum", "cell_volume",
    "InteratomicPotential", "ModelConfig", "ShEdgePotential", "build_model", "get_model_class",
    "register_model", "ForceStressOutput",
    "FullyConnectedNet", "RadialNet", "set_recompute_radial", "ConvTensorProduct",
    "Irrep", "Irreps", "tp_out_irreps_with_instructions", "wigner_3j",
]
