"""A three-layer NequIP-like stack on the C1 configuration (32 synthetic 21-atom molecules,
species {1, 6, 8}, l_max = 2, 32 channels, cutoff 5 A, float32): the HIP featurizer,
radial network and uvu convolution under the PyTorch linears and gates, with forces
through ForceStressOutput, against the float64 composition of the oracles
(``tests/nequip_stack.py``); and the same model behind the pair-style wrapper."""
import sys

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _note(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _c1_graph():
    import xnn_amd as xa
    from xnn_amd import synthetic
    mols = synthetic.random_molecules(32, seed=2)
    g = xa.collate([xa.structure_to_graph(m.as_dict(), 5.0, device=DEV) for m in mols])
    g.pos = g.pos.float()
    return g


def test_nequip_stack_on_the_c1_molecules_matches_the_oracle_composition():
    import xnn_amd as xa
    from xnn_amd import _lib
    from nequip_stack import NequIPStack, reference_energy_forces
    _note("NequIP-like stack, C1: 32 molecules x 21 atoms, 3 layers, 32 channels, l_max 2")
    g = _c1_graph()
    assert g.num_nodes == 672
    model = NequIPStack(seed=0).to(DEV)
    before = {k: _lib.calls.get(k, 0) for k in ("xnn_uvu_conv", "xnn_uvu_conv_backward",
                                                 "xnn_radial_hidden", "xnn_edge_featurize",
                                                 "xnn_radial_hidden_backward")}
    out = xa.ForceStressOutput(model).eval()(g)
    for k, v in before.items():
        assert _lib.calls.get(k, 0) > v, f"{k} did not run"
    e_ref, node_ref, f_ref = reference_energy_forces(model, g)
    from xnn_amd.functional import structure_sum
    scale = structure_sum(node_ref.abs(), g.batch.cpu(), g.num_graphs)
    err = (out["energy"].detach().cpu() - e_ref).abs()
    print(f"energy err max {float(err.max()):.3e}, err / sum|E_i| max "
          f"{float((err / scale).max()):.3e}; E[:3]={e_ref[:3].tolist()}", flush=True)
    assert bool((err <= 1e-5 * scale).all())
    f_scale = float(f_ref.abs().max())
    assert f_scale > 0.1          # forces of order one: the bar below is not vacuous
    f_err = float((out["forces"].detach().cpu().double() - f_ref).abs().max())
    print(f"forces err max {f_err:.3e} of scale {f_scale:.3e}", flush=True)
    assert f_err <= 1e-5 * f_scale
    # the net force on every molecule vanishes (translation invariance)
    net = torch.zeros(g.num_graphs, 3, dtype=torch.float64).index_add_(
        0, g.batch.cpu(), out["forces"].detach().cpu().double())
    assert float(net.abs().max()) <= 1e-5 * f_scale
    # bitwise reproducible
    out2 = xa.ForceStressOutput(model).eval()(_c1_graph())
    assert torch.equal(out["forces"], out2["forces"])
    assert torch.equal(out["energy"], out2["energy"])


def test_nequip_stack_behind_the_pair_style_wrapper():
    """A registered model other than the edge potential through deploy.LAMMPSWrapper (the
    ForceStressOutput path), one molecule: energies, forces and the virial sym(sum r (x) F)."""
    import xnn_amd as xa
    from xnn_amd import synthetic
    from xnn_amd.deploy import LAMMPSWrapper
    from nequip_stack import NequIPStack
    _note("NequIP-like stack behind LAMMPSWrapper")
    model = NequIPStack(seed=1).to(DEV)
    m = synthetic.random_molecules(1, seed=9)[0]
    g = xa.structure_to_graph(m.as_dict(), 5.0, device=DEV)
    g.pos = g.pos.float()
    out = xa.ForceStressOutput(model).eval()(g)
    pair = LAMMPSWrapper(model)(g.pos, g.edge_index, g.cell_shifts, g.atomic_numbers,
                                torch.zeros(3, 3, device=DEV))
    assert abs(float(pair["total_energy"][0]) - float(out["energy"][0])) <= 1e-6 * max(
        1.0, abs(float(out["energy"][0])))
    torch.testing.assert_close(pair["forces"].double(), out["forces"].double(), atol=1e-5, rtol=0)
    rf = g.pos.double().T @ out["forces"].double()
    torch.testing.assert_close(pair["virial"], 0.5 * (rf + rf.T), atol=1e-5, rtol=0)
