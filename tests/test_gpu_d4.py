"""GPU parity of the D4 path: the HIP coordination-number and two-body kernels and the
host-side D4 evaluation against the oracle (float64, brute-force pair images) and the
dftd4 golden values (tests/common/test_d4.py:110-126, 173-185, 202-226)."""
import math
import os
import sys

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"
HERE = os.path.dirname(os.path.abspath(__file__))
TABLES = os.path.join(HERE, "golden", "d4_tables_hcnoar.npz")
WATER = (np.array([[0.0, 0.0, 0.119262], [0.0, 0.763239, -0.477047],
                   [0.0, -0.763239, -0.477047]]), [8, 1, 1])
FAST = dict(cutoff_pair=9.0, cutoff_triple=7.0, cutoff_cn=8.0, cutoff_eeq_cn=8.0)


def _note(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def tables():
    return dict(np.load(TABLES, allow_pickle=False))


def _cluster(n, seed, box=6.0):
    rng = np.random.default_rng(seed)
    pos = rng.uniform(0, box - 1, (n, 3))
    return pos, ([1, 8, 6, 7] * (n // 4) + [1] * (n % 4))[:n]


def _eval(model, pos, z, cell=None, charges=None, grad=False):
    p = torch.tensor(pos, dtype=torch.float64, device=DEV, requires_grad=grad)
    c = None
    if cell is not None:
        c = torch.tensor(cell, dtype=torch.float64, device=DEV)[None].requires_grad_(grad)
    out = model.evaluate(torch.tensor(z, device=DEV), p, c, None if c is None else
                         torch.ones((1, 3), dtype=torch.bool), torch.tensor([len(z)]),
                         charges=charges)
    return out, p, c


def _oracle(tables, pos, z, cell, q, cutoffs, prm, width=0.0):
    """Oracle energy and its gradients in positions and cell for given charges."""
    import oracle.d4 as D
    cut_pair, cut_cn, cut_eeq = cutoffs
    dst, src, sh = D.pair_images(pos, cell, max(cutoffs))
    pt = torch.tensor(pos, dtype=torch.float64, requires_grad=True)
    ct = None if cell is None else torch.tensor(cell, dtype=torch.float64, requires_grad=True)
    v = D.edge_vectors_au(pt, ct, dst, src, sh)
    r = torch.linalg.norm(v, dim=-1)
    zt = torch.as_tensor(z)
    n = len(z)
    cn, cn_eeq, raw = D.coordination_numbers(zt, dst, src, r, tables, cut_cn / D.BOHR,
                                             cut_eeq / D.BOHR, n)
    alpha = D.dynamic_polarizabilities(zt, cn, q, tables)
    e2 = D.two_body(zt, dst, src, r, alpha, tables, prm, cut_pair / D.BOHR, width / D.BOHR, n)
    grads = torch.autograd.grad(e2.sum(), [pt] + ([ct] if ct is not None else []))
    return {"cn": cn.detach(), "raw": raw.detach(), "alpha": alpha.detach(), "e2": e2.detach(),
            "grad_pos": grads[0], "grad_cell": grads[1] if ct is not None else None}


def test_water_golden_values_on_the_gpu(tables):
    import xnn_amd.dispersion as XD
    _note("d4 water golden")
    model = XD.DFTD4(tables).to(DEV)
    out, _, _ = _eval(model, *WATER)
    np.testing.assert_allclose(out["coordination_numbers"].cpu().numpy(),
                               [1.60884227, 0.80442113, 0.80442113], atol=1e-7)
    np.testing.assert_allclose(out["charges"].cpu().numpy(),
                               [-0.58639069, 0.29319534, 0.29319534], atol=1e-7)
    np.testing.assert_allclose(out["polarizabilities"].cpu().numpy(),
                               [6.71824515, 1.35296894, 1.35296894], atol=1e-7)
    c6 = XD.c6_matrix(out["dynamic_polarizabilities"]).cpu().numpy()
    assert abs(c6[0, 0] - 24.68023585) < 1e-6 and abs(c6[0, 1] - 4.2011774) < 1e-6
    # dftd4's total, its 1.8e-11 Eh three-body part included, to the golden's 8 printed
    # digits (half a unit in the last: 5e-12)
    assert abs(float(out["energy"][0]) / XD.HARTREE - (-1.5761743e-04)) < 5e-12
    assert 1e-11 < float(out["energy_3body"][0]) / XD.HARTREE < 3e-11


def test_argon_dimer_asymptote(tables):
    import xnn_amd.dispersion as XD
    _note("d4 argon dimer")
    model = XD.DFTD4(tables).to(DEV)
    r4r2 = float(tables["r4r2"][18])
    for r in (12.0, 16.0):
        out, _, _ = _eval(model, np.array([[0.0, 0, 0], [r, 0, 0]]), [18, 18])
        c6 = float(XD.c6_matrix(out["dynamic_polarizabilities"])[0, 1])
        ra = r / XD.BOHR
        r0 = model.a1 * math.sqrt(3 * r4r2 ** 2) + model.a2
        expected = -(c6 / (ra ** 6 + r0 ** 6) + model.s8 * 3 * r4r2 ** 2 * c6 / (ra ** 8 + r0 ** 8))
        assert abs(float(out["energy"][0]) / XD.HARTREE - expected) < 1e-14


@pytest.mark.parametrize("case", ["molecule", "periodic", "triclinic_switched"])
def test_kernels_match_oracle(tables, case):
    """CN, per-atom two-body energies, and the position and cell gradients of the
    two-body energy, with the same charges on both sides, float64 (1e-11 relative)."""
    import oracle.d4 as D
    import xnn_amd.dispersion as XD
    _note(f"d4 kernels vs oracle: {case}")
    width = 0.0
    if case == "molecule":
        pos, z = _cluster(12, seed=5)
        cell = None
    elif case == "periodic":
        pos, z = _cluster(16, seed=6, box=7.0)
        cell = np.diag([7.0, 7.5, 8.0])
    else:
        pos, z = _cluster(10, seed=7)
        cell = np.array([[6.0, 0, 0], [0.8, 5.7, 0], [-0.4, 0.6, 6.2]])
        width = 2.0
    model = XD.DFTD4(tables, switch_width_pair=width, s9=0.0, **FAST).to(DEV)
    q = torch.tensor(np.random.default_rng(1).normal(0, 0.2, len(z)), dtype=torch.float64)
    out, p, c = _eval(model, pos, z, cell, charges=q.to(DEV), grad=True)
    gp, *gc = torch.autograd.grad(out["energy"].sum(), [p] + ([c] if c is not None else []))
    ref = _oracle(tables, pos, z, cell, q, (FAST["cutoff_pair"], FAST["cutoff_cn"],
                                            FAST["cutoff_eeq_cn"]), D.PBE0_D4, width)
    np.testing.assert_allclose(out["coordination_numbers"].detach().cpu(), ref["cn"], rtol=1e-12,
                               atol=1e-13)
    e2 = out["node_energy"].detach().cpu() / XD.HARTREE
    scale = float(ref["e2"].abs().max())
    np.testing.assert_allclose(e2, ref["e2"], atol=1e-11 * scale)
    g_scale = float(ref["grad_pos"].abs().max())
    np.testing.assert_allclose(gp.cpu() / XD.HARTREE, ref["grad_pos"], atol=1e-10 * g_scale)
    if cell is not None:
        np.testing.assert_allclose(gc[0][0].cpu() / XD.HARTREE, ref["grad_cell"],
                                   atol=1e-10 * float(ref["grad_cell"].abs().max()))


TILE_CASES = {
    # n atoms, seed, box (A), cell, switch width (A)
    "molecule_150": (150, 21, 13.0, None, 0.0),
    "periodic_200": (200, 22, 12.0, np.diag([12.0, 12.5, 13.0]), 0.0),
    "triclinic_170_switched": (170, 23, 11.0,
                               np.array([[11.0, 0, 0], [1.2, 10.6, 0], [-0.7, 0.9, 11.4]]), 2.0),
}


def _tile_case_check(tables, pos, z, cell, width, seed):
    import oracle.d4 as D
    import xnn_amd.dispersion as XD
    model = XD.DFTD4(tables, switch_width_pair=width, s9=0.0, **FAST).to(DEV)
    q = torch.tensor(np.random.default_rng(seed).normal(0, 0.2, len(z)), dtype=torch.float64)
    out, p, c = _eval(model, pos, z, cell, charges=q.to(DEV), grad=True)
    gp, *gc = torch.autograd.grad(out["energy"].sum(), [p] + ([c] if c is not None else []))
    ref = _oracle(tables, pos, z, cell, q, (FAST["cutoff_pair"], FAST["cutoff_cn"],
                                            FAST["cutoff_eeq_cn"]), D.PBE0_D4, width)
    np.testing.assert_allclose(out["coordination_numbers"].detach().cpu(), ref["cn"], rtol=1e-12,
                               atol=1e-13)
    e2 = out["node_energy"].detach().cpu() / XD.HARTREE
    np.testing.assert_allclose(e2, ref["e2"], atol=1e-11 * float(ref["e2"].abs().max()))
    np.testing.assert_allclose(gp.cpu() / XD.HARTREE, ref["grad_pos"],
                               atol=1e-10 * float(ref["grad_pos"].abs().max()))
    if cell is not None:
        np.testing.assert_allclose(gc[0][0].cpu() / XD.HARTREE, ref["grad_cell"],
                                   atol=1e-10 * float(ref["grad_cell"].abs().max()))
    return out, gp


@pytest.mark.parametrize("case", list(TILE_CASES))
def test_tiles_match_oracle(tables, case):
    """Structures of several 64-atom tiles, the last one partial: the kernels order the atoms
    spatially and evaluate every unordered pair of two tiles once (both atoms' shares), the
    pairs inside a tile directed. CN, per-atom two-body energies and the position and cell
    gradients against the oracle's directed brute force over all atoms (float64)."""
    n, seed, box, cell, width = TILE_CASES[case]
    _note(f"d4 tiles vs oracle: {case}")
    pos, z = _cluster(n, seed=seed, box=box)
    _tile_case_check(tables, pos, z, cell, width, seed)


def test_tiles_are_invariant_under_atom_permutation(tables):
    """Renumbering the atoms renumbers the per-atom results and gradients (the tile order is
    rebuilt from the positions; sums regroup, so to rounding)."""
    import xnn_amd.dispersion as XD
    _note("d4 tiles permutation invariance")
    pos, z = _cluster(200, seed=24, box=12.0)
    cell = np.diag([12.0, 12.5, 13.0])
    model = XD.DFTD4(tables, s9=0.0, **FAST).to(DEV)
    q = np.random.default_rng(3).normal(0, 0.2, len(z))
    perm = np.random.default_rng(4).permutation(len(z))
    res = []
    for order in (np.arange(len(z)), perm):
        out, p, c = _eval(model, pos[order], [z[k] for k in order], cell,
                          charges=torch.tensor(q[order], device=DEV), grad=True)
        gp, gc = torch.autograd.grad(out["energy"].sum(), [p, c])
        inv = np.argsort(order)
        res.append((out["node_energy"].detach().cpu().numpy()[inv], gp.cpu().numpy()[inv],
                    gc.cpu().numpy()))
    for a, b in zip(*res):
        np.testing.assert_allclose(a, b, rtol=0, atol=1e-12 * float(np.abs(a).max()))


def test_tiles_batch_of_mixed_sizes(tables):
    """One call over a 150-atom periodic cell (3 tiles), a 9-atom and a 70-atom molecule
    (1 and 2 tiles): per-atom CN, energies and gradients and each structure's cell gradient
    against the oracle run per structure (pairs never cross structures)."""
    import oracle.d4 as D
    import xnn_amd.dispersion as XD
    _note("d4 tiles batch of mixed sizes")
    model = XD.DFTD4(tables, s9=0.0, **FAST).to(DEV)
    pc, zc = _cluster(150, seed=25, box=11.0)
    cell = np.array([[11.0, 0, 0], [0.5, 10.8, 0], [0.0, -0.6, 11.3]])
    m1, z1 = _cluster(9, seed=26)
    m2, z2 = _cluster(70, seed=27, box=9.0)
    parts = [(pc, zc, cell), (m1, z1, None), (m2, z2, None)]
    q = [np.random.default_rng(5 + k).normal(0, 0.2, len(zz)) for k, (_, zz, _) in enumerate(parts)]
    pos = torch.tensor(np.concatenate([a for a, _, _ in parts]), device=DEV, requires_grad=True)
    cells = torch.tensor(np.stack([cell, np.zeros((3, 3)), np.zeros((3, 3))]), device=DEV,
                         requires_grad=True)
    pbc = torch.tensor([[True] * 3, [False] * 3, [False] * 3])
    z = zc + z1 + z2
    out = model.evaluate(torch.tensor(z, device=DEV), pos, cells, pbc,
                         torch.tensor([150, 9, 70]),
                         charges=torch.tensor(np.concatenate(q), device=DEV))
    gp, gc = torch.autograd.grad(out["energy"].sum(), [pos, cells])
    off = 0
    for k, (pp, zz, cc) in enumerate(parts):
        sl = slice(off, off + len(zz))
        off += len(zz)
        ref = _oracle(tables, pp, zz, cc, torch.tensor(q[k]), (FAST["cutoff_pair"],
                      FAST["cutoff_cn"], FAST["cutoff_eeq_cn"]), D.PBE0_D4)
        np.testing.assert_allclose(out["coordination_numbers"].detach().cpu()[sl], ref["cn"],
                                   rtol=1e-12, atol=1e-13)
        np.testing.assert_allclose(out["node_energy"].detach().cpu()[sl] / XD.HARTREE, ref["e2"],
                                   atol=1e-11 * float(ref["e2"].abs().max()))
        np.testing.assert_allclose(gp.cpu()[sl] / XD.HARTREE, ref["grad_pos"],
                                   atol=1e-10 * float(ref["grad_pos"].abs().max()))
        if cc is not None:
            np.testing.assert_allclose(gc[k].cpu() / XD.HARTREE, ref["grad_cell"],
                                       atol=1e-10 * float(ref["grad_cell"].abs().max()))


def test_tiles_structure_larger_than_max_atoms_gives_nan(tables):
    """A structure with more atoms than the max_atoms the caller promised has more tiles
    than result slots: the kernels leave it alone and its atoms come out NaN (no write
    outside the workspace)."""
    import xnn_amd.dispersion as XD
    _note("d4 tiles max_atoms guard")
    model = XD.DFTD4(tables, **FAST).to(DEV)
    pos, z = _cluster(150, seed=28, box=13.0)
    zc = torch.tensor(z, device=DEV)
    uniq, species = torch.unique(zc, return_inverse=True)
    n = len(z)
    cn, raw = XD.d4_coordination_op(
        torch.tensor(pos, device=DEV), None, species.to(torch.int32).contiguous(),
        torch.zeros(n, dtype=torch.int32, device=DEV),
        torch.tensor([0, n], dtype=torch.int64, device=DEV),
        torch.zeros((1, 3), dtype=torch.int32, device=DEV), None, model.rcov[uniq].contiguous(),
        model.en[uniq].contiguous(), [8.0 / XD.BOHR, 8.0 / XD.BOHR], 64)
    assert bool(torch.isnan(cn).all()) and bool(torch.isnan(raw).all())


def test_polarizabilities_kernel_matches_oracle(tables):
    """alpha(i w) and its chain rule to cn and q from the HIP kernel against the oracle's
    weights x charge scaling (float64 autograd): every tabulated element, CNs from 0 to
    past the weight underflow (the largest-reference fallback), charges on both sides of
    q + zeff = 0, and an atomic number outside the tables (NaN)."""
    import oracle.d4 as D
    import xnn_amd.dispersion as XD
    _note("d4 polarizabilities kernel vs oracle")
    model = XD.DFTD4(tables).to(DEV)
    rng = np.random.default_rng(21)
    elems = [int(e) for e in tables["elements"]]
    z = np.array([elems[i % len(elems)] for i in range(60)])
    cn = rng.uniform(0.0, 5.0, len(z))
    cn[:5] = 40.0                                    # exp(-wf d^2) underflows: fallback
    q = rng.normal(0.0, 0.4, len(z))
    zeff = tables["zeff"][z]
    q[5:9] = -zeff[5:9] - 0.5                        # q + zeff < 0: zeta = exp(ga)
    zt = torch.as_tensor(z)
    cn_t = torch.tensor(cn, requires_grad=True)
    q_t = torch.tensor(q, requires_grad=True)
    ref = D.dynamic_polarizabilities(zt, cn_t, q_t, tables)
    g_alpha = torch.tensor(rng.normal(size=ref.shape))
    ref_gcn, ref_gq = torch.autograd.grad((ref * g_alpha).sum(), [cn_t, q_t])
    cg = cn_t.detach().to(DEV).requires_grad_(True)
    qg = q_t.detach().to(DEV).requires_grad_(True)
    alpha = model.polarizabilities(zt.to(DEV), cg, qg)
    gcn, gq = torch.autograd.grad((alpha * g_alpha.to(DEV)).sum(), [cg, qg])
    assert _lib_calls("xnn_d4_polarizabilities") and _lib_calls("xnn_d4_polarizabilities_backward")
    np.testing.assert_allclose(alpha.detach().cpu(), ref.detach(), rtol=1e-13,
                               atol=1e-13 * float(ref.abs().max()))
    np.testing.assert_allclose(gcn.cpu(), ref_gcn, rtol=1e-12, atol=1e-12 * float(ref_gcn.abs().max()))
    np.testing.assert_allclose(gq.cpu(), ref_gq, rtol=1e-12, atol=1e-12 * float(ref_gq.abs().max()))
    assert float(gcn[:5].abs().max()) == 0.0          # the fallback weights are constant
    bad = model.polarizabilities(torch.tensor([1, 200], device=DEV),
                                 torch.tensor([1.0, 1.0], device=DEV, dtype=torch.float64),
                                 torch.zeros(2, device=DEV, dtype=torch.float64))
    assert torch.isfinite(bad[0]).all() and torch.isnan(bad[1]).all()


def _lib_calls(name):
    from xnn_amd import _lib
    return _lib.calls.get(name, 0) > 0


def test_full_molecule_with_eeq_matches_oracle_and_finite_differences(tables):
    """The whole D4 energy, EEQ charges and the ATM term (neutral-atom C6, 7 A triple
    cutoff) included, against the oracle's molecule (direct triple loop); forces against
    central differences of the GPU energy (test_d4.py:202-215: h = 1e-4 A, 1e-7 eV/A),
    which covers the ATM force's chain through the neutral polarizabilities to the CN."""
    import oracle.d4 as D
    import xnn_amd.dispersion as XD
    _note("d4 molecule full path")
    pos, z = _cluster(8, seed=2)
    model = XD.DFTD4(tables, **FAST).to(DEV)
    out, p, _ = _eval(model, pos, z, grad=True)
    (gp,) = torch.autograd.grad(out["energy"].sum(), [p])
    ref = D.d4_molecule(pos, z, tables, prm=D.PBE0_D4, with_atm=True,
                        cutoffs_au=(9.0 / D.BOHR, 7.0 / D.BOHR, 8.0 / D.BOHR, 8.0 / D.BOHR))
    np.testing.assert_allclose(out["charges"].detach().cpu(), ref["q"], atol=1e-12)
    assert float(ref["energy_3body"]) > 0
    assert abs(float(out["energy_3body"][0]) / XD.HARTREE - float(ref["energy_3body"])) \
        < 1e-12 * float(ref["energy_3body"])
    assert abs(float(out["energy"][0]) / XD.HARTREE - float(ref["energy"])) < 1e-14
    h = 1e-4
    for i, a in [(0, 0), (3, 2), (5, 1)]:
        pp, pm = pos.copy(), pos.copy()
        pp[i, a] += h
        pm[i, a] -= h
        ep = float(_eval(model, pp, z)[0]["energy"][0])
        em = float(_eval(model, pm, z)[0]["energy"][0])
        assert abs(float(gp[i, a]) - (ep - em) / (2 * h)) < 1e-7


def test_batch_equals_separate_structures(tables):
    """Two molecules and a periodic cell in one call give each structure's own energy
    and charges (pairs never cross structures)."""
    import xnn_amd.dispersion as XD
    _note("d4 batch")
    model = XD.DFTD4(tables, **FAST).to(DEV)
    m1, z1 = _cluster(9, seed=11)
    m2, z2 = _cluster(5, seed=12)
    pc, zc = _cluster(12, seed=13, box=7.0)
    cell = np.diag([7.0, 7.0, 7.0])
    pos = np.concatenate([m1, m2, pc])
    z = z1 + z2 + zc
    cells = torch.tensor(np.stack([np.zeros((3, 3)), np.zeros((3, 3)), cell]), device=DEV)
    pbc = torch.tensor([[False] * 3, [False] * 3, [True] * 3])
    out = model.evaluate(torch.tensor(z, device=DEV), torch.tensor(pos, device=DEV), cells, pbc,
                         torch.tensor([9, 5, 12]))
    e = [float(_eval(model, m1, z1)[0]["energy"][0]), float(_eval(model, m2, z2)[0]["energy"][0]),
         float(_eval(model, pc, zc, cell)[0]["energy"][0])]
    np.testing.assert_allclose(out["energy"].cpu().numpy(), e, rtol=1e-12)


def test_stress_matches_finite_strain(tables):
    """ForceStressOutput(D4Dispersion): stress against central differences of the energy
    under symmetric strain of positions and cell (test_d4.py:217-226: 1e-7)."""
    import xnn_amd as xa
    import xnn_amd.dispersion as XD
    _note("d4 stress vs finite strain")
    pos, z = _cluster(8, seed=4)
    cell = np.array([[6.0, 0, 0], [0.8, 5.7, 0], [-0.4, 0.6, 6.2]])
    model = xa.ForceStressOutput(XD.D4Dispersion(tables=tables, **FAST).to(DEV),
                                 compute_stress=True).eval()

    def graph(p, c):
        return xa.AtomicGraph(pos=torch.tensor(p, device=DEV), atomic_numbers=torch.tensor(z, device=DEV),
                              edge_index=torch.zeros((2, 0), dtype=torch.long, device=DEV),
                              cell_shifts=torch.zeros((0, 3), dtype=torch.long, device=DEV),
                              batch=torch.zeros(len(z), dtype=torch.long, device=DEV),
                              n_atoms=torch.tensor([len(z)], device=DEV),
                              cell=torch.tensor(c, device=DEV)[None],
                              pbc=torch.ones((1, 3), dtype=torch.bool, device=DEV))

    out = model(graph(pos, cell))
    vol = abs(np.linalg.det(cell))
    for (a, b) in [(0, 0), (1, 2), (2, 2)]:
        eps = np.zeros((3, 3))
        eps[a, b] = eps[b, a] = 1e-4
        ep = float(model.model(graph(pos @ (np.eye(3) + eps), cell @ (np.eye(3) + eps)))["energy"][0])
        em = float(model.model(graph(pos @ (np.eye(3) - eps), cell @ (np.eye(3) - eps)))["energy"][0])
        fd = (ep - em) / 2e-4 / vol / (1 if a == b else 2)
        assert abs(float(out["stress"][0, a, b]) - fd) < 1e-7
    # forces too, and the wrapper's bookkeeping
    assert out["forces"].shape == (len(z), 3)
    assert torch.equal(out["energy_disp"], out["energy"])


def test_periodic_three_body_matches_oracle(tables):
    """The module's ATM term in a cell narrower than a third of its 16 A triple cutoff (its
    radius graph through the replicated supercell): energy and position and cell gradients
    against the oracle's CN -> neutral alpha(i w) -> edge-list ATM over brute-force images
    (d4.py:1268-1298, dispersion.py:124-222), float64."""
    import oracle.d4 as D
    import xnn_amd.dispersion as XD
    _note("d4 periodic ATM vs oracle")
    pos, z = _cluster(4, seed=9, box=5.0)
    cell = np.diag([5.0, 5.2, 5.4])
    model = XD.DFTD4(tables, cutoff_pair=9.0, cutoff_cn=8.0, cutoff_eeq_cn=8.0,
                     cutoff_triple=16.0).to(DEV)
    q = torch.tensor(np.random.default_rng(2).normal(0, 0.2, len(z)), dtype=torch.float64)
    out, p, c = _eval(model, pos, z, cell, charges=q.to(DEV), grad=True)
    got = torch.autograd.grad(out["energy_3body"].sum(), [p, c])
    cut3 = model.cutoff_triple / D.BOHR
    dst, src, sh = D.pair_images(pos, cell, model.cutoff_triple)
    pt = torch.tensor(pos, dtype=torch.float64, requires_grad=True)
    ct = torch.tensor(cell, dtype=torch.float64, requires_grad=True)
    v = D.edge_vectors_au(pt, ct, dst, src, sh)
    r = torch.linalg.norm(v, dim=-1)
    zt = torch.as_tensor(z)
    n = len(z)
    cn, _, _ = D.coordination_numbers(zt, dst, src, r, tables, 8.0 / D.BOHR, 8.0 / D.BOHR, n)
    alpha0 = D.dynamic_polarizabilities(zt, cn, torch.zeros(n, dtype=torch.float64), tables)
    feat = alpha0 * torch.sqrt((3.0 / math.pi) * torch.as_tensor(D.cp_weights()))
    table, species = D.bj_radius_factors(zt, tables, model.a1, model.a2)
    tri = r <= cut3
    ei = torch.stack([torch.as_tensor(src), torch.as_tensor(dst)])[:, tri]
    e3 = D.atm_edges(ei, v[tri], feat, feat, species, table, 1.0, 16.0 / 3.0, cut3, 0.0, n)
    ref = torch.autograd.grad(e3.sum(), [pt, ct])
    assert float(e3.sum()) > 0
    assert abs(float(out["energy_3body"][0]) / XD.HARTREE - float(e3.sum())) \
        < 1e-11 * float(e3.sum())
    for a, b in zip(got, ref):
        a = a.reshape(b.shape).detach().cpu() / XD.HARTREE
        np.testing.assert_allclose(a, b, atol=1e-10 * float(b.abs().max()))


def _safe_coordinates(pos, cell, cutoffs, k, h, rng):
    """``k`` (atom, axis) pairs whose displacement by +-h moves no pair image across any of
    the hard ``cutoffs`` (Angstrom): central differences of an unswitched energy are then
    smooth (brute force over the images of that atom)."""
    import oracle.d4 as D
    out = []
    for i in rng.permutation(len(pos)):
        dst, src, sh = D.pair_images(pos, cell, max(cutoffs) + 1.0, receivers=[int(i)])
        d = pos[i] - pos[src] + sh @ cell
        r = np.sqrt((d * d).sum(-1))
        if all(np.abs(r - c).min() > 4 * h for c in cutoffs):
            out.append((int(i), len(out) % 3))
        if len(out) == k:
            return out
    raise RuntimeError("no safe coordinates")


def test_c5_organic_box_full_cutoffs(tables):
    """The C5 configuration at its stated size: 5,000 atoms in the 36.8 A cell, pair cutoff
    60 bohr (27 images per pair, ~6.7e7 pair-image terms), CN and EEQ-CN cutoffs 25 bohr,
    s9 = 0, charges given. Against the oracle on a 200-receiver sample (brute-force pair
    images of those receivers, d4.py:552-591, 984-1071): CN and alpha(i w) from the oracle's
    own CN to 1e-12, per-atom two-body energies to 1e-11 of scale (alpha of the sources from
    the GPU, pinned by the sample). Then the full-size gradients: the forces sum to zero,
    central differences of the GPU energy on three coordinates that no pair crosses a cutoff
    under (test_d4.py:202-215), and the strain derivative of a switched-cutoff copy against
    a finite symmetric strain (test_d4.py:217-226)."""
    import oracle.d4 as D
    import xnn_amd.dispersion as XD
    from xnn_amd import synthetic
    _note("d4 C5 organic box, 60/25/25 bohr")
    s = synthetic.organic_box(seed=0)
    pos, cell, z = np.asarray(s.pos), np.asarray(s.cell), [int(v) for v in s.numbers]
    n = len(z)
    cuts = dict(cutoff_pair=60.0 * D.BOHR, cutoff_cn=25.0 * D.BOHR, cutoff_eeq_cn=25.0 * D.BOHR)
    model = XD.DFTD4(tables, s9=0.0, **cuts).to(DEV)
    rng = np.random.default_rng(31)
    q = rng.normal(0.0, 0.15, n)
    q = torch.tensor(q - q.mean(), dtype=torch.float64)
    out, p, c = _eval(model, pos, z, cell, charges=q.to(DEV), grad=True)
    gp, gc = torch.autograd.grad(out["energy"].sum(), [p, c])
    gp, gc = gp.cpu(), gc[0].cpu()

    sample = np.sort(rng.choice(n, 200, replace=False))
    dst, src, sh = D.pair_images(pos, cell, cuts["cutoff_pair"], receivers=sample)
    v = D.edge_vectors_au(torch.tensor(pos), torch.tensor(cell), dst, src, sh)
    r = torch.linalg.norm(v, dim=-1)
    zt = torch.as_tensor(z)
    assert len(dst) > 200 * 10000                      # ~13,400 pair images per receiver
    cn, _, _ = D.coordination_numbers(zt, dst, src, r, tables, 25.0, 25.0, n)
    st = torch.as_tensor(sample)
    np.testing.assert_allclose(out["coordination_numbers"].detach().cpu()[st], cn[st],
                               rtol=1e-12, atol=1e-13)
    alpha_gpu = out["dynamic_polarizabilities"].detach().cpu()
    alpha_ref = D.dynamic_polarizabilities(zt[st], cn[st], q[st], tables)
    np.testing.assert_allclose(alpha_gpu[st], alpha_ref, rtol=1e-12,
                               atol=1e-13 * float(alpha_ref.abs().max()))
    e2 = D.two_body(zt, dst, src, r, alpha_gpu, tables, D.PBE0_D4, 60.0, 0.0, n)[st]
    got = out["node_energy"].detach().cpu()[st] / XD.HARTREE
    np.testing.assert_allclose(got, e2, atol=1e-11 * float(e2.abs().max()))

    # forces of a periodic system sum to zero
    assert float(gp.sum(0).abs().max()) <= 1e-10 * float(gp.abs().max())
    h = 1e-4
    for i, a in _safe_coordinates(pos, cell, [cuts["cutoff_pair"]], 3, h, rng):
        pp, pm = pos.copy(), pos.copy()
        pp[i, a] += h
        pm[i, a] -= h
        ep = float(_eval(model, pp, z, cell, charges=q.to(DEV))[0]["energy"][0])
        em = float(_eval(model, pm, z, cell, charges=q.to(DEV))[0]["energy"][0])
        assert abs(float(gp[i, a]) - (ep - em) / (2 * h)) < 1e-7, (i, a)

    # strain derivative (positions and cell deformed together) of a copy whose pair
    # cutoff is switched over 1 A, so that the energy is smooth in the strain
    sw = XD.DFTD4(tables, s9=0.0, switch_width_pair=1.0, **cuts).to(DEV)
    out, p, c = _eval(sw, pos, z, cell, charges=q.to(DEV), grad=True)
    gp, gc = torch.autograd.grad(out["energy"].sum(), [p, c])
    D_ab = (p.detach().t() @ gp + c.detach()[0].t() @ gc[0]).cpu()
    eps_h = 1e-5
    for a, b in [(0, 0), (1, 2)]:
        eps = np.zeros((3, 3))
        eps[a, b] = eps[b, a] = eps_h
        ep = float(_eval(sw, pos @ (np.eye(3) + eps), z, cell @ (np.eye(3) + eps),
                         charges=q.to(DEV))[0]["energy"][0])
        em = float(_eval(sw, pos @ (np.eye(3) - eps), z, cell @ (np.eye(3) - eps),
                         charges=q.to(DEV))[0]["energy"][0])
        fd = (ep - em) / (2 * eps_h)
        want = float(D_ab[a, b]) if a == b else float(D_ab[a, b] + D_ab[b, a])
        assert abs(fd - want) <= 1e-6 * max(1.0, abs(want)), (a, b, fd, want)


def test_tail_correction_restores_the_long_range_pair_sum(tables):
    """The homogeneous tail (d4.py:1073-1140, 1259-1267) stands in for the pairs beyond the
    cutoff: on the uniform 5,000-atom organic box the two-body energy at a 30-bohr cutoff
    plus its tail is much closer to that at 50 bohr plus its (smaller) tail than the bare
    energies are; the tail is negative and shrinks with the cutoff; forces and the strain
    derivative of the tail term agree with finite differences on a small cell."""
    import oracle.d4 as D
    import xnn_amd.dispersion as XD
    from xnn_amd import synthetic
    _note("d4 tail correction")
    s = synthetic.organic_box(seed=0)
    z = [int(v) for v in s.numbers]
    q = torch.zeros(len(z), dtype=torch.float64)
    out = {}
    for rc in (30.0, 50.0):
        m = XD.DFTD4(tables, s9=0.0, tail_correction=True, cutoff_pair=rc * D.BOHR,
                     cutoff_cn=25.0 * D.BOHR, cutoff_eeq_cn=25.0 * D.BOHR).to(DEV)
        o, _, _ = _eval(m, np.asarray(s.pos), z, np.asarray(s.cell), charges=q.to(DEV))
        out[rc] = (float(o["energy_2body"][0]), float(o["energy_tail"][0]))
    (e30, t30), (e50, t50) = out[30.0], out[50.0]
    assert t30 < t50 < 0
    assert abs((e30 + t30) - (e50 + t50)) < 0.05 * abs(e30 - e50), (e30, t30, e50, t50)
    # derivatives of the tail on a small cell (sharp cutoff shorter than the cell's images)
    pos, zz = _cluster(8, seed=4)
    cell = np.array([[6.0, 0, 0], [0.8, 5.7, 0], [-0.4, 0.6, 6.2]])
    m = XD.DFTD4(tables, s9=0.0, tail_correction=True, switch_width_pair=2.0, cutoff_pair=9.0,
                 cutoff_cn=8.0, cutoff_eeq_cn=8.0).to(DEV)
    qq = torch.tensor(np.random.default_rng(3).normal(0, 0.1, len(zz)), dtype=torch.float64)
    o, p, c = _eval(m, pos, zz, cell, charges=qq.to(DEV), grad=True)
    gp, gc = torch.autograd.grad(o["energy"].sum(), [p, c])
    h = 1e-4
    for i, a in [(0, 0), (5, 2)]:
        pp, pm = pos.copy(), pos.copy()
        pp[i, a] += h
        pm[i, a] -= h
        ep = float(_eval(m, pp, zz, cell, charges=qq.to(DEV))[0]["energy"][0])
        em = float(_eval(m, pm, zz, cell, charges=qq.to(DEV))[0]["energy"][0])
        assert abs(float(gp[i, a]) - (ep - em) / (2 * h)) < 1e-7
    D_ab = p.detach().t() @ gp + c.detach()[0].t() @ gc[0]
    for a, b in [(0, 0), (1, 2)]:
        eps = np.zeros((3, 3))
        eps[a, b] = eps[b, a] = h
        ep = float(_eval(m, pos @ (np.eye(3) + eps), zz, cell @ (np.eye(3) + eps),
                         charges=qq.to(DEV))[0]["energy"][0])
        em = float(_eval(m, pos @ (np.eye(3) - eps), zz, cell @ (np.eye(3) - eps),
                         charges=qq.to(DEV))[0]["energy"][0])
        want = float(D_ab[a, b]) if a == b else float(D_ab[a, b] + D_ab[b, a])
        assert abs((ep - em) / (2 * h) - want) < 1e-6, (a, b)


def test_fused_pair_matches_the_two_launch_path(tables):
    """evaluate(fused_pair=True): the two-body energies from one pair-backward launch at unit
    seeds (e_i = 1/2 alpha_i . dE/dalpha_i, the energy being bilinear in the polarizabilities)
    and their gradients scaled by the structure seeds, against the energy launch plus the
    autograd backward: two periodic structures of different size, seeds 2 and -3 on their
    energies, cutoffs with a switching window and the three-body term off."""
    import xnn_amd.dispersion as XD
    _note("d4 fused pair vs two launches")
    model = XD.DFTD4(tables, s9=0.0, cutoff_pair=12.0, cutoff_cn=9.0, cutoff_eeq_cn=9.0,
                     switch_width_pair=1.0).to(DEV)
    rng = np.random.default_rng(11)
    zs, ps, cs, ns = [], [], [], []
    for n, L in ((13, 7.5), (20, 8.5)):
        zs.append(rng.choice([1, 6, 7, 8], size=n))
        ps.append(rng.uniform(0.0, L, size=(n, 3)))
        cs.append(np.diag([L, L + 0.4, L - 0.3]) + rng.normal(scale=0.2, size=(3, 3)))
        ns.append(n)
    z = torch.tensor(np.concatenate(zs), device=DEV)
    pos0 = torch.tensor(np.concatenate(ps), dtype=torch.float64, device=DEV)
    cell0 = torch.tensor(np.stack(cs), dtype=torch.float64, device=DEV)
    pbc = torch.ones((2, 3), dtype=torch.bool)
    n_atoms = torch.tensor(ns)
    seed = torch.tensor([2.0, -3.0], dtype=torch.float64, device=DEV)
    res = []
    for fused in (False, True):
        pos = pos0.clone().requires_grad_(True)
        cell = cell0.clone().requires_grad_(True)
        out = model.evaluate(z, pos, cell, pbc, n_atoms, fused_pair=fused)
        gp, gc = torch.autograd.grad((out["energy"] * seed).sum(), [pos, cell])
        res.append((out["energy"].detach(), out["node_energy"].detach(), gp, gc,
                    out["node_energy"].requires_grad))
    (e0, n0, gp0, gc0, _), (e1, n1, gp1, gc1, req1) = res
    assert not req1
    torch.testing.assert_close(e1, e0, rtol=1e-12, atol=1e-14)
    torch.testing.assert_close(n1, n0, rtol=1e-10, atol=1e-14)
    torch.testing.assert_close(gp1, gp0, rtol=1e-11, atol=1e-13)
    torch.testing.assert_close(gc1, gc0, rtol=1e-11, atol=1e-13)
