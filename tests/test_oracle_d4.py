"""The D4 oracle pinned against the reference's golden values and closed forms
(tests/common/test_d4.py:110-126, 173-199). CPU only."""
import math
import os

import numpy as np
import pytest
import torch

import oracle.d4 as D

HERE = os.path.dirname(os.path.abspath(__file__))
TABLES = os.path.join(HERE, "golden", "d4_tables_hcnoar.npz")
WATER = (np.array([[0.0, 0.0, 0.119262], [0.0, 0.763239, -0.477047],
                   [0.0, -0.763239, -0.477047]]), [8, 1, 1])


@pytest.fixture(scope="module")
def tables():
    return dict(np.load(TABLES, allow_pickle=False))


def test_water_matches_dftd4_golden_values(tables):
    """dftd4 4.2.0, PBE0-D4 (test_d4.py:110-126): energy 1e-10 Eh, CN / charges /
    static polarizabilities 1e-7, C6 1e-6."""
    out = D.d4_molecule(WATER[0], WATER[1], tables)
    assert abs(float(out["energy"]) - (-1.5761743e-04)) < 1e-10
    np.testing.assert_allclose(out["cn"].numpy(), [1.60884227, 0.80442113, 0.80442113], atol=1e-7)
    np.testing.assert_allclose(out["q"].numpy(), [-0.58639069, 0.29319534, 0.29319534], atol=1e-7)
    np.testing.assert_allclose(out["alpha"][:, 0].numpy(), [6.71824515, 1.35296894, 1.35296894],
                               atol=1e-7)
    c6 = D.c6_pairs(out["alpha"][:, None, :], out["alpha"][None, :, :])
    assert abs(float(c6[0, 0]) - 24.68023585) < 1e-6 and abs(float(c6[0, 1]) - 4.2011774) < 1e-6
    # the three-body part is tiny for water: the two-body term alone meets the bar too
    assert abs(float(out["energy_2body"]) - (-1.5761743e-04)) < 1e-10
    assert float(out["energy_2body"]) < 0 < float(out["energy_3body"])


def test_dimer_two_body_tends_to_damped_c6_over_r6(tables):
    """Ar2 far apart: E = -(C6 / (r^6 + R0^6) + s8 3 Q^2 C6 / (r^8 + R0^8)) (test_d4.py:173-185)."""
    prm = dict(D.PBE0_D4, s9=0.0)
    r4r2 = tables["r4r2"][18]
    for r in (12.0, 16.0):
        pos = np.array([[0.0, 0, 0], [r, 0, 0]])
        out = D.d4_molecule(pos, [18, 18], tables, prm=prm, with_atm=False)
        c6 = float(D.c6_pairs(out["alpha"][0], out["alpha"][1]))
        ra = r / D.BOHR
        r0 = prm["a1"] * math.sqrt(3 * r4r2 ** 2) + prm["a2"]
        expected = -(c6 / (ra ** 6 + r0 ** 6) + prm["s8"] * 3 * r4r2 ** 2 * c6 / (ra ** 8 + r0 ** 8))
        assert abs(float(out["energy"]) - expected) < 1e-14


def test_switching_function_closed_form():
    """Quintic window: 1 below cutoff - width, 0 above, x^3 (10 - 15 x + 6 x^2) inside,
    zero slope at both ends; width <= 0 is the sharp cutoff (dispersion.py:42-67)."""
    r = torch.linspace(0.0, 12.0, 241, dtype=torch.float64, requires_grad=True)
    sw = D.switching(r, 10.0, 3.0)
    assert bool((sw[r <= 7.0] == 1.0).all()) and bool((sw[r >= 10.0] == 0.0).all())
    x = (10.0 - r.detach()) / 3.0
    mid = (x > 0) & (x < 1)
    np.testing.assert_allclose(sw.detach()[mid], (x ** 3 * (10 - 15 * x + 6 * x ** 2))[mid], rtol=1e-14)
    (g,) = torch.autograd.grad(sw.sum(), r)
    assert abs(float(g[r.detach() == 7.0])) < 1e-12 and abs(float(g[r.detach() == 10.0])) < 1e-12
    assert bool((D.switching(r, 10.0, 0.0) == 1.0).all())


def test_exact_invariances(tables):
    """Rigid rotations and translations leave CN, charges and energy unchanged."""
    rng = np.random.default_rng(3)
    pos = rng.uniform(0, 5, (8, 3))
    z = [1, 8, 6, 7, 1, 8, 6, 1]
    a = D.d4_molecule(pos, z, tables, with_atm=False)
    R, _ = np.linalg.qr(rng.normal(size=(3, 3)))
    b = D.d4_molecule(pos @ R.T + 1.7, z, tables, with_atm=False)
    for k in ("cn", "q", "e2"):
        np.testing.assert_allclose(a[k].numpy(), b[k].numpy(), atol=1e-12)


def test_tables_fixture_has_the_elements(tables):
    assert list(tables["elements"]) == [1, 6, 7, 8, 18]
    assert tables["refalpha"].shape == (23, 7, 119)
    assert int(tables["nref"][6]) == 7 and int(tables["nref"][1]) == 2
    assert 1.9 < float(tables["r4r2"][1]) < 2.1 and 3.0 < float(tables["r4r2"][6]) < 3.2
    assert float(np.abs(tables["refalpha"][:, :, 2]).sum()) == 0.0     # outside the subset


def test_public_switch_and_reference_weights_equal_the_oracle(tables):
    """xnn_amd.dispersion.switching_function and gaussian_reference_weights (the reference's
    public formulas, dispersion.py:42-121) against the oracle's switch and D4 weights."""
    import xnn_amd.dispersion as XD
    r = torch.linspace(0.0, 12.0, 97, dtype=torch.float64)
    for width in (0.0, 2.5, 20.0):
        np.testing.assert_allclose(XD.switching_function(r, 10.0, width),
                                   D.switching(r, 10.0, width), rtol=1e-15, atol=1e-16)
    z = torch.tensor([1, 6, 7, 8, 18, 6, 1])
    cn = torch.tensor([0.9, 3.1, 2.2, 1.8, 0.0, 45.0, 1.1], dtype=torch.float64)
    refcn = torch.as_tensor(tables["refcn"])[:, z].t()
    ngw = torch.as_tensor(tables["ngw"])[:, z].t()
    valid = torch.arange(refcn.shape[1])[None, :] < torch.as_tensor(tables["nref"])[z][:, None]
    got = XD.gaussian_reference_weights(cn, refcn, valid, D.WF, ngw, 1.4916681462400413e-154)
    np.testing.assert_allclose(got, D.gaussian_weights(z, cn, tables), rtol=1e-15, atol=1e-300)


def _atm_inputs(pos_aa, cell_aa, z, tables, cutoff_au, feats=None):
    dst, src, sh = D.pair_images(pos_aa, cell_aa, cutoff_au * D.BOHR)
    pos = torch.as_tensor(pos_aa)
    cell = None if cell_aa is None else torch.as_tensor(cell_aa)
    vec = D.edge_vectors_au(pos, cell, dst, src, sh)
    keep = torch.linalg.norm(vec, dim=-1) <= cutoff_au
    ei = torch.stack([torch.as_tensor(src), torch.as_tensor(dst)])[:, keep]
    table, species = D.bj_radius_factors(z, tables, D.PBE0_D4["a1"], D.PBE0_D4["a2"])
    if feats is None:
        feats = torch.rand(len(z), 23, dtype=torch.float64, generator=torch.Generator().manual_seed(1))
    return ei, vec[keep], feats, species, table


def test_atm_edges_total_equals_the_direct_triple_loop(tables):
    """The edge-list ATM (every corner visited, a third each) sums to the pinned direct
    triple loop on a molecule, with a cutoff that drops some triangles."""
    rng = np.random.default_rng(4)
    pos = rng.uniform(0.0, 5.0, size=(9, 3))
    z = torch.tensor([6, 6, 8, 1, 1, 7, 1, 8, 1])
    alpha = torch.rand(9, 23, dtype=torch.float64, generator=torch.Generator().manual_seed(2)) + 0.5
    feats = alpha * torch.sqrt((3.0 / math.pi) * torch.as_tensor(D.cp_weights()))
    for cut in (40.0, 7.0):
        ei, vec, f, sp, tab = _atm_inputs(pos, None, z, tables, cut, feats)
        e = D.atm_edges(ei, vec, f, f, sp, tab, 1.0, 16.0 / 3.0, cut, 0.0, 9)
        ref = D.atm_molecule(z, torch.as_tensor(pos) / D.BOHR, alpha, tables, D.PBE0_D4, cut)
        assert abs(float(e.sum()) - float(ref)) <= 1e-13 * abs(float(ref)) and float(ref) > 0


def test_atm_edges_per_atom_is_invariant_under_replication(tables):
    """Per-atom ATM energies of a periodic cell narrower than twice the cutoff (so with
    self-image triangles) equal those of each copy in a 2x1x1 and a 1x2x2 supercell, and a
    cell padded with vacuum reproduces the molecule."""
    rng = np.random.default_rng(7)
    cell = np.array([[5.5, 0.0, 0.0], [0.8, 5.2, 0.0], [0.3, -0.4, 5.9]])
    frac = rng.uniform(0.0, 1.0, size=(4, 3))
    pos = frac @ cell
    z = torch.tensor([6, 1, 8, 1])
    cut = 6.0 / D.BOHR
    feats = torch.rand(4, 23, dtype=torch.float64, generator=torch.Generator().manual_seed(3)) + 0.1
    ei, vec, f, sp, tab = _atm_inputs(pos, cell, z, tables, cut, feats)
    assert bool((ei[0] == ei[1]).any())               # an atom sees its own image
    e1 = D.atm_edges(ei, vec, f, f, sp, tab, 1.0, 16.0 / 3.0, cut, 1.5, 4)
    for reps in ((2, 1, 1), (1, 2, 2)):
        shifts = np.array([[i, j, k] for i in range(reps[0]) for j in range(reps[1])
                           for k in range(reps[2])])
        pos_s = np.concatenate([pos + s @ cell for s in shifts])
        cell_s = cell * np.array(reps)[:, None]
        n = len(shifts)
        ei, vec, f, sp, tab = _atm_inputs(pos_s, cell_s, z.repeat(n), tables, cut, feats.repeat(n, 1))
        es = D.atm_edges(ei, vec, f, f, sp, tab, 1.0, 16.0 / 3.0, cut, 1.5, 4 * n)
        np.testing.assert_allclose(es.reshape(n, 4), e1.expand(n, 4), rtol=1e-12)
    mol = pos - pos.mean(0)
    ei, vec, f, sp, tab = _atm_inputs(mol, None, z, tables, cut, feats)
    e_mol = D.atm_edges(ei, vec, f, f, sp, tab, 1.0, 16.0 / 3.0, cut, 1.5, 4)
    ei, vec, f, sp, tab = _atm_inputs(mol, np.eye(3) * 30.0, z, tables, cut, feats)
    e_pad = D.atm_edges(ei, vec, f, f, sp, tab, 1.0, 16.0 / 3.0, cut, 1.5, 4)
    np.testing.assert_allclose(e_pad, e_mol, rtol=1e-13)


def _triangle_closed_form(c6, r0_pair, sides, s9=1.0, alp3=16.0 / 3.0):
    """Axilrod-Teller-Muto energy of one triangle of identical atoms from its side lengths
    (bohr): s9 C6^(3/2) (3 cos a cos b cos c + 1) / (r1 r2 r3)^3, zero-damped by
    1 / (1 + 6 (R0^3 / (r1 r2 r3))^alp3), the angles from the law of cosines."""
    r1, r2, r3 = sides
    ca = (r2 * r2 + r3 * r3 - r1 * r1) / (2 * r2 * r3)
    cb = (r1 * r1 + r3 * r3 - r2 * r2) / (2 * r1 * r3)
    cc = (r1 * r1 + r2 * r2 - r3 * r3) / (2 * r1 * r2)
    prod = r1 * r2 * r3
    damp = 1.0 / (1.0 + 6.0 * (r0_pair ** 3 / prod) ** alp3)
    return s9 * c6 ** 1.5 * (3.0 * ca * cb * cc + 1.0) / prod ** 3 * damp


@pytest.mark.parametrize("shape", ["equilateral", "right_isosceles"])
def test_atm_triangle_closed_forms(tables, shape):
    """Three argon atoms: the equilateral triangle (angular factor 3/8 + 1 over r^9) and the
    right isosceles one (a right angle: factor 1 over (a a a sqrt 2)^3) against the oracle's
    triple loop and its edge-list form (dispersion.py:188-222)."""
    a = 7.0                                              # bohr
    if shape == "equilateral":
        pos = np.array([[0.0, 0, 0], [a, 0, 0], [a / 2, a * math.sqrt(3) / 2, 0]])
        sides = (a, a, a)
        factor = 1.375 / a ** 9
    else:
        pos = np.array([[0.0, 0, 0], [a, 0, 0], [0, a, 0]])
        sides = (a, a, a * math.sqrt(2))
        factor = 1.0 / (math.sqrt(2) * a ** 3) ** 3
    z = torch.tensor([18, 18, 18])
    alpha = D.dynamic_polarizabilities(z, torch.zeros(3, dtype=torch.float64),
                                       torch.zeros(3, dtype=torch.float64), tables)
    c6 = float(D.c6_pairs(alpha[0], alpha[1]))
    q4 = float(tables["r4r2"][18])
    r0 = D.PBE0_D4["a1"] * math.sqrt(3.0 * q4 * q4) + D.PBE0_D4["a2"]
    want = _triangle_closed_form(c6, r0, sides)
    prod = sides[0] * sides[1] * sides[2]
    assert abs(want / (c6 ** 1.5 / (1 + 6 * (r0 ** 3 / prod) ** (16 / 3))) - factor) < 1e-12 * factor
    pt = torch.tensor(pos)
    got = float(D.atm_molecule(z, pt, alpha, tables, D.PBE0_D4, 100.0))
    assert abs(got - want) < 1e-14 * abs(want)
    ei = torch.tensor([[j, i] for i in range(3) for j in range(3) if i != j]).t()
    vec = pt[ei[1]] - pt[ei[0]]
    feat = alpha * torch.sqrt((3.0 / math.pi) * torch.as_tensor(D.cp_weights()))
    table, species = D.bj_radius_factors(z, tables, D.PBE0_D4["a1"], D.PBE0_D4["a2"])
    e = D.atm_edges(ei, vec, feat, feat, species, table, 1.0, 16.0 / 3.0, 100.0, 0.0, 3)
    np.testing.assert_allclose(e.numpy(), want / 3.0, rtol=1e-13)


def test_cn_count_vanishes_exactly_past_its_reach(tables):
    """The D4 coordination kernels skip pairs farther than rc (1 + 27.5 / kcn): there the erf
    count (d4.py:168-170) is exactly 0.0 in float64 and so is its derivative (exp(-x^2)
    underflows for x <= -27.5), so leaving them out changes no sum. Checked with the oracle's
    own count and autograd over every element pair of the tables, at and beyond the reach,
    and just inside it (where the derivative must still be nonzero)."""
    rcov = torch.as_tensor(tables["rcov"], dtype=torch.float64)
    live = rcov[rcov > 0]
    rc = (live[:, None] + live[None, :]).reshape(-1)
    reach = rc * (1.0 + 27.5 / D.KCN)
    for scale in (1.0, 1.0001, 1.5, 3.0):
        r = (reach * scale).clone().requires_grad_(True)
        c = D.erf_count(r, rc)
        (g,) = torch.autograd.grad(c.sum(), [r])
        assert bool((c == 0.0).all()) and bool((g == 0.0).all()), scale
    r = (rc * (1.0 + 26.0 / D.KCN)).clone().requires_grad_(True)
    (g,) = torch.autograd.grad(D.erf_count(r, rc).sum(), [r])
    assert bool((g != 0.0).all())
