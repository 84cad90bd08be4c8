"""GPU parity of the D3 path: the HIP coordination-number and two-body kernels against
the oracle (float64, brute-force pair images) and the simple-dftd3 golden values
(tests/common/test_d3.py:112-157)."""
import os
import sys

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"
HERE = os.path.dirname(os.path.abspath(__file__))
WATER = (np.array([[0.0, 0.0, 0.119262], [0.0, 0.763239, -0.477047],
                   [0.0, -0.763239, -0.477047]]), [8, 1, 1])
FAST = dict(cutoff_pair=9.0, cutoff_cn=8.0)


def _note(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def tables():
    return dict(np.load(os.path.join(HERE, "golden", "d3_tables_hcnoar.npz"), allow_pickle=False))


def _cluster(n, seed, box=6.0):
    rng = np.random.default_rng(seed)
    return rng.uniform(0, box - 1, (n, 3)), ([1, 8, 6, 7] * (n // 4) + [1] * (n % 4))[:n]


def _eval(model, pos, z, cell=None, grad=False):
    p = torch.tensor(pos, dtype=torch.float64, device=DEV, requires_grad=grad)
    c = None if cell is None else torch.tensor(cell, dtype=torch.float64, device=DEV)[None].requires_grad_(grad)
    out = model.evaluate(torch.tensor(z, device=DEV), p, c,
                         None if c is None else torch.ones((1, 3), dtype=torch.bool),
                         torch.tensor([len(z)]))
    return out, p, c


def _prm(damping):
    import oracle.d3 as D3
    prm = dict(D3.PBE0_D3BJ if damping in ("bj", "op") else D3.PBE0_D3ZERO)
    if damping == "mzero":
        prm["bet"] = 0.1
    if damping == "op":
        prm["bet"] = 6.0
    return prm


def test_water_golden_values_on_the_gpu(tables):
    import xnn_amd.dispersion as XD
    _note("d3 water golden")
    bj, _, _ = _eval(XD.DFTD3(tables).to(DEV), *WATER)
    assert abs(float(bj["energy"][0]) / XD.HARTREE - (-2.768885028766e-04)) < 1e-14
    zero, _, _ = _eval(XD.DFTD3(tables, damping="zero").to(DEV), *WATER)
    assert abs(float(zero["energy"][0]) / XD.HARTREE - (-4.644598055357e-06)) < 1e-16


@pytest.mark.parametrize("damping", ["bj", "zero", "mzero", "op"])
@pytest.mark.parametrize("case", ["molecule", "triclinic_switched"])
def test_kernels_match_oracle(tables, damping, case):
    """CN, per-atom energies and the position and cell gradients (through the CN-dependent
    weights too) against autograd of the oracle, float64."""
    import oracle.d3 as D3
    import xnn_amd.dispersion as XD
    from oracle.d4 import BOHR, edge_vectors_au, pair_images
    _note(f"d3 kernels vs oracle: {damping} {case}")
    prm = _prm(damping)
    width, cell = 0.0, None
    if case == "molecule":
        pos, z = _cluster(12, seed=21)
    else:
        pos, z = _cluster(10, seed=22)
        cell = np.array([[6.0, 0, 0], [0.8, 5.7, 0], [-0.4, 0.6, 6.2]])
        width = 2.0
    model = XD.DFTD3(tables, damping=damping, switch_width_pair=width,
                     **{k: v for k, v in prm.items() if k in ("s6", "s8", "a1", "a2", "rs6", "rs8", "alp", "bet")},
                     **FAST).to(DEV)
    out, p, c = _eval(model, pos, z, cell, grad=True)
    gp, *gc = torch.autograd.grad(out["energy"].sum(), [p] + ([c] if c is not None else []))
    # oracle
    s = D3.species_of(tables, z)
    dst, src, sh = pair_images(pos, cell, max(FAST.values()))
    pt = torch.tensor(pos, dtype=torch.float64, requires_grad=True)
    ct = None if cell is None else torch.tensor(cell, dtype=torch.float64, requires_grad=True)
    r = torch.linalg.norm(edge_vectors_au(pt, ct, dst, src, sh), dim=-1)
    cn = D3.coordination_numbers(s, dst, src, r, tables, FAST["cutoff_cn"] / BOHR, len(z))
    w = D3.weights(s, cn, tables)
    c6 = D3.pair_c6(s, w, torch.as_tensor(dst), torch.as_tensor(src), tables)
    e2 = D3.two_body(s, dst, src, r, c6, tables, prm, damping, FAST["cutoff_pair"] / BOHR,
                     width / BOHR, len(z))
    grads = torch.autograd.grad(e2.sum(), [pt] + ([ct] if ct is not None else []))
    np.testing.assert_allclose(out["coordination_numbers"].detach().cpu(), cn.detach(),
                               rtol=1e-12, atol=1e-13)
    e_gpu = out["node_energy"].detach().cpu() / XD.HARTREE
    np.testing.assert_allclose(e_gpu, e2.detach(), atol=1e-11 * float(e2.abs().max()))
    np.testing.assert_allclose(gp.cpu() / XD.HARTREE, grads[0],
                               atol=1e-10 * float(grads[0].abs().max()))
    if cell is not None:
        np.testing.assert_allclose(gc[0][0].cpu() / XD.HARTREE, grads[1],
                                   atol=1e-10 * float(grads[1].abs().max()))


def test_forces_match_finite_differences(tables):
    """test_d3.py:237-256: central differences, h = 1e-4 A, 1e-7 eV/A."""
    import xnn_amd.dispersion as XD
    _note("d3 finite differences")
    pos, z = _cluster(8, seed=23)
    model = XD.DFTD3(tables, **FAST).to(DEV)
    out, p, _ = _eval(model, pos, z, grad=True)
    (gp,) = torch.autograd.grad(out["energy"].sum(), [p])
    h = 1e-4
    for i, a in [(0, 0), (3, 2), (5, 1)]:
        pp, pm = pos.copy(), pos.copy()
        pp[i, a] += h
        pm[i, a] -= h
        fd = (float(_eval(model, pp, z)[0]["energy"][0]) - float(_eval(model, pm, z)[0]["energy"][0])) / (2 * h)
        assert abs(float(gp[i, a]) - fd) < 1e-7


def test_weights_kernel_matches_oracle(tables):
    """The D3 reference weights and their chain rule to CN from the HIP kernel against the
    oracle (float64 autograd): every tabulated species, CNs from 0 to past the Gaussian
    underflow (the largest-reference fallback), and a species outside the tables (NaN)."""
    import oracle.d3 as D3
    import xnn_amd.dispersion as XD
    _note("d3 weights kernel vs oracle")
    model = XD.DFTD3(tables).to(DEV)
    rng = np.random.default_rng(31)
    n_sp = len(tables["z"])
    s = torch.as_tensor(np.arange(60) % n_sp)
    cn_np = rng.uniform(0.0, 5.0, 60)
    cn_np[:4] = 60.0                                 # exp(-4 d^2) underflows: fallback
    cn = torch.tensor(cn_np, requires_grad=True)
    ref = D3.weights(s, cn, tables)
    g_w = torch.tensor(rng.normal(size=ref.shape))
    (ref_g,) = torch.autograd.grad((ref * g_w).sum(), [cn])
    cg = cn.detach().to(DEV).requires_grad_(True)
    w = model.weights(s.to(DEV), cg)
    (g,) = torch.autograd.grad((w * g_w.to(DEV)).sum(), [cg])
    np.testing.assert_allclose(w.detach().cpu(), ref.detach(), rtol=1e-13, atol=1e-15)
    np.testing.assert_allclose(g.cpu(), ref_g, rtol=1e-12, atol=1e-12 * float(ref_g.abs().max()))
    assert float(g[:4].abs().max()) == 0.0
    bad = model.weights(torch.tensor([0, n_sp], device=DEV),
                        torch.tensor([1.0, 1.0], dtype=torch.float64, device=DEV))
    assert torch.isfinite(bad[0]).all() and torch.isnan(bad[1]).all()


@pytest.mark.parametrize("periodic", [False, True])
def test_three_body_matches_oracle(tables, periodic):
    """The D3 ATM term (s9 = 1, radii 4/3 R0_AB, exponent (alp + 2) / 3, a 1 A switch on a
    6 A triple cutoff; d3.py:840-859, 916-936): its energy and its position and cell
    gradients against the oracle's CN, weights and pair C6 (oracle/d3.py) fed as a dense C6
    matrix to the oracle's edge-list ATM (feat_a = C6 rows, feat_b = identity), which also
    checks the module's factorization of C6 over reference slots."""
    import oracle.d3 as D3
    import oracle.d4 as D4
    import xnn_amd.dispersion as XD
    _note(f"d3 three-body vs oracle: periodic={periodic}")
    pos, z = _cluster(10, seed=8)
    cell = np.diag([7.0, 7.5, 8.0]) if periodic else None
    cut_tri, width = 6.0, 1.0
    model = XD.DFTD3(tables, s9=1.0, cutoff_triple=cut_tri, switch_width_triple=width,
                     **FAST).to(DEV)
    out, p, c = _eval(model, pos, z, cell, grad=True)
    got = torch.autograd.grad(out["energy_3body"].sum(), [p] + ([c] if c is not None else []))
    n = len(z)
    s = D3.species_of(tables, z)
    dst, src, sh = D4.pair_images(pos, cell, max(FAST["cutoff_cn"], cut_tri))
    pt = torch.tensor(pos, dtype=torch.float64, requires_grad=True)
    ct = None if cell is None else torch.tensor(cell, dtype=torch.float64, requires_grad=True)
    v = D4.edge_vectors_au(pt, ct, dst, src, sh)
    r = torch.linalg.norm(v, dim=-1)
    cn = D3.coordination_numbers(s, dst, src, r, tables, FAST["cutoff_cn"] / D4.BOHR, n)
    w = D3.weights(s, cn, tables)
    ii, jj = torch.meshgrid(torch.arange(n), torch.arange(n), indexing="ij")
    c6 = D3.pair_c6(s, w, ii.reshape(-1), jj.reshape(-1), tables).reshape(n, n)
    tri = r <= cut_tri / D4.BOHR
    ei = torch.stack([torch.as_tensor(src), torch.as_tensor(dst)])[:, tri]
    uniq, spec = torch.unique(s, return_inverse=True)
    table = (4.0 / 3.0) * torch.as_tensor(tables["rvdw"])[uniq][:, uniq]
    e3 = D4.atm_edges(ei, v[tri], c6, torch.eye(n, dtype=torch.float64), spec, table, 1.0,
                      16.0 / 3.0, cut_tri / D4.BOHR, width / D4.BOHR, n)
    ref = torch.autograd.grad(e3.sum(), [pt] + ([ct] if ct is not None else []))
    assert float(e3.sum()) > 0
    assert abs(float(out["energy_3body"][0]) / XD.HARTREE - float(e3.sum())) \
        < 1e-12 * float(e3.sum())
    for a, b in zip(got, ref):
        a = a.reshape(b.shape).detach().cpu() / XD.HARTREE
        np.testing.assert_allclose(a, b, atol=1e-11 * float(b.abs().max()))


@pytest.mark.parametrize("damping", ["bj", "zero"])
def test_fused_pair_matches_the_two_launch_path(tables, damping):
    """evaluate(fused_pair=True): the two-body energies from one pair-backward launch at unit
    seeds (e_i = 1/2 w_i . dE/dw_i, bilinear in the reference weights) and their gradients
    scaled by the structure seeds, against the energy launch plus the autograd backward: two
    periodic structures, seeds 2 and -3, a switching window."""
    import xnn_amd.dispersion as XD
    _note(f"d3 fused pair vs two launches, {damping}")
    model = XD.DFTD3(tables, damping=damping, cutoff_pair=12.0, cutoff_cn=8.0,
                     switch_width_pair=1.0).to(DEV)
    rng = np.random.default_rng(12)
    zs, ps, cs, ns = [], [], [], []
    for n, L in ((14, 7.5), (19, 8.5)):
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
