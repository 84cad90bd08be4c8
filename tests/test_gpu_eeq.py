"""GPU parity of the large-regime EEQ charges (xnn_amd.eeq: the HIP real-space matrix and
its derivative kernel, the reciprocal sum and the device factorization) against the
oracle's brute-force converged Ewald operator (oracle/eeq.py, eeq.py:170-397, 664), the
rock-salt Madelung constant, finite differences of the D4 energy through the charges,
and, at the C5 size (5,000 atoms), the split and dense-regime invariances."""
import math
import os
import sys

import numpy as np
import pytest
import torch

import oracle.d4 as D

pytestmark = pytest.mark.gpu
DEV = "cuda"
HERE = os.path.dirname(os.path.abspath(__file__))


def _note(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def tables():
    return dict(np.load(os.path.join(HERE, "golden", "d4_tables_hcnoar.npz"), allow_pickle=False))


def _cell_case(seed=3, n=11):
    rng = np.random.default_rng(seed)
    cell = np.array([[9.0, 0, 0], [1.2, 8.5, 0], [-0.7, 0.9, 10.0]])
    pos = rng.uniform(0, 1, (n, 3)) @ cell
    z = ([8, 1, 1, 6, 1, 7, 8, 1, 6, 6, 1] * (n // 11 + 1))[:n]
    return pos, cell, z


def test_operator_matches_the_oracle_and_the_madelung_constant(tables):
    """R + A_rec - 2 alpha / sqrt(pi) (the assembled operator without J + sqrt(2/pi)/a) on a
    triclinic cell against the brute-force oracle to 1e-12, and a molecule's erf(gamma r)/r
    matrix; point charges on rock salt give the Madelung energy."""
    import oracle.eeq as Q
    from xnn_amd import eeq as E
    _note("eeq operator vs oracle")
    pos, cell, z = _cell_case()
    rad = tables["eeq_rad"][np.asarray(z)]
    for cutoff in (20.0, 27.0):
        alpha = E.ewald_alpha(cutoff)
        p = torch.tensor(pos / D.BOHR, device=DEV)
        c = torch.tensor(cell / D.BOHR, device=DEV)
        zeros = torch.zeros(len(z), dtype=torch.float64, device=DEV)
        sysm = E.LargeEEQSystem(p, c, torch.tensor(rad, device=DEV),
                                zeros - 2 * alpha / math.sqrt(math.pi), alpha, cutoff)
        want = Q.ewald_matrix(pos / D.BOHR, cell / D.BOHR, rad, cutoff)
        np.testing.assert_allclose(sysm.A.cpu().numpy(), want, atol=1e-12 * np.abs(want).max())
    mol = pos[:7] + 3.0
    sysm = E.LargeEEQSystem(torch.tensor(mol / D.BOHR, device=DEV), None,
                            torch.tensor(rad[:7], device=DEV),
                            torch.zeros(7, dtype=torch.float64, device=DEV), 0.0, math.inf)
    want = Q.ewald_matrix(mol / D.BOHR, None, rad[:7], 1e9)
    np.testing.assert_allclose(sysm.A.cpu().numpy(), want, atol=1e-13)
    a0 = 10.0
    base = np.array([[0, 0, 0], [0, .5, .5], [.5, 0, .5], [.5, .5, 0]])
    salt = np.concatenate([base, base + [0.5, 0, 0]]) * a0
    q = torch.tensor([1.0] * 4 + [-1.0] * 4, dtype=torch.float64, device=DEV)
    alpha = E.ewald_alpha(17.0)
    sysm = E.LargeEEQSystem(torch.tensor(salt, device=DEV), torch.eye(3, dtype=torch.float64,
                                                                       device=DEV) * a0,
                            torch.full((8,), 1e-9, dtype=torch.float64, device=DEV),
                            torch.full((8,), -2 * alpha / math.sqrt(math.pi), dtype=torch.float64,
                                       device=DEV), alpha, 17.0)
    e = 0.5 * float(q @ sysm.A @ q)
    assert abs(e - (-4 * 1.747564594633182 / (a0 / 2))) < 1e-9


def _d4_large(tables, **kw):
    """D4 on the large EEQ regime; the pair cutoff switched over 2 A so that the energy is
    smooth in the positions and strain (finite differences across a sharp cutoff jump)."""
    import xnn_amd.dispersion as XD
    return XD.DFTD4(tables, regime="large", s9=0.0, cutoff_pair=9.0, cutoff_cn=8.0,
                    cutoff_eeq_cn=8.0, switch_width_pair=2.0,
                    cutoff_eeq=kw.pop("cutoff_eeq", 11.0), **kw).to(DEV)


def _eval(model, pos, z, cell, grad=False):
    p = torch.tensor(pos, dtype=torch.float64, device=DEV, requires_grad=grad)
    c = None if cell is None else torch.tensor(cell, dtype=torch.float64, device=DEV)[None] \
        .requires_grad_(grad)
    out = model.evaluate(torch.tensor(z, device=DEV), p, c,
                         None if c is None else torch.ones((1, 3), dtype=torch.bool),
                         torch.tensor([len(z)]))
    return out, p, c


@pytest.mark.parametrize("solver", ["lu", "cg"])
def test_charges_match_the_oracle_and_finite_differences(tables, solver):
    """The charges of the large regime (regime="large", 11 A real-space range) against the
    oracle's brute-force Ewald solve with the oracle's CN, 1e-10; the D4 energy through the
    charges: forces against central differences and the strain derivative against a finite
    strain (1e-7); a molecule too; run to run bit for bit. Both solvers: the factorized
    operator and the conjugate gradients of the matrix-free one (the regime above
    LU_MAX_ATOMS atoms, forced here)."""
    import oracle.eeq as Q
    _note(f"eeq large regime charges and derivatives, solver={solver}")
    pos, cell, z = _cell_case()
    model = _d4_large(tables, eeq_solver=solver)
    out, p, c = _eval(model, pos, z, cell, grad=True)
    q = out["charges"].detach().cpu().numpy()
    zz = np.asarray(z)
    dst, src, sh = D.pair_images(pos, cell, 8.0)
    v = D.edge_vectors_au(torch.tensor(pos), torch.tensor(cell), dst, src, sh)
    _, cn_eeq, _ = D.coordination_numbers(torch.as_tensor(zz), dst, src, torch.linalg.norm(v, dim=-1),
                                          tables, 8.0 / D.BOHR, 8.0 / D.BOHR, len(z))
    cn = cn_eeq.numpy()
    rad = tables["eeq_rad"][zz]
    x = -tables["eeq_chi"][zz] + tables["eeq_kcnchi"][zz] * cn / np.sqrt(cn + 1e-14)
    diag = tables["eeq_eta"][zz] + math.sqrt(2 / math.pi) / rad
    want = Q.charges(pos / D.BOHR, cell / D.BOHR, rad, diag, x, 0.0, 11.0 / D.BOHR)
    np.testing.assert_allclose(q, want, atol=1e-10)
    gp, gc = torch.autograd.grad(out["energy"].sum(), [p, c])
    h = 1e-4
    for i, a in [(0, 0), (4, 1), (9, 2)]:
        pp, pm = pos.copy(), pos.copy()
        pp[i, a] += h
        pm[i, a] -= h
        ep = float(_eval(model, pp, z, cell)[0]["energy"][0])
        em = float(_eval(model, pm, z, cell)[0]["energy"][0])
        assert abs(float(gp[i, a]) - (ep - em) / (2 * h)) < 1e-7, (i, a)
    D_ab = (p.detach().t() @ gp + c.detach()[0].t() @ gc[0]).cpu()
    for a, b in [(0, 0), (0, 2)]:
        eps = np.zeros((3, 3))
        eps[a, b] = eps[b, a] = h
        ep = float(_eval(model, pos @ (np.eye(3) + eps), z, cell @ (np.eye(3) + eps))[0]["energy"][0])
        em = float(_eval(model, pos @ (np.eye(3) - eps), z, cell @ (np.eye(3) - eps))[0]["energy"][0])
        wantd = float(D_ab[a, b]) if a == b else float(D_ab[a, b] + D_ab[b, a])
        assert abs((ep - em) / (2 * h) - wantd) < 1e-6, (a, b)
    again = _eval(model, pos, z, cell)[0]["charges"]
    assert torch.equal(again, out["charges"].detach())
    # a molecule in the large regime: every pair, no split
    mol, zm = pos[:9] + 2.0, z[:9]
    outm, pm_, _ = _eval(model, mol, zm, None, grad=True)
    dst, src, sh = D.pair_images(mol, None, 8.0)
    v = D.edge_vectors_au(torch.tensor(mol), None, dst, src, sh)
    zz = np.asarray(zm)
    _, cn_eeq, _ = D.coordination_numbers(torch.as_tensor(zz), dst, src, torch.linalg.norm(v, dim=-1),
                                          tables, 8.0 / D.BOHR, 8.0 / D.BOHR, len(zm))
    cn = cn_eeq.numpy()
    rad = tables["eeq_rad"][zz]
    x = -tables["eeq_chi"][zz] + tables["eeq_kcnchi"][zz] * cn / np.sqrt(cn + 1e-14)
    diag = tables["eeq_eta"][zz] + math.sqrt(2 / math.pi) / rad
    want = Q.charges(mol / D.BOHR, None, rad, diag, x, 0.0, 1e9)
    np.testing.assert_allclose(outm["charges"].detach().cpu().numpy(), want,
                               atol=1e-11 if solver == "lu" else 1e-10)
    (gpm,) = torch.autograd.grad(outm["energy"].sum(), [pm_])
    pp, pm2 = mol.copy(), mol.copy()
    pp[2, 1] += h
    pm2[2, 1] -= h
    fd = (float(_eval(model, pp, zm, None)[0]["energy"][0])
          - float(_eval(model, pm2, zm, None)[0]["energy"][0])) / (2 * h)
    assert abs(float(gpm[2, 1]) - fd) < 1e-7


def test_c5_charges_large_regime(tables):
    """The C5 box (5,000 atoms, 36.8 A cell) in the large regime (the reference's default
    there, regime="auto" above 500 periodic atoms): neutral, independent of the Ewald split
    (real-space ranges of 31.75 and 21.2 A) to 1e-8, and close to the dense regime, whose
    Wigner-Seitz images over fixed +-2 windows are an approximation of the same Ewald sum
    (its supercell variation is ~3e-7 e on an 11-atom cell; here the two differ by ~1e-5 e):
    charges to 5e-5 e and the D4 energy at those charges to 1e-6 relative."""
    import time
    import xnn_amd.dispersion as XD
    from xnn_amd import synthetic
    _note("eeq C5 large regime")
    s = synthetic.organic_box(seed=0)
    z = [int(v) for v in s.numbers]
    cuts = dict(cutoff_pair=60.0 * D.BOHR, cutoff_cn=25.0 * D.BOHR, cutoff_eeq_cn=25.0 * D.BOHR,
                s9=0.0)
    auto = XD.DFTD4(tables, **cuts).to(DEV)
    assert auto.select_regime(5000, True) == "large"
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    with torch.no_grad():
        q1 = _eval(auto, s.pos, z, s.cell)[0]["charges"]
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3
    short = XD.DFTD4(tables, cutoff_eeq=40.0 * D.BOHR, **cuts).to(DEV)
    dense = XD.DFTD4(tables, regime="dense", **cuts).to(DEV)
    with torch.no_grad():
        out1 = _eval(auto, s.pos, z, s.cell)[0]
        q2 = _eval(short, s.pos, z, s.cell)[0]["charges"]
        out3 = _eval(dense, s.pos, z, s.cell)[0]
        q3 = out3["charges"]
    print(f"C5 large-regime EEQ evaluation {ms:.1f} ms (with CN, alpha, pair terms); "
          f"|q(31.75 A) - q(21.2 A)| {float((q1 - q2).abs().max()):.2e}, "
          f"|q - q_dense| {float((q1 - q3).abs().max()):.2e}", flush=True)
    assert abs(float(q1.sum())) < 1e-10
    np.testing.assert_allclose(q1.cpu(), q2.cpu(), atol=1e-8)
    np.testing.assert_allclose(q1.cpu(), q3.cpu(), atol=5e-5)
    e1, e3 = float(out1["energy"][0]), float(out3["energy"][0])
    assert abs(e1 - e3) <= 1e-6 * abs(e3), (e1, e3)


@pytest.mark.parametrize("n", [1, 128, 300, 700, 1100])
def test_blocked_cholesky_matches_lapack(n):
    """The device factorization (128-column diagonal blocks in LDS, library GEMMs for the
    panel and trailing updates) against LAPACK's on the CPU, at sizes with a partial last
    block; its factor reproduces the matrix."""
    from xnn_amd.eeq import _cholesky
    _note(f"blocked cholesky n={n}")
    g = torch.Generator().manual_seed(n)
    M = torch.randn((n, n), dtype=torch.float64, generator=g)
    A = M @ M.T + n * torch.eye(n, dtype=torch.float64)
    L, info = _cholesky(A.to(DEV))
    assert int(info) == 0
    L = L.cpu()
    ref = torch.linalg.cholesky(A)
    assert torch.equal(L, L.tril())
    assert torch.allclose(L, ref, rtol=0, atol=1e-12 * float(ref.abs().max()))
    assert torch.allclose(L @ L.T, A, rtol=0, atol=1e-12 * float(A.abs().max()))


@pytest.mark.parametrize("n", [1, 127, 128, 129, 300, 1100])
@pytest.mark.parametrize("nrhs", [1, 2, 3])
def test_blocked_substitution_solves_the_system(n, nrhs):
    """xnn_eeq_cholesky_solve (forward and backward substitution over 128-row blocks with
    the diagonal blocks' inverses) against LAPACK's solve on the CPU, at sizes with and
    without a partial last block and one, two or three right-hand sides (three: two
    passes); the same bits run to run."""
    from xnn_amd.eeq import _cholesky, _cholesky_solve
    _note(f"blocked substitution n={n} nrhs={nrhs}")
    g = torch.Generator().manual_seed(7 * n + nrhs)
    M = torch.randn((n, n), dtype=torch.float64, generator=g)
    A = M @ M.T + n * torch.eye(n, dtype=torch.float64)
    B = torch.randn((n, nrhs), dtype=torch.float64, generator=g)
    L, info, inv = _cholesky(A.to(DEV), keep_inverses=True)
    assert int(info) == 0
    X = _cholesky_solve(L, inv, B.to(DEV))
    X2 = _cholesky_solve(L, inv, B.to(DEV))
    assert torch.equal(X, X2)
    ref = torch.linalg.solve(A, B)
    assert X.shape == B.shape
    assert torch.allclose(X.cpu(), ref, rtol=0, atol=1e-12 * float(ref.abs().max()))


def test_blocked_cholesky_reports_the_first_bad_pivot():
    """An indefinite matrix: LAPACK's info (the 1-based column of the first pivot that is
    not positive), here in the second diagonal block."""
    from xnn_amd.eeq import _cholesky
    n = 300
    A = torch.eye(n, dtype=torch.float64) * 2.0
    A[200, 200] = -1.0
    _, info = _cholesky(A.to(DEV))
    _, ref = torch.linalg.cholesky_ex(A)
    assert int(info) == int(ref) == 201


def _box(n, seed):
    """An organic box of n atoms at the C5 density (bohr), its elements and cell."""
    from xnn_amd import synthetic
    s = synthetic.organic_box(n, box=36.8 * (n / 5000) ** (1.0 / 3.0), seed=seed)
    return s.pos / D.BOHR, s.cell / D.BOHR, np.asarray([int(v) for v in s.numbers])


@pytest.mark.parametrize("case", ["triclinic_11", "box_2000", "molecule_300"])
def test_matrix_free_real_product_matches_the_matrix(tables, case):
    """xnn_eeq_real_apply (no matrix; 256-atom tiles, far tiles skipped) against the formed
    matrix of xnn_eeq_real_matrix times v, one and two right-hand sides: the triclinic
    11-atom cell with an 11 A range (many images per pair), a 2,000-atom box ordered along
    a Morton curve with an 8 A range (most tile pairs skipped), a 300-atom molecule (every
    pair). With and without tile bounds the same bits (a skipped tile adds only zeros), and
    run to run the same bits."""
    from xnn_amd import eeq as E
    _note(f"eeq matrix-free real-space product, {case}")
    if case == "triclinic_11":
        pos, cell, z = _cell_case()
        pos, cell, z, cutoff = pos / D.BOHR, cell / D.BOHR, np.asarray(z), 11.0 / D.BOHR
    elif case == "box_2000":
        pos, cell, z = _box(2000, 5)
        cutoff = 8.0 / D.BOHR
    else:
        rng = np.random.default_rng(2)
        pos, cell = rng.uniform(0, 30.0, (300, 3)), None
        z, cutoff = np.asarray(([6, 1, 8] * 100)), math.inf
    alpha = E.ewald_alpha(cutoff) if cell is not None else 0.0
    rad = torch.tensor(tables["eeq_rad"][z], device=DEV)
    p = torch.tensor(pos, device=DEV)
    c = None if cell is None else torch.tensor(cell, device=DEV)
    if c is not None:                              # wrapped, along a Morton curve
        frac = p @ torch.linalg.inv(c)
        frac = frac - torch.floor(frac)
        order = E.morton_order(frac)
        p = (frac[order] @ c).contiguous()
        rad = rad[order].contiguous()
    R = E.real_matrix(p, c, rad, alpha, cutoff)
    tiles = E.tile_bounds(p) if c is not None else None
    g = torch.Generator().manual_seed(1)
    v = torch.randn(len(z), 2, dtype=torch.float64, generator=g).to(DEV)
    for nrhs in (1, 2):
        vv = v[:, :nrhs].contiguous()
        want = R @ vv
        got = E.real_apply(p, c, rad, alpha, cutoff, vv, tiles)
        scale = float(want.abs().max())
        err = float((got - want).abs().max())
        print(f"{case} nrhs={nrhs}: max |R v| {scale:.3e}, err {err:.2e}", flush=True)
        assert err <= 1e-13 * scale
        assert torch.equal(E.real_apply(p, c, rad, alpha, cutoff, vv, tiles), got)
        assert torch.equal(E.real_apply(p, c, rad, alpha, cutoff, vv, None), got)


def test_cg_regime_24000_atoms(tables):
    """The conjugate-gradient regime at 24,000 atoms (a 62 A organic box, the default
    60-bohr real-space range of D4, 5.3e3 reciprocal vectors of the half set): the charges
    against the factorized operator's to 1e-8; the operator the GPU applies against the
    oracle's matrix-free rows (oracle/eeq.py operator_rows) on a sample of 12 atoms, and
    the charges solve those rows (x - A q the same Lagrange multiplier on every sampled row,
    1e-9); memory: no (N, N) array (the conjugate-gradient solve's peak well below the
    4.6 GB of one such matrix)."""
    import time
    import oracle.eeq as Q
    from xnn_amd import eeq as E
    n = 24000
    _note(f"eeq conjugate-gradient regime, {n} atoms")
    pos, cell, z = _box(n, 1)
    rng = np.random.default_rng(7)
    cn = rng.uniform(0.0, 4.0, n)
    rad_h = tables["eeq_rad"][z]
    x_h = -tables["eeq_chi"][z] + tables["eeq_kcnchi"][z] * cn / np.sqrt(cn + 1e-14)
    diag_h = tables["eeq_eta"][z] + math.sqrt(2 / math.pi) / rad_h
    p, c = torch.tensor(pos, device=DEV), torch.tensor(cell, device=DEV)
    rad, x, diag = (torch.tensor(a, device=DEV) for a in (rad_h, x_h, diag_h))
    cutoff = 60.0
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    t0 = time.perf_counter()
    q_cg = E.eeq_charges_large(p, c, rad, diag, x, 0.0, cutoff, solver="cg")
    torch.cuda.synchronize()
    t_cg = time.perf_counter() - t0
    peak_cg = torch.cuda.max_memory_allocated() - base
    alpha = E.ewald_alpha(cutoff)
    system = E.IterativeEEQSystem(p, c, rad, diag - 2 * alpha / math.sqrt(math.pi), alpha, cutoff)
    y, mu = system.solve_augmented(x, torch.zeros((), dtype=torch.float64, device=DEV))
    print(f"CG regime, {n} atoms: {t_cg:.2f} s for the charges (solve + correction), peak "
          f"{peak_cg / 2**30:.2f} GiB above the inputs; {system.recip.C} columns x "
          f"{system.recip.K} of the reciprocal table; iterations {system.iterations}", flush=True)
    assert peak_cg < 0.5 * n * n * 8
    t0 = time.perf_counter()
    q_lu = E.eeq_charges_large(p, c, rad, diag, x, 0.0, cutoff, solver="lu")
    torch.cuda.synchronize()
    print(f"factorized operator: {time.perf_counter() - t0:.2f} s; |q_cg - q_lu| "
          f"{float((q_cg - q_lu).abs().max()):.2e}", flush=True)
    np.testing.assert_allclose(q_cg.cpu(), q_lu.cpu(), rtol=0, atol=1e-8)
    assert abs(float(q_cg.sum())) < 1e-9
    rows = np.sort(rng.choice(n, 12, replace=False))
    q_h = q_cg.cpu().numpy()
    t0 = time.perf_counter()
    want = Q.operator_rows(pos, cell, rad_h, diag_h, q_h, rows, cutoff)
    got = system.apply(q_cg).cpu().numpy()[rows]
    lam = x_h[rows] - want
    print(f"oracle rows: {time.perf_counter() - t0:.1f} s; |A q (GPU) - A q (oracle)| "
          f"{np.abs(got - want).max():.2e} of {np.abs(want).max():.2e}; multiplier spread "
          f"{np.ptp(lam):.2e}", flush=True)
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-11 * np.abs(want).max())
    assert np.ptp(lam) < 1e-9
