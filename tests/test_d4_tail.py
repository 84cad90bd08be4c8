"""The D4 tail correction's radial integrals (d4.py:1073-1107) against independent
quadrature (scipy.integrate.quad) and, for the C6 term of a sharp cutoff, the closed form
int_rc^inf r^2 / (r^6 + R^6) dr = (pi / 2 - atan(rc^3 / R^3)) / (3 R^3). CPU, float64."""
import math
import os

import numpy as np
import pytest
import torch
from scipy import integrate

HERE = os.path.dirname(os.path.abspath(__file__))


def _d4(**kw):
    import xnn_amd.dispersion as XD
    return XD.DFTD4(XD.load_d4_tables(os.path.join(HERE, "golden", "d4_tables_hcnoar.npz")), **kw)


def _window(r, rc, w):
    if w <= 0:
        return 1.0 if r < rc else 0.0
    t = min(max((rc - r) / w, 0.0), 1.0)
    return t ** 3 * (10 - 15 * t + 6 * t * t)


@pytest.mark.parametrize("width_aa", [0.0, 2.0])
def test_tail_integrals_match_quadrature(width_aa):
    import xnn_amd.dispersion as XD
    d4 = _d4(cutoff_pair=40.0 * XD.BOHR, switch_width_pair=width_aa)
    J = d4.tail_integrals()
    rc, w = 40.0, width_aa / XD.BOHR
    for za, zb in [(1, 1), (6, 8), (7, 18)]:
        qa, qb = float(d4.r4r2[za]), float(d4.r4r2[zb])
        rr = 3.0 * qa * qb
        r0 = d4.a1 * math.sqrt(rr) + d4.a2

        def f(r):
            return -(1.0 - _window(r, rc, w)) * (d4.s6 / (r ** 6 + r0 ** 6)
                                                 + d4.s8 * rr / (r ** 8 + r0 ** 8)) * r * r

        lo = rc - w
        want = integrate.quad(f, lo, rc, epsabs=0, epsrel=1e-13, limit=200)[0] if w > 0 else 0.0
        want += integrate.quad(f, rc, np.inf, epsabs=0, epsrel=1e-13, limit=200)[0]
        assert abs(float(J[za, zb]) - want) <= 1e-10 * abs(want), (za, zb)
        if w == 0:
            c6_part = (math.pi / 2 - math.atan(rc ** 3 / r0 ** 3)) / (3 * r0 ** 3)
            s8_part = integrate.quad(lambda r: rr * r * r / (r ** 8 + r0 ** 8), rc, np.inf,
                                     epsabs=0, epsrel=1e-13)[0]
            assert abs(float(J[za, zb]) + d4.s6 * c6_part + d4.s8 * s8_part) <= 1e-10 * abs(want)
    assert torch.allclose(J, J.t(), rtol=1e-14, atol=0)


def test_tail_energy_is_the_continuum_pair_sum():
    """E_tail of one atom equals (2 pi / V) sum_j J(Z_i, Z_j) C6_ij over every atom j of the
    cell (the ordered pairs of the homogeneous continuum), by a direct double loop."""
    import xnn_amd.dispersion as XD
    d4 = _d4(cutoff_pair=30.0 * XD.BOHR)
    rng = np.random.default_rng(2)
    z = torch.tensor([1, 6, 8, 7, 1, 6])
    alpha = torch.tensor(rng.uniform(0.5, 9.0, (6, 23)))
    cell = torch.tensor([[20.0, 0, 0], [1.0, 21.0, 0], [0.5, -0.3, 19.0]], dtype=torch.float64)
    got = d4.tail_energy(z, alpha, cell)
    J = d4.tail_integrals()
    c6 = XD.c6_matrix(alpha)
    vol = float(torch.linalg.det(cell).abs())
    want = torch.tensor([2 * math.pi / vol * sum(float(J[z[i], z[j]] * c6[i, j]) for j in range(6))
                         for i in range(6)], dtype=torch.float64)
    torch.testing.assert_close(got, want, rtol=1e-13, atol=0)
    assert bool((got < 0).all())
