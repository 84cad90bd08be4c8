"""Pins the featurizer oracle (oracle/reference.py) by what the mathematics fixes.

Spherical harmonics (e3nn convention, component normalization, y polar): the
per-degree norm 2l+1, Y_1 = sqrt(3) (x, y, z), the zonal m = 0 component
sqrt(2l+1) P_l(y), the addition theorem, rotation covariance through an orthogonal
matrix per degree, and e3nn's l = 2 closed forms. Radial bases and envelopes: the
closed forms of radial.py/cutoff.py written another way (sinc, expanded polynomial),
the envelope's C^2 end at the cutoff. Aggregation: loops and math.fsum.
"""
import math

import numpy as np
import pytest
import torch

import oracle.reference as R

F64 = torch.float64


def _unit(n, seed=0):
    v = torch.randn(n, 3, generator=torch.Generator().manual_seed(seed), dtype=torch.float64)
    return v / v.norm(dim=1, keepdim=True)


def test_sh_norm_per_degree():
    Y = R.e3nn_sh(3, 2.5 * _unit(500))
    for l in range(4):
        np.testing.assert_allclose((Y[:, l * l:(l + 1) ** 2] ** 2).sum(1), 2 * l + 1, rtol=1e-12)


def test_sh_degree_one_is_sqrt3_xyz():
    u = _unit(100, 1)
    np.testing.assert_allclose(R.e3nn_sh(1, u)[:, 1:4], math.sqrt(3) * u, atol=1e-14)


def test_sh_zonal_component_is_legendre_of_y():
    u = _unit(200, 2)
    Y = R.e3nn_sh(3, u)
    for l in range(4):
        P = np.polynomial.legendre.Legendre.basis(l)(u[:, 1].numpy())
        np.testing.assert_allclose(Y[:, l * l + l].numpy(), math.sqrt(2 * l + 1) * P, atol=1e-13)


def test_sh_addition_theorem():
    a, b = _unit(300, 3), _unit(300, 4)
    Ya, Yb = R.e3nn_sh(3, a), R.e3nn_sh(3, b)
    cos = (a * b).sum(1).numpy()
    for l in range(4):
        lhs = (Ya[:, l * l:(l + 1) ** 2] * Yb[:, l * l:(l + 1) ** 2]).sum(1).numpy()
        P = np.polynomial.legendre.Legendre.basis(l)(cos)
        np.testing.assert_allclose(lhs, (2 * l + 1) * P, atol=1e-12)


def test_sh_rotate_by_an_orthogonal_matrix_per_degree():
    u = _unit(400, 5)
    q, _ = torch.linalg.qr(torch.randn(3, 3, generator=torch.Generator().manual_seed(9), dtype=F64))
    Y, Yr = R.e3nn_sh(3, u), R.e3nn_sh(3, u @ q.T)
    for l in range(1, 4):
        A, B = Y[:, l * l:(l + 1) ** 2], Yr[:, l * l:(l + 1) ** 2]
        D = torch.linalg.lstsq(A, B).solution
        np.testing.assert_allclose((A @ D).numpy(), B.numpy(), atol=1e-10)
        np.testing.assert_allclose((D.T @ D).numpy(), np.eye(2 * l + 1), atol=1e-10)


def test_sh_degree_two_closed_forms():
    """e3nn's l = 2 forms: sqrt(15) xz, sqrt(15) xy, sqrt(5)(y^2 - (x^2+z^2)/2),
    sqrt(15) yz, sqrt(15)/2 (z^2 - x^2)."""
    u = _unit(50, 6)
    x, y, z = u[:, 0], u[:, 1], u[:, 2]
    want = torch.stack([math.sqrt(15) * x * z, math.sqrt(15) * x * y,
                        math.sqrt(5) * (y * y - 0.5 * (x * x + z * z)), math.sqrt(15) * y * z,
                        0.5 * math.sqrt(15) * (z * z - x * x)], 1)
    np.testing.assert_allclose(R.e3nn_sh(2, u)[:, 4:9], want, atol=1e-13)


def test_sh_degree_three_closed_forms():
    """e3nn 0.4.4's l = 3 forms (e3nn/o3/_spherical_harmonics.py, the published generated
    code), written over its component-normalized l = 2 values s20 = sqrt(15) xz and
    s24 = sqrt(15)/2 (z^2 - x^2), y polar:
    sqrt(42)/6 (s20 z + s24 x), sqrt(7) s20 y, sqrt(168)/8 (4y^2 - x^2 - z^2) x,
    sqrt(7)/2 y (2y^2 - 3x^2 - 3z^2), sqrt(168)/8 z (4y^2 - x^2 - z^2), sqrt(7) s24 y,
    sqrt(42)/6 (s24 z - s20 x). Elementwise, so a swapped or sign-flipped component fails."""
    u = _unit(400, 11)
    x, y, z = u[:, 0], u[:, 1], u[:, 2]
    s20 = math.sqrt(15) * x * z
    s24 = 0.5 * math.sqrt(15) * (z * z - x * x)
    y2, x2z2 = y * y, x * x + z * z
    want = torch.stack([math.sqrt(42) / 6 * (s20 * z + s24 * x),
                        math.sqrt(7) * s20 * y,
                        math.sqrt(168) / 8 * (4 * y2 - x2z2) * x,
                        0.5 * math.sqrt(7) * y * (2 * y2 - 3 * x2z2),
                        math.sqrt(168) / 8 * z * (4 * y2 - x2z2),
                        math.sqrt(7) * s24 * y,
                        math.sqrt(42) / 6 * (s24 * z - s20 * x)], 1)
    # the stated forms are component-normalized by themselves (sum_m Y^2 = 7)
    np.testing.assert_allclose((want * want).sum(1).numpy(), 7.0, atol=1e-12)
    np.testing.assert_allclose(R.e3nn_sh(3, u)[:, 9:16], want, atol=1e-13)
    # the package's closed forms (the kernels' polynomials) too, on unnormalized vectors
    from xnn_amd.featurizers import spherical_harmonics
    np.testing.assert_allclose(spherical_harmonics(3, 2.5 * u)[:, 9:16], want, atol=1e-13)


def test_sh_odd_degrees_flip_with_the_vector():
    u = _unit(50, 7)
    Y, Ym = R.e3nn_sh(3, u), R.e3nn_sh(3, -u)
    for l in range(4):
        np.testing.assert_allclose(Ym[:, l * l:(l + 1) ** 2], (-1) ** l * Y[:, l * l:(l + 1) ** 2],
                                   atol=1e-13)


def test_product_closed_forms_equal_the_oracle():
    """The package's closed-form polynomials (the kernels' formulas) equal the oracle's
    Legendre-recurrence harmonics."""
    from xnn_amd.featurizers import spherical_harmonics
    v = 3.0 * torch.randn(1000, 3, generator=torch.Generator().manual_seed(8), dtype=F64)
    np.testing.assert_allclose(spherical_harmonics(3, v), R.e3nn_sh(3, v), atol=1e-13)
    assert torch.equal(spherical_harmonics(3, torch.zeros(1, 3, dtype=F64))[0], torch.eye(16, dtype=F64)[0])


def test_bessel_is_a_scaled_sinc():
    r = torch.linspace(0.05, 5.0, 97, dtype=F64)
    rc, K = 5.0, 8
    got = R.bessel(r, K, rc)
    n = np.arange(1, K + 1)
    want = math.sqrt(2 / rc) * (n * np.pi / rc) * np.sinc(n[None] * r.numpy()[:, None] / rc)
    np.testing.assert_allclose(got.numpy(), want, rtol=1e-12)


def test_polynomial_envelope_expanded_form_and_smooth_end():
    rc, p = 5.0, 6
    r = torch.linspace(0.0, 4.99, 200, dtype=F64)
    x = (r / rc).numpy()
    want = 1 - (p + 1) * (p + 2) / 2 * x ** p + p * (p + 2) * x ** (p + 1) - p * (p + 1) / 2 * x ** (p + 2)
    np.testing.assert_allclose(R.polynomial_envelope(r, rc, p).numpy(), want, atol=1e-13)
    f = lambda t: float(R.polynomial_envelope(torch.tensor([t], dtype=F64), rc, p)[0])
    h = 1e-4
    assert abs(f(0.0) - 1.0) < 1e-15
    # a triple zero at rc: f ~ (1 - x)^3, so f, f' and f'' vanish there
    assert abs(f(rc - h)) < 1e-11 and f(rc) == 0.0 and f(rc + 1) == 0.0
    assert abs((f(rc - h) - f(rc - 2 * h)) / h) < 1e-6
    assert abs((f(rc - h) - 2 * f(rc - 2 * h) + f(rc - 3 * h)) / h ** 2) < 1e-2
    assert abs((f(2.0 + h) - f(2.0 - h)) / (2 * h)) > 0.1     # and not flat inside


def test_cosine_envelope_values():
    rc = 6.0
    r = torch.tensor([0.0, 3.0, 6.0, 7.0], dtype=F64)
    np.testing.assert_allclose(R.cosine_envelope(r, rc).numpy(), [1.0, 0.5, 0.0, 0.0], atol=1e-15)


def test_gaussian_centers_and_width():
    r = torch.tensor([0.0, 1.25], dtype=F64)
    g = R.gaussian(r, 5, 5.0)
    assert abs(float(g[0, 0]) - 1.0) < 1e-15 and abs(float(g[1, 1]) - 1.0) < 1e-15
    assert abs(float(g[1, 0]) - math.exp(-0.5)) < 1e-15        # one width away


def test_scatter_and_structure_sums():
    gen = torch.Generator().manual_seed(0)
    src = torch.randn(40, 3, generator=gen, dtype=F64)
    index = torch.randint(0, 7, (40,), generator=gen)
    want = torch.zeros(7, 3, dtype=F64)
    for e, i in enumerate(index.tolist()):
        want[i] += src[e]
    torch.testing.assert_close(R.scatter_sum(src, index, 7), want, rtol=1e-15, atol=1e-15)
    vals = torch.randn(1000, generator=gen, dtype=F64) * 1e3
    assert float(R.structure_sum(vals, torch.zeros(1000, dtype=torch.long), 1)[0]) == \
        pytest.approx(math.fsum(vals.tolist()), rel=1e-15, abs=1e-9)


def test_make_radial_basis_builds_the_path_bases():
    """make_radial_basis (radial.py:348-401): the Gaussian basis with float64 centers on
    [0, cutoff] and the spacing as width, the Bessel basis with trainable frequencies; the
    bases outside this path raise, unknown names are rejected, ignored options warn."""
    import warnings
    from xnn_amd.featurizers import BesselRBF, GaussianRBF, make_radial_basis
    g = make_radial_basis("gaussian", 8, 5.0)
    assert isinstance(g, GaussianRBF) and g.centers.dtype == torch.float64
    assert torch.equal(g.centers, torch.linspace(0.0, 5.0, 8, dtype=torch.float64))
    assert abs(g.gamma - 0.5 * (7 / 5.0) ** 2) < 1e-15
    r = torch.tensor([0.3, 2.0], dtype=torch.float32)
    assert g(r).dtype == torch.float32
    b = make_radial_basis("bessel", 8, 5.0, trainable=True)
    assert isinstance(b, BesselRBF) and isinstance(b.freqs, torch.nn.Parameter)
    with pytest.raises(NotImplementedError):
        make_radial_basis("expnorm", 8, 5.0)
    with pytest.raises(ValueError):
        make_radial_basis("sinc", 8, 5.0)
    with warnings.catch_warnings(record=True) as w:
        warnings.simplefilter("always")
        make_radial_basis("gaussian", 8, 5.0, trainable=True)
    assert any("trainable" in str(x.message) for x in w)
