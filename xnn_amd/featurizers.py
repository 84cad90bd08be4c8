"""Edge featurizers with the reference's parameters and a HIP evaluation.

* :class:`BesselRBF`, :class:`GaussianRBF` -- common/featurizers/radial.py:15-75, 187-268,
  and :func:`make_radial_basis` (radial.py:348-401) for those two
* :class:`CosineCutoff`, :class:`PolynomialCutoff` -- common/featurizers/cutoff.py:10-125
* :func:`spherical_harmonics` -- e3nn ``SphericalHarmonics(normalize=True,
  normalization="component")`` for ``l <= 3`` (gnn/featurizers/spherical.py:91-93): real
  harmonics without Condon-Shortley phase, ``sum_m Y_lm^2 = 2l + 1``, polar axis y
  (``Y_1 = sqrt(3) (x, y, z)``), homogeneous polynomials of the unit vector.
* :class:`SphericalHarmonicEdgeEmbedding` -- gnn/featurizers/spherical.py:28-171, whose
  ``embed`` runs one fused HIP kernel when ``fast_active``.

The modules hold exactly the reference's parameters and buffers, so a state dict
moves between the two.
"""
from __future__ import annotations

import math
from typing import Tuple

import torch
from torch import Tensor, nn

from .fast import FastPathModule


class GaussianRBF(nn.Module):
    """``exp(-gamma (r - mu_k)^2)`` on centers ``linspace(start, cutoff, n_rbf)`` (radial.py:15-75)."""

    def __init__(self, n_rbf: int = 50, cutoff: float = 5.0, gamma: float | None = None,
                 start: float = 0.0, endpoint: bool = True):
        super().__init__()
        centers = (torch.linspace(start, cutoff, n_rbf) if endpoint
                   else torch.linspace(start, cutoff, n_rbf + 1)[:n_rbf])
        self.register_buffer("centers", centers)
        self.width = (centers[1] - centers[0]).item() if n_rbf > 1 else 1.0
        self.gamma = float(gamma) if gamma is not None else 0.5 / self.width ** 2

    def forward(self, r: Tensor) -> Tensor:
        diff = r[..., None] - self.centers.to(r.dtype)
        return torch.exp(-self.gamma * diff ** 2)


class BesselRBF(nn.Module):
    """``prefactor sin(freq_n r / rc) / r``, ``freq_n = n pi`` (radial.py:187-268)."""

    def __init__(self, n_rbf: int = 8, cutoff: float = 5.0, trainable: bool = False,
                 prefactor: float | None = None):
        super().__init__()
        self.cutoff = cutoff
        freqs = math.pi * torch.arange(1, n_rbf + 1, dtype=torch.get_default_dtype())
        if trainable:
            self.freqs = nn.Parameter(freqs)
        else:
            self.register_buffer("freqs", freqs)
        self.norm = math.sqrt(2.0 / cutoff) if prefactor is None else float(prefactor)

    def exact_constants(self) -> bool:
        """Rebuild fixed float64 frequencies as the exact ``n pi`` (radial.py:233-252).

        A float32 build or checkpoint leaves them rounded to float32; learned (trainable)
        frequencies, non-float64 buffers and stored values farther than rounding (1e-6
        relative) from ``n pi`` are kept. Returns whether any value changed.
        """
        freqs = self.freqs
        if isinstance(freqs, nn.Parameter) or freqs.dtype != torch.float64:
            return False
        exact = math.pi * torch.arange(1, freqs.numel() + 1, dtype=torch.float64,
                                       device=freqs.device)
        if torch.equal(freqs, exact):
            return False
        scale = float(exact.abs().max()) if exact.numel() else 0.0
        if float((freqs - exact).abs().max()) > 1e-6 * max(scale, 1e-300):
            return False
        with torch.no_grad():
            freqs.copy_(exact)
        return True

    def forward(self, r: Tensor) -> Tensor:
        r = r.clamp(min=1e-8)[..., None]
        return self.norm * torch.sin(self.freqs * r / self.cutoff) / r


RADIAL_BASES = ("gaussian", "bessel", "expnorm", "smooth_bessel")


def make_radial_basis(name: str, n_rbf: int, cutoff: float, trainable: bool = False, *,
                      gamma: float | None = None, prefactor: float | None = None) -> nn.Module:
    """A radial basis by name (radial.py:348-401): ``"gaussian"`` (:class:`GaussianRBF`,
    ``n_rbf`` centers on ``[0, cutoff]`` kept in float64, the center spacing as width
    unless ``gamma`` is given) or ``"bessel"`` (:class:`BesselRBF`, frequencies trainable
    with ``trainable``). The reference's ``"expnorm"`` and ``"smooth_bessel"`` bases are
    not part of this path and raise ``NotImplementedError``; options the chosen basis does
    not have are ignored with a warning, as there."""
    if name not in RADIAL_BASES:
        raise ValueError(f"radial_basis must be one of {RADIAL_BASES}, got {name!r}")
    if name in ("expnorm", "smooth_bessel"):
        raise NotImplementedError(f"the {name!r} radial basis is not part of this path "
                                  "(bessel and gaussian are)")
    ignored = [k for k, bad in (("trainable", trainable and name == "gaussian"),
                                ("gamma", gamma is not None and name != "gaussian"),
                                ("prefactor", prefactor is not None and name != "bessel")) if bad]
    if ignored:
        import warnings
        warnings.warn(f"radial basis {name!r} ignores {ignored}", UserWarning, stacklevel=2)
    if name == "gaussian":
        if gamma is None and n_rbf > 1:      # the center spacing as width, in double precision
            gamma = 0.5 * ((n_rbf - 1) / cutoff) ** 2
        basis = GaussianRBF(n_rbf, cutoff, gamma=gamma)
        basis.centers = torch.linspace(0.0, cutoff, n_rbf, dtype=torch.float64)
        return basis
    return BesselRBF(n_rbf, cutoff, trainable=trainable, prefactor=prefactor)


class CosineCutoff(nn.Module):
    """``0.5 (cos(pi r / rc) + 1)`` inside the cutoff, 0 beyond (cutoff.py:10-41)."""

    def __init__(self, cutoff: float):
        super().__init__()
        self.cutoff = cutoff

    def forward(self, r: Tensor) -> Tensor:
        out = 0.5 * (torch.cos(math.pi * r / self.cutoff) + 1.0)
        return out * (r < self.cutoff)


class PolynomialCutoff(nn.Module):
    """``1 - (p+1)(p+2)/2 x^p + p(p+2) x^(p+1) - p(p+1)/2 x^(p+2)``, ``x = r / rc`` (cutoff.py:83-125)."""

    def __init__(self, cutoff: float, p: int = 6):
        super().__init__()
        self.cutoff = cutoff
        self.p = p

    def forward(self, r: Tensor) -> Tensor:
        x = r / self.cutoff
        p = self.p
        tail = ((-(p * (p + 1) / 2)) * x + p * (p + 2)) * x - (p + 1) * (p + 2) / 2
        return (1.0 + tail * x ** p) * (r < self.cutoff)


_S3, _S5, _S15 = math.sqrt(3.0), math.sqrt(5.0), math.sqrt(15.0)
_A, _B, _C = math.sqrt(35.0 / 8.0), math.sqrt(105.0), math.sqrt(21.0 / 8.0)
_D, _E = math.sqrt(7.0) / 2.0, math.sqrt(105.0) / 2.0


def spherical_harmonics(l_max: int, vec: Tensor) -> Tensor:
    """Component-normalized real SH of ``vec / |vec|`` in the e3nn order, ``(E, (l_max+1)^2)``.

    They are ``sqrt(2l+1)`` times the orthonormal real harmonics (no Condon-Shortley
    phase) in standard form with the polar axis on y: ``(x_s, y_s, z_s) = (z, x, y)``.
    A zero vector gives ``Y_0 = 1`` and zeros (``normalize`` maps it to zero).
    """
    if not 0 <= l_max <= 3:
        raise ValueError("l_max must be in [0, 3]")
    n = torch.linalg.norm(vec, dim=-1, keepdim=True)
    u = vec / n.clamp(min=1e-12)
    x, y, z = u[..., 0], u[..., 1], u[..., 2]
    out = [torch.ones_like(x)]
    if l_max >= 1:
        out += [_S3 * x, _S3 * y, _S3 * z]
    if l_max >= 2:
        x2, y2, z2 = x * x, y * y, z * z
        out += [_S15 * x * z, _S15 * x * y, _S5 * (y2 - 0.5 * (x2 + z2)), _S15 * y * z,
                0.5 * _S15 * (z2 - x2)]
    if l_max >= 3:
        x2, y2, z2 = x * x, y * y, z * z
        out += [_A * x * (3.0 * z2 - x2), _B * x * y * z, _C * x * (4.0 * y2 - x2 - z2),
                _D * y * (2.0 * y2 - 3.0 * x2 - 3.0 * z2), _C * z * (4.0 * y2 - x2 - z2),
                _E * y * (z2 - x2), _A * z * (z2 - 3.0 * x2)]
    return torch.stack(out, dim=-1)


def radial_spec(module) -> dict:
    """The HIP featurizer's description of an embedding module's radial part, read through
    the reference's attribute names only (spherical.py:86-101, radial.py:15-268,
    cutoff.py:10-125): ``module.rbf`` is a Bessel basis (``freqs``, ``norm``) or a Gaussian
    one (``centers``, ``gamma``), ``module.envelope`` a polynomial envelope (``p``) or a
    cosine one, ``module.cutoff`` the cutoff. So a reference module and this package's
    mirror of it give the same kernel arguments. Unknown bases or envelopes raise."""
    rbf, env = module.rbf, module.envelope
    if hasattr(rbf, "freqs") and hasattr(rbf, "norm"):
        basis, table, prefactor, gamma = "bessel", rbf.freqs, float(rbf.norm), 1.0
    elif hasattr(rbf, "centers") and hasattr(rbf, "gamma"):
        basis, table, prefactor, gamma = "gaussian", rbf.centers, 1.0, float(rbf.gamma)
    else:
        raise TypeError(f"no HIP radial basis for {type(rbf).__name__} (Bessel and Gaussian "
                        "bases are on the fast path)")
    if hasattr(env, "p"):
        envelope, poly_p = "polynomial", int(env.p)
    elif type(env).__name__ == "CosineCutoff":
        envelope, poly_p = "cosine", 1
    else:
        raise TypeError(f"no HIP envelope for {type(env).__name__} (polynomial and cosine "
                        "envelopes are on the fast path)")
    return dict(table=table, basis=basis, envelope=envelope, poly_p=poly_p,
                cutoff=float(module.cutoff), prefactor=prefactor, gamma=gamma)


def fast_embed(module, vec: Tensor, sh_sign: int = 1,
               want_sh: bool = True) -> Tuple[Tensor, Tensor, Tensor]:
    """``embed(vec)`` of a spherical-harmonic edge embedding on the HIP featurizer, for
    this package's module or the reference's own (spherical.py:115-138): reads
    ``module.l_max``, ``module.rbf``, ``module.envelope`` and ``module.cutoff`` and
    returns ``(length (E,), sh (E, (l_max+1)^2), radial (E, n_rbf))``. Without the
    harmonics (``want_sh=False``) only the radial part is evaluated."""
    from .ops import edge_embed
    spec = radial_spec(module)
    table = spec.pop("table")
    return edge_embed(vec, table, n_rbf=int(table.numel()),
                      l_max=int(module.l_max) if want_sh else 0, sh_sign=sh_sign,
                      want_length=want_sh, want_sh=want_sh, **spec)


class SphericalHarmonicEdgeEmbedding(nn.Module, FastPathModule):
    """Per-edge length, SH edge attributes and enveloped radial basis
    (gnn/featurizers/spherical.py:28-171).

    Same constructor as the reference, plus ``envelope`` (``"polynomial"``, the
    reference's, or ``"cosine"``) and ``sh_sign`` (``-1`` evaluates ``Y(-vec)``, as
    NequIP does with ``embed(-edge_vec)``, nequip.py:722).
    """

    def __init__(self, l_max: int = 2, n_rbf: int = 8, cutoff: float = 5.0, p: int = 6,
                 radial_type: str = "bessel", trainable_rbf: bool = False,
                 rbf_prefactor: float | None = None, envelope: str = "polynomial"):
        super().__init__()
        if not 0 <= l_max <= 3:
            raise ValueError("l_max must be in [0, 3] (the HIP harmonics stop at l = 3)")
        self.cutoff = cutoff
        self.l_max = l_max
        self.n_rbf = n_rbf
        self.radial_type = radial_type
        if radial_type == "bessel":
            self.rbf = BesselRBF(n_rbf, cutoff, trainable=trainable_rbf, prefactor=rbf_prefactor)
        elif radial_type == "gaussian":
            self.rbf = GaussianRBF(n_rbf, cutoff)
        else:
            raise ValueError(f"unknown radial_type {radial_type!r}")
        if envelope == "polynomial":
            self.envelope = PolynomialCutoff(cutoff, p=p)
        elif envelope == "cosine":
            self.envelope = CosineCutoff(cutoff)
        else:
            raise ValueError(f"unknown envelope {envelope!r}")
        self.envelope_type = envelope
        self.fast_active = False

    @property
    def output_dim(self) -> int:
        return self.n_rbf

    def _table(self) -> Tensor:
        return self.rbf.freqs if self.radial_type == "bessel" else self.rbf.centers

    def _embed_fast(self, vec: Tensor, sh_sign: int, want_sh: bool = True):
        return fast_embed(self, vec, sh_sign, want_sh)

    @property
    def radial_trainable(self) -> bool:
        return bool(self._table().requires_grad)

    def radial_message_sum(self, vec: Tensor, W: Tensor, plan, sh_sign: int = 1) -> Tensor:
        """``A_i = sum_{dst(e)=i} (radial(vec_e) W) (x) Y(sh_sign vec_e)``, ``(N, C, L)``,
        with this embedding's radial basis evaluated inside the HIP message kernels
        (float32, on a GPU; differentiable in ``vec`` only: forces and stress)."""
        from .ops import sh_radial_message_sum
        spec = radial_spec(self)
        return sh_radial_message_sum(vec, spec.pop("table"), W, plan, l_max=self.l_max,
                                     sh_sign=sh_sign, **spec)

    def radial_message_energy(self, vec: Tensor, W: Tensor, U: Tensor, z: Tensor, bias, plan,
                              sh_sign: int = 1, one_pass: bool = False) -> Tensor:
        """Per-atom ``<U, A_i> + bias[z_i]`` of the rows of :meth:`radial_message_sum`, read
        out inside the same HIP kernels (the rows never reach memory; differentiable in
        ``vec`` only)."""
        from .ops import sh_radial_message_energy
        spec = radial_spec(self)
        return sh_radial_message_energy(vec, spec.pop("table"), W, U, z, bias, plan,
                                        l_max=self.l_max, sh_sign=sh_sign, one_pass=one_pass,
                                        **spec)

    def embed(self, vec: Tensor, sh_sign: int = 1) -> Tuple[Tensor, Tensor, Tensor]:
        """``(edge_length (E,), edge_sh (E, (l_max+1)^2), edge_radial (E, n_rbf))``
        of edge vectors (spherical.py:115-138); ``Y`` is taken of ``sh_sign * vec``."""
        if self.fast_active:
            return self._embed_fast(vec, sh_sign)
        length = torch.linalg.norm(vec, dim=-1)
        edge_sh = spherical_harmonics(self.l_max, vec if sh_sign == 1 else -vec)
        radial = self.rbf(length) * self.envelope(length)[:, None]
        return length, edge_sh, radial

    def radial(self, vec: Tensor) -> Tensor:
        """The enveloped radial basis alone (no harmonics are evaluated)."""
        if self.fast_active:
            return self._embed_fast(vec, 1, want_sh=False)[2]
        length = torch.linalg.norm(vec, dim=-1)
        return self.rbf(length) * self.envelope(length)[:, None]

    def forward(self, data) -> dict:
        vec = data.edge_vectors()
        length, edge_sh, radial = self.embed(vec)
        return {"edge_vec": vec, "edge_length": length, "edge_sh": edge_sh,
                "edge_radial": radial}
