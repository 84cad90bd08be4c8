"""EEQ charges of large systems on the GPU: a converged Ewald operator, factorized on the
device, with implicit differentiation (common/models/eeq.py:170-397, 664;
dispersion_fast/eeq.py:69).

The constrained system ``[[A, 1], [1^T, 0]] [q; mu] = [x; Q]`` of the EEQ model has
``A = R + A_rec + diag(J + sqrt(2/pi) / a - 2 alpha / sqrt(pi))`` for a periodic cell:

* ``R`` (``xnn_eeq_real_matrix``, HIP): the screened kernel
  ``[erf(gamma_ij r) - erf(alpha r)] / r`` summed over every image within the real-space
  cutoff, formed densely (one thread per atom pair; 8 bytes per pair, so the MI355X's HBM
  holds it up to ~10^5 atoms);
* ``A_rec``: ``sum_G w_G cos(G . (r_i - r_j))`` over the reciprocal vectors of one
  half-space with ``exp(-G^2 / 4 alpha^2) >= eps`` and ``w_G = 2 (4 pi / V)
  exp(-G^2 / 4 alpha^2) / G^2``, as two matrix products of structure factors;
* ``alpha = erfc^-1(eps) / r_c``: both tails truncated at ``eps = 1e-10`` relative.

A molecule has ``alpha = 0``, one image and no reciprocal part. The matrix is factorized
(Cholesky) once per evaluation, and the charges are refined once with its residual. The
derivatives follow the implicit function theorem around the refined charges ``q1``:
``q = q1 + S(x - A(r) q1 - mu1, Q - 1^T q1)`` where ``S`` is the constant solve, whose
value is zero (the residual vanishes) and whose backward is the adjoint solve with the same
factor; ``A(r) q1`` is applied differentiably (the HIP derivative kernel for ``R``, PyTorch
for the reciprocal sum), so forces and stress need no second matrix. Differentiable once.
"""
from __future__ import annotations

import ctypes
import math
from typing import Optional, Tuple

import torch
from torch import Tensor

from . import _lib

#: relative truncation of the real- and reciprocal-space Ewald tails
EWALD_EPS = 1e-10
_NS = "xnn_amd"


def erfc_inverse(eps: float) -> float:
    """``x`` with ``erfc(x) = eps`` (Newton's method from the log estimate)."""
    x = math.sqrt(-math.log(eps))
    for _ in range(30):
        step = (math.erfc(x) - eps) / (-2.0 / math.sqrt(math.pi) * math.exp(-x * x))
        x -= step
        if abs(step) < 1e-15 * x:
            break
    return x


def ewald_alpha(cutoff_au: float, eps: float = EWALD_EPS) -> float:
    """Splitting parameter with ``erfc(alpha r_c) = eps`` at the real-space cutoff (bohr)."""
    return erfc_inverse(eps) / cutoff_au


def reciprocal_half_set(cell_au: Tensor, alpha: float, eps: float = EWALD_EPS) -> Tensor:
    """Integer triples ``m != 0`` of one half-space (first non-zero component positive) with
    ``|m B| <= 2 alpha sqrt(-ln eps)``, ``B = 2 pi cell^-T``, ``(M, 3)`` float64 on the
    cell's device (G and -G give the same cosine, so each pair is kept once)."""
    c = cell_au.detach().to(torch.float64).cpu()
    g_max = 2.0 * alpha * math.sqrt(-math.log(eps))
    recip = 2.0 * math.pi * torch.linalg.inv(c).t()
    # |m_a| <= g_max |a_a| / (2 pi) bounds every component
    span = [int(math.floor(g_max * float(torch.linalg.norm(c[a])) / (2.0 * math.pi))) + 1
            for a in range(3)]
    axes = [torch.arange(-s, s + 1, dtype=torch.float64) for s in span]
    m = torch.cartesian_prod(*axes)
    g = m @ recip
    keep = (g * g).sum(-1) <= g_max * g_max
    first = torch.where(m[:, 0] != 0, m[:, 0], torch.where(m[:, 1] != 0, m[:, 1], m[:, 2]))
    keep &= first > 0
    return m[keep].to(cell_au.device)


def reciprocal_weights(m: Tensor, cell_au: Tensor, alpha: float) -> Tuple[Tensor, Tensor]:
    """``G = m 2 pi cell^-T`` and ``w_G = 2 (4 pi / V) exp(-G^2 / 4 alpha^2) / G^2`` for the
    half set, differentiable in the cell."""
    vol = torch.linalg.det(cell_au).abs()
    recip = 2.0 * math.pi * torch.linalg.inv(cell_au).t()
    g = m.to(cell_au.dtype) @ recip
    g2 = (g * g).sum(-1)
    w = (8.0 * math.pi) / vol * torch.exp(-0.25 * g2 / (alpha * alpha)) / g2
    return g, w


def reciprocal_apply(pos: Tensor, g: Tensor, w: Tensor, v: Tensor) -> Tensor:
    """``A_rec v = C diag(w) C^T v + S diag(w) S^T v`` with ``C, S = cos, sin(pos G^T)``."""
    phase = pos @ g.t()
    c, s = torch.cos(phase), torch.sin(phase)
    return c @ (w * (c.t() @ v)) + s @ (w * (s.t() @ v))


# --------------------------------------------------------------------------- real space (HIP)
def _host_cell(cell: Optional[Tensor]):
    """The cell rows as 9 host doubles (the kernels take the lattice by value), or None."""
    if cell is None:
        return None
    vals = [float(v) for v in cell.detach().to(torch.float64).reshape(9).cpu()]
    return (ctypes.c_double * 9)(*vals)


def real_matrix(pos: Tensor, cell: Optional[Tensor], rad: Tensor, alpha: float,
                cutoff_au: float) -> Tensor:
    """The dense real-space matrix R (N, N) of the screened kernel (no autograd)."""
    n = pos.shape[0]
    out = torch.empty((n, n), dtype=torch.float64, device=pos.device)
    p = pos.detach().to(torch.float64).contiguous()
    _lib.call("xnn_eeq_real_matrix", _lib.ptr(p), n, _host_cell(cell),
              _lib.ptr(rad.detach().to(torch.float64).contiguous()), float(alpha),
              float(cutoff_au), _lib.ptr(out), _lib.stream(pos.device))
    return out


@torch.library.custom_op(f"{_NS}::eeq_real_apply", mutates_args=())
def real_apply_op(pos: Tensor, cell: Optional[Tensor], rad: Tensor, v: Tensor, matrix: Tensor,
                  alpha: float, cutoff_au: float) -> Tensor:
    """``R(pos, cell) v`` with the matrix formed at these positions; differentiable in
    ``pos`` and ``cell`` through ``xnn_eeq_real_grad`` (``v`` is held constant)."""
    return matrix @ v


@real_apply_op.register_fake
def _(pos, cell, rad, v, matrix, alpha, cutoff_au):
    return v.new_empty(v.shape)


def _real_apply_setup(ctx, inputs, output):
    pos, cell, rad, v, matrix, alpha, cutoff_au = inputs
    ctx.save_for_backward(pos, cell, rad, v)
    ctx.alpha, ctx.cutoff = alpha, cutoff_au


def _real_apply_backward(ctx, grad):
    if torch.is_grad_enabled():
        raise RuntimeError("the large-regime EEQ charges are differentiable once")
    pos, cell, rad, v = ctx.saved_tensors
    if ctx.needs_input_grad[3] or ctx.needs_input_grad[2]:
        raise NotImplementedError("eeq_real_apply differentiates positions and cell only")
    n = pos.shape[0]
    dev = pos.device
    grad_pos = torch.empty((n, 3), dtype=torch.float64, device=dev)
    want_cell = cell is not None and ctx.needs_input_grad[1]
    part = torch.empty((n, 9), dtype=torch.float64, device=dev) if want_cell else None
    _lib.call("xnn_eeq_real_grad", _lib.ptr(pos.detach().to(torch.float64).contiguous()), n,
              _host_cell(cell), _lib.ptr(rad.detach().to(torch.float64).contiguous()), float(ctx.alpha),
              float(ctx.cutoff), _lib.ptr(grad.to(torch.float64).contiguous()),
              _lib.ptr(v.detach().to(torch.float64).contiguous()), _lib.ptr(grad_pos),
              _lib.ptr(part), _lib.stream(dev))
    g_cell = part.sum(0).reshape(3, 3).to(cell.dtype) if want_cell else None
    return grad_pos.to(pos.dtype), g_cell, None, None, None, None, None


real_apply_op.register_autograd(_real_apply_backward, setup_context=_real_apply_setup)


# --------------------------------------------------------------------------- the system
class LargeEEQSystem:
    """The EEQ operator of one structure at fixed (detached) geometry, assembled densely and
    factorized: the constant Jacobian of the implicit differentiation."""

    def __init__(self, pos: Tensor, cell: Optional[Tensor], rad: Tensor, diag: Tensor,
                 alpha: float, cutoff_au: float, eps: float = EWALD_EPS):
        self.pos, self.cell = pos.detach(), None if cell is None else cell.detach()
        self.rad, self.alpha, self.cutoff = rad.detach(), float(alpha), float(cutoff_au)
        self.diag = diag.detach()
        self.R = real_matrix(self.pos, self.cell, self.rad, self.alpha, self.cutoff)
        A = self.R.clone()
        self.m = None
        if self.cell is not None:
            self.m = reciprocal_half_set(self.cell, self.alpha, eps)
            g, w = reciprocal_weights(self.m, self.cell.to(torch.float64), self.alpha)
            phase = self.pos.to(torch.float64) @ g.t()
            c, s = torch.cos(phase), torch.sin(phase)
            A.addmm_(c * w, c.t()).addmm_(s * w, s.t())
            del c, s, phase
        A.diagonal().add_(self.diag.to(torch.float64))
        self.A = A
        self.factor, info = _cholesky(A)
        self.cholesky = bool(int(info) == 0)
        if not self.cholesky:                  # not numerically positive definite: LU
            self.lu = torch.linalg.lu_factor(A)
        self.y_ones = None

    def _solve(self, b: Tensor) -> Tensor:
        """``A^-1 b`` for ``b`` (N, k): two triangular solves with the Cholesky factor (the
        blocked solves; the one-column path of ``cholesky_solve`` is several times slower).
        A single column is solved as two, with a zero second column: the library's
        one-column triangular solve is about six times slower than its blocked one at
        N = 5,000."""
        if b.shape[1] == 1 and b.is_cuda:
            return self._solve(torch.cat([b, torch.zeros_like(b)], 1))[:, :1]
        if self.cholesky:
            y = torch.linalg.solve_triangular(self.factor, b, upper=False)
            return torch.linalg.solve_triangular(self.factor.mT, y, upper=True)
        return torch.linalg.lu_solve(*self.lu, b)

    def solve_augmented(self, top: Tensor, bottom: Tensor) -> Tuple[Tensor, Tensor]:
        """``[[A, 1], [1^T, 0]] [y; mu] = [top; bottom]`` by eliminating the constraint:
        ``y = A^-1 top - mu A^-1 1`` with ``mu = (1^T A^-1 top - bottom) / 1^T A^-1 1``."""
        b = top.to(torch.float64).reshape(-1, 1)
        if self.y_ones is None:                # the constraint's A^-1 1, with the first solve
            y = self._solve(torch.cat([b, torch.ones_like(b)], 1))
            y1, self.y_ones = y[:, 0], y[:, 1]
        else:
            y1 = self._solve(b)[:, 0]
        mu = (y1.sum() - bottom) / self.y_ones.sum()
        return y1 - mu * self.y_ones, mu

    def apply(self, v: Tensor) -> Tensor:
        """``A v`` at the detached geometry."""
        return self.A @ v

    def apply_live(self, pos: Tensor, cell: Optional[Tensor], v: Tensor) -> Tensor:
        """``A(pos, cell) v`` with derivatives in ``pos`` and ``cell`` (``v`` constant)."""
        out = self.diag * v + real_apply_op(pos, cell, self.rad, v, self.R, self.alpha,
                                            self.cutoff)
        if cell is not None:
            g, w = reciprocal_weights(self.m, cell, self.alpha)
            out = out + reciprocal_apply(pos, g, w, v)
        return out


CHOLESKY_BLOCK = 128


def _cholesky(A: Tensor):
    """The Cholesky factor of the float64 operator and LAPACK's ``info`` (0, or the 1-based
    column of the first pivot that is not positive). On the device: right-looking blocked
    factorization, 128 columns at a time: ``xnn_eeq_cholesky_block`` factors the diagonal
    block in LDS and forms its inverse, the panel below it is ``A21 L11^-T`` and the
    trailing matrix takes ``- L21 L21^T`` (library GEMMs; a large trailing update is split
    at half height into the top rows' left square and the bottom rows, 3/4 of the square,
    and the upper triangle is discarded at the end)."""
    if not A.is_cuda:
        return torch.linalg.cholesky_ex(A)
    n, nb = A.shape[0], CHOLESKY_BLOCK
    L = A.contiguous().clone()
    info = torch.zeros(1, dtype=torch.int32, device=A.device)
    inv = torch.empty(nb * nb, dtype=torch.float64, device=A.device)
    panel = torch.empty((max(n - nb, 0), nb), dtype=torch.float64, device=A.device)
    stream = _lib.stream(A.device)
    for k in range(0, n, nb):
        b = min(nb, n - k)
        _lib.call("xnn_eeq_cholesky_block", _lib.ptr(L), n, k, b, _lib.ptr(inv),
                  _lib.ptr(info), stream)
        r = k + b
        if r < n:
            p = panel[:n - r, :b]
            torch.matmul(L[r:, k:r], inv[:b * b].view(b, b).t(), out=p)
            L[r:, k:r].copy_(p)
            m = n - r
            if m >= 4 * nb:                # the lower part only: 3/4 of the square
                h = (m // 2 + nb - 1) // nb * nb
                L[r:r + h, r:r + h].addmm_(p[:h], p[:h].t(), alpha=-1.0)
                L[r + h:, r:].addmm_(p[h:], p.t(), alpha=-1.0)
            else:
                L[r:, r:].addmm_(p, p.t(), alpha=-1.0)
    return L.tril_(), info[0]


class _ConstantSolve(torch.autograd.Function):
    """The solve with the constant Jacobian as a function of the residual: its value is
    zero (the residual of the refined charges vanishes to rounding) and its backward is the
    adjoint solve ``[[A, 1], [1^T, 0]] [lambda; kappa] = [g; 0]`` (A is symmetric)."""

    @staticmethod
    def forward(ctx, system, top, bottom):
        ctx.system = system
        return torch.zeros_like(top)

    @staticmethod
    def backward(ctx, g):
        lam, kappa = ctx.system.solve_augmented(g, torch.zeros((), dtype=torch.float64,
                                                               device=g.device))
        return None, lam.to(g.dtype), kappa.to(g.dtype)


def eeq_charges_large(pos: Tensor, cell: Optional[Tensor], rad: Tensor, diag: Tensor,
                      x: Tensor, total_charge: float, cutoff_au: float,
                      eps: float = EWALD_EPS) -> Tensor:
    """EEQ charges of one structure in the large regime (eeq.py:664-700): positions and
    cell in bohr (``cell`` None: a molecule), the charge widths ``rad``, the diagonal
    ``J + sqrt(2/pi) / a`` (the ``- 2 alpha / sqrt(pi)`` of a cell is added here), the
    right-hand side ``x`` and the total charge; ``cutoff_au`` the real-space range.
    Differentiable once in ``pos``, ``cell`` and ``x``."""
    periodic = cell is not None
    alpha = ewald_alpha(cutoff_au, eps) if periodic else 0.0
    if periodic:
        diag = diag - 2.0 * alpha / math.sqrt(math.pi)
    else:
        cutoff_au = math.inf            # a molecule: every pair (eeq.py:346-360), no split
    system = LargeEEQSystem(pos, cell, rad, diag, alpha, cutoff_au, eps)
    total = torch.as_tensor(float(total_charge), dtype=torch.float64, device=pos.device)
    with torch.no_grad():
        xd = x.detach().to(torch.float64)
        q0, mu0 = system.solve_augmented(xd, total)
        dq, dmu = system.solve_augmented(xd - system.apply(q0) - mu0, total - q0.sum())
        q1, mu1 = q0 + dq, mu0 + dmu
    live = x.requires_grad or pos.requires_grad or (periodic and cell.requires_grad)
    if not (live and torch.is_grad_enabled()):
        return q1.to(x.dtype)
    top = x.to(torch.float64) - system.apply_live(pos.to(torch.float64),
                                                  None if cell is None else cell.to(torch.float64),
                                                  q1) - mu1
    bottom = total - q1.sum()
    return (q1 + _ConstantSolve.apply(system, top, bottom)).to(x.dtype)
