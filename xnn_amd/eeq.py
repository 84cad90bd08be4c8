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
#: atoms up to which the assembled operator is factorized; conjugate gradients above
#: (eeq.py:70, 226: two (N, N) float64 matrices, 2.3 GB at 12,000 atoms)
LU_MAX_ATOMS = 12000
#: conjugate-gradient stopping rule |r| <= tol |b| per right-hand side, and its cap
#: (eeq.py:63-67)
CG_TOL = 1e-12
CG_MAXITER = 1000
#: float64 entries of the (N, 2C) column table of the factorized reciprocal product kept
#: between products (2 GB); above it the table is formed again in blocks at every product
TABLE_BUDGET = 1 << 28
#: (N, G) entries per block of the differentiable reciprocal sum (recomputed in the
#: backward)
LIVE_BUDGET = 1 << 23
#: reciprocal vectors (smallest |G|, largest weights) in the low-rank part of the
#: conjugate-gradient preconditioner (dispersion_fast/eeq.py:60-66); 0 for plain Jacobi
LOW_K_VECTORS = 256
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


def _reciprocal_block(pos: Tensor, g: Tensor, w: Tensor, v: Tensor) -> Tensor:
    phase = pos @ g.t()
    c, s = torch.cos(phase), torch.sin(phase)
    return c @ (w * (c.t() @ v)) + s @ (w * (s.t() @ v))


def reciprocal_apply(pos: Tensor, g: Tensor, w: Tensor, v: Tensor) -> Tensor:
    """``A_rec v = C diag(w) C^T v + S diag(w) S^T v`` with ``C, S = cos, sin(pos G^T)``,
    over blocks of reciprocal vectors of at most :data:`LIVE_BUDGET` phases each; a block
    that carries gradients is recomputed in the backward instead of kept (memory
    ``O(LIVE_BUDGET)`` at any size)."""
    n = max(int(pos.shape[0]), 1)
    step = max(1, LIVE_BUDGET // n)
    if g.shape[0] <= step:
        return _reciprocal_block(pos, g, w, v)
    live = torch.is_grad_enabled() and any(t.requires_grad for t in (pos, g, w, v))
    out = None
    for k0 in range(0, int(g.shape[0]), step):
        args = (pos, g[k0:k0 + step], w[k0:k0 + step], v)
        if live:
            from torch.utils.checkpoint import checkpoint
            part = checkpoint(_reciprocal_block, *args, use_reentrant=False)
        else:
            part = _reciprocal_block(*args)
        out = part if out is None else out + part
    return out


# --------------------------------------------------------------------------- real space (HIP)
def _host_cell(cell: Optional[Tensor]):
    """The cell rows as 9 host doubles (the kernels take the lattice by value), or None."""
    if cell is None:
        return None
    vals = [float(v) for v in cell.detach().to(torch.float64).reshape(9).cpu()]
    return (ctypes.c_double * 9)(*vals)


def real_matrix(pos: Tensor, cell: Optional[Tensor], rad: Tensor, alpha: float,
                cutoff_au: float, host_cell=None) -> Tensor:
    """The dense real-space matrix R (N, N) of the screened kernel (no autograd);
    ``host_cell``: the cell as :func:`_host_cell` returns it, when the caller has it."""
    n = pos.shape[0]
    out = torch.empty((n, n), dtype=torch.float64, device=pos.device)
    p = pos.detach().to(torch.float64).contiguous()
    _lib.call("xnn_eeq_real_matrix", _lib.ptr(p), n,
              host_cell if host_cell is not None else _host_cell(cell),
              _lib.ptr(rad.detach().to(torch.float64).contiguous()), float(alpha),
              float(cutoff_au), _lib.ptr(out), _lib.stream(pos.device))
    return out


def real_apply(pos: Tensor, cell, rad: Tensor, alpha: float, cutoff_au: float,
               v: Tensor, tiles: Optional[Tensor] = None, work: Optional[Tensor] = None) -> Tensor:
    """``R v`` for ``v`` (N, 1 or 2) without the matrix (``xnn_eeq_real_apply``, HIP):
    every pair and image evaluated at every product, memory O(N). ``cell``: the (3, 3)
    tensor, its 9 host doubles (:func:`_host_cell`) or None. ``tiles``: bounding
    spheres of 256-atom tiles of ``pos`` (:func:`tile_bounds`) to skip distant tiles;
    ``work``: a reusable workspace of at least the queried size (uint8)."""
    n, r = int(pos.shape[0]), int(v.shape[1])
    out = torch.empty((n, r), dtype=torch.float64, device=pos.device)
    if n == 0:
        return out
    need = ctypes.c_size_t(0)
    _lib.call("xnn_eeq_real_apply_work_size", n, r, ctypes.byref(need))
    if work is None or work.numel() < need.value:
        work = torch.empty(need.value, dtype=torch.uint8, device=pos.device)
    vv = v.detach().to(torch.float64).contiguous()
    host = cell if isinstance(cell, ctypes.Array) else _host_cell(cell)
    _lib.call("xnn_eeq_real_apply", _lib.ptr(pos.detach().to(torch.float64).contiguous()), n,
              host, _lib.ptr(rad.detach().to(torch.float64).contiguous()),
              float(alpha), float(cutoff_au), _lib.ptr(tiles), _lib.ptr(vv), r, _lib.ptr(out),
              _lib.ptr(work), int(work.numel()), _lib.stream(pos.device))
    return out


@torch.library.custom_op(f"{_NS}::eeq_real_apply", mutates_args=())
def real_apply_op(pos: Tensor, cell: Optional[Tensor], rad: Tensor, v: Tensor,
                  matrix: Optional[Tensor], alpha: float, cutoff_au: float) -> Tensor:
    """``R(pos, cell) v`` with the matrix formed at these positions, or without a matrix
    (``matrix`` None: the matrix-free HIP product); differentiable in ``pos`` and ``cell``
    through ``xnn_eeq_real_grad`` (``v`` is held constant)."""
    if matrix is not None:
        return matrix @ v
    return real_apply(pos, cell, rad, alpha, cutoff_au, v.reshape(-1, 1)).reshape(v.shape)


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
        # one read of the cell to the host; the real-space kernel runs while the host forms
        # the reciprocal vectors and weights, which go up by asynchronous copies (no drain
        # of the queue between the two parts)
        cell_h = None if self.cell is None else self.cell.to(torch.float64).cpu()
        host = None if cell_h is None else _host_cell(cell_h)
        self.R = real_matrix(self.pos, self.cell, self.rad, self.alpha, self.cutoff, host)
        A = self.R.clone()
        self.m = None
        if self.cell is not None:
            dev = self.pos.device
            m_h = reciprocal_half_set(cell_h, self.alpha, eps)
            g_h, w_h = reciprocal_weights(m_h, cell_h, self.alpha)
            up = (lambda t: t.pin_memory().to(dev, non_blocking=True)) if dev.type == "cuda" \
                else (lambda t: t)
            self.m, g, w = up(m_h), up(g_h), up(w_h)
            phase = self.pos.to(torch.float64) @ g.t()
            # A_rec = C W C^T + S W S^T = X X^T with X = [C W^1/2, S W^1/2] (w_G > 0)
            m = phase.shape[1]
            X = torch.empty((phase.shape[0], 2 * m), dtype=torch.float64, device=phase.device)
            sw = torch.sqrt(w)
            torch.cos(phase, out=X[:, :m])
            torch.sin(phase, out=X[:, m:])
            del phase
            X[:, :m].mul_(sw)
            X[:, m:].mul_(sw)
            _add_gram(A, X)
            del X
        A.diagonal().add_(self.diag.to(torch.float64))
        self.A = A
        self.factor, info, self.inv_blocks = _cholesky(A, keep_inverses=True)
        self.cholesky = bool(int(info) == 0)
        if not self.cholesky:                  # not numerically positive definite: LU
            self.lu = torch.linalg.lu_factor(A)
        self.y_ones = None

    def _solve(self, b: Tensor) -> Tensor:
        """``A^-1 b`` for ``b`` (N, k): forward and backward substitution with the Cholesky
        factor on the device (:func:`_cholesky_solve`: one launch per 128-row block, where
        the library's blocked triangular solves launch several small products per block);
        LAPACK's triangular solves on the CPU; the LU solve when the factorization failed."""
        if self.cholesky:
            if self.inv_blocks is not None:
                return _cholesky_solve(self.factor, self.inv_blocks, b)
            y = torch.linalg.solve_triangular(self.factor, b, upper=False)
            return torch.linalg.solve_triangular(self.factor.mT, y, upper=True)
        return torch.linalg.lu_solve(*self.lu, b)

    def solve_augmented(self, top: Tensor, bottom: Tensor,
                        tol_abs: Optional[float] = None) -> Tuple[Tensor, Tensor]:
        """``[[A, 1], [1^T, 0]] [y; mu] = [top; bottom]`` by eliminating the constraint:
        ``y = A^-1 top - mu A^-1 1`` with ``mu = (1^T A^-1 top - bottom) / 1^T A^-1 1``
        (direct: ``tol_abs`` is not used)."""
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


# --------------------------------------------------------------------------- CG regime
def morton_order(unit: Tensor) -> Tensor:
    """The permutation that orders points of the unit cube (N, 3) along a Morton curve
    (10 bits per axis): consecutive points are close in space."""
    q = (unit.clamp(0.0, 1.0 - 1e-12) * 1024.0).to(torch.int64)
    code = torch.zeros(unit.shape[0], dtype=torch.int64, device=unit.device)
    for bit in range(10):
        for a in range(3):
            code |= ((q[:, a] >> bit) & 1) << (3 * bit + a)
    return torch.argsort(code, stable=True)


def tile_bounds(pos: Tensor, tile: int = 256) -> Tensor:
    """Per tile of ``tile`` consecutive atoms, the center and radius of a sphere holding them,
    ``(ceil(N / tile), 4)`` (the radius rounded up: the kernels' tile test stays
    conservative)."""
    n = int(pos.shape[0])
    t = (n + tile - 1) // tile
    p = pos.to(torch.float64)
    if t * tile > n:                      # the last tile padded with copies of its last atom
        p = torch.cat([p, p[-1:].expand(t * tile - n, 3)])
    p = p.view(t, tile, 3)
    center = p.mean(1)
    radius = torch.linalg.vector_norm(p - center[:, None], dim=-1).amax(1)
    return torch.cat([center, (radius * (1.0 + 1e-12) + 1e-9)[:, None]], 1).contiguous()


def own_image_diagonal(cell: Tensor, rad: Tensor, alpha: float, cutoff_au: float) -> Tensor:
    """``R_ii``: the screened kernel summed over the atom's own lattice images ``n cell``
    (``n != 0``) within the cutoff, ``(N,)`` (zero when the cell is wider than the cutoff)."""
    c = cell.to(torch.float64)
    inv = torch.linalg.inv(c)
    reach = [int(math.floor(cutoff_au * float(torch.linalg.norm(inv[:, a])))) for a in range(3)]
    axes = [torch.arange(-k, k + 1, dtype=torch.float64, device=c.device) for k in reach]
    t = torch.cartesian_prod(*axes).reshape(-1, 3) @ c
    r = torch.linalg.vector_norm(t, dim=-1)
    r = r[(r > 1e-10) & (r <= cutoff_au)]
    if r.numel() == 0:
        return torch.zeros_like(rad, dtype=torch.float64)
    gam = 1.0 / (math.sqrt(2.0) * rad.to(torch.float64))
    k = (torch.erf(gam[:, None] * r[None]) - torch.erf(alpha * r)[None]) / r[None]
    return k.sum(1)


def _tn_product(b: Tensor, v: Tensor, chunks: int = 32) -> Tensor:
    """``b^T v`` for tall ``b`` (N, P) and ``v`` (N, Q) with a long reduction over N: split
    into ``chunks`` batched products that are summed afterwards (one library GEMM of a small
    output would run on a handful of workgroups)."""
    n = int(b.shape[0])
    m = n // chunks
    if m < 256:
        return b.t() @ v
    k = m * chunks
    out = torch.bmm(b[:k].view(chunks, m, -1).transpose(1, 2), v[:k].view(chunks, m, -1)).sum(0)
    if k < n:
        out += b[k:].t() @ v[k:]
    return out


class FactorizedReciprocal:
    """``A_rec v`` at fixed positions through factorized structure-factor phases
    (dispersion_fast/eeq.py:1-33): with ``G = m B``, ``exp(i G . r) = exp(2 pi i (m_1 f_1 +
    m_2 f_2)) exp(2 pi i m_3 f_3)`` for the fractional coordinates ``f``; the vectors of
    the half set are grouped in columns of fixed ``(m_1, m_2)``, whose phases ``Bc (N, C)``
    are products of two per-axis tables, and the third axis is ``P (N, 2 M_3 + 1)``. Then
    ``S = Bc^T (P * v)`` is the structure factor of ``v`` on every vector and ``A_rec v =
    Re[sum_k conj(P_k) (conj(Bc) (W S))_k]``: two real GEMMs per product (library GEMMs,
    real and imaginary parts stacked), no trigonometry. ``Bc`` is kept while it fits
    :data:`TABLE_BUDGET` and formed again in column blocks otherwise."""

    def __init__(self, pos: Tensor, cell: Tensor, m: Tensor, alpha: float):
        c = cell.to(torch.float64)
        f = pos.to(torch.float64) @ torch.linalg.inv(c)
        g, w = reciprocal_weights(m, c, alpha)
        mi = m.round().to(torch.int64)
        span = [int(mi[:, a].abs().max()) if mi.shape[0] else 0 for a in range(3)]
        self.tables = []
        for a in range(3):
            ms = torch.arange(-span[a], span[a] + 1, dtype=torch.float64, device=f.device)
            ph = (2.0 * math.pi) * f[:, a:a + 1] * ms[None]
            self.tables.append((torch.cos(ph), torch.sin(ph)))
        w2 = 2 * span[1] + 1
        key = (mi[:, 0] + span[0]) * w2 + (mi[:, 1] + span[1])
        cols, col_of = torch.unique(key, return_inverse=True)
        self.c1, self.c2 = cols // w2, cols % w2
        self.K = 2 * span[2] + 1
        self.C = int(cols.numel())
        W = torch.zeros((self.C, self.K), dtype=torch.float64, device=f.device)
        W[col_of, mi[:, 2] + span[2]] = w
        self.W = W
        self.n = int(f.shape[0])
        self.diagonal = float(w.sum())     # A_rec,ii = sum_G w_G
        self.block = max(1, TABLE_BUDGET // max(2 * self.n, 1))
        self.table = self._columns(0, self.C) if self.C <= self.block else None

    def _columns(self, c0: int, c1: int) -> Tensor:
        (ar, ai), (br, bi) = self.tables[0], self.tables[1]
        ar, ai = ar[:, self.c1[c0:c1]], ai[:, self.c1[c0:c1]]
        br, bi = br[:, self.c2[c0:c1]], bi[:, self.c2[c0:c1]]
        return torch.cat([ar * br - ai * bi, ar * bi + ai * br], 1)

    def apply(self, v: Tensor) -> Tensor:
        """``A_rec v`` for ``v`` (N, R)."""
        n, R = v.shape
        K, KR = self.K, self.K * v.shape[1]
        pr, pi = self.tables[2]
        vp = torch.cat([(pr[:, :, None] * v[:, None, :]).reshape(n, KR),
                        (pi[:, :, None] * v[:, None, :]).reshape(n, KR)], 1)
        ur = v.new_zeros((n, KR))
        ui = v.new_zeros((n, KR))
        for c0 in range(0, self.C, self.block):
            c1 = min(self.C, c0 + self.block)
            b = self.table if self.table is not None else self._columns(c0, c1)
            cb = c1 - c0
            x = _tn_product(b, vp)                           # (2 cb, 2 KR)
            sr = x[:cb, :KR] - x[cb:, KR:]
            si = x[:cb, KR:] + x[cb:, :KR]
            wb = self.W[c0:c1].repeat_interleave(R, dim=1)
            gr, gi = wb * sr, wb * si
            y = b @ torch.cat([torch.cat([gr, gi], 1), torch.cat([gi, -gr], 1)], 0)
            ur += y[:, :KR]
            ui += y[:, KR:]
        return (pr[:, :, None] * ur.view(n, K, R) + pi[:, :, None] * ui.view(n, K, R)).sum(1)


class IterativeEEQSystem:
    """The EEQ operator of one structure at fixed (detached) geometry, never assembled: the
    conjugate-gradient regime above :data:`LU_MAX_ATOMS` (eeq.py:226, 325-360;
    dispersion_fast/eeq.py:1-33). A product is ``diag v`` plus the matrix-free real-space
    product (``xnn_eeq_real_apply``, HIP, atoms ordered along a Morton curve of the wrapped
    fractional coordinates so that 256-atom tiles are compact and far tiles are skipped)
    plus the factorized reciprocal product (:class:`FactorizedReciprocal`). Memory O(N) in
    the real-space part and O(N C) in the reciprocal tables. Solves: preconditioned
    conjugate gradients, the preconditioner the full diagonal (``J + sqrt(2/pi)/a - 2
    alpha/sqrt(pi)``, the own images and ``sum_G w_G``) with the long-range modes of the
    smallest reciprocal vectors as a low-rank part (:meth:`_low_rank`; Jacobi for a
    molecule), the charge and the constraint right-hand sides in lockstep as two columns
    of one product. Same interface as :class:`LargeEEQSystem`."""

    def __init__(self, pos: Tensor, cell: Optional[Tensor], rad: Tensor, diag: Tensor,
                 alpha: float, cutoff_au: float, eps: float = EWALD_EPS, tol: float = CG_TOL,
                 maxiter: int = CG_MAXITER):
        self.pos = pos.detach().to(torch.float64)
        self.cell = None if cell is None else cell.detach().to(torch.float64)
        self.rad, self.alpha, self.cutoff = rad.detach().to(torch.float64), float(alpha), float(cutoff_au)
        self.diag = diag.detach().to(torch.float64)
        self.tol, self.maxiter = float(tol), int(maxiter)
        self.n = int(self.pos.shape[0])
        if self.cell is not None:
            frac = self.pos @ torch.linalg.inv(self.cell)
            frac = frac - torch.floor(frac)
            self.order = morton_order(frac)
            self.pos_s = (frac[self.order] @ self.cell).contiguous()
            self.tiles = tile_bounds(self.pos_s)
            self.m = reciprocal_half_set(self.cell, self.alpha, eps)
            self.recip = FactorizedReciprocal(self.pos_s, self.cell, self.m, self.alpha)
            own = own_image_diagonal(self.cell, self.rad, self.alpha, self.cutoff)
            full = self.diag + own + self.recip.diagonal
            self._low_rank(full[self.order])
        else:
            lo = self.pos.amin(0)
            span = (self.pos.amax(0) - lo).clamp_min(1e-12)
            self.order = morton_order((self.pos - lo) / span)
            self.pos_s = self.pos[self.order].contiguous()
            self.tiles = None                  # every pair: nothing to skip
            self.m, self.recip = None, None
            full = self.diag
        self.cell_host = _host_cell(self.cell)
        self.rad_s = self.rad[self.order].contiguous()
        self.diag_s = self.diag[self.order].contiguous()
        if self.cell is None:
            self.U = None
            self.inv_d = (1.0 / full[self.order]).contiguous()
        self.y_ones = None
        self.iterations = []                   # per conjugate-gradient solve
        self._work = None

    def _low_rank(self, full_s: Tensor) -> None:
        """The preconditioner ``M = D + U W U^T`` (dispersion_fast/eeq.py:72-86): ``U = [cos,
        sin]`` of the :data:`LOW_K_VECTORS` smallest reciprocal vectors at the (ordered)
        positions, ``W`` their weights, ``D`` the full diagonal of ``A`` less that part's
        (``sum_l w_l``); ``M^-1`` through the Woodbury identity with the Cholesky factor of
        ``W^-1 + U^T D^-1 U``. It changes how fast the iteration converges, not its limit."""
        g, w = reciprocal_weights(self.m, self.cell, self.alpha)
        L = min(LOW_K_VECTORS, int(g.shape[0]))
        if L == 0:
            self.U = None
            self.inv_d = (1.0 / full_s).contiguous()
            return
        idx = torch.argsort((g * g).sum(1))[:L]
        ph = self.pos_s @ g[idx].t()
        self.U = torch.cat([torch.cos(ph), torch.sin(ph)], 1).contiguous()
        wl = torch.cat([w[idx], w[idx]])
        self.inv_d = (1.0 / (full_s - w[idx].sum())).contiguous()
        core = torch.diag(1.0 / wl) + self.U.t() @ (self.inv_d[:, None] * self.U)
        self.core = torch.linalg.cholesky(core)

    def precondition(self, r: Tensor) -> Tensor:
        """``M^-1 r`` for the columns of ``r``."""
        z = self.inv_d[:, None] * r
        if self.U is None:
            return z
        t = torch.cholesky_solve(_tn_product(self.U, z), self.core)
        return z - self.inv_d[:, None] * (self.U @ t)

    def _matvec(self, v: Tensor) -> Tensor:
        """``A v`` in the spatial order, ``v`` (N, 1 or 2)."""
        need = ctypes.c_size_t(0)
        _lib.call("xnn_eeq_real_apply_work_size", self.n, int(v.shape[1]), ctypes.byref(need))
        if self._work is None or self._work.numel() < need.value:
            self._work = torch.empty(need.value, dtype=torch.uint8, device=v.device)
        out = real_apply(self.pos_s, self.cell_host, self.rad_s, self.alpha, self.cutoff, v,
                         self.tiles, self._work)
        out += self.diag_s[:, None] * v
        if self.recip is not None:
            out += self.recip.apply(v)
        return out

    def conjugate_gradient(self, b: Tensor, tol_abs: Tensor) -> Tensor:
        """``A^-1 b`` for the columns of ``b`` (N, 1 or 2) in the spatial order, each column
        to ``|r| <= tol_abs`` (a column that meets it is frozen while the other runs)."""
        x = self.precondition(b)
        r = b - self._matvec(x)
        z = self.precondition(r)
        p = z.clone()
        rz = (r * z).sum(0)
        for it in range(self.maxiter + 1):
            done = torch.linalg.vector_norm(r, dim=0) <= tol_abs
            if bool(done.all()):
                self.iterations.append(it)
                return x
            if it == self.maxiter:
                break
            ap = self._matvec(p)
            a = torch.where(done, torch.zeros_like(rz), rz / (p * ap).sum(0))
            x += a * p
            r -= a * ap
            z = self.precondition(r)
            rz_new = (r * z).sum(0)
            p = z + torch.where(done, torch.zeros_like(rz), rz_new / rz) * p
            rz = rz_new
        res = torch.linalg.vector_norm(r, dim=0) / torch.linalg.vector_norm(b, dim=0)
        raise RuntimeError(f"EEQ conjugate gradients did not converge in {self.maxiter} "
                           f"iterations (relative residuals {res.tolist()})")

    def solve_augmented(self, top: Tensor, bottom: Tensor,
                        tol_abs: Optional[float] = None) -> Tuple[Tensor, Tensor]:
        """``[[A, 1], [1^T, 0]] [y; mu] = [top; bottom]`` by eliminating the constraint
        (eeq.py:325-331): ``y = A^-1 top - mu A^-1 1``; ``A^-1 1`` is solved with the first
        right-hand side, as a second column of the same iteration. ``tol_abs``: an absolute
        tolerance for ``top``'s solve (default ``tol |top|``)."""
        b = top.detach().to(torch.float64).reshape(-1)[self.order]
        tb = self.tol * float(torch.linalg.vector_norm(b)) if tol_abs is None else float(tol_abs)
        if self.y_ones is None:
            ones = torch.ones_like(b)
            tols = torch.tensor([tb, self.tol * math.sqrt(self.n)], dtype=torch.float64,
                                device=b.device)
            y = self.conjugate_gradient(torch.stack([b, ones], 1), tols)
            y1, self.y_ones = y[:, 0], y[:, 1].contiguous()
        else:
            y1 = self.conjugate_gradient(b[:, None], torch.tensor([tb], dtype=torch.float64,
                                                                   device=b.device))[:, 0]
        mu = (y1.sum() - bottom) / self.y_ones.sum()
        y = y1 - mu * self.y_ones
        out = torch.empty_like(y)
        out[self.order] = y
        return out, mu

    def apply(self, v: Tensor) -> Tensor:
        """``A v`` at the detached geometry, in the atoms' order."""
        y = self._matvec(v.detach().to(torch.float64)[self.order][:, None])[:, 0]
        out = torch.empty_like(y)
        out[self.order] = y
        return out

    def apply_live(self, pos: Tensor, cell: Optional[Tensor], v: Tensor) -> Tensor:
        """``A(pos, cell) v`` with derivatives in ``pos`` and ``cell`` (``v`` constant): the
        matrix-free real-space product and the reciprocal sum in recomputed blocks."""
        out = self.diag * v + real_apply_op(pos, cell, self.rad, v, None, self.alpha, self.cutoff)
        if cell is not None:
            g, w = reciprocal_weights(self.m, cell, self.alpha)
            out = out + reciprocal_apply(pos, g, w, v)
        return out


CHOLESKY_BLOCK = 128
#: row blocks of :func:`_add_gram` (the lower block triangle: 9/16 of the square at 8)
GRAM_PARTS = 8


def _add_gram(A: Tensor, X: Tensor, parts: int = GRAM_PARTS) -> None:
    """``A += X X^T`` for a symmetric ``A`` (N, N): each of ``parts`` block rows takes the
    product up to its diagonal block (library GEMMs over the lower block triangle), then
    the blocks above the diagonal are copied from their transposes below it."""
    n = A.shape[0]
    if n < 512 or parts <= 1:
        A.addmm_(X, X.t())
        return
    step = -(-n // parts)
    cuts = list(range(0, n, step)) + [n]
    for i in range(len(cuts) - 1):
        r0, r1 = cuts[i], cuts[i + 1]
        A[r0:r1, :r1].addmm_(X[r0:r1], X[:r1].t())
    for i in range(len(cuts) - 1):
        for j in range(i + 1, len(cuts) - 1):
            A[cuts[i]:cuts[i + 1], cuts[j]:cuts[j + 1]].copy_(
                A[cuts[j]:cuts[j + 1], cuts[i]:cuts[i + 1]].t())


def _cholesky(A: Tensor, keep_inverses: bool = False):
    """The Cholesky factor of the float64 operator and LAPACK's ``info`` (0, or the 1-based
    column of the first pivot that is not positive). On the device: right-looking blocked
    factorization, 128 columns at a time: ``xnn_eeq_cholesky_block`` factors the diagonal
    block in LDS and forms its inverse, the panel below it is ``A21 L11^-T`` and the
    trailing matrix takes ``- L21 L21^T`` (library GEMMs; a large trailing update is split
    at half height into the top rows' left square and the bottom rows, 3/4 of the square,
    and the upper triangle is discarded at the end). ``keep_inverses``: also return the
    diagonal blocks' inverses (block j at ``128 * 128 j``, row stride its size; None off
    the device) for :func:`_cholesky_solve`."""
    if not A.is_cuda:
        L, info = torch.linalg.cholesky_ex(A)
        return (L, info, None) if keep_inverses else (L, info)
    n, nb = A.shape[0], CHOLESKY_BLOCK
    L = A.contiguous().clone()
    info = torch.zeros(1, dtype=torch.int32, device=A.device)
    inv_all = torch.empty(max((n + nb - 1) // nb, 1) * nb * nb, dtype=torch.float64,
                          device=A.device)
    panel = torch.empty((max(n - nb, 0), nb), dtype=torch.float64, device=A.device)
    stream = _lib.stream(A.device)
    for k in range(0, n, nb):
        b = min(nb, n - k)
        inv = inv_all[(k // nb) * nb * nb:]
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
    return (L.tril_(), info[0], inv_all) if keep_inverses else (L.tril_(), info[0])


def _cholesky_solve(L: Tensor, inv_all: Tensor, b: Tensor) -> Tensor:
    """``(L L^T)^-1 b`` for ``b`` (N, k) on the device: forward and backward blocked
    substitution with the factor and its diagonal blocks' inverses, one launch per block
    and direction (``xnn_eeq_cholesky_solve``), two columns per pass."""
    n = L.shape[0]
    x = b.to(torch.float64).contiguous().clone()
    work = torch.empty((n, min(x.shape[1], 2)), dtype=torch.float64, device=L.device)
    stream = _lib.stream(L.device)
    for c in range(0, x.shape[1], 2):
        part = x[:, c:c + 2].contiguous()
        _lib.call("xnn_eeq_cholesky_solve", _lib.ptr(L), n, _lib.ptr(inv_all), _lib.ptr(part),
                  int(part.shape[1]), _lib.ptr(work), stream)
        x[:, c:c + 2] = part
    return x


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
                      eps: float = EWALD_EPS, solver: str = "auto") -> Tensor:
    """EEQ charges of one structure in the large regime (eeq.py:664-700): positions and
    cell in bohr (``cell`` None: a molecule), the charge widths ``rad``, the diagonal
    ``J + sqrt(2/pi) / a`` (the ``- 2 alpha / sqrt(pi)`` of a cell is added here), the
    right-hand side ``x`` and the total charge; ``cutoff_au`` the real-space range.
    ``solver``: ``"auto"`` (the factorized operator up to :data:`LU_MAX_ATOMS` atoms,
    conjugate gradients above, eeq.py:226), ``"lu"`` or ``"cg"``. Differentiable once in
    ``pos``, ``cell`` and ``x``."""
    if solver not in ("auto", "lu", "cg"):
        raise ValueError(f"solver must be 'auto', 'lu' or 'cg', got {solver!r}")
    periodic = cell is not None
    alpha = ewald_alpha(cutoff_au, eps) if periodic else 0.0
    if periodic:
        diag = diag - 2.0 * alpha / math.sqrt(math.pi)
    else:
        cutoff_au = math.inf            # a molecule: every pair (eeq.py:346-360), no split
    n = int(pos.shape[0])
    iterative = solver == "cg" or (solver == "auto" and n > LU_MAX_ATOMS)
    kind = IterativeEEQSystem if iterative else LargeEEQSystem
    system = kind(pos, cell, rad, diag, alpha, cutoff_au, eps)
    total = torch.as_tensor(float(total_charge), dtype=torch.float64, device=pos.device)
    with torch.no_grad():
        xd = x.detach().to(torch.float64)
        q0, mu0 = system.solve_augmented(xd, total)
        # the residual correction (zero at convergence) to the first solve's tolerance
        tol_abs = CG_TOL * float(torch.linalg.vector_norm(xd)) if iterative else None
        dq, dmu = system.solve_augmented(xd - system.apply(q0) - mu0, total - q0.sum(), tol_abs)
        q1, mu1 = q0 + dq, mu0 + dmu
    live = x.requires_grad or pos.requires_grad or (periodic and cell.requires_grad)
    if not (live and torch.is_grad_enabled()):
        return q1.to(x.dtype)
    top = x.to(torch.float64) - system.apply_live(pos.to(torch.float64),
                                                  None if cell is None else cell.to(torch.float64),
                                                  q1) - mu1
    bottom = total - q1.sum()
    return (q1 + _ConstantSolve.apply(system, top, bottom)).to(x.dtype)
