"""D4 and D3 dispersion on the GPU: the coordination numbers, the polarizabilities, the
two-body term (pair terms over lattice images) and the three-body ATM term (triangles of a
radius graph) as HIP kernels, the charge model in PyTorch.

Mirrors ``DFTD4`` / ``D4Dispersion`` (src/xnn/common/models/d4.py:266-1309,
dispersion.py:667-878) and ``DFTD3`` / ``D3Dispersion`` (d3.py:483-1011):

* coordination numbers (d4.py:552-591) -> :func:`d4_coordination` (HIP,
  differentiable once in positions and cell);
* EEQ charges (d4.py:593-723): the dense regime (molecular matrix and dftd4's Ewald sum
  over Wigner-Seitz images, PyTorch as in the reference) and the large regime of
  eeq.py:170-397, 664 (the converged Ewald operator: its real-space part and derivative
  as HIP kernels, :mod:`xnn_amd.eeq`), chosen as ``regime="auto"`` does (d4.py:846-851);
* charge-scaled Gaussian reference weights and alpha(i w) (d4.py:984-1042,
  dispersion.py:70-121) -> :func:`d4_polarizabilities_op` (HIP, one kernel each way:
  the alpha, d alpha / d cn and d alpha / d q of the reference's native d4_alpha);
* the BJ-damped two-body energy with the quintic switch (d4.py:1044-1071,
  dispersion.py:42-67) -> :func:`d4_two_body` (HIP; gradients to positions, cell and
  alpha, the outputs of the reference's native kernel run_d4);
* the ATM three-body energy (dispersion.py:124-222, 529-647; the reference's Triton
  kernels dispersion_fast/atm.py) -> :func:`atm_energy` (HIP; gradients to the edge
  vectors and the C6 factors), with C6 from the neutral-atom polarizabilities (D4) or the
  reference-weighted C6 rows (D3).

* the optional tail correction (``tail_correction=True``, d4.py:1073-1140, 1259-1267): the
  two-body energy of a homogeneous continuum beyond the pair cutoff, per atom.

Positions in Angstrom, energies returned in eV (hartree internally). The pair kernels walk every atom pair and lattice image within
the cutoffs and the ATM term builds its own radius graph at the three-body cutoff, so the
graph may be built at the wrapped model's own cutoff.
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import Dict, List, Optional, Tuple

import numpy as np
import torch
from torch import Tensor, nn

from . import _lib

BOHR = 0.5291772109044924        # Angstrom per bohr (dispersion.py:37)
HARTREE = 27.21138624593551      # eV per hartree
KCN, K4, K5, K6 = 7.5, 4.10451, 19.08857, 2.0 * 11.28174 ** 2      # d4.py:114-117
EEQ_CN_MAX, EEQ_CN_REG = 8.0, 1.0e-14
WS_TOL, EWALD_REP = 0.01, 2
PBE0_D4 = {"s6": 1.0, "s8": 1.20065498, "a1": 0.40085597, "a2": 5.02928789}
N_FREQ = 23
EEQ_REGIMES = ("auto", "dense", "large")
AUTO_LARGE_PERIODIC, AUTO_LARGE_MOLECULAR = 500, 6000     # d4.py:137-139
DEFAULT_CUTOFF_EEQ = 16.0                                 # Angstrom, d4.py:131-134
MIN_CUTOFF_EEQ_AU = 20.0                                  # bohr, d4.py:130
TABLE_KEYS = ("rcov", "en", "zeff", "hardness", "r4r2", "eeq_chi", "eeq_eta", "eeq_kcnchi",
              "eeq_rad", "nref", "ngw", "refcn", "refq", "refalpha")

_NS = "xnn_amd"


# --------------------------------------------------------------------------- formulas
def switching_function(r: Tensor, cutoff: float, width: float) -> Tensor:
    """The quintic smoothstep window of the pair and triple sums (dispersion.py:42-67).

    With ``t = (cutoff - r) / width`` clamped to [0, 1] the window is
    ``10 t^3 - 15 t^4 + 6 t^5``: one at and below ``cutoff - width``, zero at and beyond
    ``cutoff``, with vanishing first and second derivatives at both ends. A width above the
    cutoff is taken as the cutoff; a width of zero or less means no window (all ones). The
    pair kernels evaluate the same window per term together with its slope."""
    if width <= 0.0:
        return torch.ones_like(r)
    t = ((cutoff - r) / min(width, cutoff)).clamp(0.0, 1.0)
    return t * t * t * (t * (t * 6.0 - 15.0) + 10.0)


def gaussian_reference_weights(cn: Tensor, refcn: Tensor, valid: Tensor, wf: float,
                               ngw: Optional[Tensor] = None, eps_norm: float = 0.0,
                               n_gauss: Optional[int] = None) -> Tensor:
    """Weights of an atom's reference systems from its coordination number (D3 paper
    eq 16, D4 paper eq 8; dispersion.py:70-121).

    Reference ``r`` of an atom carries ``g_r = sum_{j=1..n_r} exp(-wf j (CN - CN_r)^2)``
    (``n_r = ngw[r]`` Gaussians for D4, a single one when ``ngw`` is None as in D3), and the
    weights are ``g_r / sum_r g_r`` over the atom's ``valid`` references. When that sum is
    at most ``eps_norm`` (the Gaussians underflow far from every reference) the weight goes
    to the reference(s) with the largest ``CN_r`` instead, in equal parts of one each.
    ``refcn``, ``valid`` and ``ngw`` are per-atom ``(N, R)`` tables; ``n_gauss`` bounds the
    Gaussians per reference (default: the largest ``ngw``). The D4 polarizability and D3
    weight kernels evaluate the same weights atom by atom."""
    d2 = torch.square(cn.unsqueeze(1) - refcn)
    counts = torch.ones_like(refcn, dtype=torch.long) if ngw is None else ngw
    n_max = 1 if ngw is None else (int(ngw.max()) if n_gauss is None else int(n_gauss))
    g = torch.zeros_like(d2)
    for j in range(1, n_max + 1):
        g = g + torch.exp(d2 * (-wf * j)) * (counts >= j).to(d2.dtype)
    g = g * valid.to(d2.dtype)
    total = g.sum(dim=1, keepdim=True)
    usable = total > eps_norm
    top = refcn.masked_fill(~valid, -math.inf).amax(dim=1, keepdim=True)
    largest = (valid & ((refcn - top).abs() < 1e-12)).to(d2.dtype)
    return torch.where(usable, g / torch.where(usable, total, torch.ones_like(total)), largest)


# --------------------------------------------------------------------------- tables# --------------------------------------------------------------------------- tables
def load_d4_tables(path: str) -> Dict[str, np.ndarray]:
    """Per-element D4 tables (index = atomic number) in the derived layout: ``rcov``
    (4/3-scaled covalent radii, bohr), ``en``, ``zeff``, ``hardness``, ``r4r2``
    (sqrt(0.5 <r4>/<r2> sqrt(Z))), ``eeq_chi/eta/kcnchi/rad``, ``nref`` (119,),
    ``ngw``, ``refcn``, ``refq`` (7, 119) and ``refalpha`` (23, 7, 119), the charge-scaled
    atom-in-molecule reference polarizabilities (d4.py:444-500)."""
    with np.load(path, allow_pickle=False) as f:
        missing = [k for k in TABLE_KEYS if k not in f.files]
        if missing:
            raise ValueError(f"{path}: missing D4 tables {missing}")
        return {k: np.asarray(f[k]) for k in TABLE_KEYS}


# --------------------------------------------------------------------------- HIP ops
def _workspace(n_nodes: int, n_graphs: int, max_atoms: int, device) -> Tuple[Optional[Tensor], int]:
    need = int(_lib.load().xnn_d4_workspace_bytes(n_nodes, n_graphs, max_atoms))
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=device) if need else None
    return ws, need


def _cn_params(cut_cn: float, cut_eeq: float) -> "_lib.D4CnParams":
    return _lib.D4CnParams(cut_cn, cut_eeq, KCN, K4, K5, K6)


def d4_plan(pos: Tensor, node_ptr: Tensor, cell: Optional[Tensor], images: Tensor) -> Tensor:
    """The tile plan of the D4 pair kernels for these positions (Angstrom, float64) and
    cells: each structure's atoms in the Morton order of a bin grid over their
    (fractional, when periodic) coordinates, and the first tile of each structure, as
    int32 device memory (``xnn_d4_plan``). Built once per evaluation and shared by the
    coordination-number and two-body kernels and their backwards."""
    dev = pos.device
    n, b = pos.shape[0], node_ptr.shape[0] - 1
    nbytes = int(_lib.load().xnn_d4_plan_bytes(n, b))
    plan = torch.empty((nbytes + 3) // 4, dtype=torch.int32, device=dev)
    _lib.call("xnn_d4_plan", _lib.ptr(pos), n, _lib.ptr(node_ptr), b, _lib.ptr(cell),
              _lib.ptr(images), _lib.ptr(plan), nbytes, _lib.stream(dev))
    return plan


@torch.library.custom_op(f"{_NS}::d4_coordination", mutates_args=())
def d4_coordination_op(pos: Tensor, cell: Optional[Tensor], species: Tensor, batch32: Tensor,
                       node_ptr: Tensor, images: Tensor, plan: Optional[Tensor], rcov: Tensor,
                       en: Tensor, cutoffs: List[float], max_atoms: int) -> Tuple[Tensor, Tensor]:
    """``(cn_d4, cn_raw)``: the EN-weighted erf-count CN within ``cutoffs[0]`` and the
    plain erf count within ``cutoffs[1]`` (bohr), float64 (d4.py:552-588). ``plan`` from
    :func:`d4_plan` (None: built in the call)."""
    dev = pos.device
    n, b = pos.shape[0], node_ptr.shape[0] - 1
    cn = torch.empty(n, dtype=torch.float64, device=dev)
    raw = torch.empty(n, dtype=torch.float64, device=dev)
    ws, need = _workspace(n, b, max_atoms, dev)
    prm = _cn_params(cutoffs[0], cutoffs[1])
    _lib.call("xnn_d4_coordination", _lib.ptr(pos), n, _lib.ptr(species), _lib.ptr(batch32),
              _lib.ptr(node_ptr), b, max_atoms, _lib.ptr(cell), _lib.ptr(images), _lib.ptr(plan),
              _lib.ptr(rcov), _lib.ptr(en), prm, _lib.ptr(cn), _lib.ptr(raw), _lib.ptr(ws), need,
              _lib.stream(dev))
    return cn, raw


@d4_coordination_op.register_fake
def _(pos, cell, species, batch32, node_ptr, images, plan, rcov, en, cutoffs, max_atoms):
    n = pos.shape[0]
    return pos.new_empty(n), pos.new_empty(n)


def _cn_setup(ctx, inputs, output):
    pos, cell, species, batch32, node_ptr, images, plan, rcov, en, cutoffs, max_atoms = inputs
    ctx.save_for_backward(pos, cell, species, batch32, node_ptr, images, plan, rcov, en)
    ctx.cutoffs, ctx.max_atoms = list(cutoffs), max_atoms


def _cn_backward(ctx, g_cn, g_raw):
    if torch.is_grad_enabled():
        raise RuntimeError("the D4 kernels are differentiable once (forces and stress); a "
                           "second derivative through the dispersion term has no GPU path")
    pos, cell, species, batch32, node_ptr, images, plan, rcov, en = ctx.saved_tensors
    dev, n, b = pos.device, pos.shape[0], node_ptr.shape[0] - 1
    grad_pos = torch.empty((n, 3), dtype=torch.float64, device=dev)
    want_cell = cell is not None and ctx.needs_input_grad[1]
    part = torch.empty((n, 9), dtype=torch.float64, device=dev) if want_cell else None
    ws, need = _workspace(n, b, ctx.max_atoms, dev)
    g_cn = None if g_cn is None else g_cn.contiguous()
    g_raw = None if g_raw is None else g_raw.contiguous()
    _lib.call("xnn_d4_coordination_backward", _lib.ptr(pos), n, _lib.ptr(species),
              _lib.ptr(batch32), _lib.ptr(node_ptr), b, ctx.max_atoms, _lib.ptr(cell),
              _lib.ptr(images), _lib.ptr(plan), _lib.ptr(rcov), _lib.ptr(en),
              _cn_params(ctx.cutoffs[0], ctx.cutoffs[1]), _lib.ptr(g_cn), _lib.ptr(g_raw),
              _lib.ptr(grad_pos), _lib.ptr(part), _lib.ptr(ws), need, _lib.stream(dev))
    grad_cell = _cell_grad(part, node_ptr, b) if want_cell else None
    return grad_pos, grad_cell, None, None, None, None, None, None, None, None, None


d4_coordination_op.register_autograd(_cn_backward, setup_context=_cn_setup)


def _cell_grad(part: Tensor, node_ptr: Tensor, n_graphs: int) -> Tensor:
    out = torch.empty((n_graphs, 9), dtype=torch.float64, device=part.device)
    _lib.segment_reduce_f64(part, part.shape[0], 9, node_ptr, n_graphs, out)
    return out.view(n_graphs, 3, 3)


@torch.library.custom_op(f"{_NS}::d4_two_body", mutates_args=())
def d4_two_body_op(pos: Tensor, cell: Optional[Tensor], alpha: Tensor, species: Tensor,
                   batch32: Tensor, node_ptr: Tensor, images: Tensor, plan: Optional[Tensor],
                   r4r2: Tensor, params: List[float], max_atoms: int) -> Tensor:
    """Per-atom BJ-damped two-body energy (hartree): half of every pair image within
    ``params[4]`` bohr to each of its atoms, ``params = [s6, s8, a1, a2, cutoff, width]``
    (d4.py:1048-1071). ``plan`` from :func:`d4_plan` (None: built in the call)."""
    dev = pos.device
    n, b = pos.shape[0], node_ptr.shape[0] - 1
    e2 = torch.empty(n, dtype=torch.float64, device=dev)
    ws, need = _workspace(n, b, max_atoms, dev)
    _lib.call("xnn_d4_two_body", _lib.ptr(pos), n, _lib.ptr(species), _lib.ptr(batch32),
              _lib.ptr(node_ptr), b, max_atoms, _lib.ptr(cell), _lib.ptr(images), _lib.ptr(plan),
              _lib.ptr(r4r2), _lib.ptr(alpha), _lib.D4PairParams(*params), _lib.ptr(e2),
              _lib.ptr(ws), need, _lib.stream(dev))
    return e2


@d4_two_body_op.register_fake
def _(pos, cell, alpha, species, batch32, node_ptr, images, plan, r4r2, params, max_atoms):
    return pos.new_empty(pos.shape[0])


def _pair_setup(ctx, inputs, output):
    pos, cell, alpha, species, batch32, node_ptr, images, plan, r4r2, params, max_atoms = inputs
    ctx.save_for_backward(pos, cell, alpha, species, batch32, node_ptr, images, plan, r4r2)
    ctx.params, ctx.max_atoms = list(params), max_atoms


def _pair_backward(ctx, g_e2):
    if torch.is_grad_enabled():
        raise RuntimeError("the D4 kernels are differentiable once (forces and stress); a "
                           "second derivative through the dispersion term has no GPU path")
    pos, cell, alpha, species, batch32, node_ptr, images, plan, r4r2 = ctx.saved_tensors
    dev, n, b = pos.device, pos.shape[0], node_ptr.shape[0] - 1
    grad_pos = torch.empty((n, 3), dtype=torch.float64, device=dev)
    want_cell = cell is not None and ctx.needs_input_grad[1]
    part = torch.empty((n, 9), dtype=torch.float64, device=dev) if want_cell else None
    grad_alpha = torch.empty_like(alpha) if ctx.needs_input_grad[2] else None
    ws, need = _workspace(n, b, ctx.max_atoms, dev)
    _lib.call("xnn_d4_two_body_backward", _lib.ptr(pos), n, _lib.ptr(species), _lib.ptr(batch32),
              _lib.ptr(node_ptr), b, ctx.max_atoms, _lib.ptr(cell), _lib.ptr(images),
              _lib.ptr(plan), _lib.ptr(r4r2), _lib.ptr(alpha), _lib.D4PairParams(*ctx.params),
              _lib.ptr(g_e2.contiguous()), _lib.ptr(grad_pos), _lib.ptr(part),
              _lib.ptr(grad_alpha), _lib.ptr(ws), need, _lib.stream(dev))
    grad_cell = _cell_grad(part, node_ptr, b) if want_cell else None
    return grad_pos, grad_cell, grad_alpha, None, None, None, None, None, None, None, None


d4_two_body_op.register_autograd(_pair_backward, setup_context=_pair_setup)


def _structure_once() -> None:
    """The one-launch structure energies hold their gradients as constants: a backward
    recorded for a second derivative would drop the Hessian, so it is refused."""
    if torch.is_grad_enabled():
        raise RuntimeError("the per-structure dispersion energies of one backward launch are "
                           "differentiable once (forces and stress)")


class TwoBodyStructureEnergy(torch.autograd.Function):
    """The two-body energies per structure (B,) and, detached, per atom (N,), with their
    gradients, from one launch of the pair backward at unit seeds, as the reference's native
    kernel returns energy and gradient together (``run_d4``, dispersion_fast/cpu.py:834-935).

    The energy is bilinear in the polarizabilities (C6_ij = sum_w cp3(w) alpha_i(w)
    alpha_j(w), the damping and the switch do not depend on them), and every pair gives half
    to each of its atoms, so an atom's share is e_i = 1/2 sum_w alpha_i(w) dE/dalpha_i(w) with
    dE/dalpha at unit seeds: the energy-only pair kernel is not needed. The backward scales
    the stored gradients by each structure's seed, exact for any seed on the per-structure
    energies; the per-atom energies carry no gradient."""

    @staticmethod
    def forward(ctx, pos, cell, alpha, species, batch32, node_ptr, images, plan, r4r2, params,
                max_atoms):
        dev, n, b = pos.device, pos.shape[0], node_ptr.shape[0] - 1
        grad_pos = torch.empty((n, 3), dtype=torch.float64, device=dev)
        part = torch.empty((n, 9), dtype=torch.float64, device=dev) if cell is not None else None
        grad_alpha = torch.empty_like(alpha)
        ones = torch.ones(n, dtype=torch.float64, device=dev)
        ws, need = _workspace(n, b, max_atoms, dev)
        _lib.call("xnn_d4_two_body_backward", _lib.ptr(pos), n, _lib.ptr(species),
                  _lib.ptr(batch32), _lib.ptr(node_ptr), b, max_atoms, _lib.ptr(cell),
                  _lib.ptr(images), _lib.ptr(plan), _lib.ptr(r4r2), _lib.ptr(alpha),
                  _lib.D4PairParams(*params), _lib.ptr(ones), _lib.ptr(grad_pos), _lib.ptr(part),
                  _lib.ptr(grad_alpha), _lib.ptr(ws), need, _lib.stream(dev))
        from .ops import structure_sum_op
        e2 = 0.5 * (alpha * grad_alpha).sum(1)
        e2_b = structure_sum_op(e2, node_ptr, batch32)
        ctx.save_for_backward(batch32, node_ptr, grad_pos, part, grad_alpha)
        ctx.mark_non_differentiable(e2)
        return e2_b, e2

    @staticmethod
    def backward(ctx, g_b, _g_e2):
        _structure_once()
        batch32, node_ptr, grad_pos, part, grad_alpha = ctx.saved_tensors
        gs = g_b.index_select(0, batch32.long())[:, None]   # each atom's structure seed
        g_pos = grad_pos * gs if ctx.needs_input_grad[0] else None
        g_cell = None
        if part is not None and ctx.needs_input_grad[1]:
            g_cell = _cell_grad(part, node_ptr, g_b.shape[0]) * g_b[:, None, None]
        g_alpha = grad_alpha * gs if ctx.needs_input_grad[2] else None
        return g_pos, g_cell, g_alpha, None, None, None, None, None, None, None, None


def _alpha_tables(nref, ngw, refcn, refq, zeff, gi, refalpha, ga: float,
                  wf: float) -> "_lib.D4AlphaTables":
    return _lib.D4AlphaTables(nref.shape[0], _lib.ptr(nref), _lib.ptr(ngw), _lib.ptr(refcn),
                              _lib.ptr(refq), _lib.ptr(zeff), _lib.ptr(gi), _lib.ptr(refalpha),
                              ga, wf)


@torch.library.custom_op(f"{_NS}::d4_polarizabilities", mutates_args=())
def d4_polarizabilities_op(z: Tensor, cn: Tensor, q: Tensor, nref: Tensor, ngw: Tensor,
                           refcn: Tensor, refq: Tensor, zeff: Tensor, gi: Tensor,
                           refalpha: Tensor, ga: float, wf: float) -> Tensor:
    """alpha(i w) (N, 23) at the coordination numbers ``cn`` and charges ``q``: the
    charge-scaled Gaussian reference weights contracted with the reference
    polarizabilities in one HIP kernel (d4.py:984-1042; the reference's native d4_alpha,
    dispersion_fast/cpu.py:774-829). Tables indexed by atomic number, in the kernel's
    layout (see ``DFTD4``); differentiable once in ``cn`` and ``q``."""
    n = cn.shape[0]
    alpha = torch.empty((n, N_FREQ), dtype=torch.float64, device=cn.device)
    _lib.call("xnn_d4_polarizabilities", n, _lib.ptr(z), _lib.ptr(cn), _lib.ptr(q),
              _alpha_tables(nref, ngw, refcn, refq, zeff, gi, refalpha, ga, wf),
              _lib.ptr(alpha), _lib.stream(cn.device))
    return alpha


@d4_polarizabilities_op.register_fake
def _(z, cn, q, nref, ngw, refcn, refq, zeff, gi, refalpha, ga, wf):
    return cn.new_empty((cn.shape[0], N_FREQ))


def _alpha_setup(ctx, inputs, output):
    z, cn, q, nref, ngw, refcn, refq, zeff, gi, refalpha, ga, wf = inputs
    ctx.save_for_backward(z, cn, q, nref, ngw, refcn, refq, zeff, gi, refalpha)
    ctx.ga, ctx.wf = ga, wf


def _alpha_backward(ctx, g_alpha):
    if torch.is_grad_enabled():
        raise RuntimeError("the D4 kernels are differentiable once (forces and stress); a "
                           "second derivative through the dispersion term has no GPU path")
    z, cn, q, nref, ngw, refcn, refq, zeff, gi, refalpha = ctx.saved_tensors
    n = cn.shape[0]
    g_cn = torch.empty_like(cn) if ctx.needs_input_grad[1] else None
    g_q = torch.empty_like(q) if ctx.needs_input_grad[2] else None
    if g_cn is not None or g_q is not None:
        _lib.call("xnn_d4_polarizabilities_backward", n, _lib.ptr(z), _lib.ptr(cn), _lib.ptr(q),
                  _alpha_tables(nref, ngw, refcn, refq, zeff, gi, refalpha, ctx.ga, ctx.wf),
                  _lib.ptr(g_alpha.contiguous()), _lib.ptr(g_cn), _lib.ptr(g_q),
                  _lib.stream(cn.device))
    return (None, g_cn, g_q) + (None,) * 9


d4_polarizabilities_op.register_autograd(_alpha_backward, setup_context=_alpha_setup)


# --------------------------------------------------------------------------- ATM
@dataclass
class ATMConstants:
    """The scalars and tables of one ATM term (dispersion_fast/atm.py:355-363): per-atom
    ``species`` (N,) indexing the ``table`` (S, S) of damping-radius pair factors (the
    triangle's R0 is the product of its three), ``s9``, the exponent ``alp3``, the
    three-body ``cutoff`` and switching ``width`` (bohr; <= 0: sharp)."""

    species: Tensor
    table: Tensor
    s9: float
    alp3: float
    cutoff: float
    width: float


def atm_plan(edge_index: Tensor, n_atoms: int) -> Tuple[Tensor, List[int]]:
    """The triplet plan of an edge list on the GPU (dispersion_fast/atm.py:318-352): the
    edges sorted by (center, neighbor) with the per-center ranges, as an opaque byte
    tensor, and ``[tiles, has_repeats]`` (the busiest center's tiles of 64 edges to
    larger-index neighbors; whether some center has repeated-atom triangles). One small
    synchronous device-to-host copy."""
    dev = edge_index.device
    ei = edge_index.to(torch.long).contiguous()
    n_edges = int(ei.shape[1])
    nbytes = ctypes.c_size_t()
    _lib.call("xnn_atm_plan_size", n_edges, int(n_atoms), ctypes.byref(nbytes))
    plan = torch.empty(max(int(nbytes.value), 1), dtype=torch.uint8, device=dev)
    info = (ctypes.c_int64 * 2)()
    _lib.call("xnn_atm_plan", _lib.ptr(ei), n_edges, int(n_atoms), _lib.ptr(plan),
              int(nbytes.value), info, _lib.stream(dev))
    return plan, [int(info[0]), int(info[1])]


def _atm_work(n_edges: int, n_atoms: int, k: int, backward: bool, dev) -> Tensor:
    nbytes = ctypes.c_size_t()
    _lib.call("xnn_atm_work_size", n_edges, n_atoms, k, int(backward), ctypes.byref(nbytes))
    return torch.empty(max(int(nbytes.value), 1), dtype=torch.uint8, device=dev)


def _atm_params(p: List[float]) -> "_lib.AtmParams":
    return _lib.AtmParams(float(p[0]), float(p[1]), float(p[2]), float(p[3]))


@torch.library.custom_op(f"{_NS}::atm_energy", mutates_args=())
def atm_energy_op(plan: Tensor, edge_vec: Tensor, feat_a: Tensor, feat_b: Tensor,
                  species: Tensor, table: Tensor, params: List[float], n_atoms: int,
                  max_tiles: int, has_repeats: int) -> Tensor:
    """Per-atom ATM energies (N,) in hartree over the planned edges (bohr vectors, input
    order), pair C6 = <feat_a[x], feat_b[y]>, ``params`` = [s9, alp3, cutoff, width];
    differentiable twice in ``edge_vec``, ``feat_a`` and ``feat_b`` (the gradient is
    :func:`atm_energy_grad_op`, itself differentiable)."""
    dev = edge_vec.device
    n_edges, k = int(edge_vec.shape[0]), int(feat_a.shape[1])
    energy = torch.empty(n_atoms, dtype=torch.float64, device=dev)
    work = _atm_work(n_edges, n_atoms, k, False, dev)
    _lib.call("xnn_atm_energy", _lib.ptr(plan), n_edges, n_atoms, max_tiles, has_repeats,
              _lib.ptr(edge_vec), _lib.ptr(feat_a), _lib.ptr(feat_b), k, _lib.ptr(species),
              _lib.ptr(table), int(table.shape[0]), _atm_params(params), _lib.ptr(energy),
              _lib.ptr(work), work.numel(), _lib.stream(dev))
    return energy


@atm_energy_op.register_fake
def _(plan, edge_vec, feat_a, feat_b, species, table, params, n_atoms, max_tiles, has_repeats):
    return edge_vec.new_empty(n_atoms)


def _atm_setup(ctx, inputs, output):
    plan, edge_vec, feat_a, feat_b, species, table, params, n_atoms, max_tiles, has_repeats = inputs
    ctx.save_for_backward(plan, edge_vec, feat_a, feat_b, species, table)
    ctx.meta = (list(params), n_atoms, max_tiles, has_repeats)


def _atm_backward(ctx, g_energy):
    plan, vec, fa, fb, species, table = ctx.saved_tensors
    params, n_atoms, max_tiles, has_repeats = ctx.meta
    g_vec, g_fa, g_fb = atm_energy_grad_op(plan, vec, fa, fb, g_energy.to(torch.float64),
                                           species, table, params, n_atoms, max_tiles,
                                           has_repeats)
    need = ctx.needs_input_grad
    return (None, g_vec if need[1] else None, g_fa if need[2] else None,
            g_fb if need[3] else None) + (None,) * 6


@torch.library.custom_op(f"{_NS}::atm_energy_grad", mutates_args=())
def atm_energy_grad_op(plan: Tensor, edge_vec: Tensor, feat_a: Tensor, feat_b: Tensor,
                       grad_energy: Tensor, species: Tensor, table: Tensor, params: List[float],
                       n_atoms: int, max_tiles: int,
                       has_repeats: int) -> Tuple[Tensor, Tensor, Tensor]:
    """The gradients of ``sum_i grad_energy[i] E_i`` in the edge vectors and both factor
    matrices (dispersion_fast/atm.py:413-443). Differentiable once more: its Jacobian in
    the first three inputs is the (symmetric) Hessian of that sum, so its backward is the
    Hessian times the incoming cotangents, and in ``grad_energy`` the energies' derivative
    along them (xnn_atm_energy_backward_tangent, atm.py:475-509)."""
    dev = edge_vec.device
    n_edges, k = int(edge_vec.shape[0]), int(feat_a.shape[1])
    g_vec = torch.empty_like(edge_vec)
    g_fa = torch.empty_like(feat_a)
    g_fb = torch.empty_like(feat_b)
    work = _atm_work(n_edges, n_atoms, k, True, dev)
    _lib.call("xnn_atm_energy_backward", _lib.ptr(plan), n_edges, n_atoms, max_tiles,
              has_repeats, _lib.ptr(edge_vec), _lib.ptr(feat_a), _lib.ptr(feat_b), k,
              _lib.ptr(species), _lib.ptr(table), int(table.shape[0]), _atm_params(params),
              _lib.ptr(grad_energy.contiguous()), _lib.ptr(g_vec), _lib.ptr(g_fa),
              _lib.ptr(g_fb), _lib.ptr(work), work.numel(), _lib.stream(dev))
    return g_vec, g_fa, g_fb


@atm_energy_grad_op.register_fake
def _(plan, edge_vec, feat_a, feat_b, grad_energy, species, table, params, n_atoms, max_tiles,
      has_repeats):
    return torch.empty_like(edge_vec), torch.empty_like(feat_a), torch.empty_like(feat_b)


def _atm_grad_setup(ctx, inputs, output):
    plan, vec, fa, fb, go, species, table, params, n_atoms, max_tiles, has_repeats = inputs
    ctx.save_for_backward(plan, vec, fa, fb, go, species, table)
    ctx.meta = (list(params), n_atoms, max_tiles, has_repeats)


def _atm_grad_backward(ctx, u_vec, u_fa, u_fb):
    if torch.is_grad_enabled():
        raise RuntimeError("the ATM kernels are differentiable twice (forces, stress and their "
                           "derivatives); a third derivative has no GPU path")
    plan, vec, fa, fb, go, species, table = ctx.saved_tensors
    params, n_atoms, max_tiles, has_repeats = ctx.meta
    dev = vec.device
    n_edges, k = int(vec.shape[0]), int(fa.shape[1])
    # an output that reached no loss has no cotangent: a zero direction
    dirs = [torch.zeros_like(x) if u is None else u.to(torch.float64).contiguous()
            for x, u in ((vec, u_vec), (fa, u_fa), (fb, u_fb))]
    energy_t = torch.empty(n_atoms, dtype=torch.float64, device=dev)
    h_vec, h_fa, h_fb = (torch.empty_like(x) for x in (vec, fa, fb))
    nbytes = ctypes.c_size_t()
    _lib.call("xnn_atm_tangent_work_size", n_edges, n_atoms, k, ctypes.byref(nbytes))
    work = torch.empty(max(int(nbytes.value), 1), dtype=torch.uint8, device=dev)
    _lib.call("xnn_atm_energy_backward_tangent", _lib.ptr(plan), n_edges, n_atoms, max_tiles,
              has_repeats, _lib.ptr(vec), _lib.ptr(fa), _lib.ptr(fb), k, _lib.ptr(species),
              _lib.ptr(table), int(table.shape[0]), _atm_params(params),
              _lib.ptr(go.contiguous()), _lib.ptr(dirs[0]), _lib.ptr(dirs[1]),
              _lib.ptr(dirs[2]), _lib.ptr(energy_t), _lib.ptr(h_vec), _lib.ptr(h_fa),
              _lib.ptr(h_fb), _lib.ptr(work), work.numel(), _lib.stream(dev))
    need = ctx.needs_input_grad
    return (None, h_vec if need[1] else None, h_fa if need[2] else None,
            h_fb if need[3] else None, energy_t.to(go.dtype) if need[4] else None) + (None,) * 6


atm_energy_grad_op.register_autograd(_atm_grad_backward, setup_context=_atm_grad_setup)


atm_energy_op.register_autograd(_atm_backward, setup_context=_atm_setup)


def atm_energy(edge_index: Tensor, edge_vec: Tensor, feat_a: Tensor, feat_b: Tensor,
               consts: ATMConstants, n_atoms: int) -> Tensor:
    """Per-atom ATM energies (N,) in hartree with the HIP kernels
    (dispersion_fast/atm.py:512-535): ``edge_index`` (2, E) ``[src, dst]`` within the
    three-body cutoff, both directions of every pair; ``edge_vec`` (E, 3) in bohr;
    ``feat_a``, ``feat_b`` (N, K <= 32) with pair C6 = <feat_a[x], feat_b[y]> (may be the
    same tensor). Differentiable twice in ``edge_vec``, ``feat_a`` and ``feat_b`` (forces,
    stress, and the second derivatives of a force loss); float64 throughout; GPU only."""
    if not edge_vec.is_cuda:
        raise RuntimeError("xnn_amd ATM runs on the GPU (HIP kernels); there is no CPU path")
    plan, info = atm_plan(edge_index, n_atoms)
    f64 = torch.float64
    return atm_energy_op(plan, edge_vec.to(f64).contiguous(), feat_a.to(f64).contiguous(),
                         feat_b.to(f64).contiguous(),
                         consts.species.to(device=edge_vec.device, dtype=torch.int32).contiguous(),
                         consts.table.to(device=edge_vec.device, dtype=f64).contiguous(),
                         [float(consts.s9), float(consts.alp3), float(consts.cutoff),
                          float(consts.width)], int(n_atoms), info[0], info[1])


class ATMStructureEnergy(torch.autograd.Function):
    """ATM energies per structure (B,) and, detached, per atom (N,), with their gradients,
    from one launch of the ATM backward at unit seeds (no energy launch).

    A triangle's energy goes with C9 = sqrt(C6_ij C6_jk C6_ik), each pair C6 bilinear in the
    features, so it is homogeneous of degree one in each member atom's features (both
    operands scaled together): an atom's share is e_i = 1/3 (feat_a_i . dE/dfeat_a_i +
    feat_b_i . dE/dfeat_b_i) at unit seeds, and the structure total is their sum. The
    backward scales the stored gradients by the structure seeds (an edge's by the seed of
    its structure), exact for any seed on the per-structure energies."""

    @staticmethod
    def forward(ctx, plan, edge_vec, feat_a, feat_b, species, table, params, n_atoms, max_tiles,
                has_repeats, edge_graph, node_ptr, batch32):
        dev = edge_vec.device
        n_edges, k = int(edge_vec.shape[0]), int(feat_a.shape[1])
        g_vec = torch.empty_like(edge_vec)
        g_fa = torch.empty_like(feat_a)
        g_fb = torch.empty_like(feat_b)
        ones = torch.ones(n_atoms, dtype=torch.float64, device=dev)
        work = _atm_work(n_edges, n_atoms, k, True, dev)
        _lib.call("xnn_atm_energy_backward", _lib.ptr(plan), n_edges, n_atoms, max_tiles,
                  has_repeats, _lib.ptr(edge_vec), _lib.ptr(feat_a), _lib.ptr(feat_b), k,
                  _lib.ptr(species), _lib.ptr(table), int(table.shape[0]), _atm_params(params),
                  _lib.ptr(ones), _lib.ptr(g_vec), _lib.ptr(g_fa), _lib.ptr(g_fb),
                  _lib.ptr(work), work.numel(), _lib.stream(dev))
        from .ops import structure_sum_op
        e = ((feat_a * g_fa).sum(1) + (feat_b * g_fb).sum(1)) / 3.0
        e_b = structure_sum_op(e, node_ptr, batch32)
        ctx.save_for_backward(g_vec, g_fa, g_fb, edge_graph, batch32)
        ctx.mark_non_differentiable(e)
        return e_b, e

    @staticmethod
    def backward(ctx, g_b, _g_e):
        _structure_once()
        g_vec, g_fa, g_fb, edge_graph, batch32 = ctx.saved_tensors
        ga = g_b.index_select(0, batch32.long())[:, None]
        need = ctx.needs_input_grad
        gv = g_vec * g_b.index_select(0, edge_graph)[:, None] if need[1] else None
        return (None, gv, g_fa * ga if need[2] else None, g_fb * ga if need[3] else None) + \
            (None,) * 9


def atm_structure_energy(edge_index: Tensor, edge_vec: Tensor, feat_a: Tensor, feat_b: Tensor,
                         consts: ATMConstants, node_ptr: Tensor,
                         batch32: Tensor) -> Tuple[Tensor, Tensor]:
    """ATM energies per structure (B,) with gradients and per atom (N,) detached, from one
    launch of the ATM backward (:class:`ATMStructureEnergy`); arguments as
    :func:`atm_energy`, plus the structures' atom ranges ``node_ptr`` (B + 1) and each atom's
    structure ``batch32`` (N,). For forces and stress from the structure energies."""
    if not edge_vec.is_cuda:
        raise RuntimeError("xnn_amd ATM runs on the GPU (HIP kernels); there is no CPU path")
    n_atoms = int(batch32.shape[0])
    plan, info = atm_plan(edge_index, n_atoms)
    f64 = torch.float64
    dev = edge_vec.device
    edge_graph = batch32.to(dev).long().index_select(0, edge_index[0].to(dev).long())
    return ATMStructureEnergy.apply(
        plan, edge_vec.to(f64).contiguous(), feat_a.to(f64).contiguous(),
        feat_b.to(f64).contiguous(), consts.species.to(device=dev, dtype=torch.int32).contiguous(),
        consts.table.to(device=dev, dtype=f64).contiguous(),
        [float(consts.s9), float(consts.alp3), float(consts.cutoff), float(consts.width)],
        n_atoms, info[0], info[1], edge_graph, node_ptr, batch32)


def _ewald_rows(i0: int, i1: int, a: float, pos: Tensor, cell: Tensor, vol: Tensor,
                recip: Tensor, rad: Tensor) -> Tensor:
    """Rows i0..i1 of the off-diagonal Ewald EEQ matrix (d4.py:608-680), see
    ``DFTD4._coulomb_periodic``."""
    n, dev, dt = pos.shape[0], pos.device, pos.dtype
    one = torch.arange(-1, 2, device=dev)
    t27 = torch.cartesian_prod(one, one, one).to(dt) @ cell
    two = torch.arange(-EWALD_REP, EWALD_REP + 1, device=dev)
    grid = torch.cartesian_prod(two, two, two)
    t125 = grid.to(dt) @ cell
    g = grid[(grid != 0).any(1)].to(dt) @ recip
    g2 = (g * g).sum(-1)
    gfac = 4.0 * math.pi / vol * torch.exp(-0.25 * g2 / (a * a)) / g2
    m = i1 - i0
    gamma = torch.rsqrt(rad[i0:i1, None] ** 2 + rad[None, :] ** 2)
    d = pos[None, :, :] - pos[i0:i1, None, :]
    d = d - torch.round(d.detach() @ torch.linalg.inv(cell.detach())) @ cell
    dimg = d[:, :, None, :] + t27[None, None]
    r2 = (dimg * dimg).sum(-1)
    thr = 1.4901161193847656e-08
    r2 = torch.where(r2 < thr, torch.full_like(r2, math.inf), r2)
    sel = (r2 - r2.min(-1, keepdim=True).values) <= WS_TOL
    nimg = sel.sum(-1).to(dt)
    ii, jj, kk = torch.nonzero(sel, as_tuple=True)
    vec = dimg[ii, jj, kk]
    vt = vec[:, None, :] + t125[None]
    rt2 = (vt * vt).sum(-1)
    keep = rt2 >= thr * thr
    rs = torch.sqrt(torch.where(keep, rt2, torch.ones_like(rt2)))
    kern = (torch.erf(gamma[ii, jj][:, None] * rs) - torch.erf(a * rs)) / rs
    adir = torch.where(keep, kern, torch.zeros_like(kern)).sum(-1)
    arec = (torch.cos(vec @ g.t()) * gfac[None]).sum(-1)
    return torch.zeros(m * n, dtype=dt, device=dev).index_add(
        0, ii * n + jj, (adir + arec) / nimg[ii, jj]).view(m, n)


# --------------------------------------------------------------------------- host pieces
def image_counts(cell: Tensor, pbc: Optional[Tensor], cutoff_aa: float) -> Tensor:
    """Translations per axis that cover ``cutoff_aa``: ceil(cutoff / interplanar spacing),
    the spacing of axis c being the cell volume over |a_(c+1) x a_(c+2)| (the image range
    of neighborlist.py:74-104). (B, 3) int32 on the cell's device; 0 on non-periodic axes
    and for an all-zero cell. On the GPU one HIP launch (``xnn_d4_image_counts``) and no
    host synchronization."""
    c = cell.detach().reshape(-1, 3, 3).to(torch.float64).contiguous()
    if c.is_cuda:
        out = torch.empty((c.shape[0], 3), dtype=torch.int32, device=c.device)
        flags = None if pbc is None else _pbc_flags(pbc, c.device)
        _lib.call("xnn_d4_image_counts", _lib.ptr(c), _lib.ptr(flags), c.shape[0],
                  float(cutoff_aa), _lib.ptr(out), _lib.stream(c.device))
        return out
    a0, a1, a2 = c[:, 0], c[:, 1], c[:, 2]
    x = torch.stack([torch.cross(a1, a2, dim=-1), torch.cross(a2, a0, dim=-1),
                     torch.cross(a0, a1, dim=-1)], dim=1)
    vol = (a0 * x[:, 0]).sum(-1).abs()
    norm = torch.linalg.norm(x, dim=-1)
    live = (c.abs().sum((1, 2)) > 1e-8)[:, None] & (norm > 0) & (vol[:, None] > 0)
    if pbc is not None:
        live = live & pbc.reshape(-1, 3).to(torch.bool)
    n = torch.ceil(cutoff_aa * norm / torch.where(live, vol[:, None], torch.ones_like(norm)))
    return torch.where(live, n.clamp(0.0, 32767.0), torch.zeros_like(n)).to(torch.int32)


_PBC: Dict[Tuple, Tensor] = {}


def _pbc_flags(pbc: Tensor, dev) -> Tensor:
    """pbc as (B, 3) uint8 on ``dev``; a host tensor is moved once per distinct value."""
    if pbc.is_cuda:
        return pbc.reshape(-1, 3).to(device=dev, dtype=torch.uint8).contiguous()
    key = (tuple(bool(v) for v in pbc.reshape(-1).tolist()), str(dev))
    hit = _PBC.get(key)
    if hit is None:
        if len(_PBC) >= 64:
            _PBC.clear()
        hit = _PBC[key] = pbc.reshape(-1, 3).to(torch.uint8).to(dev)
    return hit


_LAYOUTS: Dict[Tuple, Tuple[Tensor, Tensor]] = {}


def _batch_tensors(counts: List[int], dev) -> Tuple[Tensor, Tensor]:
    """node_ptr (B+1) int64 and batch (N) int32 of structures of these sizes on ``dev``,
    built once per layout (no host synchronization after the first call)."""
    key = (tuple(counts), str(dev))
    hit = _LAYOUTS.get(key)
    if hit is None:
        node_ptr = torch.tensor(np.concatenate([[0], np.cumsum(counts)]), dtype=torch.int64)
        batch32 = torch.repeat_interleave(torch.arange(len(counts), dtype=torch.int32),
                                          torch.tensor(counts, dtype=torch.int64))
        if len(_LAYOUTS) >= 64:
            _LAYOUTS.clear()
        hit = _LAYOUTS[key] = (node_ptr.to(dev), batch32.to(dev))
    return hit


def _ewald_alpha(rlen: float, dlen: float, vol: float) -> float:
    """Ewald splitting parameter balancing the decay of the +-2 real and reciprocal
    windows (the upstream search of d4.py:183-224: doubling from 1e-8, then bisection to
    sqrt(eps); 0.25 when the search fails)."""
    def rec(g, a):
        return 4.0 * math.pi * math.exp(-0.25 * g * g / (a * a)) / (vol * g * g)

    def drt(r, a):
        return math.erfc(a * r) / r

    def bal(a):
        return (rec(4.0 * rlen, a) - rec(5.0 * rlen, a)) - (drt(2.0 * dlen, a) - drt(3.0 * dlen, a))

    tol = 1.4901161193847656e-08
    a = 1.0e-8
    d = bal(a)
    k = 0
    while d < -tol and k < 2000:
        a *= 2.0
        d = bal(a)
        k += 1
    if k == 0 or k >= 2000:
        return 0.25
    left = 0.5 * a
    k = 0
    while d < tol and k < 2000:
        a *= 2.0
        d = bal(a)
        k += 1
    if k >= 2000:
        return 0.25
    right = a
    a = 0.5 * (left + right)
    d = bal(a)
    k = 0
    while abs(d) > tol and k <= 30:
        if d < 0.0:
            left = a
        else:
            right = a
        a = 0.5 * (left + right)
        d = bal(a)
        k += 1
    return 0.25 if k > 30 else a


class DFTD4(nn.Module):
    """D4 (PBE0-D4 defaults: BJ two-body and the ATM three-body term, ``s9 = 1``) on the
    GPU; ``evaluate`` takes a batch of structures, ``forward`` an
    :class:`~xnn_amd.data.AtomicGraph`. Cutoffs in Angstrom (defaults: the upstream
    60 / 40 / 30 / 25 bohr for pair / triple / CN / EEQ CN, d4.py:121-127)."""

    # ``forward``'s ``fused_pair`` (see ``evaluate``); set by DispersionCorrection while only
    # the per-structure energies are differentiated
    fused_pair = False

    def __init__(self, tables: Dict[str, np.ndarray], s6: float = 1.0, s8: float = 1.20065498,
                 a1: float = 0.40085597, a2: float = 5.02928789, s9: float = 1.0,
                 alp: float = 16.0, ga: float = 3.0, gc: float = 2.0, wf: float = 6.0,
                 cutoff_pair: float = 60.0 * BOHR, cutoff_triple: float = 40.0 * BOHR,
                 cutoff_cn: float = 30.0 * BOHR, cutoff_eeq_cn: float = 25.0 * BOHR,
                 switch_width_pair: float = 0.0, switch_width_triple: float = 0.0,
                 tail_correction: bool = False, regime: str = "auto",
                 cutoff_eeq: Optional[float] = None, eeq_solver: str = "auto"):
        super().__init__()
        self.tail_correction = bool(tail_correction)
        if eeq_solver not in ("auto", "lu", "cg"):
            raise ValueError(f"eeq_solver must be 'auto', 'lu' or 'cg', got {eeq_solver!r}")
        # the large regime's solve: the factorized operator up to LU_MAX_ATOMS atoms,
        # conjugate gradients above (eeq.py:194, 226)
        self.eeq_solver = eeq_solver
        regime = str(regime).lower()
        if regime not in EEQ_REGIMES:
            raise ValueError(f"regime must be one of {EEQ_REGIMES}, got {regime!r}")
        self.regime = regime
        self.s6, self.s8, self.a1, self.a2 = float(s6), float(s8), float(a1), float(a2)
        self.s9, self.alp = float(s9), float(alp)
        self.ga, self.gc, self.wf = float(ga), float(gc), float(wf)
        self.cutoff_pair, self.cutoff_cn = float(cutoff_pair), float(cutoff_cn)
        self.cutoff_triple = float(cutoff_triple)
        self.cutoff_eeq_cn = float(cutoff_eeq_cn)
        self.switch_width_pair = float(switch_width_pair)
        self.switch_width_triple = float(switch_width_triple)
        self.cutoff = max(self.cutoff_pair, self.cutoff_cn, self.cutoff_eeq_cn)
        # the real-space range of the large regime's Ewald split (d4.py:461-473): at least
        # the other terms' radius and 16 A unless given
        base = max(self.cutoff_pair, self.cutoff_triple, self.cutoff_cn, self.cutoff_eeq_cn)
        self.cutoff_eeq = (float(cutoff_eeq) if cutoff_eeq is not None
                           else (base if regime == "dense" else max(base, DEFAULT_CUTOFF_EEQ)))
        for k in TABLE_KEYS:
            v = tables[k]
            dt = torch.long if np.issubdtype(v.dtype, np.integer) else torch.float64
            self.register_buffer(k, torch.as_tensor(v, dtype=dt), persistent=False)
        # the polarizability kernel's layout: element-major rows
        kt = {"k_nref": self.nref.to(torch.int32), "k_ngw": self.ngw.t().to(torch.int32),
              "k_refcn": self.refcn.t(), "k_refq": self.refq.t(),
              "k_gi": self.hardness * self.gc, "k_refalpha": self.refalpha.permute(2, 1, 0)}
        for k, v in kt.items():
            self.register_buffer(k, v.contiguous(), persistent=False)

    # ---- building blocks
    def select_regime(self, n_atoms: int, periodic: bool) -> str:
        """``"dense"`` or ``"large"`` for one structure: ``regime="auto"`` takes the large
        regime above 500 periodic or 6000 molecular atoms (d4.py:846-851)."""
        if self.regime != "auto":
            return self.regime
        return "large" if n_atoms > (AUTO_LARGE_PERIODIC if periodic else AUTO_LARGE_MOLECULAR) \
            else "dense"

    def charges(self, z: Tensor, pos_au: Tensor, cn_eeq: Tensor, total_charge: float,
                cell_au: Optional[Tensor]) -> Tensor:
        """EEQ charges of one structure (d4.py:682-723): the dense restatement of dftd4, or
        the large regime's converged Ewald operator on the GPU (:mod:`xnn_amd.eeq`)."""
        n = pos_au.shape[0]
        if self.select_regime(n, cell_au is not None) == "large" and n > 0:
            from .eeq import eeq_charges_large
            if cell_au is not None and self.cutoff_eeq < MIN_CUTOFF_EEQ_AU * BOHR:
                raise ValueError(f"the large EEQ regime needs cutoff_eeq >= {MIN_CUTOFF_EEQ_AU:.0f} "
                                 f"bohr ({MIN_CUTOFF_EEQ_AU * BOHR:.1f} A), got {self.cutoff_eeq:.2f} A")
            rad = self.eeq_rad[z]
            diag = self.eeq_eta[z] + math.sqrt(2.0 / math.pi) / rad
            x = -self.eeq_chi[z] + self.eeq_kcnchi[z] * cn_eeq / torch.sqrt(cn_eeq + EEQ_CN_REG)
            return eeq_charges_large(pos_au, cell_au, rad, diag, x, float(total_charge),
                                     self.cutoff_eeq / BOHR, solver=self.eeq_solver)
        A = self._coulomb_periodic(z, pos_au, cell_au) if cell_au is not None else \
            self._coulomb_molecular(z, pos_au)
        x = -self.eeq_chi[z] + self.eeq_kcnchi[z] * cn_eeq / torch.sqrt(cn_eeq + EEQ_CN_REG)
        ones = torch.ones((n, 1), dtype=pos_au.dtype, device=pos_au.device)
        M = torch.cat([torch.cat([A, ones], 1),
                       torch.cat([ones.t(), torch.zeros((1, 1), dtype=pos_au.dtype,
                                                         device=pos_au.device)], 1)], 0)
        rhs = torch.cat([x, torch.full((1,), float(total_charge), dtype=pos_au.dtype,
                                       device=pos_au.device)])
        return torch.linalg.solve(M, rhs[:, None])[:n, 0]

    def _coulomb_molecular(self, z, pos):
        n = pos.shape[0]
        rad = self.eeq_rad[z]
        gamma = torch.rsqrt(rad[:, None] ** 2 + rad[None, :] ** 2)
        eye = torch.eye(n, dtype=torch.bool, device=pos.device)
        d = pos[None, :, :] - pos[:, None, :]
        r2 = (d * d).sum(-1)
        r = torch.sqrt(torch.where(eye, torch.ones_like(r2), r2))
        off = torch.where(eye, torch.zeros_like(r), torch.erf(gamma * r) / r)
        return off + torch.diag(self.eeq_eta[z] + math.sqrt(2.0 / math.pi) / rad)

    def _coulomb_periodic(self, z, pos, cell):
        """Ewald-summed EEQ matrix over Wigner-Seitz images (d4.py:608-680): every pair
        vector is represented by its minimum-distance image(s) within +-1 cells (ties
        within 0.01 bohr^2 averaged), summed over +-2 cells in real space with the
        erf(gamma r)/r - erf(a r)/r kernel and over +-2 reciprocal cells. Rows are formed in
        chunks of bounded memory (about 1 GB of temporaries each, so thousands of atoms
        fit), recomputed in the backward when positions or cell need gradients."""
        n, dev, dt = pos.shape[0], pos.device, pos.dtype
        vol = torch.linalg.det(cell).abs()
        recip = 2.0 * math.pi * torch.linalg.inv(cell).t()
        # the Ewald parameter is a constant of the evaluation (a search on the host)
        a = _ewald_alpha(float(torch.linalg.norm(recip.detach(), dim=1).min()),
                         float(torch.linalg.norm(cell.detach(), dim=1).min()), float(vol.detach()))
        rad = self.eeq_rad[z]
        rows = max(1, int((1 << 30) // (8 * 3 * 125 * max(n, 1))))
        parts = []
        for i0 in range(0, n, rows):
            i1 = min(n, i0 + rows)
            args = (pos, cell, vol, recip, rad)
            if torch.is_grad_enabled() and (pos.requires_grad or cell.requires_grad):
                from torch.utils.checkpoint import checkpoint
                parts.append(checkpoint(_ewald_rows, i0, i1, a, *args, use_reentrant=False))
            else:
                parts.append(_ewald_rows(i0, i1, a, *args))
        A = torch.cat(parts, 0) if parts else pos.new_zeros((0, 0))
        return A + torch.diag(self.eeq_eta[z] + math.sqrt(2.0 / math.pi) / rad
                              - 2.0 * a / math.sqrt(math.pi))

    def weights(self, z: Tensor, cn: Tensor, q: Tensor) -> Tensor:
        """Gaussian reference weights times the charge scaling, (N, 7) (d4.py:984-1023,
        dispersion.py:70-121)."""
        refcn = self.refcn[:, z].t()
        ngw = self.ngw[:, z].t()
        valid = torch.arange(refcn.shape[1], device=z.device)[None, :] < self.nref[z][:, None]
        d2 = (cn[:, None] - refcn) ** 2
        gw = torch.zeros_like(d2)
        for j in range(1, int(self.ngw.max()) + 1):
            gw = gw + torch.where(ngw >= j, torch.exp(-self.wf * j * d2), torch.zeros_like(d2))
        gw = torch.where(valid, gw, torch.zeros_like(gw))
        norm = gw.sum(1)
        ok = norm > 1.4916681462400413e-154
        w = gw / torch.where(ok, norm, torch.ones_like(norm))[:, None]
        top = torch.where(valid, refcn, torch.full_like(refcn, -math.inf)).max(1).values
        fb = (valid & ((refcn - top[:, None]).abs() < 1e-12)).to(cn.dtype)
        w = torch.where(ok[:, None], w, fb)
        zi = self.zeff[z][:, None]
        gi = (self.hardness[z] * self.gc)[:, None]
        qmod = q[:, None] + zi
        qref = self.refq[:, z].t() + zi
        neg = qmod < 0.0
        safe = torch.where(neg, torch.ones_like(qmod), qmod)
        zeta = torch.exp(self.ga * (1.0 - torch.exp(gi * (1.0 - qref / safe))))
        zeta = torch.where(neg, torch.full_like(qmod, math.exp(self.ga)), zeta)
        return w * zeta

    def polarizabilities(self, z: Tensor, cn: Tensor, q: Tensor) -> Tensor:
        """alpha(i w), (N, 23) bohr^3 (d4.py:1036-1042): the weights above contracted
        with the reference polarizabilities, one HIP kernel each way
        (:func:`d4_polarizabilities_op`)."""
        if not cn.is_cuda:
            raise RuntimeError("xnn_amd D4 runs on the GPU (HIP kernels); there is no CPU path")
        return d4_polarizabilities_op(z.long().contiguous(), cn.to(torch.float64).contiguous(),
                                      q.to(torch.float64).contiguous(), self.k_nref, self.k_ngw,
                                      self.k_refcn, self.k_refq, self.zeff, self.k_gi,
                                      self.k_refalpha, self.ga, self.wf)

    # ---- evaluation
    def evaluate(self, z: Tensor, pos: Tensor, cell: Optional[Tensor], pbc: Optional[Tensor],
                 n_atoms: Tensor, total_charge: Optional[Tensor] = None,
                 charges: Optional[Tensor] = None, fused_pair: bool = False) -> Dict[str, Tensor]:
        """Energies and D4 properties of a batch (atoms of a structure contiguous).
        ``cell`` (B, 3, 3) Angstrom or None; ``charges`` replaces the EEQ solve when
        given. Differentiable once in ``pos`` and ``cell``.

        ``fused_pair``: the two-body energies and their gradients come from one pair-kernel
        launch (:class:`TwoBodyStructureEnergy`) instead of an energy launch in the forward
        and a gradient launch in the backward; then only the per-structure energies
        (``"energy"``, ``"energy_2body"``, ...) carry gradients and ``"node_energy"`` is
        returned detached. For forces and stress from the structure energies (without
        gradients wanted, the energy-only kernel runs as usual)."""
        if not pos.is_cuda:
            raise RuntimeError("xnn_amd D4 runs on the GPU (HIP kernels); there is no CPU path")
        dev = pos.device
        if self.refalpha.device != dev:
            raise RuntimeError(f"the D4 tables are on {self.refalpha.device}, the positions on "
                               f"{dev}: move the module with .to(device)")
        pos = pos.to(torch.float64)
        n_atoms_h = [int(x) for x in n_atoms.cpu()]
        B = len(n_atoms_h)
        node_ptr, batch32 = _batch_tensors(n_atoms_h, dev)
        zc = z.to(dev).long()
        # the pair tables are indexed by atomic number; a number outside them is clamped for
        # the lookups and its polarizabilities, hence the energies, come out NaN
        species = zc.clamp(0, self.r4r2.shape[0] - 1).to(torch.int32).contiguous()
        cell64 = None
        images = torch.zeros((B, 3), dtype=torch.int32, device=dev)
        if cell is not None:
            cell64 = cell.reshape(-1, 3, 3).to(dev, torch.float64).contiguous()
            images = image_counts(cell64, pbc, self.cutoff)
        max_atoms = max(n_atoms_h) if n_atoms_h else 1
        pos = pos.contiguous()
        plan = d4_plan(pos.detach(), node_ptr, None if cell64 is None else cell64.detach(), images)
        cut_cn, cut_eeq = self.cutoff_cn / BOHR, self.cutoff_eeq_cn / BOHR
        cn, raw = d4_coordination_op(pos, cell64, species, batch32, node_ptr, images, plan,
                                     self.rcov, self.en, [cut_cn, cut_eeq], max_atoms)
        periodic = None  # host flags per structure, read only where needed (a synchronization)
        if charges is None:
            periodic = [bool(x) for x in (images != 0).any(1).cpu()]
            cn_eeq = math.log(1.0 + math.exp(EEQ_CN_MAX)) - torch.log(1.0 + torch.exp(EEQ_CN_MAX - raw))
            qs = []
            for b in range(B):
                s0, s1 = sum(n_atoms_h[:b]), sum(n_atoms_h[:b + 1])
                qt = 0.0 if total_charge is None else float(total_charge.reshape(-1)[b])
                cell_b = cell64[b] / BOHR if (cell64 is not None and periodic[b]) else None
                qs.append(self.charges(zc[s0:s1], pos[s0:s1] / BOHR, cn_eeq[s0:s1], qt, cell_b))
            q = torch.cat(qs) if qs else pos.new_zeros(0)
        else:
            q = charges.to(dev, torch.float64)
        alpha = self.polarizabilities(zc, cn, q).contiguous()
        params = [self.s6, self.s8, self.a1, self.a2, self.cutoff_pair / BOHR,
                  self.switch_width_pair / BOHR]
        e2_b = None
        wants_grad = torch.is_grad_enabled() and (
            pos.requires_grad or (cell64 is not None and cell64.requires_grad))
        if fused_pair and wants_grad:
            e2_b, e2 = TwoBodyStructureEnergy.apply(pos, cell64, alpha, species, batch32,
                                                    node_ptr, images, plan, self.r4r2, params,
                                                    max_atoms)
        else:
            e2 = d4_two_body_op(pos, cell64, alpha, species, batch32, node_ptr, images, plan,
                                self.r4r2, params, max_atoms)
        from .ops import structure_sum_op
        e3, e3_b = None, None
        if self.s9 != 0.0:
            if e2_b is not None:
                e3_b, e3 = self.three_body(zc, pos, cell64, pbc, n_atoms_h, cn,
                                           structures=(node_ptr, batch32))
            else:
                e3 = self.three_body(zc, pos, cell64, pbc, n_atoms_h, cn)
        e_tail = None
        if self.tail_correction and cell64 is not None:
            if periodic is None:
                periodic = [bool(x) for x in (images != 0).any(1).cpu()]
            parts = []
            for b in range(B):
                s0, s1 = sum(n_atoms_h[:b]), sum(n_atoms_h[:b + 1])
                if periodic[b]:
                    parts.append(self.tail_energy(zc[s0:s1], alpha[s0:s1], cell64[b] / BOHR))
                else:
                    parts.append(torch.zeros_like(e2[s0:s1]))
            e_tail = torch.cat(parts) if parts else None
        # the sums in a fixed order (float64); absent terms are one shared zero (few launches:
        # the evaluation is short enough for their issue time to show)
        node = e2
        for extra in (e3, e_tail):
            if extra is not None:
                node = node + extra
        node_energy = node * HARTREE
        zero = None if (e3 is not None and e_tail is not None) else node_energy.new_zeros(B)
        parts_sum = {k: (zero if t is None else structure_sum_op(t, node_ptr, batch32) * HARTREE)
                     for k, t in (("energy_3body", e3), ("energy_tail", e_tail))}
        if e2_b is not None:
            # the structure totals from the fused two- and three-body sums plus the tail's
            energy_2 = e2_b * HARTREE
            energy = energy_2
            if e3_b is not None:
                parts_sum["energy_3body"] = e3_b * HARTREE
                energy = energy + parts_sum["energy_3body"]
            if e_tail is not None:
                energy = energy + parts_sum["energy_tail"]
            node_energy = node_energy.detach()
        else:
            energy = structure_sum_op(node_energy, node_ptr, batch32)
            energy_2 = energy if node is e2 else structure_sum_op(e2, node_ptr, batch32) * HARTREE
        return {"node_energy": node_energy, "energy": energy, "energy_2body": energy_2,
                **parts_sum,
                "coordination_numbers": cn, "charges": q,
                "polarizabilities": alpha[:, 0], "dynamic_polarizabilities": alpha,
                "node_features": torch.stack([cn, q, alpha[:, 0]], dim=1)}

    # ---- homogeneous tail of the pair sum beyond its cutoff (d4.py:1073-1140)
    def tail_integrals(self, n_points: int = 48) -> Tensor:
        """Per element pair (A, B), the radial integral of the BJ-damped two-body kernel that
        the pair cutoff leaves out, ``J_AB = -int (1 - sw(r)) [s6 / (r^6 + R0^6) +
        s8 rr / (r^8 + R0^8)] r^2 dr`` from the start of the switching window (the cutoff
        when it is sharp) to infinity, bohr^-3, with ``rr = 3 Q_A Q_B`` and
        ``R0 = a1 sqrt(rr) + a2``. The part beyond the cutoff is integrated in ``x = 1 / r``
        (then ``r^2 dr / (r^n + R0^n) = x^(n-4) dx / (1 + R0^n x^n)`` on ``(0, 1 / rc]``), the
        window in ``r``, each with ``n_points``-point Gauss-Legendre quadrature. Shape
        ``(Z, Z)`` over the tables' atomic numbers."""
        nodes, weights = np.polynomial.legendre.leggauss(n_points)
        t = torch.as_tensor(nodes, dtype=torch.float64, device=self.r4r2.device)
        w = torch.as_tensor(weights, dtype=torch.float64, device=self.r4r2.device)
        rc = self.cutoff_pair / BOHR
        rr = 3.0 * self.r4r2[:, None] * self.r4r2[None, :]
        r0 = self.a1 * torch.sqrt(rr) + self.a2
        p6, p8 = (r0 ** 6).unsqueeze(-1), (r0 ** 8).unsqueeze(-1)
        rr3 = rr.unsqueeze(-1)
        # x = 1 / r over (0, 1 / rc]: the midpoint map of [-1, 1] onto it
        x, wx = (t + 1.0) * (0.5 / rc), w * (0.5 / rc)
        beyond = self.s6 * x * x / (1.0 + p6 * x ** 6) + self.s8 * rr3 * x ** 4 / (1.0 + p8 * x ** 8)
        total = (beyond * wx).sum(-1)
        width = min(self.switch_width_pair, self.cutoff_pair) / BOHR
        if width > 0.0:
            r = (rc - width) + (t + 1.0) * (0.5 * width)
            wr = w * (0.5 * width)
            lost = (1.0 - switching_function(r, rc, width)) * r * r
            inside = self.s6 / (r ** 6 + p6) + self.s8 * rr3 / (r ** 8 + p8)
            total = total + (inside * lost * wr).sum(-1)
        return -total

    def tail_energy(self, z: Tensor, alpha: Tensor, cell_au: Tensor) -> Tensor:
        """Per-atom tail correction of one periodic structure (hartree, d4.py:1109-1140):
        each atom's pairs with every atom beyond the cutoff in a homogeneous continuum,
        ``E_i = (2 pi / V) sum_B J(Z_i, B) C6(i, B)`` with ``C6(i, B)`` the Casimir-Polder
        product of ``alpha_i`` with the summed polarizabilities of the structure's atoms of
        element ``B``. Differentiable in ``alpha`` and the cell."""
        vol = torch.linalg.det(cell_au).abs()
        n_z = self.r4r2.shape[0]
        by_element = torch.zeros((n_z, alpha.shape[1]), dtype=alpha.dtype,
                                 device=alpha.device).index_add(0, z, alpha)
        field = self.tail_integrals() @ by_element                     # (Z, 23)
        # (2 pi / V) (3 / pi) sum_w cp_w alpha_i(w) field(Z_i, w)
        return (6.0 / vol) * (alpha * cp_weights(alpha) * field.index_select(0, z)).sum(-1)

    def three_body(self, z: Tensor, pos: Tensor, cell64: Optional[Tensor], pbc: Optional[Tensor],
                   counts: List[int], cn: Tensor, structures: Optional[Tuple[Tensor, Tensor]] = None):
        """Per-atom ATM energies (hartree, d4.py:1268-1298): C6 from the polarizabilities
        of the neutral atoms (q = 0), damping radii ``a1 sqrt(3 Q_A Q_B) + a2``, exponent
        ``alp / 3``, edges of the radius graph within ``cutoff_triple``; the HIP
        triplet kernels (:func:`atm_energy`), over the species present. With
        ``structures = (node_ptr, batch32)``: (per-structure energies with gradients,
        per-atom energies detached) from :func:`atm_structure_energy`."""
        uniq, species = torch.unique(z, return_inverse=True)
        species = species.to(torch.int32).contiguous()
        alpha0 = self.polarizabilities(z, cn, torch.zeros_like(cn))
        feat = alpha0 * torch.sqrt((3.0 / math.pi) * cp_weights(alpha0))
        edge_index, vec = triple_graph(pos, cell64, pbc, counts, self.cutoff_triple)
        q4 = self.r4r2[uniq]
        table = self.a1 * torch.sqrt(3.0 * q4[:, None] * q4[None, :]) + self.a2
        consts = ATMConstants(species, table, self.s9, self.alp / 3.0, self.cutoff_triple / BOHR,
                              self.switch_width_triple / BOHR)
        if structures is not None:
            return atm_structure_energy(edge_index, vec, feat, feat, consts, *structures)
        return atm_energy(edge_index, vec, feat, feat, consts, pos.shape[0])

    def forward(self, data) -> Dict[str, Tensor]:
        return self.evaluate(data.atomic_numbers, data.pos, data.cell, data.pbc, data.n_atoms,
                             data.total_charge, fused_pair=self.fused_pair)


def cp_weights(like: Tensor) -> Tensor:
    """Casimir-Polder trapezoid weights of the 23 imaginary frequencies (d4.py:130-141)."""
    f = [0.000001, 0.05, 0.1, 0.2, 0.3, 0.4, 0.5, 0.6, 0.7, 0.8, 0.9, 1.0,
         1.2, 1.4, 1.6, 1.8, 2.0, 2.5, 3.0, 4.0, 5.0, 7.5, 10.0]
    cp = [0.5 * ((f[k] - f[k - 1] if k > 0 else 0.0) + (f[k + 1] - f[k] if k < 22 else 0.0))
          for k in range(23)]
    return torch.tensor(cp, dtype=like.dtype, device=like.device)


def c6_matrix(alpha_iw: Tensor) -> Tensor:
    """(3/pi) sum_w cp_w alpha_i(w) alpha_j(w) for all pairs, (N, N) (d4.py:251-266)."""
    return (3.0 / math.pi) * (alpha_iw * cp_weights(alpha_iw)) @ alpha_iw.T


def triple_graph(pos: Tensor, cell64: Optional[Tensor], pbc: Optional[Tensor], counts: List[int],
                 cutoff_aa: float) -> Tuple[Tensor, Tensor]:
    """Edges ``[src, dst]`` within ``cutoff_aa`` of a batch (structures contiguous, HIP
    radius graph per structure) and their vectors in bohr,
    ``(pos[dst] - pos[src] + shift @ cell) / bohr``, differentiable in ``pos`` and the
    cell (d4.py:1201-1207 with the in-cutoff mask of 1277)."""
    from .data import build_neighbor_list
    eis, vecs = [], []
    s0 = 0
    for b, n in enumerate(counts):
        p = pos[s0:s0 + n]
        cell_b = None if cell64 is None else cell64[b]
        pbc_b = None
        if cell_b is not None:
            pbc_b = (torch.ones(3, dtype=torch.bool) if pbc is None
                     else pbc.reshape(-1, 3)[b].detach().cpu().bool())
            if not bool(pbc_b.any()):
                cell_b = None
        if cell_b is None:
            ei, _ = build_neighbor_list(p.detach(), cutoff_aa)
            v = p[ei[1]] - p[ei[0]]
        else:
            ei, sh = build_neighbor_list(p.detach(), cutoff_aa, cell_b.detach(), pbc_b)
            v = p[ei[1]] - p[ei[0]] + sh.to(pos.dtype) @ cell_b
        eis.append(ei + s0)
        vecs.append(v)
        s0 += n
    if not eis:
        return (torch.zeros((2, 0), dtype=torch.long, device=pos.device),
                pos.new_zeros((0, 3)))
    return torch.cat(eis, 1), torch.cat(vecs) / BOHR


# --------------------------------------------------------------------------- potentials
class DispersionCorrection(nn.Module):
    """A dispersion term as a potential, standalone or added to a short-range model
    (dispersion.py:667-842): ``forward(data)`` returns the combined ``"energy"`` (B,) and
    ``"node_energy"`` (eV) plus ``"energy_sr"``, ``"energy_disp"`` and the term's per-atom
    quantities (``"eeq_charges"`` for the D4 charges). The HIP term needs no edges, so
    ``cutoff`` is the wrapped model's own (0 standalone): graphs are built for the model
    alone, and the wrapped model sees them unchanged."""

    _RENAME = {"charges": "eeq_charges"}
    edge_virial = False          # the term depends on the cell beyond the edge vectors
    # False while ForceStressOutput differentiates the per-structure energies only: the
    # term then takes its two-body energies and gradients from one pair launch and returns
    # its per-atom energies detached
    node_energy_grads = True

    def __init__(self, term: nn.Module, model: Optional[nn.Module] = None):
        super().__init__()
        self.term = term
        self.model = model
        self.cutoff = float(getattr(model, "cutoff", 0.0)) if model is not None else 0.0

    def forward(self, data) -> Dict[str, Tensor]:
        fuse = not self.node_energy_grads and hasattr(self.term, "fused_pair")
        if fuse:
            self.term.fused_pair = True
        try:
            disp = dict(self.term(data))
        finally:
            if fuse:
                self.term.fused_pair = False
        node_disp = disp.pop("node_energy")
        energy_disp = disp.pop("energy")
        if self.model is None:
            out = {"node_energy": node_disp, "energy": energy_disp,
                   "energy_sr": torch.zeros_like(energy_disp)}
        else:
            out = dict(self.model(data))
            out["energy_sr"] = out["energy"]
            out["energy"] = out["energy"] + energy_disp
            out["node_energy"] = out["node_energy"] + node_disp.to(out["node_energy"].dtype)
        out["energy_disp"] = energy_disp
        for k, v in disp.items():
            out[self._RENAME.get(k, k)] = v
        return out


class D4Dispersion(DispersionCorrection):
    """D4 dispersion (two- and three-body) as a potential, standalone or wrapped around a model
    (d4.py:1321-1365). ``tables``: the per-element tables (dict or a path for
    :func:`load_d4_tables`); ``d4_options``: keyword arguments of :class:`DFTD4`."""

    def __init__(self, model: Optional[nn.Module] = None, tables=None, **d4_options):
        if tables is None:
            raise ValueError("D4Dispersion needs the per-element D4 tables (dict or .npz path)")
        if isinstance(tables, str):
            tables = load_d4_tables(tables)
        super().__init__(DFTD4(tables, **d4_options), model)

    @property
    def d4(self) -> DFTD4:
        return self.term


# --------------------------------------------------------------------------- D3
D3_DAMPINGS = {"bj": 0, "zero": 1, "mzero": 2, "op": 3}
D3_KCN, D3_WF = 16.0, 4.0                                           # d3.py:464-465
D3_RS9 = 4.0 / 3.0                  # ATM damping radii scale (d3.py:466)
PBE0_D3BJ = {"s6": 1.0, "s8": 1.2177, "a1": 0.4145, "a2": 4.8593}   # d3.py:477-478
PBE0_D3ZERO = {"s6": 1.0, "s8": 0.928, "rs6": 1.287, "rs8": 1.0}
D3_TABLE_KEYS = ("z", "rcov", "r4r2", "rvdw", "nref", "refcn", "c6ref")


def load_d3_tables(path: str) -> Dict[str, np.ndarray]:
    """Compact per-element D3 tables: ``z`` (S,) element list, ``rcov`` (4/3-scaled,
    bohr), ``r4r2``, ``rvdw`` (S, S, bohr), ``nref`` (S,), ``refcn`` (7, S) and ``c6ref``
    (7, 7, S, S) [ref_i, ref_j, species_i, species_j] (d3.py:194-219, 617-628)."""
    with np.load(path, allow_pickle=False) as f:
        missing = [k for k in D3_TABLE_KEYS if k not in f.files]
        if missing:
            raise ValueError(f"{path}: missing D3 tables {missing}")
        return {k: np.asarray(f[k]) for k in D3_TABLE_KEYS}


@torch.library.custom_op(f"{_NS}::d3_coordination", mutates_args=())
def d3_coordination_op(pos: Tensor, cell: Optional[Tensor], species: Tensor, batch32: Tensor,
                       node_ptr: Tensor, images: Tensor, rcov: Tensor, cutoff_cn: float,
                       max_atoms: int) -> Tensor:
    """Exponential-count D3 coordination numbers within ``cutoff_cn`` bohr (d3.py:632-642)."""
    dev = pos.device
    n, b = pos.shape[0], node_ptr.shape[0] - 1
    cn = torch.empty(n, dtype=torch.float64, device=dev)
    ws, need = _workspace(n, b, max_atoms, dev)
    _lib.call("xnn_d3_coordination", _lib.ptr(pos), n, _lib.ptr(species), _lib.ptr(batch32),
              _lib.ptr(node_ptr), b, max_atoms, _lib.ptr(cell), _lib.ptr(images), _lib.ptr(rcov),
              cutoff_cn, D3_KCN, _lib.ptr(cn), _lib.ptr(ws), need, _lib.stream(dev))
    return cn


@d3_coordination_op.register_fake
def _(pos, cell, species, batch32, node_ptr, images, rcov, cutoff_cn, max_atoms):
    return pos.new_empty(pos.shape[0])


def _d3cn_setup(ctx, inputs, output):
    pos, cell, species, batch32, node_ptr, images, rcov, cutoff_cn, max_atoms = inputs
    ctx.save_for_backward(pos, cell, species, batch32, node_ptr, images, rcov)
    ctx.cutoff_cn, ctx.max_atoms = cutoff_cn, max_atoms


def _d3cn_backward(ctx, g_cn):
    if torch.is_grad_enabled():
        raise RuntimeError("the D3 kernels are differentiable once")
    pos, cell, species, batch32, node_ptr, images, rcov = ctx.saved_tensors
    dev, n, b = pos.device, pos.shape[0], node_ptr.shape[0] - 1
    grad_pos = torch.empty((n, 3), dtype=torch.float64, device=dev)
    want_cell = cell is not None and ctx.needs_input_grad[1]
    part = torch.empty((n, 9), dtype=torch.float64, device=dev) if want_cell else None
    ws, need = _workspace(n, b, ctx.max_atoms, dev)
    _lib.call("xnn_d3_coordination_backward", _lib.ptr(pos), n, _lib.ptr(species),
              _lib.ptr(batch32), _lib.ptr(node_ptr), b, ctx.max_atoms, _lib.ptr(cell),
              _lib.ptr(images), _lib.ptr(rcov), ctx.cutoff_cn, D3_KCN,
              _lib.ptr(g_cn.contiguous()), _lib.ptr(grad_pos), _lib.ptr(part), _lib.ptr(ws), need,
              _lib.stream(dev))
    grad_cell = _cell_grad(part, node_ptr, b) if want_cell else None
    return grad_pos, grad_cell, None, None, None, None, None, None, None


d3_coordination_op.register_autograd(_d3cn_backward, setup_context=_d3cn_setup)


@torch.library.custom_op(f"{_NS}::d3_weights", mutates_args=())
def d3_weights_op(species: Tensor, cn: Tensor, nref: Tensor, refcn: Tensor) -> Tensor:
    """D3 reference weights (N, 7): Gaussians exp(-4 (CN - CN_ref)^2) normalized per atom,
    the largest-CN fallback where all vanish (d3.py:644-649), one HIP kernel; ``nref`` (S,)
    int32 and ``refcn`` (S, 7) species-major. Differentiable once in ``cn``."""
    n = cn.shape[0]
    w = torch.empty((n, 7), dtype=torch.float64, device=cn.device)
    _lib.call("xnn_d3_weights", n, _lib.ptr(species), _lib.ptr(cn), nref.shape[0],
              _lib.ptr(nref), _lib.ptr(refcn), D3_WF, _lib.ptr(w), _lib.stream(cn.device))
    return w


@d3_weights_op.register_fake
def _(species, cn, nref, refcn):
    return cn.new_empty((cn.shape[0], 7))


def _d3w_setup(ctx, inputs, output):
    species, cn, nref, refcn = inputs
    ctx.save_for_backward(species, cn, nref, refcn)


def _d3w_backward(ctx, g_w):
    if torch.is_grad_enabled():
        raise RuntimeError("the D3 kernels are differentiable once")
    species, cn, nref, refcn = ctx.saved_tensors
    g_cn = torch.empty_like(cn)
    _lib.call("xnn_d3_weights_backward", cn.shape[0], _lib.ptr(species), _lib.ptr(cn),
              nref.shape[0], _lib.ptr(nref), _lib.ptr(refcn), D3_WF,
              _lib.ptr(g_w.contiguous()), _lib.ptr(g_cn), _lib.stream(cn.device))
    return None, g_cn, None, None


d3_weights_op.register_autograd(_d3w_backward, setup_context=_d3w_setup)


def _d3_params(p: List[float]) -> "_lib.D3PairParams":
    return _lib.D3PairParams(*p[:10], int(p[10]))


@torch.library.custom_op(f"{_NS}::d3_two_body", mutates_args=())
def d3_two_body_op(pos: Tensor, cell: Optional[Tensor], weights: Tensor, species: Tensor,
                   batch32: Tensor, node_ptr: Tensor, images: Tensor, r4r2: Tensor, rvdw: Tensor,
                   c6ref: Tensor, params: List[float], max_atoms: int) -> Tensor:
    """Per-atom D3 two-body energy (hartree); ``params = [s6, s8, a1, a2, rs6, rs8, alp,
    bet, cutoff, width, damping]`` (bohr), ``c6ref`` (S, S, 7, 7) (d3.py:651-722)."""
    dev = pos.device
    n, b = pos.shape[0], node_ptr.shape[0] - 1
    e2 = torch.empty(n, dtype=torch.float64, device=dev)
    ws, need = _workspace(n, b, max_atoms, dev)
    _lib.call("xnn_d3_two_body", _lib.ptr(pos), n, _lib.ptr(species), _lib.ptr(batch32),
              _lib.ptr(node_ptr), b, max_atoms, _lib.ptr(cell), _lib.ptr(images), _lib.ptr(r4r2),
              _lib.ptr(rvdw), _lib.ptr(c6ref), r4r2.shape[0], _lib.ptr(weights),
              _d3_params(params), _lib.ptr(e2), _lib.ptr(ws), need, _lib.stream(dev))
    return e2


@d3_two_body_op.register_fake
def _(pos, cell, weights, species, batch32, node_ptr, images, r4r2, rvdw, c6ref, params, max_atoms):
    return pos.new_empty(pos.shape[0])


def _d3pair_setup(ctx, inputs, output):
    (pos, cell, weights, species, batch32, node_ptr, images, r4r2, rvdw, c6ref, params,
     max_atoms) = inputs
    ctx.save_for_backward(pos, cell, weights, species, batch32, node_ptr, images, r4r2, rvdw, c6ref)
    ctx.params, ctx.max_atoms = list(params), max_atoms


def _d3pair_backward(ctx, g_e2):
    if torch.is_grad_enabled():
        raise RuntimeError("the D3 kernels are differentiable once")
    pos, cell, weights, species, batch32, node_ptr, images, r4r2, rvdw, c6ref = ctx.saved_tensors
    dev, n, b = pos.device, pos.shape[0], node_ptr.shape[0] - 1
    grad_pos = torch.empty((n, 3), dtype=torch.float64, device=dev)
    want_cell = cell is not None and ctx.needs_input_grad[1]
    part = torch.empty((n, 9), dtype=torch.float64, device=dev) if want_cell else None
    grad_w = torch.empty_like(weights) if ctx.needs_input_grad[2] else None
    ws, need = _workspace(n, b, ctx.max_atoms, dev)
    _lib.call("xnn_d3_two_body_backward", _lib.ptr(pos), n, _lib.ptr(species), _lib.ptr(batch32),
              _lib.ptr(node_ptr), b, ctx.max_atoms, _lib.ptr(cell), _lib.ptr(images),
              _lib.ptr(r4r2), _lib.ptr(rvdw), _lib.ptr(c6ref), r4r2.shape[0], _lib.ptr(weights),
              _d3_params(ctx.params), _lib.ptr(g_e2.contiguous()), _lib.ptr(grad_pos),
              _lib.ptr(part), _lib.ptr(grad_w), _lib.ptr(ws), need, _lib.stream(dev))
    grad_cell = _cell_grad(part, node_ptr, b) if want_cell else None
    return grad_pos, grad_cell, grad_w, None, None, None, None, None, None, None, None, None


d3_two_body_op.register_autograd(_d3pair_backward, setup_context=_d3pair_setup)


class D3TwoBodyStructureEnergy(torch.autograd.Function):
    """D3 two-body energies per structure (B,) and, detached, per atom (N,), with their
    gradients, from one launch of the pair backward at unit seeds: C6_ij = sum_ab w_ia w_jb
    C6ref_ab is bilinear in the reference weights and the damping radii do not depend on
    them, so an atom's share is e_i = 1/2 w_i . dE/dw_i. The backward scales the stored
    gradients by the structure seeds (as :class:`TwoBodyStructureEnergy`)."""

    @staticmethod
    def forward(ctx, pos, cell, weights, species, batch32, node_ptr, images, r4r2, rvdw, c6ref,
                params, max_atoms):
        dev, n, b = pos.device, pos.shape[0], node_ptr.shape[0] - 1
        grad_pos = torch.empty((n, 3), dtype=torch.float64, device=dev)
        part = torch.empty((n, 9), dtype=torch.float64, device=dev) if cell is not None else None
        grad_w = torch.empty_like(weights)
        ones = torch.ones(n, dtype=torch.float64, device=dev)
        ws, need = _workspace(n, b, max_atoms, dev)
        _lib.call("xnn_d3_two_body_backward", _lib.ptr(pos), n, _lib.ptr(species),
                  _lib.ptr(batch32), _lib.ptr(node_ptr), b, max_atoms, _lib.ptr(cell),
                  _lib.ptr(images), _lib.ptr(r4r2), _lib.ptr(rvdw), _lib.ptr(c6ref),
                  r4r2.shape[0], _lib.ptr(weights), _d3_params(params), _lib.ptr(ones),
                  _lib.ptr(grad_pos), _lib.ptr(part), _lib.ptr(grad_w), _lib.ptr(ws), need,
                  _lib.stream(dev))
        from .ops import structure_sum_op
        e2 = 0.5 * (weights * grad_w).sum(1)
        e2_b = structure_sum_op(e2, node_ptr, batch32)
        ctx.save_for_backward(batch32, node_ptr, grad_pos, part, grad_w)
        ctx.mark_non_differentiable(e2)
        return e2_b, e2

    @staticmethod
    def backward(ctx, g_b, _g_e2):
        _structure_once()
        batch32, node_ptr, grad_pos, part, grad_w = ctx.saved_tensors
        gs = g_b.index_select(0, batch32.long())[:, None]
        g_pos = grad_pos * gs if ctx.needs_input_grad[0] else None
        g_cell = None
        if part is not None and ctx.needs_input_grad[1]:
            g_cell = _cell_grad(part, node_ptr, g_b.shape[0]) * g_b[:, None, None]
        g_w = grad_w * gs if ctx.needs_input_grad[2] else None
        return (g_pos, g_cell, g_w) + (None,) * 9


def _batch_layout(n_atoms: Tensor, dev) -> Tuple[List[int], Tensor, Tensor]:
    counts = [int(x) for x in n_atoms.cpu()]
    node_ptr, batch32 = _batch_tensors(counts, dev)
    return counts, node_ptr, batch32


class DFTD3(nn.Module):
    """D3 on the GPU (d3.py:483-960): ``damping`` in {"bj", "zero", "mzero", "op"}, PBE0
    defaults, cutoffs in Angstrom (upstream 60 / 40 / 40 bohr for pairs / triples / CN);
    ``s9 != 0`` adds the ATM term (zero damping with radii ``4/3 R0_AB``, exponent
    ``(alp + 2) / 3``; the upstream default is off)."""

    fused_pair = False       # as DFTD4.fused_pair

    def __init__(self, tables: Dict[str, np.ndarray], damping: str = "bj", s6: float = 1.0,
                 s8: Optional[float] = None, a1: float = 0.4145, a2: float = 4.8593,
                 rs6: float = 1.287, rs8: float = 1.0, alp: float = 14.0, bet: float = 0.0,
                 s9: float = 0.0, cutoff_pair: float = 60.0 * BOHR,
                 cutoff_triple: float = 40.0 * BOHR, cutoff_cn: float = 40.0 * BOHR,
                 switch_width_pair: float = 0.0, switch_width_triple: float = 0.0):
        super().__init__()
        damping = {"rational": "bj", "d3bj": "bj"}.get(damping.lower(), damping.lower())
        if damping not in D3_DAMPINGS:
            raise ValueError(f"damping must be one of {tuple(D3_DAMPINGS)}, got {damping!r}")
        self.s9 = float(s9)
        self.cutoff_triple = float(cutoff_triple)
        self.switch_width_triple = float(switch_width_triple)
        if s8 is None:
            s8 = PBE0_D3BJ["s8"] if damping in ("bj", "op") else PBE0_D3ZERO["s8"]
        self.damping = damping
        self.s6, self.s8, self.a1, self.a2 = float(s6), float(s8), float(a1), float(a2)
        self.rs6, self.rs8, self.alp, self.bet = float(rs6), float(rs8), float(alp), float(bet)
        self.cutoff_pair, self.cutoff_cn = float(cutoff_pair), float(cutoff_cn)
        self.switch_width_pair = float(switch_width_pair)
        self.cutoff = max(self.cutoff_pair, self.cutoff_cn)
        self.elements = [int(v) for v in tables["z"]]
        for k in D3_TABLE_KEYS:
            if k == "z":
                continue
            v = tables[k]
            dt = torch.long if np.issubdtype(v.dtype, np.integer) else torch.float64
            self.register_buffer(k, torch.as_tensor(v, dtype=dt), persistent=False)
        # species-major layouts of the reference CNs and counts for the weights kernel
        self.register_buffer("k_refcn", self.refcn.t().contiguous(), persistent=False)
        self.register_buffer("k_nref", self.nref.to(torch.int32), persistent=False)
        # species-pair major layout of the reference block for the kernel
        self.register_buffer("c6pair", torch.as_tensor(
            np.ascontiguousarray(np.asarray(tables["c6ref"]).transpose(2, 3, 0, 1)),
            dtype=torch.float64), persistent=False)

    def species(self, z: Tensor) -> Tensor:
        lut = torch.full((max(self.elements) + 1,), -1, dtype=torch.long)
        lut[torch.tensor(self.elements)] = torch.arange(len(self.elements))
        zc = z.detach().cpu().long()
        if bool((zc > max(self.elements)).any()) or bool((lut[zc.clamp(max=max(self.elements))] < 0).any()):
            raise ValueError(f"the D3 tables cover the elements {self.elements} only")
        return lut[zc]

    def weights(self, s: Tensor, cn: Tensor) -> Tensor:
        """Gaussian reference weights exp(-4 (CN - CN_ref)^2), normalized, with the
        largest-CN fallback (d3.py:644-649, dispersion.py:70-121): one HIP kernel each
        way (:func:`d3_weights_op`)."""
        if not cn.is_cuda:
            raise RuntimeError("xnn_amd D3 runs on the GPU (HIP kernels); there is no CPU path")
        return d3_weights_op(s.to(torch.int32).contiguous(), cn.to(torch.float64).contiguous(),
                             self.k_nref, self.k_refcn)

    def evaluate(self, z: Tensor, pos: Tensor, cell: Optional[Tensor], pbc: Optional[Tensor],
                 n_atoms: Tensor, fused_pair: bool = False) -> Dict[str, Tensor]:
        """Energies of a batch; ``fused_pair`` as in :meth:`DFTD4.evaluate` (the two-body
        energies and gradients from one launch; ``"node_energy"`` then detached)."""
        if not pos.is_cuda:
            raise RuntimeError("xnn_amd D3 runs on the GPU (HIP kernels); there is no CPU path")
        dev = pos.device
        if self.refcn.device != dev:
            raise RuntimeError("move the D3 module to the positions' device with .to(device)")
        pos = pos.to(torch.float64)
        counts, node_ptr, batch32 = _batch_layout(n_atoms, dev)
        s = self.species(z).to(dev)
        species = s.to(torch.int32).contiguous()
        cell64 = None
        images = torch.zeros((len(counts), 3), dtype=torch.int32, device=dev)
        if cell is not None:
            cell64 = cell.reshape(-1, 3, 3).to(dev, torch.float64).contiguous()
            images = image_counts(cell64, pbc, self.cutoff).to(dev)
        max_atoms = max(counts) if counts else 1
        cn = d3_coordination_op(pos.contiguous(), cell64, species, batch32, node_ptr, images,
                                self.rcov, self.cutoff_cn / BOHR, max_atoms)
        w = self.weights(species, cn).contiguous()
        params = [self.s6, self.s8, self.a1, self.a2, self.rs6, self.rs8, self.alp, self.bet,
                  self.cutoff_pair / BOHR, self.switch_width_pair / BOHR,
                  float(D3_DAMPINGS[self.damping])]
        wants_grad = torch.is_grad_enabled() and (
            pos.requires_grad or (cell64 is not None and cell64.requires_grad))
        e2_b = None
        if fused_pair and wants_grad:
            e2_b, e2 = D3TwoBodyStructureEnergy.apply(
                pos.contiguous(), cell64, w, species, batch32, node_ptr, images, self.r4r2,
                self.rvdw.contiguous(), self.c6pair, params, max_atoms)
        else:
            e2 = d3_two_body_op(pos.contiguous(), cell64, w, species, batch32, node_ptr, images,
                                self.r4r2, self.rvdw.contiguous(), self.c6pair, params, max_atoms)
        from .ops import structure_sum_op
        e3 = torch.zeros_like(e2)
        if self.s9 != 0.0:
            e3 = self.three_body(s.to(dev), w, pos, cell64, pbc, counts)
        energy_2 = structure_sum_op(e2, node_ptr, batch32) if e2_b is None else e2_b
        energy_3 = structure_sum_op(e3, node_ptr, batch32)
        node_energy = (e2 + e3) * HARTREE
        if e2_b is not None:
            node_energy = node_energy.detach()
        return {"node_energy": node_energy, "energy": (energy_2 + energy_3) * HARTREE,
                "energy_2body": energy_2 * HARTREE, "energy_3body": energy_3 * HARTREE,
                "coordination_numbers": cn, "weights": w}

    def c6_factors(self, s: Tensor, w: Tensor) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
        """The pair C6 ``W_i^T C6ref[Z_i, Z_j] W_j`` (d3.py:651-674) as ``<f_i, g_j>`` over
        the reference slots of the elements present (d3.py:840-859): ``f_i[p, b] =
        sum_a W_i[a] C6ref[a, b, Z_i, E_p]`` and ``g_j[p, b] = W_j[b]`` at the atom's own
        element ``E_p``; returns ``f, g`` (N, K), the present elements and each atom's
        index among them."""
        uniq, spec = torch.unique(s, return_inverse=True)
        block = self.c6ref[:, :, s][:, :, :, uniq]                   # (7, 7, N, P)
        f = torch.einsum("na,abnp->npb", w, block)                    # (N, P, 7)
        own = torch.nn.functional.one_hot(spec, uniq.shape[0]).to(w.dtype)
        g = own[:, :, None] * w[:, None, :]                           # (N, P, 7)
        slots = (torch.arange(7, device=s.device)[None, :] < self.nref[uniq][:, None]).reshape(-1)
        return f.reshape(s.shape[0], -1)[:, slots], g.reshape(s.shape[0], -1)[:, slots], uniq, spec

    def three_body(self, s: Tensor, w: Tensor, pos: Tensor, cell64: Optional[Tensor],
                   pbc: Optional[Tensor], counts: List[int]) -> Tensor:
        """Per-atom ATM energies (hartree, d3.py:916-936) on the HIP triplet kernels."""
        f, g, uniq, spec = self.c6_factors(s, w)
        if f.shape[1] > 32:
            raise NotImplementedError(
                f"the D3 ATM term takes at most 32 reference slots over the elements present "
                f"(these have {f.shape[1]}); set s9 = 0")
        edge_index, vec = triple_graph(pos, cell64, pbc, counts, self.cutoff_triple)
        table = D3_RS9 * self.rvdw[uniq][:, uniq]
        consts = ATMConstants(spec, table, self.s9, (self.alp + 2.0) / 3.0,
                              self.cutoff_triple / BOHR, self.switch_width_triple / BOHR)
        return atm_energy(edge_index, vec, f.contiguous(), g.contiguous(), consts, pos.shape[0])

    def forward(self, data) -> Dict[str, Tensor]:
        return self.evaluate(data.atomic_numbers, data.pos, data.cell, data.pbc, data.n_atoms,
                             fused_pair=self.fused_pair)


class D3Dispersion(DispersionCorrection):
    """D3 dispersion (two-body; ATM with ``s9 != 0``) as a potential, standalone or wrapped
    around a model (d3.py:965-1016); ``tables``: dict or path for :func:`load_d3_tables`."""

    def __init__(self, model: Optional[nn.Module] = None, tables=None, **d3_options):
        if tables is None:
            raise ValueError("D3Dispersion needs the per-element D3 tables (dict or .npz path)")
        if isinstance(tables, str):
            tables = load_d3_tables(tables)
        super().__init__(DFTD3(tables, **d3_options), model)

    @property
    def d3(self) -> DFTD3:
        return self.term
