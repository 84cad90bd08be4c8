"""HIP-backed operators of the per-edge path, registered as ``torch.library`` custom ops.

Each op is a thin call into ``libxnn_amd.so`` on the current stream, with its
autograd formula registered next to it. The ops run on GPU tensors only; on any
other device, or without the library, they raise (there is no fallback).

Reference counterparts (file:line in molssi-ai/xnn):

=====================  ==============================================================
op                     replaces
=====================  ==============================================================
``edge_vectors``       ``AtomicGraph.edge_vectors`` / ``_EdgeVectors``
                       (common/data/atomic_data.py:371-467)
``edge_embed``         ``SphericalHarmonicEdgeEmbedding.embed``
                       (gnn/featurizers/spherical.py:115-138) with ``BesselRBF`` /
                       ``GaussianRBF`` (common/featurizers/radial.py:15-75, 187-268)
                       and ``PolynomialCutoff`` / ``CosineCutoff`` (cutoff.py:10-125)
``sh_message_sum``     ``ConvTensorProduct.conv`` reference path for scalar edge
                       weights (gnn/fast/conv.py:137-143) + ``scatter_sum``
``sh_linear_message_   the same with the edge weights formed in the kernel by the last
sum``                  linear layer of the weight network (``h @ W``)
``sh_radial_message_   the same with ``h`` the enveloped radial basis of the edge length,
sum``                  evaluated in the kernel (spherical.py:135-138): featurizer,
                       linear layer and message in one launch each way
``strain_apply``,      the strain deformation, strain gradient and stress of
``virial_finish``,     ``ForceStressOutput`` (common/models/outputs.py:166-239)
``stress_finish``
``segment_sum``        ``scatter_sum`` (common/models/ops.py:403-448)
``gather_rows``        ``gather_rows`` (common/models/ops.py:494-528)
``structure_sum``      ``structure_sum`` (common/models/ops.py:531-557), float64 totals
``node_readout``       no reference op: the measured model's linear per-atom readout
                       ``E_i = <U, A_i> + atom_ref[Z_i]`` (one streaming pass each way)
=====================  ==============================================================

All reductions walk CSR rows in a fixed order (no float atomics), so every op
is bitwise reproducible run to run. The linear ops (edge vectors, segment sums,
gathers, structure sums) are differentiable to any order: each backward is its
adjoint op. The nonlinear ones (edge embedding, SH message sums) are
differentiable once; a double backward through them (force training with
``create_graph=True``) raises, and the modules take the PyTorch formulation there.
"""
from __future__ import annotations

from typing import List, Optional, Tuple

import torch
from torch import Tensor

from . import _lib
from .plan import EdgePlan

_NS = "xnn_amd"


def _require_gpu(*tensors: Optional[Tensor]) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError("xnn_amd ops run on the GPU only (got a tensor on "
                               f"{t.device}); there is no CPU fallback")
        dev = t.device
    _lib.load()
    return dev


def _once_differentiable() -> None:
    if torch.is_grad_enabled():
        raise RuntimeError("the xnn_amd backward is differentiable once; double backward "
                           "(create_graph=True) needs the reference path (use_fast=False)")


def _opt(t: Optional[Tensor]) -> Optional[Tensor]:
    return None if t is None or t.numel() == 0 else t


# --------------------------------------------------------------------------- edge vectors
@torch.library.custom_op(f"{_NS}::edge_vectors", mutates_args=())
def edge_vectors_op(pos: Tensor, cell: Optional[Tensor], batch32: Tensor, src: Tensor, dst: Tensor,
                    shift: Tensor, ptr_dst: Tensor, perm_dst: Optional[Tensor], ptr_src: Tensor,
                    perm_src: Tensor, visit: Optional[Tensor], node_ptr: Tensor,
                    out_dtype: int) -> Tensor:
    """``pos[dst] - pos[src] + shift @ cell`` per edge, formed in the geometry dtype and
    returned in ``out_dtype`` (atomic_data.py:371-418)."""
    dev = _require_gpu(pos)
    n_edges = src.shape[0]
    odt = torch.float32 if out_dtype == _lib.XNN_F32 else torch.float64
    vec = torch.empty((n_edges, 3), dtype=odt, device=dev)
    cell = _opt(cell)
    prm = _lib.FeaturizeParams(0, 0, 2, 1, 0, 1, 1.0, 1.0, 1.0)
    _lib.call("xnn_edge_featurize", _lib.dtype_code(pos.dtype), out_dtype, None,
              _lib.ptr(pos), pos.shape[0], _lib.ptr(cell),
              0 if cell is None else cell.shape[0], _lib.ptr(batch32), _lib.ptr(src),
              _lib.ptr(dst), _lib.ptr(shift), n_edges, prm, None, _lib.ptr(vec), None, None, None,
              _lib.stream(dev))
    return vec


@edge_vectors_op.register_fake
def _(pos, cell, batch32, src, dst, shift, ptr_dst, perm_dst, ptr_src, perm_src, visit, node_ptr,
      out_dtype):
    odt = torch.float32 if out_dtype == _lib.XNN_F32 else torch.float64
    return pos.new_empty((src.shape[0], 3), dtype=odt)


@torch.library.custom_op(f"{_NS}::force_reduce", mutates_args=())
def force_reduce_op(g_edge: Tensor, cell_like: Optional[Tensor], batch32: Tensor, src: Tensor,
                    dst: Tensor, shift: Tensor, ptr_dst: Tensor, perm_dst: Optional[Tensor],
                    ptr_src: Tensor, perm_src: Tensor, visit: Optional[Tensor],
                    node_ptr: Tensor, n_nodes: int, geom_code: int,
                    want_cell: bool) -> Tuple[Tensor, Tensor]:
    """Adjoint of :func:`edge_vectors_op`: ``grad_pos[i] = sum_{dst=i} g - sum_{src=i} g``
    and, when ``want_cell``, ``grad_cell[b] = sum_{edges of b} shift^T g`` (float64
    accumulation, returned in the geometry dtype) (atomic_data.py:452-467)."""
    dev = _require_gpu(g_edge)
    g_edge = g_edge.contiguous()
    gdt = torch.float32 if geom_code == _lib.XNN_F32 else torch.float64
    n_graphs = node_ptr.shape[0] - 1
    grad_pos = torch.empty((n_nodes, 3), dtype=gdt, device=dev)
    partial = torch.empty((n_nodes, 9), dtype=torch.float64, device=dev) if want_cell else None
    s = _lib.stream(dev)
    _lib.call("xnn_edge_force_reduce", geom_code, _lib.dtype_code(g_edge.dtype), _lib.ptr(g_edge),
              g_edge.shape[0], _lib.ptr(ptr_dst), _lib.ptr(perm_dst), _lib.ptr(ptr_src),
              _lib.ptr(perm_src), _lib.ptr(shift), _lib.ptr(visit), n_nodes,
              _lib.ptr(grad_pos), _lib.ptr(partial), None, None, s)
    if not want_cell:
        return grad_pos, grad_pos.new_zeros((0,))
    return grad_pos, _lib.virial_reduce(partial, n_nodes, node_ptr, n_graphs, None, False, gdt)


@force_reduce_op.register_fake
def _(g_edge, cell_like, batch32, src, dst, shift, ptr_dst, perm_dst, ptr_src, perm_src, visit,
      node_ptr, n_nodes, geom_code, want_cell):
    gdt = torch.float32 if geom_code == _lib.XNN_F32 else torch.float64
    n_graphs = node_ptr.shape[0] - 1
    return (g_edge.new_empty((n_nodes, 3), dtype=gdt),
            g_edge.new_empty((n_graphs, 3, 3) if want_cell else (0,), dtype=gdt))


def _edge_vectors_setup(ctx, inputs, output):
    (pos, cell, batch32, src, dst, shift, ptr_dst, perm_dst, ptr_src, perm_src, visit,
     node_ptr, out_dtype) = inputs
    ctx.save_for_backward(batch32, src, dst, shift, ptr_dst, perm_dst, ptr_src, perm_src, visit,
                          node_ptr)
    ctx.n_nodes = pos.shape[0]
    ctx.geom_code = _lib.dtype_code(pos.dtype)
    ctx.has_cell = cell is not None and cell.numel() > 0


def _edge_vectors_backward(ctx, grad):
    (batch32, src, dst, shift, ptr_dst, perm_dst, ptr_src, perm_src, visit,
     node_ptr) = ctx.saved_tensors
    want_cell = bool(ctx.has_cell and ctx.needs_input_grad[1])
    grad_pos, grad_cell = force_reduce_op(grad.contiguous(), None, batch32, src, dst, shift,
                                          ptr_dst, perm_dst, ptr_src, perm_src, visit, node_ptr,
                                          ctx.n_nodes, ctx.geom_code, want_cell)
    return (grad_pos if ctx.needs_input_grad[0] else None, grad_cell if want_cell else None,
            None, None, None, None, None, None, None, None, None, None, None)


edge_vectors_op.register_autograd(_edge_vectors_backward, setup_context=_edge_vectors_setup)


def _force_reduce_setup(ctx, inputs, output):
    (g_edge, cell_like, batch32, src, dst, shift, ptr_dst, perm_dst, ptr_src, perm_src, visit,
     node_ptr, n_nodes, geom_code, want_cell) = inputs
    ctx.save_for_backward(batch32, src, dst, shift, ptr_dst, perm_dst, ptr_src, perm_src, visit,
                          node_ptr)
    ctx.out_code = _lib.dtype_code(g_edge.dtype)
    ctx.want_cell = want_cell


def _force_reduce_backward(ctx, d_pos, d_cell):
    # the adjoint of the reduction is the edge-vector map applied to the cotangents
    (batch32, src, dst, shift, ptr_dst, perm_dst, ptr_src, perm_src, visit,
     node_ptr) = ctx.saved_tensors
    cell = d_cell.contiguous() if (ctx.want_cell and d_cell is not None) else None
    if d_pos is None:
        d_pos = torch.zeros((ptr_dst.shape[0] - 1, 3), dtype=cell.dtype if cell is not None
                            else torch.float32, device=ptr_dst.device)
    if cell is not None:
        cell = cell.to(d_pos.dtype)
    g = edge_vectors_op(d_pos.contiguous(), cell, batch32, src, dst, shift, ptr_dst, perm_dst,
                        ptr_src, perm_src, visit, node_ptr, ctx.out_code)
    return (g, None, None, None, None, None, None, None, None, None, None, None, None, None, None)


force_reduce_op.register_autograd(_force_reduce_backward, setup_context=_force_reduce_setup)


def virial_finish(M: Tensor, term: Optional[Tensor], dtype: torch.dtype) -> Tensor:
    """``sym(M + term)`` per structure, (B, 3, 3) in ``dtype``, from float64 (B, 9) sums."""
    n_graphs = M.shape[0]
    out = torch.empty((n_graphs, 3, 3), dtype=dtype, device=M.device)
    _lib.call("xnn_virial_finish", _lib.dtype_code(dtype), _lib.ptr(M), _lib.ptr(term), n_graphs,
              1, _lib.ptr(out), _lib.stream(M.device))
    return out


def _stress_operands(g: Tensor, cell: Tensor, pbc: Optional[Tensor]):
    """The cell as (B, 3, 3) float32/float64 and the pbc flags as uint8 (None: all periodic)
    for the stress kernels."""
    c = cell.reshape(-1, 3, 3)
    if c.dtype not in (torch.float32, torch.float64):
        c = c.to(g.dtype)
    c = c.contiguous()
    flags = None
    if pbc is not None:
        if pbc.is_cuda:
            flags = pbc.reshape(-1, 3).to(torch.bool).contiguous().view(torch.uint8)
        elif not bool(pbc.reshape(-1, 3).any(-1).all()):
            # some structure is non-periodic in every direction (host check: pbc is on
            # the CPU, so this is no device sync)
            flags = pbc.reshape(-1, 3).to(device=g.device, dtype=torch.uint8)
    return c, flags


def energy_stress_supported(node_energy: Tensor) -> bool:
    """Whether :func:`energy_stress_finish` takes this structure (one block of threads)."""
    return (node_energy.is_cuda and node_energy.dim() == 1
            and node_energy.shape[0] <= int(_lib.load().xnn_energy_stress_max_nodes()))


def energy_stress_finish(node_energy: Tensor, strain_gradient: Tensor, cell: Tensor,
                         pbc: Optional[Tensor], scale: float = 1.0) -> Tuple[Tensor, Tensor]:
    """One structure's energy ``sum_i E_i`` (float64, shape (1,)) and stress
    ``scale * strain_gradient / V`` (zero for a molecule) in one kernel: the structure sum
    (base.py:161-180) and the stress of outputs.py:227-239; not differentiable."""
    g = strain_gradient.contiguous()
    c, flags = _stress_operands(g, cell, pbc)
    e = node_energy.contiguous()
    energy = torch.empty(1, dtype=torch.float64, device=e.device)
    stress = torch.empty_like(g)
    _lib.call("xnn_energy_stress_finish", _lib.dtype_code(e.dtype), _lib.ptr(e), e.shape[0],
              _lib.dtype_code(g.dtype), _lib.ptr(g), _lib.dtype_code(c.dtype), _lib.ptr(c),
              _lib.ptr(flags), float(scale), _lib.ptr(energy), _lib.ptr(stress),
              _lib.stream(e.device))
    return energy, stress


def stress_finish(strain_gradient: Tensor, cell: Tensor, pbc: Optional[Tensor],
                  scale: float = 1.0) -> Tensor:
    """``scale * strain_gradient / V`` for periodic structures, zero for molecules
    (outputs.py:227-239), one kernel; not differentiable (forces and stress only)."""
    g = strain_gradient.contiguous()
    c, flags = _stress_operands(g, cell, pbc)
    out = torch.empty_like(g)
    _lib.call("xnn_stress_finish", _lib.dtype_code(g.dtype), _lib.ptr(g), _lib.dtype_code(c.dtype),
              _lib.ptr(c), _lib.ptr(flags), g.shape[0], float(scale), _lib.ptr(out),
              _lib.stream(g.device))
    return out


# --------------------------------------------------------------------------- strain probe
@torch.library.custom_op(f"{_NS}::edge_vectors_strain_probe", mutates_args=())
def edge_vectors_strain_probe_op(pos: Tensor, strain_probe: Tensor, cell: Optional[Tensor],
                                 batch32: Tensor, src: Tensor, dst: Tensor, shift: Tensor,
                                 ptr_dst: Tensor, perm_dst: Optional[Tensor], ptr_src: Tensor,
                                 perm_src: Tensor, visit: Optional[Tensor], node_ptr: Tensor,
                                 out_dtype: int) -> Tensor:
    """Edge vectors of the configuration deformed by the strain ``strain_probe`` (B, 3, 3)
    about zero: ``r_e (I + sym(strain))`` with ``sym(s) = (s + s^T) / 2``, the deformation
    of ForceStressOutput (outputs.py:166-180; it moves positions and cell, hence every
    edge vector, by the same linear map). The probe is zero by contract (its value is not
    read), so the vectors are the undeformed ones; what it carries is its gradient, which
    the backward forms directly: ``dE/d strain = sym(sum_e r_e (x) dE/dr_e)`` per structure,
    float64 accumulation, from the force-reduction kernel. Differentiable once."""
    return edge_vectors_op(pos, cell, batch32, src, dst, shift, ptr_dst, perm_dst, ptr_src,
                           perm_src, visit, node_ptr, out_dtype)


@edge_vectors_strain_probe_op.register_fake
def _(pos, strain_probe, cell, batch32, src, dst, shift, ptr_dst, perm_dst, ptr_src, perm_src,
      visit, node_ptr, out_dtype):
    odt = torch.float32 if out_dtype == _lib.XNN_F32 else torch.float64
    return pos.new_empty((src.shape[0], 3), dtype=odt)


def _probe_setup(ctx, inputs, output):
    (pos, strain_probe, cell, batch32, src, dst, shift, ptr_dst, perm_dst, ptr_src, perm_src,
     visit, node_ptr, out_dtype) = inputs
    ctx.save_for_backward(output, batch32, src, dst, shift, ptr_dst, perm_dst, ptr_src, perm_src,
                          visit, node_ptr)
    ctx.n_nodes = pos.shape[0]
    ctx.geom_code = _lib.dtype_code(pos.dtype)
    ctx.has_cell = cell is not None and cell.numel() > 0
    ctx.probe_dtype = strain_probe.dtype


def _probe_backward(ctx, grad):
    _once_differentiable()
    (vec, batch32, src, dst, shift, ptr_dst, perm_dst, ptr_src, perm_src, visit,
     node_ptr) = ctx.saved_tensors
    grad = grad.contiguous()
    dev = grad.device
    n_nodes = ctx.n_nodes
    n_graphs = node_ptr.shape[0] - 1
    gdt = torch.float32 if ctx.geom_code == _lib.XNN_F32 else torch.float64
    want_cell = bool(ctx.has_cell and ctx.needs_input_grad[2])
    grad_pos = torch.empty((n_nodes, 3), dtype=gdt, device=dev)
    if n_graphs == 1 and not want_cell:
        # one structure: block sums of the strain derivative, added by one finishing block
        grad_probe = torch.empty((1, 3, 3), dtype=ctx.probe_dtype, device=dev)
        need = int(_lib.load().xnn_edge_force_reduce_virial_workspace_bytes(grad.shape[0],
                                                                            n_nodes))
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
        _lib.call("xnn_edge_force_reduce_virial", ctx.geom_code, _lib.dtype_code(grad.dtype),
                  _lib.ptr(grad), grad.shape[0], _lib.ptr(ptr_dst), _lib.ptr(perm_dst),
                  _lib.ptr(ptr_src), _lib.ptr(perm_src), _lib.ptr(visit), n_nodes,
                  _lib.ptr(grad_pos), _lib.ptr(vec), _lib.dtype_code(ctx.probe_dtype),
                  _lib.ptr(grad_probe), _lib.ptr(ws), need, _lib.stream(dev))
        return (grad_pos if ctx.needs_input_grad[0] else None, grad_probe, None,
                None, None, None, None, None, None, None, None, None, None, None)
    cell_partial = torch.empty((n_nodes, 9), dtype=torch.float64, device=dev) if want_cell else None
    virial_partial = torch.empty((n_nodes, 9), dtype=torch.float64, device=dev)
    _lib.call("xnn_edge_force_reduce", ctx.geom_code, _lib.dtype_code(grad.dtype), _lib.ptr(grad),
              grad.shape[0], _lib.ptr(ptr_dst), _lib.ptr(perm_dst), _lib.ptr(ptr_src),
              _lib.ptr(perm_src), _lib.ptr(shift), _lib.ptr(visit), n_nodes, _lib.ptr(grad_pos),
              _lib.ptr(cell_partial), _lib.ptr(vec), _lib.ptr(virial_partial), _lib.stream(dev))
    grad_probe = _lib.virial_reduce(virial_partial, n_nodes, node_ptr, n_graphs, None, True,
                                    ctx.probe_dtype)
    grad_cell = None
    if want_cell:
        grad_cell = _lib.virial_reduce(cell_partial, n_nodes, node_ptr, n_graphs, None, False, gdt)
    return (grad_pos if ctx.needs_input_grad[0] else None, grad_probe, grad_cell,
            None, None, None, None, None, None, None, None, None, None, None)


edge_vectors_strain_probe_op.register_autograd(_probe_backward, setup_context=_probe_setup)


def edge_vectors(pos: Tensor, cell: Optional[Tensor], plan: EdgePlan,
                 out_dtype: Optional[torch.dtype] = None,
                 strain_probe: Optional[Tensor] = None) -> Tensor:
    """Edge vectors of a planned graph; differentiable to ``pos`` and ``cell`` to any
    order (the backward is the CSR force reduction, whose adjoint is this map again).
    With ``strain_probe`` (a zero (B, 3, 3) tensor) the strain gradient comes from the
    same backward pass (differentiable once)."""
    out_dtype = out_dtype or pos.dtype
    if cell is not None:
        cell = cell.reshape(-1, 3, 3).to(pos.dtype)
        if not cell.is_contiguous():
            cell = cell.contiguous()
    if strain_probe is not None:
        return edge_vectors_strain_probe_op(
            pos.contiguous(), strain_probe, cell, plan.batch32, plan.src, plan.dst, plan.shift,
            plan.ptr_dst, plan.perm_dst, plan.ptr_src, plan.perm_src, plan.visit, plan.node_ptr,
            _lib.dtype_code(out_dtype))
    return edge_vectors_op(pos.contiguous(), cell, plan.batch32, plan.src, plan.dst, plan.shift,
                           plan.ptr_dst, plan.perm_dst, plan.ptr_src, plan.perm_src,
                           plan.visit, plan.node_ptr, _lib.dtype_code(out_dtype))


# --------------------------------------------------------------------------- strain deformation
@torch.library.custom_op(f"{_NS}::strain_apply", mutates_args=())
def strain_apply_op(pos: Tensor, cell: Optional[Tensor], strain: Tensor, batch32: Tensor,
                    node_ptr: Tensor) -> Tuple[Tensor, Tensor]:
    """``pos (I + sym(strain)[batch])`` and ``cell (I + sym(strain))``, the deformation
    of ForceStressOutput (outputs.py:166-180); an empty cell comes back empty."""
    dev = _require_gpu(pos, strain)
    code = _lib.dtype_code(pos.dtype)
    cell = _opt(cell)
    pos_out = torch.empty_like(pos)
    cell_out = torch.empty_like(cell) if cell is not None else pos.new_zeros((0,))
    n_graphs = node_ptr.shape[0] - 1
    _lib.call("xnn_strain_apply", code, _lib.ptr(pos), pos.shape[0],
              _lib.ptr(batch32) if n_graphs > 1 else None, _lib.ptr(cell), n_graphs,
              _lib.ptr(strain), _lib.ptr(pos_out), _lib.ptr(cell_out) if cell is not None else None,
              _lib.stream(dev))
    return pos_out, cell_out


@strain_apply_op.register_fake
def _(pos, cell, strain, batch32, node_ptr):
    return torch.empty_like(pos), (torch.empty_like(cell) if cell is not None and cell.numel()
                                   else pos.new_zeros((0,)))


def _strain_setup(ctx, inputs, output):
    pos, cell, strain, batch32, node_ptr = inputs
    ctx.save_for_backward(pos, _opt(cell), strain, batch32, node_ptr)


def _strain_backward(ctx, g_pos, g_cell):
    _once_differentiable()
    pos, cell, strain, batch32, node_ptr = ctx.saved_tensors
    dev, n = pos.device, pos.shape[0]
    n_graphs = node_ptr.shape[0] - 1
    code = _lib.dtype_code(pos.dtype)
    g_pos = torch.zeros_like(pos) if g_pos is None else g_pos.contiguous()
    grad_pos = torch.empty_like(pos)
    partial = torch.empty((n, 9), dtype=torch.float64, device=dev)
    grad_cell = term = None
    if cell is not None:
        g_cell = torch.zeros_like(cell) if (g_cell is None or g_cell.numel() == 0) else g_cell.contiguous()
        grad_cell = torch.empty_like(cell)
        term = torch.empty((n_graphs, 9), dtype=torch.float64, device=dev)
    _lib.call("xnn_strain_apply_backward", code, _lib.ptr(pos), n,
              _lib.ptr(batch32) if n_graphs > 1 else None, _lib.ptr(cell), n_graphs,
              _lib.ptr(strain), _lib.ptr(g_pos), _lib.ptr(g_cell) if cell is not None else None,
              _lib.ptr(grad_pos), _lib.ptr(grad_cell), _lib.ptr(partial), _lib.ptr(term),
              _lib.stream(dev))
    grad_strain = _lib.virial_reduce(partial, n, node_ptr, n_graphs, term, True, strain.dtype)
    return grad_pos, grad_cell, grad_strain, None, None


strain_apply_op.register_autograd(_strain_backward, setup_context=_strain_setup)


# --------------------------------------------------------------------------- edge embedding
def _params(iparams: List[int], fparams: List[float]) -> "_lib.FeaturizeParams":
    n_rbf, basis, envelope, p, l_max, sign = iparams
    cutoff, prefactor, gamma = fparams
    return _lib.FeaturizeParams(n_rbf, basis, envelope, p, l_max, sign, cutoff, prefactor, gamma)


@torch.library.custom_op(f"{_NS}::edge_embed", mutates_args=())
def edge_embed_op(vec: Tensor, rbf_table: Tensor, iparams: List[int], fparams: List[float],
                  want_length: bool, want_sh: bool, want_radial: bool
                  ) -> Tuple[Tensor, Tensor, Tensor]:
    """``(|v|, Y(sign v / |v|), rbf(|v|) * envelope(|v|))`` per edge vector
    (spherical.py:135-138); unrequested outputs come back empty."""
    dev = _require_gpu(vec)
    n_edges = vec.shape[0]
    n_rbf, l_max = iparams[0], iparams[4]
    L = (l_max + 1) ** 2
    length = vec.new_empty((n_edges,) if want_length else (0,))
    sh = vec.new_empty((n_edges, L) if want_sh else (0,))
    radial = vec.new_empty((n_edges, n_rbf) if want_radial else (0,))
    code = _lib.dtype_code(vec.dtype)
    _lib.call("xnn_edge_featurize", code, code, _lib.ptr(vec), None, 0, None, 0, None, None, None,
              None, n_edges, _params(iparams, fparams), _lib.ptr(rbf_table), None,
              _lib.ptr(length) if want_length else None, _lib.ptr(sh) if want_sh else None,
              _lib.ptr(radial) if want_radial else None, _lib.stream(dev))
    return length, sh, radial


@edge_embed_op.register_fake
def _(vec, rbf_table, iparams, fparams, want_length, want_sh, want_radial):
    n_edges = vec.shape[0]
    L = (iparams[4] + 1) ** 2
    return (vec.new_empty((n_edges,) if want_length else (0,)),
            vec.new_empty((n_edges, L) if want_sh else (0,)),
            vec.new_empty((n_edges, iparams[0]) if want_radial else (0,)))


def _edge_embed_setup(ctx, inputs, output):
    vec, rbf_table, iparams, fparams, want_length, want_sh, want_radial = inputs
    ctx.save_for_backward(vec, rbf_table)
    ctx.iparams, ctx.fparams = list(iparams), list(fparams)
    ctx.wants = (want_length, want_sh, want_radial)


def _edge_embed_backward(ctx, d_length, d_sh, d_radial):
    _once_differentiable()
    vec, rbf_table = ctx.saved_tensors
    if ctx.needs_input_grad[1]:
        raise NotImplementedError("the fast edge embedding does not differentiate the radial "
                                  "basis parameters; use use_fast=False to train them")
    want_length, want_sh, want_radial = ctx.wants
    d_length = d_length.contiguous() if want_length and d_length is not None else None
    d_sh = d_sh.contiguous() if want_sh and d_sh is not None else None
    d_radial = d_radial.contiguous() if want_radial and d_radial is not None else None
    g = torch.empty_like(vec)
    code = _lib.dtype_code(vec.dtype)
    _lib.call("xnn_edge_featurize_backward", code, code, _lib.ptr(vec), None, 0, None, 0, None,
              None, None, None, vec.shape[0], _params(ctx.iparams, ctx.fparams),
              _lib.ptr(rbf_table), None, _lib.ptr(d_length), _lib.ptr(d_sh), _lib.ptr(d_radial),
              None, _lib.ptr(g), _lib.stream(vec.device))
    return g, None, None, None, None, None, None


edge_embed_op.register_autograd(_edge_embed_backward, setup_context=_edge_embed_setup)


def edge_embed(vec: Tensor, rbf_table: Tensor, *, n_rbf: int, basis: str, envelope: str,
               poly_p: int, l_max: int, cutoff: float, prefactor: float = 1.0,
               gamma: float = 1.0, sh_sign: int = 1, want_length: bool = True,
               want_sh: bool = True, want_radial: bool = True) -> Tuple[Tensor, Tensor, Tensor]:
    """Length, spherical harmonics and enveloped radial basis of edge vectors."""
    iparams = [int(n_rbf), _lib.BASIS[basis], _lib.ENVELOPE[envelope], int(poly_p), int(l_max),
               int(sh_sign)]
    fparams = [float(cutoff), float(prefactor), float(gamma)]
    table = rbf_table.to(device=vec.device, dtype=vec.dtype).contiguous()
    return edge_embed_op(vec.contiguous(), table, iparams, fparams, bool(want_length),
                         bool(want_sh), bool(want_radial))


# --------------------------------------------------------------------------- SH message sum
@torch.library.custom_op(f"{_NS}::sh_message_sum", mutates_args=())
def sh_message_sum_op(vec: Tensor, phi: Tensor, ptr_dst: Tensor, perm_dst: Optional[Tensor],
                      l_max: int, sh_sign: int) -> Tensor:
    """``A[i, c, lm] = sum_{dst(e)=i} phi[e, c] Y_lm(sign vec_e)`` (float32)."""
    dev = _require_gpu(vec, phi)
    n_nodes = ptr_dst.shape[0] - 1
    C = phi.shape[1]
    L = (l_max + 1) ** 2
    out = torch.empty((n_nodes, C, L), dtype=torch.float32, device=dev)
    _lib.call("xnn_sh_message_sum", _lib.XNN_F32, _lib.ptr(vec), None, n_nodes, None, 0, None,
              None, None, vec.shape[0], _lib.ptr(ptr_dst), _lib.ptr(perm_dst), l_max, sh_sign, C,
              _lib.ptr(phi), _lib.ptr(out), _lib.stream(dev))
    return out


@sh_message_sum_op.register_fake
def _(vec, phi, ptr_dst, perm_dst, l_max, sh_sign):
    return phi.new_empty((ptr_dst.shape[0] - 1, phi.shape[1], (l_max + 1) ** 2))


def _sh_msg_setup(ctx, inputs, output):
    vec, phi, ptr_dst, perm_dst, l_max, sh_sign = inputs
    ctx.save_for_backward(vec, phi, ptr_dst, perm_dst)
    ctx.l_max, ctx.sh_sign = l_max, sh_sign


def _sh_msg_backward(ctx, d_out):
    _once_differentiable()
    vec, phi, ptr_dst, perm_dst = ctx.saved_tensors
    d_out = d_out.contiguous()
    n_nodes = ptr_dst.shape[0] - 1
    d_phi = torch.empty_like(phi)
    g_vec = torch.empty_like(vec) if ctx.needs_input_grad[0] else None
    _lib.call("xnn_sh_message_sum_backward", _lib.XNN_F32, _lib.ptr(vec), None, n_nodes, None, 0,
              None, None, None, vec.shape[0], _lib.ptr(ptr_dst), _lib.ptr(perm_dst), ctx.l_max,
              ctx.sh_sign, phi.shape[1], _lib.ptr(phi), _lib.ptr(d_out), _lib.ptr(d_phi),
              _lib.ptr(g_vec), _lib.stream(vec.device))
    return g_vec, d_phi, None, None, None, None


sh_message_sum_op.register_autograd(_sh_msg_backward, setup_context=_sh_msg_setup)


def sh_message_sum(vec: Tensor, phi: Tensor, plan: EdgePlan, l_max: int,
                   sh_sign: int = 1) -> Tensor:
    """Aggregate ``phi[e, c] * Y_lm(sign vec_e)`` onto receivers: ``(N, C, (l_max+1)^2)``."""
    if vec.dtype != torch.float32 or phi.dtype != torch.float32:
        raise TypeError("sh_message_sum computes in float32")
    if phi.shape[0] != vec.shape[0]:
        raise ValueError("phi and vec need one row per edge")
    if not 1 <= phi.shape[1] <= 256:
        raise ValueError("sh_message_sum takes 1 to 256 channels")
    return sh_message_sum_op(vec.contiguous(), phi.contiguous(), plan.ptr_dst, plan.perm_dst,
                             int(l_max), int(sh_sign))


# --------------------------------------------------------------------------- fused linear + SH message sum
LINEAR_MESSAGE_CHANNELS = (32, 64, 128)
LINEAR_MESSAGE_MAX_FEATURES = 8


@torch.library.custom_op(f"{_NS}::sh_linear_message_sum", mutates_args=())
def sh_linear_message_sum_op(vec: Tensor, h: Tensor, W: Tensor, ptr_dst: Tensor,
                             perm_dst: Optional[Tensor], l_max: int, sh_sign: int) -> Tensor:
    """``A[i, c, lm] = sum_{dst(e)=i} (h_e W)[c] Y_lm(sign vec_e)`` (float32); ``h W`` is
    formed in the kernel and never stored."""
    dev = _require_gpu(vec, h, W)
    n_nodes = ptr_dst.shape[0] - 1
    K, C = W.shape
    L = (l_max + 1) ** 2
    out = torch.empty((n_nodes, C, L), dtype=torch.float32, device=dev)
    _lib.call("xnn_sh_linear_message_sum", _lib.XNN_F32, _lib.ptr(vec), None, n_nodes, None, 0,
              None, None, None, vec.shape[0], _lib.ptr(ptr_dst), _lib.ptr(perm_dst), l_max,
              sh_sign, K, C, _lib.ptr(h), _lib.ptr(W), _lib.ptr(out), _lib.stream(dev))
    return out


@sh_linear_message_sum_op.register_fake
def _(vec, h, W, ptr_dst, perm_dst, l_max, sh_sign):
    return h.new_empty((ptr_dst.shape[0] - 1, W.shape[1], (l_max + 1) ** 2))


def _lin_msg_setup(ctx, inputs, output):
    vec, h, W, ptr_dst, perm_dst, l_max, sh_sign = inputs
    ctx.save_for_backward(vec, h, W, ptr_dst, perm_dst)
    ctx.l_max, ctx.sh_sign = l_max, sh_sign


def _lin_msg_backward(ctx, d_out):
    _once_differentiable()
    vec, h, W, ptr_dst, perm_dst = ctx.saved_tensors
    d_out = d_out.contiguous()
    n_nodes = ptr_dst.shape[0] - 1
    K, C = W.shape
    dev = vec.device
    need_vec, need_h, need_W = ctx.needs_input_grad[0], ctx.needs_input_grad[1], ctx.needs_input_grad[2]
    g_vec = torch.empty_like(vec) if need_vec else None
    d_h = torch.empty_like(h) if (need_h or need_vec) else None
    if need_vec or need_h:
        _lib.call("xnn_sh_linear_message_sum_backward", _lib.XNN_F32, _lib.ptr(vec), None,
                  n_nodes, None, 0, None, None, None, vec.shape[0], _lib.ptr(ptr_dst),
                  _lib.ptr(perm_dst), ctx.l_max, ctx.sh_sign, K, C, _lib.ptr(h), _lib.ptr(W),
                  _lib.ptr(d_out), _lib.ptr(d_h), _lib.ptr(g_vec), _lib.stream(dev))
    d_W = None
    if need_W:
        # d_W = h^T d_phi needs d_phi itself: one pass of the unfused backward forms it
        phi = h @ W
        d_phi = torch.empty_like(phi)
        _lib.call("xnn_sh_message_sum_backward", _lib.XNN_F32, _lib.ptr(vec), None, n_nodes, None,
                  0, None, None, None, vec.shape[0], _lib.ptr(ptr_dst), _lib.ptr(perm_dst),
                  ctx.l_max, ctx.sh_sign, C, _lib.ptr(phi), _lib.ptr(d_out), _lib.ptr(d_phi),
                  None, _lib.stream(dev))
        d_W = h.t() @ d_phi
    return g_vec, (d_h if need_h else None), d_W, None, None, None, None


sh_linear_message_sum_op.register_autograd(_lin_msg_backward, setup_context=_lin_msg_setup)


def linear_message_supported(n_features: int, n_channels: int, l_max: int) -> bool:
    """Shapes the fused kernels take; others use the linear layer + :func:`sh_message_sum`."""
    return (n_channels in LINEAR_MESSAGE_CHANNELS and 1 <= n_features <= LINEAR_MESSAGE_MAX_FEATURES
            and 1 <= l_max <= 3)


def sh_linear_message_sum(vec: Tensor, h: Tensor, W: Tensor, plan: EdgePlan, l_max: int,
                          sh_sign: int = 1) -> Tensor:
    """``sh_message_sum(vec, h @ W, ...)`` with the linear layer inside the kernel."""
    if vec.dtype != torch.float32 or h.dtype != torch.float32 or W.dtype != torch.float32:
        raise TypeError("sh_linear_message_sum computes in float32")
    if h.shape[0] != vec.shape[0] or h.shape[1] != W.shape[0]:
        raise ValueError("h needs one row per edge and W one row per feature of h")
    if not linear_message_supported(W.shape[0], W.shape[1], l_max):
        raise ValueError(f"sh_linear_message_sum takes {LINEAR_MESSAGE_CHANNELS} channels, at "
                         f"most {LINEAR_MESSAGE_MAX_FEATURES} features and l_max in [1, 3]")
    return sh_linear_message_sum_op(vec.contiguous(), h.contiguous(), W.contiguous(),
                                    plan.ptr_dst, plan.perm_dst, int(l_max), int(sh_sign))


@torch.library.custom_op(f"{_NS}::sh_radial_message_sum", mutates_args=())
def sh_radial_message_sum_op(vec: Tensor, rbf_table: Tensor, W: Tensor, ptr_dst: Tensor,
                             perm_dst: Optional[Tensor], iparams: List[int],
                             fparams: List[float]) -> Tensor:
    """``A[i, c, lm] = sum_{dst(e)=i} (h_e W)[c] Y_lm(sign vec_e)`` with
    ``h_e = rbf(|vec_e|) envelope(|vec_e|)`` evaluated in the kernel (float32): the
    featurizer's radial part, the linear layer and the message in one launch."""
    dev = _require_gpu(vec, W)
    n_nodes = ptr_dst.shape[0] - 1
    C = W.shape[1]
    L = (iparams[4] + 1) ** 2
    out = torch.empty((n_nodes, C, L), dtype=torch.float32, device=dev)
    _lib.call("xnn_sh_radial_message_sum", _lib.XNN_F32, _lib.ptr(vec), None, n_nodes, None, 0,
              None, None, None, vec.shape[0], _lib.ptr(ptr_dst), _lib.ptr(perm_dst),
              _params(iparams, fparams), _lib.ptr(rbf_table), C, _lib.ptr(W), _lib.ptr(out),
              _lib.stream(dev))
    return out


@sh_radial_message_sum_op.register_fake
def _(vec, rbf_table, W, ptr_dst, perm_dst, iparams, fparams):
    return vec.new_empty((ptr_dst.shape[0] - 1, W.shape[1], (iparams[4] + 1) ** 2))


def _rad_msg_setup(ctx, inputs, output):
    vec, rbf_table, W, ptr_dst, perm_dst, iparams, fparams = inputs
    ctx.save_for_backward(vec, rbf_table, W, ptr_dst, perm_dst)
    ctx.iparams, ctx.fparams = list(iparams), list(fparams)


def _rad_msg_backward(ctx, d_out):
    _once_differentiable()
    if ctx.needs_input_grad[1] or ctx.needs_input_grad[2]:
        raise NotImplementedError("sh_radial_message_sum differentiates the edge vectors only; "
                                  "train W with edge_embed + sh_linear_message_sum")
    vec, rbf_table, W, ptr_dst, perm_dst = ctx.saved_tensors
    d_out = d_out.contiguous()
    g_vec = torch.empty_like(vec)
    _lib.call("xnn_sh_radial_message_sum_backward", _lib.XNN_F32, _lib.ptr(vec), None,
              ptr_dst.shape[0] - 1, None, 0, None, None, None, vec.shape[0], _lib.ptr(ptr_dst),
              _lib.ptr(perm_dst), _params(ctx.iparams, ctx.fparams), _lib.ptr(rbf_table),
              W.shape[1], _lib.ptr(W), _lib.ptr(d_out), _lib.ptr(g_vec), _lib.stream(vec.device))
    return g_vec, None, None, None, None, None, None


sh_radial_message_sum_op.register_autograd(_rad_msg_backward, setup_context=_rad_msg_setup)


def sh_radial_message_sum(vec: Tensor, rbf_table: Tensor, W: Tensor, plan: EdgePlan, *,
                          basis: str, envelope: str, poly_p: int, l_max: int, cutoff: float,
                          prefactor: float = 1.0, gamma: float = 1.0,
                          sh_sign: int = 1) -> Tensor:
    """``sh_linear_message_sum(vec, radial(vec), W, ...)`` with the radial basis (``W.shape[0]``
    functions) evaluated inside the kernels; differentiable in ``vec`` only."""
    if vec.dtype != torch.float32 or W.dtype != torch.float32:
        raise TypeError("sh_radial_message_sum computes in float32")
    n_rbf = W.shape[0]
    if rbf_table.numel() != n_rbf:
        raise ValueError("W needs one row per radial basis function")
    if not linear_message_supported(n_rbf, W.shape[1], l_max):
        raise ValueError(f"sh_radial_message_sum takes {LINEAR_MESSAGE_CHANNELS} channels, at "
                         f"most {LINEAR_MESSAGE_MAX_FEATURES} basis functions and l_max in [1, 3]")
    iparams = [int(n_rbf), _lib.BASIS[basis], _lib.ENVELOPE[envelope], int(poly_p), int(l_max),
               int(sh_sign)]
    fparams = [float(cutoff), float(prefactor), float(gamma)]
    table = rbf_table.to(device=vec.device, dtype=torch.float32).contiguous()
    return sh_radial_message_sum_op(vec.contiguous(), table, W.contiguous(), plan.ptr_dst,
                                    plan.perm_dst, iparams, fparams)


@torch.library.custom_op(f"{_NS}::sh_radial_message_energy", mutates_args=())
def sh_radial_message_energy_op(vec: Tensor, rbf_table: Tensor, W: Tensor, U: Tensor,
                                z: Tensor, bias: Optional[Tensor], ptr_dst: Tensor,
                                perm_dst: Optional[Tensor], iparams: List[int],
                                fparams: List[float]) -> Tensor:
    """Per-atom energies ``E_i = <U, A_i> + bias[z_i]`` of the rows
    ``A_i = sum_{dst(e)=i} (h_e W) (x) Y(sign vec_e)`` (float32), formed and read out in
    one kernel: the (N, C, L) rows never reach memory."""
    dev = _require_gpu(vec, W)
    n_nodes = ptr_dst.shape[0] - 1
    out = torch.empty(n_nodes, dtype=torch.float32, device=dev)
    _lib.call("xnn_sh_radial_message_energy", _lib.XNN_F32, _lib.ptr(vec), None, n_nodes, None, 0,
              None, None, None, vec.shape[0], _lib.ptr(ptr_dst), _lib.ptr(perm_dst),
              _params(iparams, fparams), _lib.ptr(rbf_table), W.shape[1], _lib.ptr(W),
              _lib.ptr(U), _lib.ptr(z), _lib.ptr(bias), 0 if bias is None else bias.shape[0],
              _lib.ptr(out), _lib.stream(dev))
    return out


@sh_radial_message_energy_op.register_fake
def _(vec, rbf_table, W, U, z, bias, ptr_dst, perm_dst, iparams, fparams):
    return vec.new_empty(ptr_dst.shape[0] - 1)


def _rad_energy_setup(ctx, inputs, output):
    vec, rbf_table, W, U, z, bias, ptr_dst, perm_dst, iparams, fparams = inputs
    ctx.save_for_backward(vec, rbf_table, W, U, ptr_dst, perm_dst)
    ctx.iparams, ctx.fparams = list(iparams), list(fparams)


def _rad_energy_backward(ctx, g):
    _once_differentiable()
    if any(ctx.needs_input_grad[1:4]) or ctx.needs_input_grad[5]:
        raise NotImplementedError("sh_radial_message_energy differentiates the edge vectors "
                                  "only; train the weights with the A-row kernels")
    vec, rbf_table, W, U, ptr_dst, perm_dst = ctx.saved_tensors
    # a broadcast cotangent (d sum_i E_i, or its -1 seed) is read as one value
    stride = 0 if (g.dim() == 1 and g.stride(0) == 0) else 1
    g = g.to(torch.float32)
    if stride == 1:
        g = g.contiguous()
    g_vec = torch.empty_like(vec)
    _lib.call("xnn_sh_radial_message_energy_backward", _lib.XNN_F32, _lib.ptr(vec), None,
              ptr_dst.shape[0] - 1, None, 0, None, None, None, vec.shape[0], _lib.ptr(ptr_dst),
              _lib.ptr(perm_dst), _params(ctx.iparams, ctx.fparams), _lib.ptr(rbf_table),
              W.shape[1], _lib.ptr(W), _lib.ptr(U), _lib.ptr(g), stride, _lib.ptr(g_vec),
              _lib.stream(vec.device))
    return (g_vec,) + (None,) * 9


sh_radial_message_energy_op.register_autograd(_rad_energy_backward,
                                              setup_context=_rad_energy_setup)


class MessageEnergyOnePass(torch.autograd.Function):
    """Per-atom energies ``<U, A_i> + bias[z_i]`` and their edge-vector gradients from one
    launch of the readout backward (``xnn_sh_radial_message_energy_forces``): each edge's
    share ``(phi_e U) . Y_e`` of its receiver's ``<U, A_i>`` comes out of the backward's own
    dY, the atoms' energies are their CSR sums plus the bias (``xnn_node_energy_from_edges``),
    and no forward launch runs. The gradients are formed for the cotangent -1 of every atom
    (the forces' seed, the tensor the force outputs pass); an edge feeds its receiver's
    energy only, so another cotangent scales each edge's stored gradient by its receiver's
    value: exact for any cotangent."""

    @staticmethod
    def forward(ctx, vec, rbf_table, W, U, z, bias, ptr_dst, perm_dst, dst, iparams, fparams):
        from .outputs import _minus_one
        dev = vec.device
        n_nodes = ptr_dst.shape[0] - 1
        g_vec = torch.empty_like(vec)
        edge_energy = torch.empty(vec.shape[0], dtype=torch.float32, device=dev)
        seed = _minus_one(edge_energy)
        _lib.call("xnn_sh_radial_message_energy_forces", _lib.XNN_F32, _lib.ptr(vec), None,
                  n_nodes, None, 0, None, None, None, vec.shape[0], _lib.ptr(ptr_dst),
                  _lib.ptr(perm_dst), _params(iparams, fparams), _lib.ptr(rbf_table),
                  W.shape[1], _lib.ptr(W), _lib.ptr(U), _lib.ptr(seed), 0,
                  _lib.ptr(g_vec), _lib.ptr(edge_energy), _lib.stream(dev))
        node = torch.empty(n_nodes, dtype=torch.float32, device=dev)
        _lib.call("xnn_node_energy_from_edges", _lib.ptr(edge_energy), _lib.ptr(ptr_dst),
                  _lib.ptr(perm_dst), n_nodes, _lib.ptr(z), _lib.ptr(bias),
                  0 if bias is None else bias.shape[0], _lib.ptr(node), _lib.stream(dev))
        ctx.save_for_backward(g_vec, dst, seed)
        return node

    @staticmethod
    def backward(ctx, g):
        _once_differentiable()
        g_vec, dst, seed = ctx.saved_tensors
        g = g.to(torch.float32)
        broadcast = g.dim() == 1 and g.stride(0) == 0
        if broadcast and g.data_ptr() == seed.data_ptr():   # the forces' own -1 seed
            return (g_vec,) + (None,) * 10
        if broadcast:                                       # one value for every atom
            return (g_vec * (-g[:1]),) + (None,) * 10
        return (g_vec * (-g).index_select(0, dst.long())[:, None],) + (None,) * 10


def sh_radial_message_energy(vec: Tensor, rbf_table: Tensor, W: Tensor, U: Tensor, z: Tensor,
                             bias: Optional[Tensor], plan: EdgePlan, *, basis: str,
                             envelope: str, poly_p: int, l_max: int, cutoff: float,
                             prefactor: float = 1.0, gamma: float = 1.0,
                             sh_sign: int = 1, one_pass: bool = False) -> Tensor:
    """:func:`sh_radial_message_sum` read out in the kernel: the per-atom energies
    ``<U, A_i> + bias[z_i]`` (U: (C, (l_max+1)^2), bias indexed by ``z``, may be None);
    differentiable in ``vec`` only. ``one_pass``: when ``vec`` wants gradients, energies
    and gradients from one backward launch (:class:`MessageEnergyOnePass`)."""
    if vec.dtype != torch.float32 or W.dtype != torch.float32 or U.dtype != torch.float32:
        raise TypeError("sh_radial_message_energy computes in float32")
    n_rbf, C = W.shape
    L = (int(l_max) + 1) ** 2
    if rbf_table.numel() != n_rbf:
        raise ValueError("W needs one row per radial basis function")
    if U.numel() != C * L:
        raise ValueError(f"U needs {C} x {L} readout weights")
    if not linear_message_supported(n_rbf, C, l_max):
        raise ValueError(f"sh_radial_message_energy takes {LINEAR_MESSAGE_CHANNELS} channels, at "
                         f"most {LINEAR_MESSAGE_MAX_FEATURES} basis functions and l_max in [1, 3]")
    iparams = [int(n_rbf), _lib.BASIS[basis], _lib.ENVELOPE[envelope], int(poly_p), int(l_max),
               int(sh_sign)]
    fparams = [float(cutoff), float(prefactor), float(gamma)]
    table = rbf_table.to(device=vec.device, dtype=torch.float32).contiguous()
    b = None if bias is None else bias.to(device=vec.device, dtype=torch.float32).contiguous()
    if one_pass and torch.is_grad_enabled() and vec.requires_grad:
        return MessageEnergyOnePass.apply(vec.contiguous(), table, W.contiguous(),
                                          U.reshape(-1).contiguous(),
                                          z.to(torch.int64).contiguous(), b, plan.ptr_dst,
                                          plan.perm_dst, plan.dst, iparams, fparams)
    return sh_radial_message_energy_op(vec.contiguous(), table, W.contiguous(),
                                       U.reshape(-1).contiguous(), z.to(torch.int64).contiguous(),
                                       b, plan.ptr_dst, plan.perm_dst, iparams, fparams)


# --------------------------------------------------------------------------- segment sums
@torch.library.custom_op(f"{_NS}::segment_sum", mutates_args=())
def segment_sum_op(src: Tensor, index32: Tensor, ptr: Tensor, perm: Optional[Tensor]) -> Tensor:
    """``out[i] = sum over rows e with index[e] = i of src[e]`` via the CSR ``ptr``/``perm``."""
    dev = _require_gpu(src)
    n_seg = ptr.shape[0] - 1
    feat = src.shape[1:]
    F = 1
    for d in feat:
        F *= int(d)
    out = src.new_empty((n_seg, *feat))
    _lib.call("xnn_segment_sum", _lib.dtype_code(src.dtype), _lib.ptr(src), src.shape[0], F,
              _lib.ptr(ptr), _lib.ptr(perm), n_seg, _lib.ptr(out), _lib.stream(dev))
    return out


@segment_sum_op.register_fake
def _(src, index32, ptr, perm):
    return src.new_empty((ptr.shape[0] - 1, *src.shape[1:]))


def _gather(src: Tensor, index32: Tensor) -> Tensor:
    src = src.contiguous()
    feat = src.shape[1:]
    F = 1
    for d in feat:
        F *= int(d)
    out = src.new_empty((index32.shape[0], *feat))
    _lib.call("xnn_gather_rows", _lib.dtype_code(src.dtype), _lib.ptr(src), src.shape[0], F,
              _lib.ptr(index32), index32.shape[0], _lib.ptr(out), _lib.stream(src.device))
    return out


def _segment_sum_setup(ctx, inputs, output):
    src, index32, ptr, perm = inputs
    ctx.save_for_backward(index32, ptr, perm)


def _segment_sum_backward(ctx, grad):
    index32, ptr, perm = ctx.saved_tensors
    return gather_rows_op(grad.contiguous(), index32, ptr, perm), None, None, None


segment_sum_op.register_autograd(_segment_sum_backward, setup_context=_segment_sum_setup)


@torch.library.custom_op(f"{_NS}::gather_rows", mutates_args=())
def gather_rows_op(src: Tensor, index32: Tensor, ptr: Tensor, perm: Optional[Tensor]) -> Tensor:
    """``src[index]`` along dim 0; its adjoint is the CSR segment sum."""
    _require_gpu(src)
    return _gather(src, index32)


@gather_rows_op.register_fake
def _(src, index32, ptr, perm):
    return src.new_empty((index32.shape[0], *src.shape[1:]))


def _gather_setup(ctx, inputs, output):
    src, index32, ptr, perm = inputs
    ctx.save_for_backward(index32, ptr, perm)


def _gather_backward(ctx, grad):
    index32, ptr, perm = ctx.saved_tensors
    return segment_sum_op(grad.contiguous(), index32, ptr, perm), None, None, None


gather_rows_op.register_autograd(_gather_backward, setup_context=_gather_setup)


@torch.library.custom_op(f"{_NS}::structure_sum", mutates_args=())
def structure_sum_op(src: Tensor, node_ptr: Tensor, batch32: Tensor) -> Tensor:
    """Per-structure totals of per-atom values, accumulated and returned in float64."""
    dev = _require_gpu(src)
    n_seg = node_ptr.shape[0] - 1
    src = src.contiguous()
    F = 1
    for d in src.shape[1:]:
        F *= int(d)
    out = torch.empty((n_seg, *src.shape[1:]), dtype=torch.float64, device=dev)
    _lib.segment_reduce_f64(src, src.shape[0], F, node_ptr, n_seg, out)
    return out


@structure_sum_op.register_fake
def _(src, node_ptr, batch32):
    return src.new_empty((node_ptr.shape[0] - 1, *src.shape[1:]), dtype=torch.float64)


def _structure_sum_setup(ctx, inputs, output):
    src, node_ptr, batch32 = inputs
    ctx.save_for_backward(node_ptr, batch32)
    ctx.src_dtype = src.dtype
    ctx.src_shape = src.shape


def _structure_sum_backward(ctx, grad):
    # broadcast of every structure's cotangent to its atoms: the gather over batch,
    # whose own adjoint is the segment sum over node_ptr; one structure is a plain
    # broadcast (a stride-0 view, no kernel)
    node_ptr, batch32 = ctx.saved_tensors
    if node_ptr.shape[0] == 2:
        return grad.to(ctx.src_dtype).expand(ctx.src_shape), None, None
    g = gather_rows_op(grad.contiguous(), batch32, node_ptr.to(torch.int32), None)
    return g.to(ctx.src_dtype), None, None


structure_sum_op.register_autograd(_structure_sum_backward, setup_context=_structure_sum_setup)


@torch.library.custom_op(f"{_NS}::node_readout", mutates_args=())
def node_readout_op(rows: Tensor, weight: Tensor, z: Tensor, bias: Tensor) -> Tensor:
    """``out[i] = bias[z[i]] + rows[i] . weight`` for ``rows (N, F)``, in the rows' dtype:
    one wave per row streams it once (``torch.addmv`` with the gathered bias, as one
    launch). Differentiable once in every tensor input."""
    dev = _require_gpu(rows, weight, z, bias)
    rows = rows.contiguous()
    weight = weight.to(rows.dtype).contiguous()
    bias = bias.to(rows.dtype).contiguous()
    z = z.to(torch.int64).contiguous()
    n, F = rows.shape
    out = torch.empty(n, dtype=rows.dtype, device=dev)
    _lib.call("xnn_node_readout", _lib.dtype_code(rows.dtype), _lib.ptr(rows), n, F,
              _lib.ptr(weight), _lib.ptr(z), _lib.ptr(bias), bias.shape[0], _lib.ptr(out),
              _lib.stream(dev))
    return out


@node_readout_op.register_fake
def _(rows, weight, z, bias):
    return rows.new_empty(rows.shape[0])


def _readout_setup(ctx, inputs, output):
    rows, weight, z, bias = inputs
    ctx.save_for_backward(rows if ctx.needs_input_grad[1] else None, weight, z)
    ctx.n_bias, ctx.bias_dtype, ctx.weight_dtype = bias.shape[0], bias.dtype, weight.dtype


def _readout_backward(ctx, grad):
    _once_differentiable()
    rows, weight, z = ctx.saved_tensors
    n = grad.shape[0]
    d_rows = d_weight = d_bias = None
    if ctx.needs_input_grad[0]:
        w = weight.to(grad.dtype).contiguous()
        F = w.shape[0]
        # a broadcast cotangent (the -1 seed of a force evaluation) is read as one value
        g = grad if (grad.dim() == 1 and grad.stride(0) == 0) else grad.contiguous()
        d_rows = torch.empty((n, F), dtype=grad.dtype, device=grad.device)
        _lib.call("xnn_node_readout_backward", _lib.dtype_code(grad.dtype), _lib.ptr(g),
                  0 if g.stride(0) == 0 else 1, n, F, _lib.ptr(w), _lib.ptr(d_rows),
                  _lib.stream(grad.device))
    if ctx.needs_input_grad[1]:
        d_weight = (rows.t() @ grad).to(ctx.weight_dtype)
    if ctx.needs_input_grad[3]:
        d_bias = torch.zeros(ctx.n_bias, dtype=grad.dtype, device=grad.device).index_add_(
            0, z, grad).to(ctx.bias_dtype)
    return d_rows, d_weight, None, d_bias


node_readout_op.register_autograd(_readout_backward, setup_context=_readout_setup)


# --------------------------------------------------------------------------- radial network
@torch.library.custom_op(f"{_NS}::radial_hidden", mutates_args=())
def radial_hidden_op(x: Tensor, weights: List[Tensor], scales: List[float]) -> Tensor:
    """``s_n = silu(c_n s_{n-1} A_n)`` over 1-3 hidden layers (``xnn_radial_hidden``);
    differentiable through :class:`xnn_amd.radial.FusedHidden`."""
    _require_gpu(x, *weights)
    out = x.new_empty((x.shape[0], weights[-1].shape[1]))
    _lib.radial_hidden(x, weights, scales, out)
    return out


@radial_hidden_op.register_fake
def _(x, weights, scales):
    return x.new_empty((x.shape[0], weights[-1].shape[1]))


@torch.library.custom_op(f"{_NS}::radial_hidden_backward", mutates_args=())
def radial_hidden_backward_op(x: Tensor, grad_out: Tensor, weights: List[Tensor],
                              scales: List[float]) -> Tensor:
    """Input gradient of :func:`radial_hidden_op`, activations recomputed."""
    _require_gpu(x, grad_out, *weights)
    gx = torch.empty_like(x)
    _lib.radial_hidden(x, weights, scales, gx, grad_out=grad_out)
    return gx


@radial_hidden_backward_op.register_fake
def _(x, grad_out, weights, scales):
    return torch.empty_like(x)


# --------------------------------------------------------------------------- uvu convolution
def _uvu_dims(h: Tensor, y: Tensor, w: Tensor):
    return int(h.shape[1]), int(y.shape[1]), int(w.shape[1])


@torch.library.custom_op(f"{_NS}::uvu_conv", mutates_args=())
def uvu_conv_op(h: Tensor, y: Tensor, w: Tensor, weight_index: Optional[Tensor], src: Tensor,
                dst: Tensor, ptr_dst: Tensor, perm_dst: Optional[Tensor], ptr_src: Tensor,
                perm_src: Tensor, paths: List[int], coefs: List[float], dim_out: int,
                zero_grad_h: bool) -> Tensor:
    """Gather + uvu tensor product + receiver sum (``xnn_uvu_conv``); ``paths`` holds 9
    ints per path (``xnn_uvu_path``), ``coefs`` their scales (the divisor folded in)."""
    dev = _require_gpu(h, y, w)
    d1, d2, dw = _uvu_dims(h, y, w)
    n, e = int(h.shape[0]), int(src.shape[0])
    out = torch.empty((n, dim_out), dtype=torch.float32, device=dev)
    _lib.call("xnn_uvu_conv", _lib.ptr(h), n, d1, _lib.ptr(y), d2, _lib.ptr(w), int(w.shape[0]),
              dw, _lib.ptr(weight_index), _lib.ptr(src), e, _lib.ptr(ptr_dst), _lib.ptr(perm_dst),
              _lib.uvu_paths(paths, coefs), len(coefs), _lib.ptr(out), dim_out, _lib.stream(dev))
    return out


@uvu_conv_op.register_fake
def _(h, y, w, weight_index, src, dst, ptr_dst, perm_dst, ptr_src, perm_src, paths, coefs,
      dim_out, zero_grad_h):
    return h.new_empty((h.shape[0], dim_out))


@torch.library.custom_op(f"{_NS}::uvu_conv_backward", mutates_args=())
def uvu_conv_backward_op(g: Tensor, h: Tensor, y: Tensor, w: Tensor,
                         weight_index: Optional[Tensor], src: Tensor, dst: Tensor,
                         ptr_dst: Tensor, perm_dst: Optional[Tensor], ptr_src: Tensor,
                         perm_src: Tensor, paths: List[int], coefs: List[float],
                         zero_grad_h: bool, want_h: bool, want_y: bool,
                         want_w: bool) -> Tuple[Tensor, Tensor, Tensor]:
    """``(d h, d Y, d w per edge)`` of :func:`uvu_conv_op` (empty tensors where not wanted)."""
    dev = _require_gpu(g, h, y, w)
    d1, d2, dw = _uvu_dims(h, y, w)
    n, e = int(h.shape[0]), int(src.shape[0])
    f32 = dict(dtype=torch.float32, device=dev)
    gh = ((torch.zeros if zero_grad_h else torch.empty)((n, d1), **f32) if want_h
          else torch.empty(0, **f32))
    gy = torch.empty((e, d2), **f32) if want_y else torch.empty(0, **f32)
    gw = torch.empty((e, dw), **f32) if want_w else torch.empty(0, **f32)
    table = _lib.uvu_paths(paths, coefs)
    need = (int(_lib.load().xnn_uvu_conv_workspace_bytes(e, d2, table, len(coefs)))
            if (want_y or want_h) else 0)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=dev) if need else None
    _lib.call("xnn_uvu_conv_backward", _lib.ptr(h), n, d1, _lib.ptr(y), d2, _lib.ptr(w),
              int(w.shape[0]), dw, _lib.ptr(weight_index), _lib.ptr(src), _lib.ptr(dst), e,
              _lib.ptr(ptr_dst), _lib.ptr(perm_dst), _lib.ptr(ptr_src), _lib.ptr(perm_src),
              table, len(coefs), _lib.ptr(g.contiguous()), int(g.shape[1]),
              _lib.ptr(gh) if want_h else None, _lib.ptr(gy) if want_y else None,
              _lib.ptr(gw) if want_w else None, _lib.ptr(ws), need, _lib.stream(dev))
    return gh, gy, gw


@uvu_conv_backward_op.register_fake
def _(g, h, y, w, weight_index, src, dst, ptr_dst, perm_dst, ptr_src, perm_src, paths, coefs,
      zero_grad_h, want_h, want_y, want_w):
    e = src.shape[0]
    return (h.new_empty(h.shape if want_h else (0,)), y.new_empty((e, y.shape[1]) if want_y else (0,)),
            w.new_empty((e, w.shape[1]) if want_w else (0,)))


def _uvu_setup(ctx, inputs, output):
    (h, y, w, widx, src, dst, ptr_dst, perm_dst, ptr_src, perm_src, paths, coefs, dim_out,
     zero_grad_h) = inputs
    ctx.save_for_backward(h, y, w, widx, src, dst, ptr_dst, perm_dst, ptr_src, perm_src)
    ctx.paths, ctx.coefs, ctx.zero_grad_h = paths, coefs, zero_grad_h


def _uvu_backward(ctx, g):
    _once_differentiable()
    h, y, w, widx, src, dst, ptr_dst, perm_dst, ptr_src, perm_src = ctx.saved_tensors
    need = ctx.needs_input_grad
    gh, gy, gw = uvu_conv_backward_op(g, h, y, w, widx, src, dst, ptr_dst, perm_dst, ptr_src,
                                      perm_src, ctx.paths, ctx.coefs, ctx.zero_grad_h,
                                      bool(need[0]), bool(need[1]), bool(need[2]))
    if need[2] and widx is not None:
        gw = torch.zeros_like(w).index_add_(0, widx.to(torch.int64), gw)
    return (gh if need[0] else None, gy if need[1] else None, gw if need[2] else None,
            None, None, None, None, None, None, None, None, None, None, None)


uvu_conv_op.register_autograd(_uvu_backward, setup_context=_uvu_setup)
