"""Edge plans: the int32 edge streams and CSR orderings the HIP kernels walk.

An :class:`EdgePlan` is built once per edge list (on the device, by
``xnn_edge_plan``) and cached on the graph. It holds

* ``src``, ``dst`` (int32) and ``shift`` (three signed 10-bit fields in one
  int32) for every edge, in the edge list's own order;
* the receiver CSR ``ptr_dst`` with ``perm_dst`` (``None`` when the edges are
  already grouped by receiver, as :func:`~xnn_amd.data.build_neighbor_list`
  returns them), and the sender CSR ``ptr_src`` / ``perm_src``;
* the structure of every atom (``batch32``) and the structures' atom ranges
  (``node_ptr``, int64).

This mirrors the orderings of the reference's no-atomics kernels
(``common/models/csr.py:20-51``): every per-atom sum walks one CSR row in a
fixed order, so results are bitwise reproducible.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch
from torch import Tensor

from . import _lib


@dataclass
class EdgePlan:
    n_nodes: int
    n_edges: int
    n_graphs: int
    src: Tensor
    dst: Tensor
    shift: Tensor
    ptr_dst: Tensor
    perm_dst: Optional[Tensor]
    ptr_src: Tensor
    perm_src: Tensor
    batch32: Tensor
    node_ptr: Tensor
    # a space-filling-curve order of the atoms (structure by structure), the order in
    # which the force reductions take them; None: index order
    visit: Optional[Tensor] = None

    @property
    def device(self) -> torch.device:
        return self.ptr_dst.device


def build_plan(edge_index: Tensor, cell_shifts: Optional[Tensor], n_nodes: int,
               batch: Optional[Tensor] = None, n_atoms: Optional[Tensor] = None) -> EdgePlan:
    """Build the plan of an edge list on its (GPU) device.

    Raises ``ValueError`` for edge indices outside ``[0, n_nodes)``, image
    shifts outside ``[-512, 511]`` or atoms not grouped by structure.
    """
    device = edge_index.device
    if device.type != "cuda":
        raise ValueError("edge plans live on the GPU; move the graph to the device first")
    n_edges = int(edge_index.shape[1])
    edge_index = edge_index.to(torch.int64).contiguous()
    if cell_shifts is None or cell_shifts.numel() == 0:
        shifts = None
    else:
        shifts = cell_shifts.to(torch.int64).contiguous()
    i32 = dict(dtype=torch.int32, device=device)
    src = torch.empty(n_edges, **i32)
    dst = torch.empty(n_edges, **i32)
    shift = torch.empty(n_edges, **i32)
    ptr_dst = torch.empty(n_nodes + 1, **i32)
    ptr_src = torch.empty(n_nodes + 1, **i32)
    perm_dst = torch.empty(n_edges, **i32)
    perm_src = torch.empty(n_edges, **i32)
    flag = torch.empty(1, **i32)
    ws_bytes = int(_lib.load().xnn_edge_plan_workspace_bytes(n_edges, n_nodes))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=device)
    _lib.call("xnn_edge_plan", _lib.ptr(edge_index), _lib.ptr(shifts), n_edges, n_nodes,
              _lib.ptr(src), _lib.ptr(dst), _lib.ptr(shift), _lib.ptr(ptr_dst), _lib.ptr(perm_dst),
              _lib.ptr(ptr_src), _lib.ptr(perm_src), _lib.ptr(flag), _lib.ptr(ws), ws_bytes,
              _lib.stream(device))
    if batch is None:
        batch = torch.zeros(n_nodes, dtype=torch.int64, device=device)
    batch = batch.to(device)
    if n_atoms is None:
        n_atoms = torch.tensor([n_nodes], dtype=torch.int64, device=device)
    n_atoms = n_atoms.to(device=device, dtype=torch.int64)
    node_ptr = torch.zeros(n_atoms.shape[0] + 1, dtype=torch.int64, device=device)
    node_ptr[1:] = torch.cumsum(n_atoms, 0)
    # one host read: overflow flag, receiver grouping, structure grouping, atom count
    checks = [flag[0].to(torch.int64),
              (dst[1:] >= dst[:-1]).all().to(torch.int64) if n_edges > 1 else
              torch.ones((), dtype=torch.int64, device=device),
              (batch[1:] >= batch[:-1]).all().to(torch.int64) if n_nodes > 1 else
              torch.ones((), dtype=torch.int64, device=device),
              node_ptr[-1],
              ((batch >= 0) & (batch < n_atoms.shape[0])).all().to(torch.int64) if n_nodes > 0
              else torch.ones((), dtype=torch.int64, device=device)]
    overflow, grouped, batch_sorted, total, batch_ok = torch.stack(checks).tolist()
    if overflow & 2:
        raise ValueError(f"edge_index holds atom indices outside [0, {n_nodes})")
    if overflow & 1:
        raise ValueError("cell_shifts outside [-512, 511]: the packed int32 shifts cannot hold "
                         "them (wrap the positions into the cell first)")
    if not batch_ok:
        raise ValueError("batch holds structure indices outside [0, B)")
    if not batch_sorted:
        raise ValueError("the atoms of a batch must be grouped by structure (as collate does)")
    if total != n_nodes:
        raise ValueError(f"n_atoms sums to {total}, the graph has {n_nodes} atoms")
    return EdgePlan(n_nodes=n_nodes, n_edges=n_edges, n_graphs=int(n_atoms.shape[0]), src=src,
                    dst=dst, shift=shift, ptr_dst=ptr_dst, perm_dst=None if grouped else perm_dst,
                    ptr_src=ptr_src, perm_src=perm_src, batch32=batch.to(torch.int32),
                    node_ptr=node_ptr)


def _spread10(q: Tensor) -> Tensor:
    """The 10 low bits of ``q`` (int64) spread to every third bit (Morton interleave)."""
    q = (q | (q << 16)) & 0x030000FF
    q = (q | (q << 8)) & 0x0300F00F
    q = (q | (q << 4)) & 0x030C30C3
    return (q | (q << 2)) & 0x09249249


def spatial_order(pos: Tensor, cell: Optional[Tensor], batch: Tensor, n_graphs: int) -> Tensor:
    """The atoms sorted along a Morton (Z-order) curve of their positions, structure by
    structure, int32: fractional coordinates of the cell for one periodic structure, else
    the batch's bounding box, 10 bits per axis. Neighbours in space end up near one another
    in the order; an ordering hint only (nothing computed depends on it)."""
    p = pos.detach().to(torch.float64)
    if cell is not None and n_graphs == 1 and bool(torch.isfinite(p).all()):
        c = cell.detach().reshape(-1, 3, 3)[0].to(torch.float64)
        frac = p @ torch.linalg.inv(c)
        frac = frac - torch.floor(frac)
    else:
        lo, hi = p.min(0).values, p.max(0).values
        frac = (p - lo) / (hi - lo).clamp(min=1e-9)
    q = (frac * 1024.0).to(torch.int64).clamp(0, 1023)
    code = _spread10(q[:, 0]) | (_spread10(q[:, 1]) << 1) | (_spread10(q[:, 2]) << 2)
    key = (batch.to(torch.int64) << 30) | code
    return torch.argsort(key, stable=True).to(torch.int32)


def plan_for(graph) -> EdgePlan:
    """The cached plan of an :class:`~xnn_amd.data.AtomicGraph` (rebuilt when its edge
    list, shifts or atom count change identity)."""
    cached = getattr(graph, "_xnn_plan", None)
    # identity of the (held) tensors, as the reference's orderings cache (csr.py:35-51)
    if (cached is not None and cached[0] is graph.edge_index and cached[1] is graph.cell_shifts
            and cached[2] == graph.num_nodes):
        return cached[3]
    plan = build_plan(graph.edge_index, graph.cell_shifts, graph.num_nodes, graph.batch,
                      graph.n_atoms)
    if plan.n_nodes > 0:
        plan.visit = spatial_order(graph.pos, graph.cell, plan.batch32, plan.n_graphs)
    object.__setattr__(graph, "_xnn_plan",
                       (graph.edge_index, graph.cell_shifts, graph.num_nodes, plan))
    return plan
