"""The message step of an equivariant convolution (gnn/fast/conv.py:24-441).

:class:`ConvTensorProduct` is the ``uvu`` tensor product of e3nn 0.5's ``TensorProduct``
(the reference subclasses it): for each instruction ``(i_in1, i_in2, i_out)``

    out[z, u, k] += c_p sum_{v, i, j} w[z, u, v] C[i, j, k] x1[z, u, i] x2[z, v, j]

with ``C`` the real Wigner 3j tensor (:func:`xnn_amd.irreps.wigner_3j`) and
``c_p = sqrt(alpha)`` from e3nn's normalization: ``alpha = dim(out irrep)`` for
``irrep_normalization="component"`` divided by, for ``path_normalization="element"``, the
sum over the instructions into the same output of ``in1_var in2_var mul2`` (times
``out_var`` and the path weight). Called as a module it is that product (PyTorch);
:meth:`ConvTensorProduct.conv` is the whole message step, gather + product + receiver sum
+ the message divisor, which on the fast path runs as one HIP kernel each way
(``xnn_uvu_conv``, ``xnn_uvu_conv_backward``) that never stores a per-edge message.
Fast-eligible products are those of the reference's fast path (conv.py:35-45): every
instruction ``uvu``, second operand of multiplicity one, one instruction per output
block, per-edge weights; here also degrees at most 3, at most 48 paths and 16 node-feature
blocks, and one second-operand block per degree (as the harmonics have).
"""
from __future__ import annotations

import math
from typing import List, Optional, Sequence, Tuple

import torch
from torch import Tensor, nn

from .fast import FastPathModule
from .irreps import Instruction, Irreps, wigner_3j

MAX_L = 3
MAX_PATHS = 48
MAX_DIM2 = 16
MAX_BLOCKS = 16


class ConvTensorProduct(nn.Module, FastPathModule):
    """``uvu`` tensor product with per-edge weights and a fused message pass."""

    def __init__(self, irreps_in1, irreps_in2, irreps_out, instructions: Sequence,
                 in1_var: Optional[List[float]] = None, in2_var: Optional[List[float]] = None,
                 out_var: Optional[List[float]] = None, irrep_normalization: str = "component",
                 path_normalization: str = "element", internal_weights: Optional[bool] = None,
                 shared_weights: Optional[bool] = None):
        super().__init__()
        self.irreps_in1 = Irreps(irreps_in1)
        self.irreps_in2 = Irreps(irreps_in2)
        self.irreps_out = Irreps(irreps_out)
        if shared_weights is None:
            shared_weights = True
        if internal_weights is None:
            internal_weights = shared_weights
        if internal_weights and not shared_weights:
            raise ValueError("internal weights are shared weights")
        self.shared_weights, self.internal_weights = bool(shared_weights), bool(internal_weights)
        ins = []
        for item in instructions:
            i1, i2, io, mode, has_w = item[:5]
            pw = float(item[5]) if len(item) > 5 else 1.0
            if mode != "uvu":
                raise NotImplementedError(f"connection mode {mode!r}: only 'uvu' is implemented")
            m1, m2, mo = self.irreps_in1[i1], self.irreps_in2[i2], self.irreps_out[io]
            if m1.mul != mo.mul:
                raise ValueError("uvu needs equal multiplicities of the first input and the output")
            if m1.ir.p * m2.ir.p != mo.ir.p or not abs(m1.ir.l - m2.ir.l) <= mo.ir.l <= m1.ir.l + m2.ir.l:
                raise ValueError(f"instruction {item} breaks the selection rules")
            ins.append(Instruction(i1, i2, io, mode, bool(has_w), pw))
        self.instructions = ins
        in1_var = in1_var or [1.0] * len(self.irreps_in1)
        in2_var = in2_var or [1.0] * len(self.irreps_in2)
        out_var = out_var or [1.0] * len(self.irreps_out)
        self.path_coefficients: List[float] = []
        for p in ins:
            mo = self.irreps_out[p.i_out]
            alpha = {"component": mo.ir.dim,
                     "norm": self.irreps_in1[p.i_in1].ir.dim * self.irreps_in2[p.i_in2].ir.dim,
                     "none": 1}[irrep_normalization]
            if path_normalization == "element":
                x = sum(in1_var[q.i_in1] * in2_var[q.i_in2] * self.irreps_in2[q.i_in2].mul
                        for q in ins if q.i_out == p.i_out)
            elif path_normalization == "path":
                x = in1_var[p.i_in1] * in2_var[p.i_in2] * self.irreps_in2[p.i_in2].mul
                x *= len([q for q in ins if q.i_out == p.i_out])
            else:
                x = 1.0
            if x > 0:
                alpha /= x
            alpha *= out_var[p.i_out] * p.path_weight
            self.path_coefficients.append(math.sqrt(alpha))
        # per-instruction weight offsets (path shape (mul1, mul2), instruction order)
        self.weight_offsets: List[int] = []
        n = 0
        for p in ins:
            self.weight_offsets.append(n)
            if p.has_weight:
                n += self.irreps_in1[p.i_in1].mul * self.irreps_in2[p.i_in2].mul
        self.weight_numel = n
        if self.internal_weights and n > 0:
            self.weight = nn.Parameter(torch.randn(n))
        else:
            self.register_parameter("weight", None)
        self.fast_active = False
        self.fast_eligible = (
            not self.shared_weights and not self.internal_weights
            and all(m.mul == 1 for m in self.irreps_in2)
            and len({p.i_out for p in ins}) == len(ins) == len(self.irreps_out)
            and all(p.has_weight for p in ins)
            and len(ins) <= MAX_PATHS and self.irreps_in2.dim <= MAX_DIM2
            and len(self.irreps_in1) <= MAX_BLOCKS
            and len({m.ir.l for m in self.irreps_in2}) == len(self.irreps_in2)
            and len({(p.i_in1, self.irreps_in2[p.i_in2].ir.l, self.irreps_out[p.i_out].ir.l)
                     for p in ins}) == len(ins)
            and max(m.ir.l for m in list(self.irreps_in1) + list(self.irreps_in2)
                    + list(self.irreps_out)) <= MAX_L)
        self.__dict__["_w3j"] = {}
        self.__dict__["_paths"] = None

    # ------------------------------------------------------------------ reference path
    def _c(self, l1: int, l2: int, l3: int, like: Tensor) -> Tensor:
        key = (l1, l2, l3, like.dtype, like.device)
        c = self._w3j.get(key)
        if c is None:
            c = torch.as_tensor(wigner_3j(l1, l2, l3), dtype=like.dtype, device=like.device)
            self._w3j[key] = c
        return c

    def forward(self, x1: Tensor, x2: Tensor, weight: Optional[Tensor] = None) -> Tensor:
        """The tensor product of ``x1`` (..., irreps_in1.dim) and ``x2`` (..., irreps_in2.dim)."""
        if weight is None:
            if not self.internal_weights:
                raise ValueError("the weights are an input of this product")
            weight = self.weight
        lead = torch.broadcast_shapes(x1.shape[:-1], x2.shape[:-1])
        x1 = x1.expand(lead + x1.shape[-1:]).reshape(-1, x1.shape[-1])
        x2 = x2.expand(lead + x2.shape[-1:]).reshape(-1, x2.shape[-1])
        z = x1.shape[0]
        w = weight.reshape(-1, self.weight_numel) if self.weight_numel else weight
        if w.dim() == 2 and w.shape[0] == 1 and z != 1:
            w = w.expand(z, -1)
        s1, s2, so = self.irreps_in1.slices(), self.irreps_in2.slices(), self.irreps_out.slices()
        blocks = [None] * len(self.irreps_out)
        for p, coef, off in zip(self.instructions, self.path_coefficients, self.weight_offsets):
            m1, m2, mo = self.irreps_in1[p.i_in1], self.irreps_in2[p.i_in2], self.irreps_out[p.i_out]
            a = x1[:, s1[p.i_in1]].reshape(z, m1.mul, m1.ir.dim)
            b = x2[:, s2[p.i_in2]].reshape(z, m2.mul, m2.ir.dim)
            c = self._c(m1.ir.l, m2.ir.l, mo.ir.l, x1)
            ab = torch.einsum("zui,zvj,ijk->zuvk", a, b, c)
            if p.has_weight:
                wp = w[:, off:off + m1.mul * m2.mul].reshape(z, m1.mul, m2.mul)
                r = torch.einsum("zuv,zuvk->zuk", wp, ab)
            else:
                r = ab.sum(2)
            r = (coef * r).reshape(z, mo.dim)
            blocks[p.i_out] = r if blocks[p.i_out] is None else blocks[p.i_out] + r
        out = [blk if blk is not None else x1.new_zeros(z, self.irreps_out[i].dim)
               for i, blk in enumerate(blocks)]
        out = torch.cat(out, dim=1) if out else x1.new_zeros(z, 0)
        return out.reshape(lead + (self.irreps_out.dim,))

    # ------------------------------------------------------------------ fast path
    def fast_supported(self, device: torch.device, dtype: torch.dtype) -> bool:
        return self.fast_eligible and device.type == "cuda" and dtype == torch.float32

    def weight_map(self, like: Tensor, message_divisor: Optional[float] = None
                   ) -> Tuple[Optional[Tensor], Optional[Tensor]]:
        """The kernels take the weights in the instruction order and scale them
        themselves: there is no column map (conv.py:47-80 returns one for its kernel)."""
        return None, None

    def path_table(self) -> Tuple[List[int], List[float]]:
        """``(ints, coefs)``: per path ``l1, l2, l3, mul, off1, off2, off_out, off_w,
        block`` (the node block read) and the path coefficients, in instruction order
        (``xnn_uvu_path``)."""
        if self._paths is None:
            s1, s2, so = self.irreps_in1.slices(), self.irreps_in2.slices(), self.irreps_out.slices()
            ints, seen = [], set()
            for p, off in zip(self.instructions, self.weight_offsets):
                m1, m2, mo = self.irreps_in1[p.i_in1], self.irreps_in2[p.i_in2], self.irreps_out[p.i_out]
                seen.add(p.i_in1)
                ints += [m1.ir.l, m2.ir.l, mo.ir.l, m1.mul, s1[p.i_in1].start, s2[p.i_in2].start,
                         so[p.i_out].start, off, p.i_in1]
            self.__dict__["_paths"] = (ints, list(self.path_coefficients),
                                       len(seen) == len(self.irreps_in1))
        return self._paths[0], self._paths[1]

    def conv(self, node_feats: Tensor, edge_attrs: Tensor, edge_weights: Tensor,
             edge_index: Tensor, num_nodes: int, message_divisor: Optional[float] = None,
             weights_mapped: bool = False, weight_index: Optional[Tensor] = None,
             plan=None) -> Tensor:
        """Gather, tensor product and sum onto the receivers (conv.py:93-143).

        ``edge_index`` (2, E): row 0 the senders, row 1 the receivers; ``weight_index``
        (E,): edge ``e`` takes weight row ``weight_index[e]``; ``message_divisor`` divides
        the sums. ``plan``: the :class:`~xnn_amd.plan.EdgePlan` of ``edge_index`` (built and
        cached here when omitted) on the fast path.
        """
        if self.fast_active:
            return self._conv_fast(node_feats, edge_attrs, edge_weights, edge_index, num_nodes,
                                   message_divisor, weight_index, plan)
        if weight_index is not None:
            edge_weights = edge_weights.index_select(0, weight_index)
        messages = self(node_feats.index_select(0, edge_index[0]), edge_attrs, edge_weights)
        out = messages.new_zeros(num_nodes, messages.shape[1]).index_add_(0, edge_index[1], messages)
        if message_divisor is not None:
            out = out / message_divisor
        return out

    def _conv_fast(self, node_feats, edge_attrs, edge_weights, edge_index, num_nodes,
                   message_divisor, weight_index, plan):
        from . import ops
        if plan is None:
            plan = plan_of(edge_index, num_nodes)
        ints, coefs = self.path_table()
        if message_divisor is not None:
            coefs = [c / message_divisor for c in coefs]
        widx = None
        if weight_index is not None:
            widx = weight_index.to(torch.int32).contiguous()
            if widx.numel() and (int(widx.min()) < 0 or int(widx.max()) >= edge_weights.shape[0]):
                raise IndexError("weight_index out of range of the weight rows")
        return ops.uvu_conv_op(node_feats.contiguous(), edge_attrs.contiguous(),
                               edge_weights.contiguous(), widx, plan.src, plan.dst, plan.ptr_dst,
                               plan.perm_dst, plan.ptr_src, plan.perm_src, ints, coefs,
                               self.irreps_out.dim, not self._paths[2])


_plan_cache = [None]


def plan_of(edge_index: Tensor, num_nodes: int):
    """The edge plan of ``edge_index`` (the last one is kept, keyed by identity)."""
    hit = _plan_cache[0]
    if hit is not None and hit[0] is edge_index and hit[1] == num_nodes \
            and hit[2] == edge_index._version:
        return hit[3]
    from .plan import build_plan
    plan = build_plan(edge_index, None, num_nodes)
    _plan_cache[0] = (edge_index, num_nodes, edge_index._version, plan)
    return plan
