"""The reference's aggregation functions with the same signatures
(common/models/ops.py:403-557, 754-764), deterministic on the GPU.

On GPU tensors ``scatter_sum`` / ``gather_rows`` / ``structure_sum`` run the HIP
segmented reductions over a CSR of ``index`` (built once per index tensor and
cached by identity and contents version, like the reference's ``orderings``,
csr.py:35-51); on CPU
tensors they are the reference's ``index_add`` formulation.
"""
from __future__ import annotations

from typing import Tuple

import torch
from torch import Tensor

from . import _lib

_last = [None]


def _csr_key(index: Tensor, n: int) -> tuple:
    # the same tensor object with the same storage, contents version and size: an index
    # changed in place (its _version moves) or rebound to other memory gets a new CSR
    return (index.data_ptr(), index._version, index.numel(), index.dtype, n)


def csr_of(index: Tensor, n: int) -> Tuple[Tensor, Tensor, object]:
    """``(index32, ptr (n+1), perm or None)`` of a 1-D index over ``n`` buckets; the last
    one is cached for the same index tensor while its contents are unchanged."""
    hit = _last[0]
    key = _csr_key(index, n)
    if hit is not None and hit[0] is index and hit[1] == key:
        return hit[2]
    from .plan import build_plan
    pair = torch.stack([index, index]).to(torch.int64)
    plan = build_plan(pair, None, n)
    out = (plan.dst, plan.ptr_dst, plan.perm_dst)
    _last[0] = (index, key, out)
    return out


def scatter_sum(src: Tensor, index: Tensor, dim_size: int) -> Tensor:
    """``out[index[e]] += src[e]`` over dim 0 (ops.py:403-448), without atomics on a GPU."""
    if not src.is_cuda:
        if dim_size == 1:
            return src.sum(0, keepdim=True)
        out = torch.zeros([dim_size] + list(src.shape[1:]), dtype=src.dtype, device=src.device)
        return out.index_add_(0, index, src)
    from .ops import segment_sum_op
    index32, ptr, perm = csr_of(index, dim_size)
    return segment_sum_op(src.contiguous(), index32, ptr, perm)


def gather_rows(src: Tensor, index: Tensor) -> Tensor:
    """``src[index]`` along dim 0 (ops.py:494-528); its adjoint is :func:`scatter_sum`."""
    if not src.is_cuda:
        return src.index_select(0, index)
    from .ops import gather_rows_op
    index32, ptr, perm = csr_of(index, src.shape[0])
    return gather_rows_op(src.contiguous(), index32, ptr, perm)


def structure_sum(src: Tensor, index: Tensor, dim_size: int) -> Tensor:
    """Per-structure totals accumulated in float64 (ops.py:531-557), for any ``index``.

    On a GPU the rows are summed along the CSR of ``index``: an index grouped by
    structure (as :func:`~xnn_amd.data.collate` builds it) is summed in place, any other
    is first gathered into structure order by the CSR's stable permutation (each
    structure's rows keep their relative order, as the CPU ``index_add`` visits them)."""
    if not src.is_cuda:
        if dim_size == 1:
            return src.to(torch.float64).sum(0, keepdim=True)
        out = torch.zeros(dim_size, dtype=torch.float64, device=src.device)
        return out.index_add(0, index, src.to(torch.float64))
    from .ops import structure_sum_op
    index32, ptr, perm = csr_of(index, dim_size)
    node_ptr = ptr.to(torch.int64)
    if perm is None:
        return structure_sum_op(src, node_ptr, index32)
    order = perm.to(torch.int64)
    return structure_sum_op(src.index_select(0, order), node_ptr,
                            index32.index_select(0, order))


def cell_volume(cell: Tensor) -> Tensor:
    """Volume of row-vector cells ``(..., 3, 3)`` by the triple product (ops.py:754-764)."""
    cross = torch.linalg.cross(cell[..., 1, :], cell[..., 2, :])
    return (cell[..., 0, :] * cross).sum(-1).abs()


__all__ = ["scatter_sum", "gather_rows", "structure_sum", "cell_volume", "csr_of"]
_ = _lib
