"""TEST INFRASTRUCTURE ONLY: CPU restatement of the equivariant convolution's message step.

Checker of ``xnn_amd.conv`` / ``xnn_amd.irreps`` (the ``uvu`` tensor product of
``ConvTensorProduct.conv``, gnn/fast/conv.py:93-143, reference path 137-143: gather the
sender rows, e3nn ``TensorProduct``, ``scatter_sum``, divide). Float64 NumPy, edge by edge.

* :func:`wigner_3j` -- the real-basis Clebsch-Gordan tensor of e3nn 0.5: SymPy's
  Clebsch-Gordan coefficients (``sympy.physics.wigner.clebsch_gordan``, Condon-Shortley
  phase; an implementation independent of the product's Racah sum) carried to the real
  basis by e3nn's ``change_basis_real_to_complex`` (rows complex m, columns real m', times
  ``(-i)^l``), unit Frobenius norm.
* :func:`path_coefficients` -- e3nn's normalization of each instruction
  (``irrep_normalization="component"``, ``path_normalization="element"``, unit variances):
  ``sqrt(dim(l_out) / sum over the instructions into that output of mul_2)``.
* :func:`uvu_conv` -- the message step by brute force.
* :func:`uvu_conv_torch` -- the same sums in float64 PyTorch, each instruction over all
  edges at once, differentiable (for forces of a stacked model); pinned to
  :func:`uvu_conv` by ``tests/test_conv.py``.
"""
from __future__ import annotations

import functools
from typing import List, Optional, Sequence, Tuple

import numpy as np


def _q(l: int) -> np.ndarray:
    q = np.zeros((2 * l + 1, 2 * l + 1), dtype=np.complex128)
    s = 1.0 / np.sqrt(2.0)
    for m in range(1, l + 1):
        q[l - m, l + m] = s                     # complex -m from real +m and -m
        q[l - m, l - m] = -1j * s
        q[l + m, l + m] = (-1) ** m * s         # complex +m
        q[l + m, l - m] = 1j * (-1) ** m * s
    q[l, l] = 1.0
    return (-1j) ** l * q


@functools.lru_cache(maxsize=None)
def wigner_3j(l1: int, l2: int, l3: int) -> np.ndarray:
    from sympy.physics.wigner import clebsch_gordan
    cg = np.zeros((2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1))
    for m1 in range(-l1, l1 + 1):
        for m2 in range(-l2, l2 + 1):
            m3 = m1 + m2
            if abs(m3) <= l3:
                cg[l1 + m1, l2 + m2, l3 + m3] = float(clebsch_gordan(l1, l2, l3, m1, m2, m3))
    c = np.einsum("ij,kl,mn,ikn->jlm", _q(l1), _q(l2), np.conj(_q(l3).T), cg.astype(np.complex128))
    assert np.abs(c.imag).max() < 1e-12
    c = c.real
    return c / np.linalg.norm(c)


def parse_irreps(s: str) -> List[Tuple[int, int, int]]:
    """``"8x0e+8x1o"`` -> ``[(mul, l, p)]``."""
    out = []
    for part in s.split("+"):
        part = part.strip()
        mul, ir = part.split("x") if "x" in part else ("1", part)
        out.append((int(mul), int(ir[:-1]), 1 if ir[-1] == "e" else -1))
    return out


def offsets(irreps: Sequence[Tuple[int, int, int]]) -> List[int]:
    out, i = [], 0
    for mul, l, _ in irreps:
        out.append(i)
        i += mul * (2 * l + 1)
    return out


def path_coefficients(irreps1, irreps2, irreps_out, instructions) -> List[float]:
    coefs = []
    for a, b, c in instructions:
        x = sum(irreps2[bb][0] for _, bb, cc in instructions if cc == c)
        coefs.append(float(np.sqrt((2 * irreps_out[c][1] + 1) / x)))
    return coefs


def uvu_conv(h: np.ndarray, y: np.ndarray, w: np.ndarray, src: np.ndarray, dst: np.ndarray,
             n_nodes: int, irreps1: str, irreps2: str, irreps_out: str,
             instructions: Sequence[Tuple[int, int, int]], divisor: Optional[float] = None,
             weight_index: Optional[np.ndarray] = None) -> np.ndarray:
    """Sum over edges of the uvu product of ``h[src]`` with ``y`` under ``w``, onto ``dst``."""
    i1, i2, io = parse_irreps(irreps1), parse_irreps(irreps2), parse_irreps(irreps_out)
    o1, o2, oo = offsets(i1), offsets(i2), offsets(io)
    coefs = path_coefficients(i1, i2, io, instructions)
    dim_out = sum(m * (2 * l + 1) for m, l, _ in io)
    out = np.zeros((n_nodes, dim_out))
    w_off, offs = 0, []
    for a, b, c in instructions:
        offs.append(w_off)
        w_off += i1[a][0] * i2[b][0]
    for e in range(len(src)):
        row = e if weight_index is None else int(weight_index[e])
        for (a, b, c), coef, wo in zip(instructions, coefs, offs):
            mul, l1, _ = i1[a]
            _, l2, _ = i2[b]
            _, l3, _ = io[c]
            x1 = h[src[e], o1[a]:o1[a] + mul * (2 * l1 + 1)].reshape(mul, 2 * l1 + 1)
            x2 = y[e, o2[b]:o2[b] + 2 * l2 + 1]
            wp = w[row, wo:wo + mul]
            C = wigner_3j(l1, l2, l3)
            msg = coef * np.einsum("u,ijk,ui,j->uk", wp, C, x1, x2)
            out[dst[e], oo[c]:oo[c] + mul * (2 * l3 + 1)] += msg.reshape(-1)
    if divisor is not None:
        out = out / divisor
    return out


def uvu_conv_torch(h, y, w, src, dst, n_nodes: int, irreps1: str, irreps2: str,
                   irreps_out: str, instructions: Sequence[Tuple[int, int, int]],
                   divisor: Optional[float] = None):
    """:func:`uvu_conv` on torch tensors (float64), every edge of an instruction at once:
    ``out[dst, c] += coef w[e, path] C x1[src] x2[e]`` by ``index_add``; differentiable in
    ``h``, ``y`` and ``w``."""
    import torch
    i1, i2, io = parse_irreps(irreps1), parse_irreps(irreps2), parse_irreps(irreps_out)
    o1, o2, oo = offsets(i1), offsets(i2), offsets(io)
    coefs = path_coefficients(i1, i2, io, instructions)
    dim_out = sum(m * (2 * l + 1) for m, l, _ in io)
    E = y.shape[0]
    blocks = [None] * len(io)
    wo = 0
    for (a, b, c), coef in zip(instructions, coefs):
        mul, l1, _ = i1[a]
        _, l2, _ = i2[b]
        _, l3, _ = io[c]
        x1 = h.index_select(0, src)[:, o1[a]:o1[a] + mul * (2 * l1 + 1)].reshape(E, mul, 2 * l1 + 1)
        x2 = y[:, o2[b]:o2[b] + 2 * l2 + 1]
        wp = w[:, wo:wo + mul]
        wo += mul * i2[b][0]
        C = torch.as_tensor(wigner_3j(l1, l2, l3), dtype=h.dtype, device=h.device)
        msg = coef * torch.einsum("eu,ijk,eui,ej->euk", wp, C, x1, x2)
        part = h.new_zeros(n_nodes, mul * (2 * l3 + 1)).index_add(0, dst, msg.reshape(E, -1))
        blocks[c] = part if blocks[c] is None else blocks[c] + part
    out = torch.cat([blk if blk is not None else h.new_zeros(n_nodes, io[k][0] * (2 * io[k][1] + 1))
                     for k, blk in enumerate(blocks)], dim=1) if io else h.new_zeros(n_nodes, 0)
    assert out.shape[1] == dim_out
    return out / divisor if divisor is not None else out
