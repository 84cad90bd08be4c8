"""TEST INFRASTRUCTURE ONLY: CPU restatement of the per-edge radial network.

Checker of ``xnn_amd.radial`` (``RadialNet`` and the fused hidden-layer kernel). It
evaluates the network the way e3nn 0.5's ``FullyConnectedNet`` does, layer by layer and
unfolded, in float64 NumPy (the layer rule of e3nn's ``nn._fc._Layer``, which the
reference's ``RadialNet`` subclasses, gnn/models/blocks.py:223-260):

    act layer:   y = cst f(x W / sqrt(h_in var_in)) sqrt(var_out)
    last layer:  y = x W / sqrt(h_in var_in / var_out)      (act too when out_act)

with ``cst = E[f(z)^2]^(-1/2)``, ``z ~ N(0, 1)`` (e3nn ``normalize2mom``), which this module
computes by Gauss-Hermite quadrature (the exact integral; e3nn and the product estimate
it from 10^6 seeded draws, so the two agree to the sampling error only).
"""
from __future__ import annotations

import math
from typing import Callable, Optional, Sequence

import numpy as np


def silu(z: np.ndarray) -> np.ndarray:
    return z / (1.0 + np.exp(-z))


def dsilu(z: np.ndarray) -> np.ndarray:
    s = 1.0 / (1.0 + np.exp(-z))
    return s * (1.0 + z * (1.0 - s))


def exact_second_moment_constant(f: Callable[[np.ndarray], np.ndarray], n: int = 200) -> float:
    """``E[f(z)^2]^(-1/2)`` for ``z ~ N(0, 1)`` by probabilists' Gauss-Hermite quadrature."""
    x, w = np.polynomial.hermite_e.hermegauss(n)
    return float((np.sum(w * f(x) ** 2) / math.sqrt(2.0 * math.pi)) ** -0.5)


def fully_connected(x: np.ndarray, weights: Sequence[np.ndarray], cst: float,
                    f: Callable[[np.ndarray], np.ndarray] = silu, variance_in: float = 1.0,
                    variance_out: float = 1.0, out_act: bool = False) -> np.ndarray:
    """The network on ``x`` (E, hs[0]) layer by layer, float64."""
    x = np.asarray(x, dtype=np.float64)
    var_in = variance_in
    n = len(weights)
    for i, w in enumerate(weights):
        w = np.asarray(w, dtype=np.float64)
        last = i == n - 1
        var_out = variance_out if last else 1.0
        h_in = w.shape[0]
        if (not last) or out_act:
            x = cst * f(x @ (w / math.sqrt(h_in * var_in))) * math.sqrt(var_out)
        else:
            x = x @ (w / math.sqrt(h_in * var_in / var_out))
        var_in = var_out
    return x


def hidden_chain(x: np.ndarray, weights: Sequence[np.ndarray], scales: Sequence[float]):
    """``s_n = silu(c_n s_{n-1} A_n)``: the fused kernel's contract, float64; returns the
    output and a function of the output cotangent giving the input cotangent."""
    s = [np.asarray(x, dtype=np.float64)]
    z = []
    for w, c in zip(weights, scales):
        z.append(c * (s[-1] @ np.asarray(w, dtype=np.float64)))
        s.append(silu(z[-1]))

    def vjp(g: np.ndarray) -> np.ndarray:
        g = np.asarray(g, dtype=np.float64)
        for n in range(len(weights) - 1, -1, -1):
            g = (scales[n] * (g * dsilu(z[n]))) @ np.asarray(weights[n], dtype=np.float64).T
        return g

    return s[-1], vjp


def fully_connected_torch(x, weights, cst: float, f=None, variance_in: float = 1.0,
                          variance_out: float = 1.0):
    """:func:`fully_connected` on torch tensors (float64, SiLU by default), differentiable."""
    import torch
    f = torch.nn.functional.silu if f is None else f
    var_in = variance_in
    n = len(weights)
    for i, w in enumerate(weights):
        last = i == n - 1
        var_out = variance_out if last else 1.0
        h_in = w.shape[0]
        if not last:
            x = cst * f(x @ (w / math.sqrt(h_in * var_in))) * math.sqrt(var_out)
        else:
            x = x @ (w / math.sqrt(h_in * var_in / var_out))
        var_in = var_out
    return x
