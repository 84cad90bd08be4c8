"""The per-edge radial network (``RadialNet``) with its hidden layers on one HIP kernel.

* :class:`Normalize2Mom` -- e3nn 0.5's ``normalize2mom`` (an activation scaled to unit
  second moment under a standard normal input), the activation wrapper of the reference's
  networks (gnn/models/blocks.py:17, 194; e3nn is a dependency the reference imports).
* :class:`FullyConnectedNet` -- e3nn 0.5's ``FullyConnectedNet`` layers: the parameters
  ``layer{i}.weight`` of shape ``(h_in, h_out)`` and
  ``act(x @ W / sqrt(h_in var_in)) sqrt(var_out)`` per layer, the last one without the
  activation unless ``out_act``.
* :class:`RadialNet` -- gnn/models/blocks.py:223-417: the same network with the scalar
  factors folded into one product per layer and an optional column map of the output
  (``out_index``, ``out_scale``); on the fast path its hidden SiLU layers run as one HIP
  kernel per direction (``xnn_radial_hidden``), which replaces the reference's Triton
  ``FusedHidden`` (gnn/fast/radial_kernels.py:43-152). The kernel takes one to three hidden
  layers (the reference's takes exactly three).
* :class:`FusedHidden` -- the autograd of that kernel: the input gradient on the HIP
  backward kernel, and the PyTorch formula (differentiable again) when the weights'
  gradients are wanted or the backward is itself differentiated, as in
  radial_kernels.py:98-133.
"""
from __future__ import annotations

import math
from typing import Callable, List, NamedTuple, Optional, Sequence, Tuple

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from .fast import FastPathModule

#: hidden layers of a radial network recompute their activations in the backward from
#: this many edges on (``recompute="auto"``, evaluation mode; blocks.py:212-220)
RECOMPUTE_MIN_EDGES = 1_000_000
#: limits of the fused kernel
MAX_FUSED_LAYERS = 3
MAX_FUSED_WIDTH = 128
MAX_FUSED_INPUTS = 32


def shifted_softplus(x: Tensor) -> Tensor:
    """``softplus(x) - log 2`` (blocks.py:31-38)."""
    return F.softplus(x) - math.log(2.0)


#: scalar activations by name (blocks.py:31-38)
SCALAR_ACTIVATIONS = {"silu": F.silu, "tanh": torch.tanh, "abs": torch.abs,
                      "ssp": shifted_softplus, "None": None, None: None}


def second_moment_constant(f: Callable[[Tensor], Tensor]) -> float:
    """``E[f(z)^2]^(-1/2)`` for ``z ~ N(0, 1)`` as e3nn 0.5 estimates it: the mean over
    10^6 float64 draws of a CPU generator seeded with 0 (``e3nn.math.moment``)."""
    gen = torch.Generator(device="cpu").manual_seed(0)
    z = torch.randn(1_000_000, generator=gen, dtype=torch.float64)
    with torch.no_grad():
        return float(f(z).pow(2).mean().pow(-0.5))


class Normalize2Mom(nn.Module):
    """``cst * f(x)`` with ``cst`` = :func:`second_moment_constant` of ``f``; the identity
    scale when ``cst`` is within 1e-4 of one (e3nn 0.5 ``normalize2mom``)."""

    def __init__(self, f: Callable[[Tensor], Tensor]):
        super().__init__()
        self.f = f
        self.cst = second_moment_constant(f)
        self._is_id = abs(self.cst - 1.0) < 1e-4

    def forward(self, x: Tensor) -> Tensor:
        return self.f(x) if self._is_id else self.f(x).mul(self.cst)


class _Layer(nn.Module):
    """One layer of :class:`FullyConnectedNet` (e3nn 0.5 ``nn._fc._Layer``)."""

    def __init__(self, h_in: int, h_out: int, act: Optional[nn.Module], var_in: float,
                 var_out: float):
        super().__init__()
        self.weight = nn.Parameter(torch.randn(h_in, h_out))
        self.act = act
        self.h_in, self.h_out = h_in, h_out
        self.var_in, self.var_out = var_in, var_out

    def forward(self, x: Tensor) -> Tensor:
        if self.act is not None:
            x = x @ (self.weight / (self.h_in * self.var_in) ** 0.5)
            return self.act(x) * self.var_out ** 0.5
        return x @ (self.weight / (self.h_in * self.var_in / self.var_out) ** 0.5)


class FullyConnectedNet(nn.Sequential):
    """e3nn 0.5 ``FullyConnectedNet``: layers ``layer0 .. layer{n-1}`` between the widths
    ``hs``, each ``act`` (normalized to unit second moment) but the last."""

    def __init__(self, hs: Sequence[int], act: Optional[Callable] = None,
                 variance_in: float = 1.0, variance_out: float = 1.0, out_act: bool = False):
        super().__init__()
        self.hs = tuple(int(h) for h in hs)
        act = Normalize2Mom(act) if act is not None else None
        var_in = variance_in
        n = len(self.hs) - 1
        for i, (h1, h2) in enumerate(zip(self.hs, self.hs[1:])):
            last = i == n - 1
            var_out = variance_out if last else 1.0
            self.add_module(f"layer{i}", _Layer(h1, h2, act if (out_act or not last) else None,
                                                var_in, var_out))
            var_in = var_out


def _dsilu(z: Tensor) -> Tensor:
    s = torch.sigmoid(z)
    return s * (1.0 + z * (1.0 - s))


def _vjp_torch(x: Tensor, a: Sequence[Tensor], scales: Sequence[float],
               g: Tensor) -> List[Tensor]:
    """The backward of the fused layers in PyTorch operations (differentiable again):
    gradients of ``x`` and of each ``a_n`` (radial_kernels.py:90-101, with the factors)."""
    s = [x]
    z = []
    for w, c in zip(a, scales):
        z.append((s[-1] @ w) * c)
        s.append(F.silu(z[-1]))
    grads_w: List[Tensor] = [None] * len(a)  # type: ignore[list-item]
    for n in range(len(a) - 1, -1, -1):
        delta = g * _dsilu(z[n]) * scales[n]
        grads_w[n] = s[n].t() @ delta
        g = delta @ a[n].t()
    return [g] + grads_w


def _grad_node(t: Tensor):
    """The autograd node that produces ``t``'s gradient (its AccumulateGrad for a leaf)."""
    if t.grad_fn is not None:
        return t.grad_fn
    if not t.requires_grad:
        return None
    return t.view_as(t).grad_fn.next_functions[0][0]


def _executes(node) -> bool:
    """Whether the running backward reaches ``node`` (``True`` when unknown)."""
    if node is None:
        return False
    try:
        return bool(torch._C._will_engine_execute_node(node))
    except Exception:
        return True


class FusedHidden(torch.autograd.Function):
    """``silu(c_L silu(... silu(c_1 x A_1) ...) A_L)`` for ``x`` (E, K) in float32."""

    @staticmethod
    def forward(ctx, x: Tensor, scales: Tuple[float, ...], nodes, *a: Tensor) -> Tensor:
        from . import ops
        x = x.contiguous()
        a = tuple(w.contiguous() for w in a)
        out = ops.radial_hidden_op(x, list(a), list(scales))
        ctx.save_for_backward(x, *a)
        ctx.scales, ctx.nodes = scales, nodes
        return out

    @staticmethod
    def backward(ctx, g: Tensor):
        from . import ops
        x, *a = ctx.saved_tensors
        need = ctx.needs_input_grad
        want_w = [need[3 + i] and _executes(ctx.nodes[i]) for i in range(len(a))]
        if torch.is_grad_enabled() or any(want_w):
            grads = _vjp_torch(x, a, ctx.scales, g)
            gx = grads[0] if need[0] else None
            gw = [gr if nd else None for gr, nd in zip(grads[1:], need[3:])]
            return (gx, None, None, *gw)
        gx = ops.radial_hidden_backward_op(x, g.contiguous(), list(a), list(ctx.scales)) \
            if need[0] else None
        return (gx, None, None, *([None] * len(a)))


def fused_hidden(x: Tensor, weights: Sequence[Tensor], scales: Sequence[float]) -> Tensor:
    """The hidden SiLU layers on the HIP kernel; ``weights[n]`` of shape (in, out) carries
    the scalar factor ``scales[n]`` (applied to the product)."""
    nodes = tuple(_grad_node(w) if torch.is_grad_enabled() else None for w in weights)
    return FusedHidden.apply(x, tuple(float(c) for c in scales), nodes, *weights)


class _Stage(NamedTuple):
    """One layer as ``post * act(gain * (x @ weight))`` (``act`` None: ``gain * (x @ weight)``,
    the output variance already in ``gain``)."""
    weight: Tensor
    gain: float
    act: Optional[Callable[[Tensor], Tensor]]
    post: float


def _stages(net: nn.Module) -> Optional[List[_Stage]]:
    """The layers of a :class:`FullyConnectedNet` as stages (``None`` when a child is not
    one of its layers). e3nn's layer is ``act(x W / sqrt(h_in var_in)) sqrt(var_out)``, and a
    normalized activation carries its constant: both scalars are pulled out of the
    activation so that a stage's ``post`` can be merged into the next stage's ``gain``."""
    out: List[_Stage] = []
    for layer in net.children():
        if not isinstance(layer, _Layer):
            return None
        act, post = layer.act, math.sqrt(layer.var_out)
        if isinstance(act, Normalize2Mom):
            post = post if act._is_id else post * act.cst
            act = act.f
        gain = 1.0 / math.sqrt(layer.h_in * layer.var_in)
        if act is None:
            gain, post = gain * post, 1.0
        out.append(_Stage(layer.weight, gain, act, post))
    return out


def _wants_checkpoint(mode: str, training: bool, x: Tensor, depth: int) -> bool:
    """Whether the hidden activations are recomputed in the backward instead of kept:
    never for ``"off"``, a single layer or an input that needs no gradient; always for
    ``"on"``; for ``"auto"`` in evaluation mode from :data:`RECOMPUTE_MIN_EDGES` rows."""
    if mode == "off" or depth < 2 or not (torch.is_grad_enabled() and x.requires_grad):
        return False
    return mode == "on" or (not training and x.shape[0] >= RECOMPUTE_MIN_EDGES)


def _select_columns(y: Tensor, index: Optional[Tensor], scale: Optional[Tensor]) -> Tensor:
    if scale is None:
        return y
    if index is not None:
        y = y.index_select(-1, index)
    return y * scale


class RadialNet(FullyConnectedNet, FastPathModule):
    """Per-edge radial network (gnn/models/blocks.py:223-417).

    A :class:`FullyConnectedNet` (same parameters and ``state_dict`` keys) evaluated as
    stages ``post * act(gain * (x @ W))`` in which each stage's ``post`` is merged into the
    next stage's ``gain``, so that every layer costs one product and one scalar. With
    ``out_scale`` it returns the output columns ``out_index`` (all when None) times
    ``out_scale``; for a linear last layer the selection and scale are applied to its weight
    before the product. On the fast path (``fast_active``, evaluation mode, float32 on the
    GPU, one to three hidden SiLU layers of at most 128 units, at most 32 inputs) the hidden
    layers run on :func:`fused_hidden`; otherwise, with ``recompute`` ("auto": evaluation
    mode from :data:`RECOMPUTE_MIN_EDGES` edges; "on"; "off") they are recomputed in the
    backward by checkpointing, or kept.
    """

    def __init__(self, hs, act=None, variance_in=1, variance_out=1, out_act=False):
        super().__init__(hs, act, variance_in, variance_out, out_act)
        self.recompute = "auto"
        self.fast_active = False

    def fast_supported(self, device: torch.device, dtype: torch.dtype) -> bool:
        stages = _stages(self)
        if device.type != "cuda" or dtype != torch.float32 or stages is None:
            return False
        hidden = stages[:-1]
        return (1 <= len(hidden) <= MAX_FUSED_LAYERS and self.hs[0] <= MAX_FUSED_INPUTS
                and all(st.act is F.silu and st.weight.shape[1] <= MAX_FUSED_WIDTH
                        for st in hidden))

    @staticmethod
    def _run_hidden(x: Tensor, hidden: Sequence[_Stage]) -> Tensor:
        carry = 1.0
        for st in hidden:
            x = x @ (st.weight * (st.gain * carry))
            if st.act is not None:
                x = st.act(x)
            carry = st.post
        return x

    def forward(self, x: Tensor, out_index: Optional[Tensor] = None,
                out_scale: Optional[Tensor] = None) -> Tensor:
        stages = _stages(self)
        if stages is None:
            for layer in self:
                x = layer(x)
            return _select_columns(x, out_index, out_scale)
        shape = x.shape
        x = x.reshape(-1, shape[-1])
        hidden, last = stages[:-1], stages[-1]
        if (self.fast_active and not self.training and x.is_cuda
                and x.dtype == torch.float32 and hidden):
            carried = [1.0] + [st.post for st in hidden[:-1]]
            h = fused_hidden(x, [st.weight for st in hidden],
                             [st.gain * c for st, c in zip(hidden, carried)])
        elif _wants_checkpoint(self.recompute, self.training, x, len(stages)):
            from torch.utils.checkpoint import checkpoint
            h = checkpoint(self._run_hidden, x, hidden, use_reentrant=False)
        else:
            h = self._run_hidden(x, hidden)
        scale = last.gain * (hidden[-1].post if hidden else 1.0)
        if last.act is None:
            y = h @ (_select_columns(last.weight, out_index, out_scale) * scale)
        else:
            y = _select_columns(last.act(h @ (last.weight * scale)) * last.post, out_index,
                                out_scale)
        return y.reshape(shape[:-1] + y.shape[-1:])


def set_recompute_radial(model: nn.Module, recompute: str = "auto") -> nn.Module:
    """Set ``recompute`` ("auto", "on" or "off") on every :class:`RadialNet` of ``model``."""
    if recompute not in ("auto", "on", "off"):
        raise ValueError(f"recompute must be 'auto', 'on' or 'off', got {recompute!r}")
    for m in model.modules():
        if isinstance(m, RadialNet):
            m.recompute = recompute
    return model
