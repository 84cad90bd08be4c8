"""Fast-path selection, as in the reference (common/models/fast.py:60-219).

A :class:`FastPathModule` keeps the parameters and buffers of its reference
formulation and adds a HIP evaluation; the owning model sets ``fast_active``
once per evaluation through :func:`select`. ``use_fast``:

``True``    the HIP kernels (raises if they cannot run on this device/dtype)
``False``   the PyTorch formulation of the reference
``"auto"``  the HIP kernels on a GPU (the MI355X entry of :data:`MI355X_POLICY`
            takes them from the first edge) for the modules that have them, the
            PyTorch formulation elsewhere

The HIP backward is differentiable once, so a training step that needs the
force loss's second derivative (``create_graph=True``) takes the PyTorch
formulation; :func:`select` sees it through ``double_backward``.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional, Union

import warnings

import torch
from torch import nn

from . import _lib

UseFast = Union[bool, str]


class FastPathPrecisionWarning(UserWarning):
    """A fast path ran in float32: results differ from the reference at ~1e-6
    (fast.py:41-42)."""


_warned_float32 = [False]


def warn_float32_once() -> None:
    """The float32 precision warning, once per process (fast.py:48-59)."""
    if _warned_float32[0]:
        return
    _warned_float32[0] = True
    warnings.warn(
        "The HIP fast path is running in float32: it evaluates the reference's function "
        "with another summation order, so energies and forces differ from the reference "
        "at about 1e-6 relative (float64: about 1e-14). use_fast=False selects the "
        "reference formulation.", FastPathPrecisionWarning, stacklevel=3)


def resolve_use_fast(use_fast: UseFast) -> UseFast:
    """Validate ``use_fast`` (``True``, ``False`` or ``"auto"``)."""
    if isinstance(use_fast, str):
        if use_fast.lower() != "auto":
            raise ValueError(f"use_fast must be True, False or 'auto', got {use_fast!r}")
        return "auto"
    if isinstance(use_fast, bool):
        return use_fast
    raise TypeError(f"use_fast must be True, False or 'auto', got {type(use_fast).__name__}")


class FastPathModule:
    """Mixin of a module with a reference and a HIP evaluation (fast.py:73-91)."""

    fast_active: bool = False

    def fast_supported(self, device: torch.device, dtype: torch.dtype) -> bool:
        return device.type == "cuda" and dtype in (torch.float32, torch.float64)


@dataclass
class AutoPolicy:
    """Minimum edge counts for ``use_fast="auto"`` keyed by a device-name substring
    (fast.py:99-168)."""

    min_edges: Dict[str, int] = field(default_factory=dict)
    default_min_edges: int = 0

    def decide(self, device: torch.device, dtype: torch.dtype, num_edges: int) -> bool:
        if device.type != "cuda":
            return False
        name = torch.cuda.get_device_name(device).lower()
        for key, value in self.min_edges.items():
            if key.lower() in name:
                return num_edges >= int(value)
        return num_edges >= self.default_min_edges


#: the kernels win from the first edge on MI355X (one launch per stage, no host syncs)
MI355X_POLICY = AutoPolicy(min_edges={"MI355": 0, "gfx950": 0}, default_min_edges=0)


def fast_modules(model: nn.Module) -> List[FastPathModule]:
    return [m for m in model.modules() if isinstance(m, FastPathModule)]


def select(modules: List[FastPathModule], use_fast: UseFast, policy: Optional[AutoPolicy],
           device: torch.device, dtype: torch.dtype, num_edges: int,
           double_backward: bool = False) -> bool:
    """Set ``fast_active`` on ``modules`` for one evaluation (fast.py:171-201).

    ``use_fast=True`` on a device or dtype the kernels do not take, or with the HIP
    library missing on a GPU, raises instead of silently running the reference.
    """
    use_fast = resolve_use_fast(use_fast)
    if use_fast is False or double_backward:
        want = False
    elif use_fast is True:
        want = True
    else:
        want = (policy or MI355X_POLICY).decide(device, dtype, num_edges)
    if want and device.type == "cuda":
        _lib.load()  # raises when the HIP library is missing: no silent fallback
    any_fast = False
    for m in modules:
        ok = m.fast_supported(device, dtype)
        if want and not ok and use_fast is True:
            # asked for explicitly: a module without a HIP path is an error, not a fallback
            raise RuntimeError(f"{type(m).__name__} has no HIP path for {device}/{dtype}")
        m.fast_active = bool(want and ok)
        any_fast = any_fast or m.fast_active
    if any_fast and dtype == torch.float32:
        warn_float32_once()
    return any_fast


def set_use_fast(model: nn.Module, use_fast: UseFast) -> nn.Module:
    """Set ``use_fast`` on every model inside ``model`` that has one (fast.py:204-219)."""
    mode = resolve_use_fast(use_fast)
    for m in model.modules():
        if hasattr(m, "use_fast"):
            m.use_fast = mode
    return model
