"""Argument rules shared by the operator wrappers.

Every public operator checks its arguments before anything reaches the GPU and raises
``ValueError`` at the first rule an argument breaks.  A wrapper states its rules as a
sequence of calls on one ``Rules`` object, in a fixed order: with several bad
arguments, the first rule in that order decides the error.  Messages name the
operator, the argument, and what was expected against what was given.
"""

from __future__ import annotations

from typing import Iterable, Optional

import torch


def _dtype_names(dtypes: Iterable[torch.dtype]) -> str:
    return ", ".join(str(d).replace("torch.", "") for d in dtypes)


class Rules:
    """The checks of one operator call; each failure message starts with ``op``."""

    def __init__(self, op: str):
        self.op = op

    def fail(self, message: str, error=ValueError):
        raise error(f"{self.op}: {message}")

    def require(self, ok: bool, message: str):
        """Fail with ``message`` unless ``ok``."""
        if not ok:
            self.fail(message)

    def dims(self, name: str, t: torch.Tensor, n: int, layout: str):
        """``t`` has ``n`` axes, described by ``layout`` (e.g. "(batch, dim, length)")."""
        if t.dim() != n:
            self.fail(f"{name} should be {layout}, a {n}-d tensor; its shape is {tuple(t.shape)}")

    def shape(self, name: str, t: Optional[torch.Tensor], *allowed):
        """``t`` is absent or has one of the ``allowed`` shapes."""
        if t is None:
            return
        got = tuple(t.shape)
        if got not in [tuple(a) for a in allowed]:
            wanted = " or ".join(str(tuple(a)) for a in allowed)
            self.fail(f"{name} should have shape {wanted}; its shape is {got}")

    def same_device(self, device: torch.device, **tensors):
        """Every given tensor lives on ``device`` (in keyword order)."""
        for name, t in tensors.items():
            if t is not None and t.device != device:
                self.fail(f"{name} lives on {t.device}, the other operands on {device}")

    def dtype_in(self, allowed, **tensors):
        """Every given tensor has a dtype in ``allowed`` (in keyword order)."""
        for name, t in tensors.items():
            if t is not None and t.dtype not in allowed:
                self.fail(f"{name} has dtype {str(t.dtype).replace('torch.', '')}; this operator takes "
                          f"{_dtype_names(allowed)}")
