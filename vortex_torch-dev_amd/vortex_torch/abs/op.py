"""``vOp``: base class of all flow operators.

An op is called twice per layout: once while the context is in
``Mode.profile`` (validate shapes and layout tags, pick the kernel, allocate
persistent output buffers) and then in ``Mode.execute`` (launch).  Dispatch
follows the reference (vortex_torch/abs/op.py:77-104): ``ctx.mode`` None or
``execute`` -> :meth:`execute`, ``profile`` -> :meth:`profile`, anything else
-> ``ValueError``.
"""
from __future__ import annotations

from abc import ABC, abstractmethod
from typing import Any

from ..utils import Mode
from .context_base import ContextBase


class vOp(ABC):
    def __init__(self) -> None:
        super().__init__()

    @abstractmethod
    def profile(self, *args: Any, ctx: ContextBase = None, **kwargs: Any) -> Any:
        raise NotImplementedError

    @abstractmethod
    def execute(self, *args: Any, ctx: ContextBase = None, **kwargs: Any) -> Any:
        raise NotImplementedError

    def __call__(self, *args: Any, ctx: ContextBase = None, **kwargs: Any) -> Any:
        mode = ctx.mode
        if mode is None or mode == Mode.execute:
            return self.execute(*args, ctx=ctx, **kwargs)
        if mode == Mode.profile:
            return self.profile(*args, ctx=ctx, **kwargs)
        raise ValueError(f"Unknown mode: {mode!r}, expected 'profile' or 'execute'")

    def _prefix(self) -> str:
        return f"{type(self).__name__}: "
