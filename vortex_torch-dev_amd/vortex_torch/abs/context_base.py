"""Base class of the runtime contexts (indexer and cache side).

Contract follows the reference (vortex_torch/abs/context_base.py:7-116): a
context has a ``name``, a ``mode`` (``Mode.profile`` while flows are traced to
plan buffers, ``Mode.execute`` while they run) and a ``_created`` flag set by
``create``.  It also accumulates the auxiliary bytes and flops the ops declare
while profiling (``add_aux_memory`` / ``add_aux_flops``), which
``vFlow.run_indexer_virtual`` reports as a per-page cost model.
"""
from __future__ import annotations

from abc import ABC, abstractmethod
from typing import Any, Union

import torch

from ..utils import UNSET, Mode


class ContextBase(ABC):
    __slots__ = ("name", "mode", "_created")

    @property
    def created(self) -> bool:
        return self._created

    @abstractmethod
    def create(self, *args: Any, **kwargs: Any) -> "ContextBase":
        """Populates the context from the serving runtime's objects."""
        raise NotImplementedError

    def profile(self) -> None:
        self.mode = Mode.profile

    def execute(self) -> None:
        self.mode = Mode.execute

    def assert_created(self) -> None:
        if not self._created:
            raise RuntimeError("Context is not created yet.")

    def missing(self) -> list:
        """Names of slots that still hold UNSET."""
        return [n for n in self.__slots__ if n != "_created" and getattr(self, n) is UNSET]

    # ---------------------------------------------------------------- costs
    @staticmethod
    def _tensor_nbytes(t: torch.Tensor) -> int:
        return int(t.element_size() * t.nelement())

    def add_aux_memory(self, obj: Union[int, torch.Tensor]) -> int:
        """Adds `obj` bytes (an int, or a tensor's size) to the auxiliary total."""
        if isinstance(obj, bool) or not isinstance(obj, (int, torch.Tensor)):
            raise TypeError("add_aux_memory expects an int (bytes) or a torch.Tensor")
        nbytes = obj if isinstance(obj, int) else self._tensor_nbytes(obj)
        if nbytes < 0:
            raise ValueError("nbytes must be non-negative")
        self._aux_total_bytes += nbytes
        return nbytes

    def add_aux_flops(self, nflops: int) -> int:
        self._aux_total_flops += nflops
        return nflops

    def clear_aux_memory(self) -> None:
        self._aux_total_bytes = 0

    def clear_aux_flops(self) -> None:
        self._aux_total_flops = 0

    def summary(self) -> dict:
        """Bytes held by the context's tensors (by device, storage counted
        once) plus the auxiliary byte and flop totals."""
        seen = set()
        by_device: dict = {}
        for n in self.__slots__:
            if n.startswith("_"):
                continue
            v = getattr(self, n, None)
            if not isinstance(v, torch.Tensor):
                continue
            st = v.untyped_storage()
            key = (str(v.device), st.data_ptr())
            if key in seen:
                continue
            seen.add(key)
            by_device[str(v.device)] = by_device.get(str(v.device), 0) + int(st.nbytes())
        return {
            "internal_bytes": by_device,
            "aux_bytes": int(getattr(self, "_aux_total_bytes", 0)),
            "aux_flops": int(getattr(self, "_aux_total_flops", 0)),
        }
