"""Cache-side runtime context (page size, pool size, head geometry).

Fields and :meth:`Context.create` follow the reference
(vortex_torch/cache/context.py:7-59).
"""
from __future__ import annotations

from typing import Any

from ..abs import ContextBase
from ..utils import UNSET, Mode

_FIELDS = ("max_new_tokens_per_batch", "page_size", "total_num_pages", "head_dim", "head_num")


class Context(ContextBase):
    """Mutable single-instance context, populated by :meth:`create`."""

    __slots__ = ContextBase.__slots__ + _FIELDS + ("_aux_total_bytes", "_aux_total_flops")

    def __init__(self) -> None:
        for n in self.__slots__:
            object.__setattr__(self, n, UNSET)
        self.name = "Cache"
        self.mode = Mode.profile
        self._created = False
        self._aux_total_bytes = 0
        self._aux_total_flops = 0

    def create(self, parent: Any, model_runner: Any, *, overwrite: bool = False) -> "Context":
        """Not thread-safe: call once, from one thread."""
        if self._created and not overwrite:
            raise RuntimeError("Context.create() already called; pass overwrite=True to reinitialize.")
        sa = model_runner.server_args
        self.page_size = parent.page_size
        self.total_num_pages = parent.num_pages
        self.max_new_tokens_per_batch = max(sa.max_prefill_tokens, model_runner.req_to_token_pool.size)
        self.head_num = parent.head_num
        self.head_dim = parent.head_dim
        self._created = True
        return self


__all__ = ["Context"]
