"""``vFlow``: the user-facing base class of a sparse-attention algorithm.

A flow declares its extra cache tensors (:meth:`create_cache`), how they are
updated when pages fill (:meth:`forward_cache`) and how the indexer turns a
decode query into the sparse block table (:meth:`forward_indexer`).  The
contract follows the reference (vortex_torch/flow/flow.py:6-460):

* ``forward_indexer(q, o, cache, ctx)``: q ``[B*H_kv, G, D]``; ``o`` the packed
  sparse index buffer, written in place; each cache tensor is seen as
  ``[S, r, c]`` (page-packed).
* ``forward_cache(cache, loc, ctx)``: each cache tensor seen as ``[rows, r, c]``
  (pool rows); ``loc`` the token slots written this step.
* ``create_cache(page_size, head_dim)`` returns ``{name: (r, c)}`` for the
  extra tensors; ``"k"`` and ``"v"`` are added by :meth:`get_cache_meta_info`.

Per segment the sparse list holds ``min(n_pages, topk + bos + eos)`` pages.
"""
from __future__ import annotations

import functools
from abc import ABC, abstractmethod
from typing import Dict, Tuple

import torch

from .. import _deferred
from ..abs import ContextBase
from ..utils import Mode


def _ctx_of(args, kwargs, pos: int):
    if "ctx" in kwargs:
        return kwargs["ctx"]
    return args[pos] if len(args) > pos else None


def _scoped(fn, ctx_pos: int, kind: str):
    """Runs a forward_indexer / forward_cache inside a deferral scope when its
    context is in execute mode (see vortex_torch._deferred): recorded work is
    fused where possible and everything is finished when the method returns.
    ctx_pos: position of ctx among the method's arguments after self."""

    @functools.wraps(fn)
    def scoped(self, *args, **kwargs):
        ctx = _ctx_of(args, kwargs, ctx_pos)
        mode = getattr(ctx, "mode", None)
        with _deferred.scope(active=mode is None or mode == Mode.execute, kind=kind):
            return fn(self, *args, **kwargs)

    scoped._vtx_scoped = True
    return scoped


class vFlow(ABC):
    def __init__(self):
        super().__init__()

    def __init_subclass__(cls, **kwargs):
        super().__init_subclass__(**kwargs)
        for name, ctx_pos, kind in (("forward_indexer", 3, "indexer"), ("forward_cache", 2, "cache")):
            fn = cls.__dict__.get(name)
            if fn is not None and not getattr(fn, "_vtx_scoped", False) and callable(fn):
                setattr(cls, name, _scoped(fn, ctx_pos, kind))

    @abstractmethod
    def forward_indexer(self, q: torch.Tensor, o: torch.Tensor, cache: Dict[str, torch.Tensor],
                        ctx: ContextBase):
        """Scores pages for the decode query and writes the sparse indices into o."""

    @abstractmethod
    def forward_cache(self, cache: Dict[str, torch.Tensor], loc: torch.Tensor, ctx: ContextBase):
        """Updates the flow's cache tensors for the token slots in loc."""

    @abstractmethod
    def create_cache(self, page_size: int, head_dim: int) -> Dict[str, Tuple[int, int]]:
        """Inner shapes (r, c) of the extra cache tensors (not "k"/"v")."""

    def get_cache_meta_info(self, page_size: int, head_dim: int) -> Dict[str, Tuple[int, int]]:
        """:meth:`create_cache` plus ``"k"`` and ``"v"`` of shape (page_size, head_dim)."""
        meta = self.create_cache(page_size, head_dim)
        assert "k" not in meta.keys()
        assert "v" not in meta.keys()
        meta["k"] = (page_size, head_dim)
        meta["v"] = (page_size, head_dim)
        return meta

    def get_token_ratio(self, page_size: int, head_dim: int) -> float:
        """Cache size per page in units of one (page_size x head_dim) page."""
        unit = page_size * head_dim
        return sum(r * c / unit for (r, c) in self.get_cache_meta_info(page_size, head_dim).values())

    def run_indexer_virtual(self, group_size: int, page_size: int, head_dim: int):
        """Profiles :meth:`forward_indexer` on empty inputs and returns the
        auxiliary flops per page the ops declared (the reference's offline
        cost model, vortex_torch/flow/flow.py:420-460)."""
        from ..abs import FORMAT, as_vtensor
        from ..indexer import Context as IContext

        ctx = IContext()
        ctx.group_size = group_size
        ctx.num_kv_heads = 1
        ctx.num_qo_heads = group_size
        ctx.head_dim = head_dim
        ctx.page_size = page_size
        ctx.max_num_pages = 0
        ctx.max_num_pages_per_request = 0
        device = "cuda" if torch.cuda.is_available() else "cpu"
        dtype = torch.bfloat16
        with torch.no_grad():
            q = as_vtensor(torch.empty((1, group_size, head_dim), device=device, dtype=dtype), FORMAT.BATCHED)
            o = as_vtensor(torch.empty((0, 1, 1), device=device, dtype=dtype), FORMAT.RAGGED)
            cache = {
                name: as_vtensor(torch.zeros((0, r, c), dtype=dtype, device=device), FORMAT.PAGED)
                for name, (r, c) in self.get_cache_meta_info(page_size, head_dim).items()
            }
            self.forward_indexer(q, o, cache, ctx=ctx)
        return ctx._aux_total_flops
