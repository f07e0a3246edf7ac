"""Indexer topK: turns per-page scores into the sparse block table.

``topK()(x, o, ctx=ctx)`` takes the RAGGED score vector ``[S, 1, 1]`` and
writes, for every segment that has more than ``topk_val`` middle pages, the
``topk_val`` best-scoring middle pages (best first, ties to the lower page
position) into ``o`` after the segment's reserved BOS pages.  Segments with
fewer middle pages are left as the planner wrote them (all pages).

Profile / execute contract follows the reference
(vortex_torch/indexer/output_func.py:8-235); execute calls ``topk_output``
with the reference's argument list, which launches the gfx950 select kernel.
When its input is a GeMV result recorded inside the same forward_indexer, it
launches the fused mean + GeMV + select kernel instead; when it is the
maximum over query heads of a recorded GeMM (the GQA flow), the fused
GeMM + softmax + max + select kernel.
"""
from __future__ import annotations

from typing import Callable, Dict, Optional

import torch

from .. import _deferred, _hip
from .._C import topk_output
from ..abs import FORMAT, vOp, vTensor
from .context import Context
from .matmul import PendingGemm, PendingGemv, _schedule_of


class topK(vOp):
    _impl_map: Dict[FORMAT, Callable] = {
        FORMAT.RAGGED: topk_output,
    }

    def __init__(self):
        super().__init__()
        self.impl: Optional[Callable] = None
        # workspace of the fused kernel's split layout: an arrival counter per
        # segment the block table can hold (zero between launches) and the
        # staging zone of its pre-selection
        self.seg_counters: Optional[torch.Tensor] = None

    def profile(self, x: vTensor, o: vTensor, ctx: Context) -> None:
        p = self._prefix()
        assert isinstance(x, vTensor), f"{p}profile expects x to be vTensor, got {type(x)}"
        assert isinstance(o, vTensor), f"{p}profile expects o to be vTensor, got {type(o)}"
        assert x.dim() == 3, f"{p}expected x to be 3D, got ndim={x.dim()} shape={tuple(x.shape)}"
        assert o.dim() == 3, f"{p}expected o to be 3D, got ndim={o.dim()} shape={tuple(o.shape)}"
        assert x.shape[1] == 1 and x.shape[2] == 1, (
            f"{p}expected x.shape[1] == x.shape[2] == 1, got {tuple(x.shape)}")
        assert x._format in self._impl_map, (
            f"{p}no implementation for x._format={x._format}. "
            f"Available: {list(self._impl_map.keys())}")
        self.impl = self._impl_map[x._format]
        assert x.device == o.device, (
            f"{p}x and o must be on the same device (x.device={x.device}, o.device={o.device})")
        indptr = ctx.dense_kv_indptr
        if isinstance(indptr, torch.Tensor) and indptr.numel() > 1 and x.device.type == "cuda":
            # one arrival counter per segment and the staging zone, sized by
            # the library for every batch the block table can hold
            S = indptr.numel() - 1
            self.seg_counters = torch.zeros((_hip.indexer_fused_workspace_len(S),), dtype=torch.int32,
                                            device=x.device)

    def execute(self, x: torch.Tensor, o: torch.Tensor, ctx: Context) -> torch.Tensor:
        assert self.impl is not None, f"{self._prefix()}execute called before profile() (impl is None)"
        pending = _deferred.pending_of(x)
        if self.impl is topk_output and isinstance(pending, PendingGemv) and pending.ctx is ctx:
            pending.fuse_with_topk(o, ctx, self.seg_counters)
            return o
        if self.impl is topk_output and isinstance(pending, PendingGemm) and pending.fuses_with_topk(x, ctx):
            pending.fuse_with_topk(o, ctx)
            return o
        if self.impl is topk_output and _quest_chain(pending, ctx) is not None:
            _fuse_quest(_quest_chain(pending, ctx), o, ctx)
            return o
        _deferred.materialize(x)
        self.impl(
            x,
            ctx.dense_kv_indptr,
            ctx.sparse_kv_indptr,
            ctx.dense_kv_indices,
            o,
            ctx.batch_size * ctx.num_kv_heads,
            ctx.topk_val,
            ctx.page_reserved_bos,
            ctx.page_reserved_eos,
            ctx.max_num_pages_per_request,
        )
        return o


def _quest_chain(aggr, ctx: Context):
    """(mul_a, mul_b, maximum, row sum, page maximum) recorded for the fused
    Quest kernel and ending in `aggr`, or None."""
    if not (isinstance(aggr, _deferred.PendingOp) and aggr.kind == "quest_aggr" and not aggr.done
            and aggr.info.get("ctx") is ctx):
        return None
    rsum = aggr.deps[0]
    mx = rsum.deps[0]
    pa, pb = mx.deps
    chain = (pa, pb, mx, rsum, aggr)
    if any(p.done or p.elided for p in chain):
        return None
    return chain


def _fuse_quest(chain, o: torch.Tensor, ctx: Context) -> None:
    """Runs the Quest chain's row sums, page maxima and top-k as one kernel;
    the products and their maximum become elided work."""
    pa, pb, mx, rsum, aggr = chain
    sc = _deferred.current_scope()
    if sc is not None:  # earlier recorded work runs first, in program order
        for p in list(sc.pending):
            if p is pa or p is pb:
                break
            p.flush()
    for d in pa.deps + pb.deps:  # recorded producers of q and the envelopes
        d.flush()
    # the CMax + CMin forward_cache left for these envelopes run in the same
    # launch (their results, then these); the score is symmetric in the two
    ya, yb = pa.info["y"], pb.info["y"]
    env = _deferred.take_carry_envelope(ya, yb)
    if env is not None:
        ya, yb = env[1], env[2]
    _hip.indexer_quest_fused(
        pa.info["x"], ya, yb, rsum.info["out"], aggr.info["out"],
        ctx.dense_kv_indptr, ctx.sparse_kv_indptr, ctx.dense_kv_indices, o,
        ctx.batch_size * ctx.num_kv_heads, ctx.topk_val, ctx.page_reserved_bos,
        ctx.page_reserved_eos, ctx.max_num_pages_per_request,
        envelope=None if env is None else (env[0].x, env[0].loc, env[0].ctx.head_num),
        schedule=_schedule_of(ctx))
    if env is not None:
        env[0].done = True
    rsum.done = aggr.done = True
    for p in (pa, pb, mx):
        p.elided = True


__all__ = ["topK"]
