"""Indexer reductions over one tile axis: ``Max``, ``Mean``, ``Min``,
``L2Norm``, ``Sum`` (reference vortex_torch/indexer/reduce.py:8-438).

x is a RAGGED score tensor [S, D0, D1]; the output, [ctx.max_num_pages, 1,
D1] (dim 1) or [ctx.max_num_pages, D0, 1] (dim 2), is written at the
positions of the planner's workload list by ``vtx_ragged_reduce``
(replacing the Triton ``reduce_rr``, indexer/triton_kernels/reduce_impl.py:8-146).
"""
from __future__ import annotations

from typing import Callable, Dict, Optional, Tuple

import torch

from .. import _deferred, _hip
from ..abs import FORMAT, as_vtensor, vOp, vTensor
from ..utils import ReduceType
from ._walk import ready, winfo
from .context import Context
from .matmul import PendingGemm


def reduce_rr(x: torch.Tensor, o: torch.Tensor, dim: int, reduce_type: ReduceType, ctx: Context) -> None:
    """RAGGED x -> RAGGED o over ctx's workload list."""
    ready(x)
    _hip.ragged_reduce(x, o, dim, reduce_type.value, winfo(ctx))


class Reduce(vOp):
    _impl_map: Dict[FORMAT, Tuple[Callable, FORMAT]] = {
        FORMAT.RAGGED: (reduce_rr, FORMAT.RAGGED),
    }

    def __init__(self, dim: int = 1):
        super().__init__()
        self.dim = dim
        self.reduce_type: Optional[ReduceType] = None
        self.impl: Optional[Callable] = None
        self.output_format: Optional[FORMAT] = None
        self.output_buffer: Optional[torch.Tensor] = None
        p = self._prefix()
        assert self.dim in (1, 2), f"{p}__init__: dim must be 1 or 2, got dim={self.dim}"

    def profile(self, x: vTensor, ctx: Context) -> vTensor:
        p = self._prefix()
        assert isinstance(x, vTensor), f"{p}profile expects x to be vTensor, got {type(x)}"
        assert x.dim() == 3, f"{p}expected 3D input [N, D0, D1], got ndim={x.dim()} shape={tuple(x.shape)}"
        assert x._format in self._impl_map, (
            f"{p}no implementation for x_fmt={x._format}. Available keys: {list(self._impl_map.keys())}")
        self.impl, self.output_format = self._impl_map[x._format]
        D0, D1 = x.shape[1], x.shape[2]
        out_d0 = 1 if self.dim == 1 else D0
        out_d1 = 1 if self.dim == 2 else D1
        self.output_buffer = torch.empty((ctx.max_num_pages, out_d0, out_d1), device=x.device, dtype=x.dtype)
        ctx.add_aux_memory(self.output_buffer)
        if x._format == FORMAT.PAGED:
            ctx.add_aux_flops(x.shape[1] * x.shape[2])
        return as_vtensor(self.output_buffer, self.output_format)

    def execute(self, x: torch.Tensor, ctx: Context) -> torch.Tensor:
        p = self._prefix()
        assert self.impl is not None, f"{p}execute called before profile() (impl is None)"
        assert self.output_buffer is not None, f"{p}output buffer is None; did profile() run?"
        pending = _deferred.pending_of(x)
        role = _quest_role(self, pending, ctx)
        if role is not None:
            # the row sum / page maximum of the Quest chain: a following topK fuses it
            xp, out, dim, rt = _deferred.plain(x), self.output_buffer, self.dim, self.reduce_type
            rec = _deferred.PendingOp(role, lambda: reduce_rr(xp, out, dim, rt, ctx), [pending], ctx=ctx, out=out)
            _deferred.current_scope().add(rec)
            return _deferred.DeferredTensor.make(out, self.output_format, rec)
        if (self.impl is reduce_rr and self.dim == 2 and self.reduce_type == ReduceType.Max
                and isinstance(pending, PendingGemm) and pending.ctx is ctx and pending.accepts_max()):
            # max over the query heads of a recorded GeMM: a following topK fuses all of it
            xp, out, dim, rt = _deferred.plain(x), self.output_buffer, self.dim, self.reduce_type
            pending.add_max(out, lambda: reduce_rr(xp, out, dim, rt, ctx))
            return _deferred.DeferredTensor.make(out, self.output_format, pending)
        self.impl(x, self.output_buffer, self.dim, self.reduce_type, ctx)
        return self.output_buffer


def _quest_role(op: Reduce, pending, ctx: Context):
    """"quest_sum" for Sum(dim=2) of a recorded Quest maximum, "quest_aggr" for
    Max(dim=1) of a recorded Quest row sum; None otherwise."""
    if op.impl is not reduce_rr or not isinstance(pending, _deferred.PendingOp) or pending.elided:
        return None
    if pending.info.get("ctx") is not ctx:
        return None
    if pending.kind == "quest_max" and op.dim == 2 and op.reduce_type == ReduceType.Sum:
        return "quest_sum"
    if pending.kind == "quest_sum" and op.dim == 1 and op.reduce_type == ReduceType.Max:
        return "quest_aggr"
    return None


class Max(Reduce):
    def __init__(self, dim: int = 1):
        super().__init__(dim)
        self.reduce_type = ReduceType.Max


class Min(Reduce):
    def __init__(self, dim: int = 1):
        super().__init__(dim)
        self.reduce_type = ReduceType.Min


class Mean(Reduce):
    def __init__(self, dim: int = 1):
        super().__init__(dim)
        self.reduce_type = ReduceType.Mean


class L2Norm(Reduce):
    def __init__(self, dim: int = 1):
        super().__init__(dim)
        self.reduce_type = ReduceType.L2Norm


class Sum(Reduce):
    def __init__(self, dim: int = 1):
        super().__init__(dim)
        self.reduce_type = ReduceType.Sum


__all__ = ["Reduce", "Max", "Min", "Mean", "L2Norm", "Sum", "reduce_rr"]
