"""In-place segment ops over the packed page axis: ``Softmax`` and
``Normalize`` (reference vortex_torch/indexer/scan.py:8-388).

For every segment with more than topk middle pages, over its middle
positions and per tile column: softmax of ``x * scale``, or division by the
column's L2 norm (floored at 1e-12), rounded to bf16 in place.  Kernel:
``vtx_segment_scan`` (replacing the Triton softmax_inplace_r /
normalize_inplace_r, indexer/triton_kernels/softmax_impl.py:6-130,
normalize_impl.py:6-118).
"""
from __future__ import annotations

from typing import Callable, Dict, Optional, Tuple

import torch

from .. import _deferred, _hip
from ..abs import FORMAT, vOp, vTensor
from ._walk import ready
from .context import Context
from .matmul import PendingGemm


def _segments(ctx: Context) -> int:
    return int(ctx.batch_size) * int(ctx.num_kv_heads)


def softmax_inplace_r(x: torch.Tensor, dim: int, scale: float, ctx: Context) -> None:
    ready(x)
    _hip.segment_scan(_hip.SEGMENT_SOFTMAX, scale, x, ctx.dense_kv_indptr, _segments(ctx), ctx.topk_val,
                      ctx.page_reserved_bos, ctx.page_reserved_eos)


def normalize_inplace_r(x: torch.Tensor, dim: int, ctx: Context) -> None:
    ready(x)
    _hip.segment_scan(_hip.SEGMENT_NORMALIZE, 1.0, x, ctx.dense_kv_indptr, _segments(ctx), ctx.topk_val,
                      ctx.page_reserved_bos, ctx.page_reserved_eos)


class _SegmentOp(vOp):
    _impl_map: Dict[FORMAT, Tuple[Callable, FORMAT]] = {}

    def __init__(self, dim: int = 0):
        super().__init__()
        self.dim = dim
        self.impl: Optional[Callable] = None
        self.output_format: Optional[FORMAT] = None
        p = self._prefix()
        assert self.dim in (0,), f"{p}__init__: dim must be 0, got dim={self.dim}"

    def profile(self, x: vTensor, ctx: Context) -> vTensor:
        p = self._prefix()
        assert isinstance(x, vTensor), f"{p}profile expects x to be vTensor, got {type(x)}"
        assert x.dim() == 3, f"{p}expected 3D input [S_pack, D0, D1], got ndim={x.dim()} shape={tuple(x.shape)}"
        assert x._format in self._impl_map, (
            f"{p}no implementation for x_fmt={x._format}. Available keys: {list(self._impl_map.keys())}")
        self.impl, self.output_format = self._impl_map[x._format]
        if x._format == FORMAT.PAGED:
            ctx.add_aux_flops(x.shape[1] * x.shape[2])
        return x


class Softmax(_SegmentOp):
    _impl_map = {FORMAT.RAGGED: (softmax_inplace_r, FORMAT.RAGGED)}

    def __init__(self, dim: int = 0, scale: float = 1.0):
        super().__init__(dim)
        self.scale = scale

    def execute(self, x: torch.Tensor, ctx: Context) -> torch.Tensor:
        p = self._prefix()
        assert self.impl is not None, f"{p}execute called before profile() (impl is None)"
        pending = _deferred.pending_of(x)
        if (self.impl is softmax_inplace_r and isinstance(pending, PendingGemm) and pending.ctx is ctx
                and pending.accepts_softmax()):
            # joins the recorded GeMM; runs right after it (or inside the fused GQA kernel)
            xp, dim, scale = _deferred.plain(x), self.dim, self.scale
            pending.add_softmax(scale, lambda: softmax_inplace_r(xp, dim, scale, ctx))
            return x
        self.impl(x, self.dim, self.scale, ctx)
        return x


class Normalize(_SegmentOp):
    _impl_map = {FORMAT.RAGGED: (normalize_inplace_r, FORMAT.RAGGED)}

    def execute(self, x: torch.Tensor, ctx: Context) -> torch.Tensor:
        p = self._prefix()
        assert self.impl is not None, f"{p}execute called before profile() (impl is None)"
        self.impl(x, self.dim, ctx)
        return x


__all__ = ["Softmax", "Normalize", "softmax_inplace_r", "normalize_inplace_r"]
