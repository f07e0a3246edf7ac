"""Indexer GeMV: scores every page of every segment against the segment's query.

``GeMV()(x, y, ctx=ctx)`` with x ``[B*H_kv, 1, D]`` (BATCHED) and y the
centroid pool ``[pool_rows, 1, D]`` (PAGED) returns a RAGGED score vector
``[ctx.max_num_pages, 1, 1]`` of x's dtype, where for each planner workload
(segment q, offset, length) ``score[p] = x[q] . y[dense_kv_indices[p]]``.
Only the positions of the workloads (the middle pages of segments that need a
top-k) are written.

Profile / execute contract and checks follow the reference
(vortex_torch/indexer/matmul.py:10-189).  The execute path launches the gfx950
kernel of ``libvortex_hip.so`` (``vtx_gemv_paged``), or — inside a flow's
forward_indexer, when a topK consumes the scores — records the launch so
that the topK runs mean + GeMV + select as one kernel (``vtx_indexer_fused``).
"""
from __future__ import annotations

from typing import Callable, Dict, Optional, Tuple

import torch

from .. import _deferred, _hip
from ..abs import FORMAT, as_vtensor, vOp, vTensor
from . import _walk
from .context import Context


#: Largest query group the fused kernel averages itself (torch.mean's order).
MEAN_IN_KERNEL_MAX_G = 16


class PendingGemv(_deferred.Pending):
    """A recorded ``GeMV`` launch.  ``topK`` on its result replaces it (and
    the recorded mean of its query, if any) by one fused launch."""

    def __init__(self, op: "GeMV", x: torch.Tensor, y: torch.Tensor, ctx: Context):
        super().__init__()
        self.op, self.x, self.y, self.ctx = op, x, y, ctx

    def _run(self) -> None:
        _deferred.materialize(self.x)
        self.op.impl(self.x, self.y, self.op.output_buffer, self.ctx)

    def fuse_with_topk(self, o: torch.Tensor, ctx: Context,
                       seg_counters: Optional[torch.Tensor] = None) -> None:
        """q-mean (if recorded) + GeMV + topK into ``o`` in one kernel.
        ``seg_counters`` (the topK op's zeroed int32 workspace, one counter per
        segment) lets the kernel split long segments over several workgroups."""
        sc = _deferred.current_scope()
        mean = _deferred.pending_of(self.x)
        # earlier recorded work runs first, in program order
        if sc is not None:
            for p in list(sc.pending):
                if p is mean or p is self:
                    break
                p.flush()
        # The kernel folds the mean in with torch's summation order, which
        # torch keeps for up to 16 query heads per kv head (four fp32
        # accumulators over the heads, one thread per column); past that
        # torch's mean runs first and the kernel starts from its result.
        if isinstance(mean, _deferred.PendingMean) and int(mean.q.shape[1]) <= MEAN_IN_KERNEL_MAX_G:
            q, x_out = mean.q, mean.out
        else:
            _deferred.materialize(self.x)
            q, x_out, mean = self.x, None, None
        # the page-finish mean forward_cache left for these centroids runs in
        # the same launch (its results, then these)
        cm = _deferred.take_carry(self.y)
        _hip.indexer_fused(
            q, x_out, self.y, self.op.output_buffer,
            ctx.dense_kv_indptr, ctx.sparse_kv_indptr, ctx.dense_kv_indices, o,
            ctx.batch_size * ctx.num_kv_heads, ctx.topk_val, ctx.page_reserved_bos,
            ctx.page_reserved_eos, ctx.max_num_pages_per_request, seg_counters=seg_counters,
            mode=_deferred.fused_layout(),
            cmean=None if cm is None else (cm.x, cm.loc, cm.ctx.head_num),
            schedule=_schedule_of(ctx))
        if cm is not None:
            cm.done = True
        if mean is not None:
            mean.done = True
        self.done = True


def _schedule_of(ctx: Context) -> Optional[torch.Tensor]:
    """The fused-indexer schedule plan_decode wrote into the context, if any."""
    s = getattr(ctx, "_fused_schedule", None)
    return s if isinstance(s, torch.Tensor) and s.is_cuda else None


def _fusable(x: torch.Tensor, y: torch.Tensor, ctx: Context) -> bool:
    """Whether GeMV may wait for a following topK to run fused with it.

    The fused kernel scores each segment's middle pages from the block table
    (dense_kv_indptr, bos, eos, topk) instead of walking the workload list;
    both describe the same pages for a plan_decode block table as long as a
    segment's middle count fits the planner's int16 (the reference caps
    requests at 4096 pages, far below)."""
    if _deferred.current_scope() is None or not _deferred.fusion_enabled():
        return False
    with torch._C.DisableTorchFunctionSubclass():
        if not (x.is_cuda and y.is_cuda and x.dtype == torch.bfloat16 and y.dtype == torch.bfloat16):
            return False
        D = int(x.shape[-1])
    try:
        span = int(ctx.max_num_pages_per_request) - int(ctx.page_reserved_bos) - int(ctx.page_reserved_eos)
        if span >= 32768 or int(ctx.topk_val) > 4096:
            return False
    except (TypeError, ValueError):
        return False
    return _hip.indexer_fused_supported(D)


def mv_bpr(x: torch.Tensor, y: torch.Tensor, o: torch.Tensor, ctx: Context) -> None:
    """(BATCHED x, PAGED y) -> RAGGED o, walking ctx's workload list."""
    _hip.gemv_paged(
        x, y, o,
        ctx.dense_kv_indices,
        ctx.winfo_q_indices,
        ctx.winfo_kv_offsets,
        ctx.winfo_kv_lens,
        ctx.winfo_num_workloads,
        ctx.max_chunk_size,
    )


class GeMV(vOp):
    _impl_map: Dict[Tuple[FORMAT, FORMAT], Tuple[Callable, FORMAT]] = {
        (FORMAT.BATCHED, FORMAT.PAGED): (mv_bpr, FORMAT.RAGGED),
    }

    def __init__(self):
        super().__init__()
        self.impl: Optional[Callable] = None
        self.output_format: Optional[FORMAT] = None
        self.output_buffer: Optional[torch.Tensor] = None

    def profile(self, x: vTensor, y: vTensor, ctx: Context) -> vTensor:
        p = self._prefix()
        assert isinstance(x, vTensor), f"{p}profile expects x to be vTensor, got {type(x)}"
        assert isinstance(y, vTensor), f"{p}profile expects y to be vTensor, got {type(y)}"
        assert x.dim() == 3 and y.dim() == 3, (
            f"{p}expected 3D inputs; got x.ndim={x.dim()}, y.ndim={y.dim()}")
        assert x.shape[1] == 1, f"{p}expected x.shape[1] == 1, got {tuple(x.shape)}"
        assert y.shape[1] == 1, f"{p}expected y.shape[1] == 1, got {tuple(y.shape)}"
        assert x.shape[2] == y.shape[2], (
            f"{p}last dimension mismatch: x.shape[2]={x.shape[2]} vs y.shape[2]={y.shape[2]}")
        key = (x._format, y._format)
        assert key in self._impl_map, (
            f"{p}no implementation for (x_fmt={key[0]}, y_fmt={key[1]}). "
            f"Available: {list(self._impl_map.keys())}")
        self.impl, self.output_format = self._impl_map[key]

        self.output_buffer = torch.empty((ctx.max_num_pages, 1, 1), device=x.device, dtype=x.dtype)
        ctx.add_aux_memory(self.output_buffer)
        for t in (x, y):
            if t._format == FORMAT.PAGED:
                ctx.add_aux_flops(t.shape[1] * t.shape[2])
        return as_vtensor(self.output_buffer, self.output_format)

    def execute(self, x: torch.Tensor, y: torch.Tensor, ctx: Context) -> torch.Tensor:
        p = self._prefix()
        assert self.impl is not None, f"{p}execute called before profile() (impl is None)"
        assert self.output_buffer is not None, f"{p}output buffer is None; did profile() run?"
        assert x.device == y.device == self.output_buffer.device, (
            f"{p}device mismatch: x={x.device}, y={y.device}, o={self.output_buffer.device}")
        if self.impl is mv_bpr and _fusable(x, y, ctx):
            pending = PendingGemv(self, x, y, ctx)
            _deferred.current_scope().add(pending)
            return _deferred.DeferredTensor.make(self.output_buffer, self.output_format, pending)
        _deferred.materialize(x)
        self.impl(x, y, self.output_buffer, ctx)
        return self.output_buffer


def _mm(x_fmt: FORMAT, y_fmt: FORMAT) -> Callable:
    def impl(x: torch.Tensor, y: torch.Tensor, o: torch.Tensor, ctx: Context) -> None:
        _walk.ready(x, y)
        _hip.ragged_gemm(x, _walk.ROW_MODE[x_fmt], y, _walk.ROW_MODE[y_fmt], o, ctx.dense_kv_indices,
                         _walk.winfo(ctx))
    return impl


#: o[p] = y[p] x[p]^T ([C, G] per position) over ctx's workload list
#: (reference indexer/triton_kernels/matmul_impl.py: mm_bpr 6-113, mm_rrr and mm_rpr 127-391).
mm_bpr = _mm(FORMAT.BATCHED, FORMAT.PAGED)
mm_rrr = _mm(FORMAT.RAGGED, FORMAT.RAGGED)
mm_rpr = _mm(FORMAT.RAGGED, FORMAT.PAGED)


class PendingGemm(_deferred.Pending):
    """A recorded ``GeMM`` (BATCHED queries x PAGED centroids, one centroid
    per page) and what follows it in the GQA flow: an in-place ``Softmax`` of
    its output and a ``Max`` over the query heads.  ``topK`` on the maximum
    replaces the chain by one fused launch (``vtx_indexer_gqa_fused``);
    flushed any other way, the recorded launches run in order.

    A follow-on op joins the chain only when the chain is the newest recorded
    work of the scope, so no other recorded computation can observe its
    output between the ops."""

    def __init__(self, op: "GeMM", x: torch.Tensor, y: torch.Tensor, ctx: Context):
        super().__init__()
        self.op, self.x, self.y, self.ctx = op, x, y, ctx
        self.softmax: Optional[Tuple[float, Callable[[], None]]] = None  # (scale, launch)
        self.max_out: Optional[torch.Tensor] = None
        self.max_run: Optional[Callable[[], None]] = None

    def _newest(self) -> bool:
        sc = _deferred.current_scope()
        return sc is not None and bool(sc.pending) and sc.pending[-1] is self and not self.done

    def accepts_softmax(self) -> bool:
        return self._newest() and self.softmax is None and self.max_out is None

    def accepts_max(self) -> bool:
        return self._newest() and self.max_out is None

    def add_softmax(self, scale: float, run: Callable[[], None]) -> None:
        self.softmax = (float(scale), run)

    def add_max(self, out: torch.Tensor, run: Callable[[], None]) -> None:
        self.max_out, self.max_run = out, run

    def _run(self) -> None:
        _deferred.materialize(self.x)
        self.op.impl(self.x, self.y, self.op.output_buffer, self.ctx)
        if self.softmax is not None:
            self.softmax[1]()
        if self.max_run is not None:
            self.max_run()

    def fuses_with_topk(self, x: torch.Tensor, ctx: Context) -> bool:
        if self.done or self.max_out is None or ctx is not self.ctx:
            return False
        with torch._C.DisableTorchFunctionSubclass():
            return x.data_ptr() == self.max_out.data_ptr()

    def fuse_with_topk(self, o: torch.Tensor, ctx: Context) -> None:
        """GeMM + softmax (if recorded) + max + topK into ``o`` in one kernel."""
        sc = _deferred.current_scope()
        if sc is not None:  # earlier recorded work runs first, in program order
            for p in list(sc.pending):
                if p is self:
                    break
                p.flush()
        _deferred.materialize(self.x)
        # the page-finish mean forward_cache left for these centroids runs in
        # the same launch (its results, then these)
        cm = _deferred.take_carry(self.y)
        _hip.indexer_gqa_fused(
            self.x, self.y, self.op.output_buffer, self.max_out,
            ctx.dense_kv_indptr, ctx.sparse_kv_indptr, ctx.dense_kv_indices, o,
            ctx.batch_size * ctx.num_kv_heads, ctx.topk_val, ctx.page_reserved_bos,
            ctx.page_reserved_eos, ctx.max_num_pages_per_request,
            softmax_scale=None if self.softmax is None else self.softmax[0],
            cmean=None if cm is None else (cm.x, cm.loc, cm.ctx.head_num), schedule=_schedule_of(ctx))
        if cm is not None:
            cm.done = True
        self.done = True


def _gemm_fusable(x: torch.Tensor, y: torch.Tensor, ctx: Context) -> bool:
    """Whether GeMM may wait for the softmax / max / topK that may follow.

    Like GeMV's, the fused kernel walks each segment's middle pages from the
    block table instead of the workload list, which describe the same pages
    for a plan_decode block table; the queries must be BATCHED [S, G, D] with
    one row per segment and one centroid per page."""
    if _deferred.current_scope() is None or not _deferred.fusion_enabled():
        return False
    with torch._C.DisableTorchFunctionSubclass():
        if not (x.is_cuda and y.is_cuda and x.dtype == torch.bfloat16 and y.dtype == torch.bfloat16):
            return False
        if x.dim() != 3 or y.dim() != 3 or int(y.shape[1]) != 1 or not x.is_contiguous():
            return False
        S, G, D = (int(v) for v in x.shape)
    try:
        span = int(ctx.max_num_pages_per_request) - int(ctx.page_reserved_bos) - int(ctx.page_reserved_eos)
        if span >= 32768 or int(ctx.topk_val) > 4096:
            return False
        if S < int(ctx.batch_size) * int(ctx.num_kv_heads):
            return False
    except (TypeError, ValueError):
        return False
    return _hip.indexer_gqa_fused_supported(D, G)


class GeMM(vOp):
    """O[s] = Y[s] X[s]^T per packed position: x [B or S, N_x, K], y [S, N_y, K]
    -> RAGGED [ctx.max_num_pages, N_y, N_x] (reference vortex_torch/indexer/matmul.py:193-398)."""

    _impl_map: Dict[Tuple[FORMAT, FORMAT], Tuple[Callable, FORMAT]] = {
        (FORMAT.BATCHED, FORMAT.PAGED): (mm_bpr, FORMAT.RAGGED),
        (FORMAT.RAGGED, FORMAT.RAGGED): (mm_rrr, FORMAT.RAGGED),
        (FORMAT.RAGGED, FORMAT.PAGED): (mm_rpr, FORMAT.RAGGED),
    }

    def __init__(self):
        super().__init__()
        self.impl: Optional[Callable] = None
        self.output_format: Optional[FORMAT] = None
        self.output_buffer: Optional[torch.Tensor] = None

    def profile(self, x: vTensor, y: vTensor, ctx: Context) -> vTensor:
        p = self._prefix()
        assert isinstance(x, vTensor), f"{p}profile expects x to be vTensor, got {type(x)}"
        assert isinstance(y, vTensor), f"{p}profile expects y to be vTensor, got {type(y)}"
        assert x.dim() == 3 and y.dim() == 3, (
            f"{p}expected 3D inputs; got x.ndim={x.dim()}, y.ndim={y.dim()}")
        assert x.shape[2] == y.shape[2], (
            f"{p}last dimension mismatch: x.shape[2]={x.shape[2]} vs y.shape[2]={y.shape[2]}")
        key = (x._format, y._format)
        assert key in self._impl_map, (
            f"{p}no implementation for (x_fmt={key[0]}, y_fmt={key[1]}). "
            f"Available: {list(self._impl_map.keys())}")
        self.impl, self.output_format = self._impl_map[key]
        Ny, Nx = y.shape[1], x.shape[1]
        self.output_buffer = torch.empty((ctx.max_num_pages, Ny, Nx), device=x.device, dtype=x.dtype)
        ctx.add_aux_memory(self.output_buffer)
        for t in (x, y):
            if t._format == FORMAT.PAGED:
                ctx.add_aux_flops(t.shape[1] * t.shape[2])
        return as_vtensor(self.output_buffer, self.output_format)

    def execute(self, x: torch.Tensor, y: torch.Tensor, ctx: Context) -> torch.Tensor:
        p = self._prefix()
        assert self.impl is not None, f"{p}execute called before profile() (impl is None)"
        assert self.output_buffer is not None, f"{p}output buffer is None; did profile() run?"
        assert x.device == y.device == self.output_buffer.device, (
            f"{p}device mismatch: x={x.device}, y={y.device}, o={self.output_buffer.device}")
        if self.impl is mm_bpr and _gemm_fusable(x, y, ctx):
            pending = PendingGemm(self, x, y, ctx)
            _deferred.current_scope().add(pending)
            return _deferred.DeferredTensor.make(self.output_buffer, self.output_format, pending)
        self.impl(x, y, self.output_buffer, ctx)
        return self.output_buffer


__all__ = ["GeMV", "GeMM", "PendingGemm", "mv_bpr", "mm_bpr", "mm_rrr", "mm_rpr"]
