"""Elementwise binary indexer ops with broadcasting: ``Maximum``,
``Minimum``, ``Add`` (alpha * x + beta * y), ``Multiply`` (reference
vortex_torch/indexer/elementwise_binary.py:8-326).

Operand formats (x, y): (RAGGED, RAGGED), (BATCHED, PAGED), (RAGGED,
PAGED); the output [ctx.max_num_pages, max(C), max(D)] is RAGGED and is
written at the positions of the planner's workload list by
``vtx_ragged_binary`` (replacing the Triton
elementwise_binary_{rrr,bpr,rpr}, indexer/triton_kernels/elementwise_binary_impl.py:7-510).
"""
from __future__ import annotations

from typing import Callable, Dict, Optional, Tuple

import torch

from .. import _deferred, _hip
from ..abs import FORMAT, as_vtensor, vOp, vTensor
from ..utils import ElementwiseBinaryOpType
from ._walk import ROW_MODE, ready, winfo
from .context import Context


def _binary(x_fmt: FORMAT, y_fmt: FORMAT) -> Callable:
    def impl(x, y, o, op_type: ElementwiseBinaryOpType, alpha: float, beta: float, ctx: Context) -> None:
        ready(x, y)
        _hip.ragged_binary(op_type.value, alpha, beta, x, ROW_MODE[x_fmt], y, ROW_MODE[y_fmt], o,
                           ctx.dense_kv_indices, winfo(ctx))
    return impl


elementwise_binary_rrr = _binary(FORMAT.RAGGED, FORMAT.RAGGED)
elementwise_binary_bpr = _binary(FORMAT.BATCHED, FORMAT.PAGED)
elementwise_binary_rpr = _binary(FORMAT.RAGGED, FORMAT.PAGED)


class Elementwise_Binary(vOp):
    _impl_map: Dict[Tuple[FORMAT, FORMAT], Tuple[Callable, FORMAT]] = {
        (FORMAT.RAGGED, FORMAT.RAGGED): (elementwise_binary_rrr, FORMAT.RAGGED),
        (FORMAT.BATCHED, FORMAT.PAGED): (elementwise_binary_bpr, FORMAT.RAGGED),
        (FORMAT.RAGGED, FORMAT.PAGED): (elementwise_binary_rpr, FORMAT.RAGGED),
    }

    def __init__(self, alpha: float = 1.0, beta: float = 1.0):
        super().__init__()
        self.impl: Optional[Callable] = None
        self.op_type: Optional[ElementwiseBinaryOpType] = None
        self.alpha = alpha
        self.beta = beta
        self.output_format: Optional[FORMAT] = None
        self.output_buffer: Optional[torch.Tensor] = None

    def profile(self, x: vTensor, y: vTensor, ctx: Context) -> vTensor:
        p = self._prefix()
        assert isinstance(x, vTensor), f"{p}profile expects x to be vTensor, got {type(x)}"
        assert isinstance(y, vTensor), f"{p}profile expects y to be vTensor, got {type(y)}"
        assert x.dim() == 3 and y.dim() == 3, (
            f"{p}expected 3D inputs [S, C, D]; got x.ndim={x.dim()}, y.ndim={y.dim()}")
        assert x.shape[1] == y.shape[1] or x.shape[1] == 1 or y.shape[1] == 1, (
            f"{p}dim-1 not broadcastable: x.shape={tuple(x.shape)}, y.shape={tuple(y.shape)}")
        assert x.shape[2] == y.shape[2] or x.shape[2] == 1 or y.shape[2] == 1, (
            f"{p}dim-2 not broadcastable: x.shape={tuple(x.shape)}, y.shape={tuple(y.shape)}")
        key = (x._format, y._format)
        assert key in self._impl_map, (
            f"{p}no implementation for (x_fmt={key[0]}, y_fmt={key[1]}). Available: {list(self._impl_map.keys())}")
        self.impl, self.output_format = self._impl_map[key]
        assert x.device == y.device, f"{p}device mismatch (x.device={x.device}, y.device={y.device})"
        C_out = max(x.shape[1], y.shape[1])
        D_out = max(x.shape[2], y.shape[2])
        self.output_buffer = torch.empty((ctx.max_num_pages, C_out, D_out), device=x.device, dtype=x.dtype)
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
        kind = self._quest_role(x, y, ctx)
        if kind is not None:
            return self._record(kind, x, y, ctx)
        self.impl(x, y, self.output_buffer, self.op_type, self.alpha, self.beta, ctx)
        return self.output_buffer

    # -- recording for the fused Quest kernel (see vortex_torch/_deferred.py)
    def _quest_role(self, x, y, ctx: Context) -> Optional[str]:
        """"quest_mul" for q x envelope products, "quest_max" for the maximum
        of two recorded products of the same queries; None otherwise."""
        if _deferred.current_scope() is None or not _deferred.fusion_enabled():
            return None
        if self.op_type == ElementwiseBinaryOpType.Mul and self.impl is elementwise_binary_bpr:
            return "quest_mul" if _quest_operands(x, y, ctx) else None
        if self.op_type == ElementwiseBinaryOpType.Maximum and self.impl is elementwise_binary_rrr:
            pa, pb = _deferred.pending_of(x), _deferred.pending_of(y)
            if (isinstance(pa, _deferred.PendingOp) and isinstance(pb, _deferred.PendingOp) and pa is not pb
                    and pa.kind == pb.kind == "quest_mul" and pa.info["ctx"] is ctx and pb.info["ctx"] is ctx
                    and not pa.elided and not pb.elided):
                with torch._C.DisableTorchFunctionSubclass():
                    same_q = pa.info["x"].data_ptr() == pb.info["x"].data_ptr()
                    same_y = pa.info["y"].shape == pb.info["y"].shape
                if same_q and same_y:
                    return "quest_max"
        return None

    def _record(self, kind: str, x, y, ctx: Context):
        xp, yp, out = _deferred.plain(x), _deferred.plain(y), self.output_buffer
        deps = [d for d in (_deferred.pending_of(x), _deferred.pending_of(y)) if d is not None]
        op_type, alpha, beta, impl = self.op_type, self.alpha, self.beta, self.impl
        pending = _deferred.PendingOp(kind, lambda: impl(xp, yp, out, op_type, alpha, beta, ctx), deps,
                                      x=xp, y=yp, ctx=ctx)
        _deferred.current_scope().add(pending)
        return _deferred.DeferredTensor.make(out, self.output_format, pending)


def _quest_operands(x, y, ctx: Context) -> bool:
    """Queries [S, G, D] (BATCHED) times a per-page envelope pool [rows, 1, D]
    (PAGED), both bf16 on the GPU, in a shape the fused Quest kernel takes."""
    with torch._C.DisableTorchFunctionSubclass():
        if not (x.is_cuda and y.is_cuda and x.dtype == torch.bfloat16 and y.dtype == torch.bfloat16):
            return False
        if x.dim() != 3 or y.dim() != 3 or int(y.shape[1]) != 1 or int(x.shape[2]) != int(y.shape[2]):
            return False
        if not (x.is_contiguous() and y.is_contiguous()):
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
    return _hip.indexer_quest_fused_supported(D, G)


class Maximum(Elementwise_Binary):
    def __init__(self, alpha: float = 1.0, beta: float = 1.0):
        super().__init__(alpha, beta)
        self.op_type = ElementwiseBinaryOpType.Maximum


class Minimum(Elementwise_Binary):
    def __init__(self, alpha: float = 1.0, beta: float = 1.0):
        super().__init__(alpha, beta)
        self.op_type = ElementwiseBinaryOpType.Minimum


class Add(Elementwise_Binary):
    def __init__(self, alpha: float = 1.0, beta: float = 1.0):
        super().__init__(alpha, beta)
        self.op_type = ElementwiseBinaryOpType.Add


class Multiply(Elementwise_Binary):
    def __init__(self, alpha: float = 1.0, beta: float = 1.0):
        super().__init__(alpha, beta)
        self.op_type = ElementwiseBinaryOpType.Mul


__all__ = ["Elementwise_Binary", "Maximum", "Minimum", "Add", "Multiply"]
