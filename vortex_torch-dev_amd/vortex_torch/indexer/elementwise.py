"""Elementwise unary indexer ops with an affine pre-transform: ``Relu``,
``Sigmoid``, ``Silu``, ``Add_Mul``, ``Abs`` (reference
vortex_torch/indexer/elementwise.py:8-297).

With a = alpha, b = beta (both rounded to bf16) and z = b * x + a (bf16
arithmetic): Relu x >= a ? x : b; Sigmoid 1 / (1 + exp(z)); Silu
x / (1 + exp(z)); Abs |z|; Add_Mul z.  RAGGED in and out, written at the
positions of the planner's workload list by ``vtx_ragged_unary``
(replacing the Triton elementwise_rr, indexer/triton_kernels/elementwise_impl.py:7-171).
"""
from __future__ import annotations

from typing import Callable, Dict, Optional, Tuple

import torch

from .. import _hip
from ..abs import FORMAT, as_vtensor, vOp, vTensor
from ..utils import ElementwiseOpType
from ._walk import ready, winfo
from .context import Context


def elementwise_rr(x: torch.Tensor, o: torch.Tensor, op_type: ElementwiseOpType, alpha: float, beta: float,
                   ctx: Context) -> None:
    ready(x)
    _hip.ragged_unary(op_type.value, alpha, beta, x, o, winfo(ctx))


class Elementwise(vOp):
    _impl_map: Dict[FORMAT, Tuple[Callable, FORMAT]] = {
        FORMAT.RAGGED: (elementwise_rr, FORMAT.RAGGED),
    }

    def __init__(self, alpha: float = 1.0, beta: float = 1.0):
        super().__init__()
        self.impl: Optional[Callable] = None
        self.op_type: Optional[ElementwiseOpType] = None
        self.alpha = alpha
        self.beta = beta
        self.output_format: Optional[FORMAT] = None
        self.output_buffer: Optional[torch.Tensor] = None

    def profile(self, x: vTensor, ctx: Context) -> vTensor:
        p = self._prefix()
        assert isinstance(x, vTensor), f"{p}profile expects x to be vTensor, got {type(x)}"
        assert x.dim() == 3, f"{p}expected 3D input [S, C, D], got ndim={x.dim()} shape={tuple(x.shape)}"
        assert x._format in self._impl_map, (
            f"{p}no implementation for x_fmt={x._format}. Available keys: {list(self._impl_map.keys())}")
        self.impl, self.output_format = self._impl_map[x._format]
        S, C, D = ctx.max_num_pages, x.shape[1], x.shape[2]
        self.output_buffer = torch.empty((S, C, D), device=x.device, dtype=x.dtype)
        ctx.add_aux_memory(self.output_buffer)
        if x._format == FORMAT.PAGED:
            ctx.add_aux_flops(x.shape[1] * x.shape[2])
        return as_vtensor(self.output_buffer, self.output_format)

    def execute(self, x: torch.Tensor, ctx: Context) -> torch.Tensor:
        p = self._prefix()
        assert self.impl is not None, f"{p}execute called before profile() (impl is None)"
        assert self.output_buffer is not None, f"{p}output buffer is None; did profile() run?"
        assert x.device == self.output_buffer.device, (
            f"{p}device mismatch: x={x.device}, o={self.output_buffer.device}")
        self.impl(x, self.output_buffer, self.op_type, self.alpha, self.beta, ctx)
        return self.output_buffer


class Relu(Elementwise):
    def __init__(self, alpha: float = 0.0, beta: float = 0.0):
        super().__init__(alpha, beta)
        self.op_type = ElementwiseOpType.Relu


class Silu(Elementwise):
    def __init__(self, alpha: float = 0.0, beta: float = 0.0):
        super().__init__(alpha, beta)
        self.op_type = ElementwiseOpType.Silu


class Sigmoid(Elementwise):
    def __init__(self, alpha: float = 0.0, beta: float = 0.0):
        super().__init__(alpha, beta)
        self.op_type = ElementwiseOpType.Sigmoid


class Add_Mul(Elementwise):
    def __init__(self, alpha: float = 0.0, beta: float = 1.0):
        super().__init__(alpha, beta)
        self.op_type = ElementwiseOpType.Add_Mul


class Abs(Elementwise):
    def __init__(self, alpha: float = 0.0, beta: float = 1.0):
        super().__init__(alpha, beta)
        self.op_type = ElementwiseOpType.Abs


__all__ = ["Elementwise", "Relu", "Silu", "Sigmoid", "Add_Mul", "Abs"]
