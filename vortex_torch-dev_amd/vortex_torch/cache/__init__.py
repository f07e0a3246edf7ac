"""Cache-side operators (run when KV pages fill).

Implemented on gfx950: the page-finish reductions :class:`Mean`,
:class:`Max`, :class:`Min`, :class:`L2Norm` (PAGED -> PAGED), the fused
:class:`MultiReduce`, and the runtime :class:`Context`.
"""
from .context import Context
from .reduce import L2Norm, Max, Mean, Min, MultiReduce

__all__ = ["Mean", "Max", "Min", "L2Norm", "MultiReduce", "Context"]
