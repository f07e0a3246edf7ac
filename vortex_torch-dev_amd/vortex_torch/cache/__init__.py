"""Cache-side operators (run when KV pages fill).

Implemented on gfx950: the page-finish reductions :class:`Mean`,
:class:`Max`, :class:`Min`, :class:`L2Norm` (PAGED -> PAGED), the fused
:class:`MultiReduce`, the pool writer :func:`set_kv_buffer_launcher`, and
the runtime :class:`Context`.
"""
from .context import Context
from .reduce import L2Norm, Max, Mean, Min, MultiReduce
from .set_kv import set_kv_buffer_launcher

__all__ = ["Mean", "Max", "Min", "L2Norm", "MultiReduce", "Context", "set_kv_buffer_launcher"]
