"""Shared helpers of the workload-walking indexer ops."""
from __future__ import annotations

from .. import _deferred
from ..abs import FORMAT
from .context import Context

# Reference FORMAT of an operand -> its row mode in the kernel library.
ROW_MODE = {FORMAT.BATCHED: 0, FORMAT.PAGED: 1, FORMAT.RAGGED: 2}


def winfo(ctx: Context):
    """The planner's workload list: (q indices, kv offsets, kv lens, count)."""
    return (ctx.winfo_q_indices, ctx.winfo_kv_offsets, ctx.winfo_kv_lens, ctx.winfo_num_workloads)


def ready(*tensors):
    """Runs any recorded work that writes these tensors before a kernel reads them."""
    for t in tensors:
        _deferred.materialize(t)
