"""Indexer-side operators (run every decode step in every sparse layer).

Implemented on gfx950: :class:`GeMV` (page scoring), :class:`topK` (sparse
page select), :mod:`utils_sglang` (``plan_decode``), the runtime
:class:`Context`.  The reference's other scoring ops (GeMM, Softmax, the
reductions and elementwise ops used by other flows) are not part of this
build's hot path.
"""
from . import utils_sglang
from .context import Context, get_ctx
from .matmul import GeMV
from .output_func import topK

__all__ = ["GeMV", "topK", "utils_sglang", "Context", "get_ctx"]
