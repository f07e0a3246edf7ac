"""Indexer-side operators (run every decode step in every sparse layer).

Scoring: :class:`GeMV`, :class:`GeMM`; output routing: :class:`topK`;
reductions over a tile axis: :class:`Max`, :class:`Mean`, :class:`Min`,
:class:`L2Norm`, :class:`Sum`; in-place segment scans: :class:`Softmax`,
:class:`Normalize`; elementwise: :class:`Maximum`, :class:`Minimum`,
:class:`Multiply`, :class:`Add`, :class:`Relu`, :class:`Sigmoid`,
:class:`Silu`, :class:`Add_Mul`, :class:`Abs`; the planner in
:mod:`utils_sglang`; the runtime :class:`Context`.  Every op runs on the
gfx950 kernel library (reference vortex_torch/indexer/__init__.py:50-72
lists the same names; Transpose and Save/Load are not part of this build).
"""
from . import utils_sglang
from .context import Context, get_ctx
from .elementwise import Abs, Add_Mul, Relu, Sigmoid, Silu
from .elementwise_binary import Add, Maximum, Minimum, Multiply
from .matmul import GeMM, GeMV
from .output_func import topK
from .reduce import L2Norm, Max, Mean, Min, Sum
from .scan import Normalize, Softmax

__all__ = [
    "GeMM", "GeMV",
    "topK",
    "Max", "Mean", "Min", "L2Norm", "Sum",
    "Softmax", "Normalize",
    "Maximum", "Minimum", "Multiply", "Add",
    "Relu", "Sigmoid", "Silu", "Add_Mul", "Abs",
    "utils_sglang",
    "Context",
    "get_ctx",
]
