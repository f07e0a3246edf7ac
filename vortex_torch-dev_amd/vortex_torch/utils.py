"""Shared enums and sentinels of the vortex_torch API.

Names and values mirror the reference (vortex_torch/utils.py:1-31): they are
part of the public surface (flows compare ``ctx.mode`` against ``Mode`` and
reduction ops carry a ``ReduceType``).
"""
from enum import Enum


class _Unset:
    """Marker for context fields that have not been populated yet."""

    _instance = None

    def __new__(cls):
        if cls._instance is None:
            cls._instance = super().__new__(cls)
        return cls._instance

    def __repr__(self) -> str:
        return "UNSET"

    def __bool__(self) -> bool:
        return False


UNSET = _Unset()


class Mode(Enum):
    profile = 0
    execute = 1


class ReduceType(Enum):
    Mean = 0
    Max = 1
    Min = 2
    L2Norm = 3
    Sum = 4


class ElementwiseBinaryOpType(Enum):
    Maximum = 0
    Minimum = 1
    Add = 2
    Mul = 3


class ElementwiseOpType(Enum):
    Relu = 0
    Sigmoid = 1
    Silu = 2
    Abs = 3
    Add_Mul = 4
