"""Flow API: :class:`vFlow`, :func:`register`, :func:`build_vflow` and the
registered :mod:`algorithms`."""
from . import algorithms
from .flow import vFlow
from .loader import build_vflow
from .registry import register

__all__ = ["vFlow", "register", "build_vflow", "algorithms"]
