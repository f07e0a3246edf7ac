"""``build_vflow``: instantiate a registered flow by name, optionally after
executing a user file that registers it (reference
vortex_torch/flow/loader.py:19-94)."""
from __future__ import annotations

import importlib.util
import inspect
import os
import types
import uuid
from typing import Any, Dict, Optional

from .flow import vFlow
from .registry import RegistryError, get as _get, list_keys


class FlowLoadError(Exception):
    """The user file could not be executed, or the flow name is unknown."""


class FlowInitError(Exception):
    """Constructor arguments do not fit, or the constructor raised."""


def _load_module_from_file(file_path: str) -> types.ModuleType:
    """Executes `file_path` under a fresh module name so its @register calls run."""
    if not os.path.isfile(file_path):
        raise FlowLoadError(f"File does not exist: {file_path}")
    name = f"user_flow_{uuid.uuid4().hex}"
    spec = importlib.util.spec_from_file_location(name, file_path)
    if spec is None or spec.loader is None:
        raise FlowLoadError(f"Failed to create import spec for: {file_path}")
    module = importlib.util.module_from_spec(spec)
    try:
        spec.loader.exec_module(module)
    except Exception as e:
        raise FlowLoadError(f"Failed to import user module: {e}") from e
    return module


def _validate_kwargs(cls: type, init_kwargs: Dict[str, Any]) -> None:
    sig = inspect.signature(cls.__init__)
    try:
        sig.bind_partial(None, **(init_kwargs or {}))
    except TypeError as e:
        raise FlowInitError(f"Constructor arguments mismatch: {e}") from e


def build_vflow(selected: str, init_kwargs: Optional[Dict[str, Any]] = None,
                user_file: Optional[str] = None) -> vFlow:
    if user_file:
        _load_module_from_file(user_file)
    try:
        cls = _get(selected)
    except RegistryError as e:
        raise FlowLoadError(f"{e} (available: {list_keys()})")
    kwargs = init_kwargs or {}
    _validate_kwargs(cls, kwargs)
    try:
        return cls(**kwargs)
    except Exception as e:
        raise FlowInitError(f"Failed to instantiate: {e}") from e
