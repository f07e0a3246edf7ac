"""``vTensor``: a torch.Tensor carrying a layout tag (``FORMAT``).

Behaviour follows the reference (vortex_torch/abs/tensor.py:8-165):

* torch operations on vTensors return vTensors with the same tag;
* all vTensors taking part in one operation must carry the same tag,
  otherwise ``RuntimeError``;
* a vTensor cannot be combined with a plain ``torch.Tensor`` in one
  operation (``RuntimeError``); Python scalars are fine;
* wrapping never copies storage, and pickling keeps the tag.

The tag is what the ops use to pick an implementation (e.g. GeMV on
(BATCHED, PAGED) inputs produces a RAGGED score vector).
"""
from __future__ import annotations

from enum import Enum
from typing import Any, Iterator

import torch


class FORMAT(Enum):
    """Logical layout of a tensor in a flow.

    BATCHED: one row per (request, kv head) — queries.
    RAGGED: rows packed segment after segment (scores, sparse indices).
    PAGED: rows addressed through the block table (cache pools).
    """

    BATCHED = 0
    RAGGED = 1
    PAGED = 2


_deferred_mod = None


def _deferral():
    """vortex_torch._deferred (imported on first use: it subclasses vTensor)."""
    global _deferred_mod
    if _deferred_mod is None:
        from .. import _deferred

        _deferred_mod = _deferred
    return _deferred_mod


def _tensors_in(obj: Any) -> Iterator[torch.Tensor]:
    if isinstance(obj, torch.Tensor):
        yield obj
    elif isinstance(obj, (list, tuple)):
        for item in obj:
            yield from _tensors_in(item)
    elif isinstance(obj, dict):
        for item in obj.values():
            yield from _tensors_in(item)


def _op_format(args, kwargs) -> "FORMAT | None":
    formats = set()
    plain = False
    for t in _tensors_in((args, kwargs)):
        if isinstance(t, vTensor):
            formats.add(t._format)
        else:
            plain = True
    if formats and plain:
        raise RuntimeError("vTensor cannot operate with plain torch.Tensor in the same op.")
    if len(formats) > 1:
        raise RuntimeError(f"vTensor _format mismatch in op: {formats}")
    return next(iter(formats)) if formats else None


def _tag(result: Any, fmt: FORMAT) -> Any:
    if isinstance(result, torch.Tensor):
        if isinstance(result, vTensor):
            result._format = fmt
            return result
        return vTensor._wrap(result, fmt)
    if isinstance(result, (list, tuple)):
        return type(result)(_tag(r, fmt) for r in result)
    if isinstance(result, dict):
        return {k: _tag(v, fmt) for k, v in result.items()}
    return result


class vTensor(torch.Tensor):
    """torch.Tensor subclass with a ``_format`` layout tag."""

    _format: FORMAT

    def __new__(cls, data, _format: FORMAT = FORMAT.BATCHED, **kwargs):
        if not isinstance(data, torch.Tensor):
            data = torch.as_tensor(data, **kwargs)
        return cls._wrap(data, _format)

    @classmethod
    def _wrap(cls, base: torch.Tensor, fmt: FORMAT) -> "vTensor":
        out = torch.Tensor._make_subclass(cls, base, require_grad=base.requires_grad)
        out._format = fmt
        return out

    # Backwards-compatible name used by the reference's helpers.
    _from_base = _wrap

    def __repr__(self, *, tensor_contents=None):
        with torch._C.DisableTorchFunctionSubclass():
            body = torch.Tensor.__repr__(self.as_subclass(torch.Tensor))
        return f"vTensor(format={self._format}, {body})"

    def __reduce_ex__(self, protocol):
        with torch._C.DisableTorchFunctionSubclass():
            base = torch.Tensor(self)
        return (_rebuild_vtensor, (base, self._format, self.requires_grad))

    @classmethod
    def __torch_function__(cls, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        if not any(issubclass(t, vTensor) for t in types):
            return super().__torch_function__(func, types, args, kwargs)
        d = _deferral()
        if d.current_scope() is not None and not d.is_metadata(func):
            # inside an execute-mode forward_indexer: record the head-group
            # mean, and let any other operation see finished data
            deferred = d.try_defer_mean(func, args, kwargs)
            if deferred is not None:
                return deferred
            d.flush_all()
        if d.current_carry() is not None and not d.is_metadata(func) and d.carry_touched_by(args, kwargs):
            d.flush_carry()  # a carried page-finish mean reads or writes these
        fmt = _op_format(args, kwargs)
        with torch._C.DisableTorchFunctionSubclass():
            out = func(*args, **kwargs)
        if fmt is None:
            return out
        return _tag(out, fmt)


def _rebuild_vtensor(base: torch.Tensor, fmt: FORMAT, requires_grad: bool) -> vTensor:
    out = torch.Tensor._make_subclass(vTensor, base, require_grad=requires_grad)
    out._format = fmt
    return out


def as_vtensor(x: Any, _format: FORMAT = FORMAT.BATCHED) -> vTensor:
    """Tags ``x`` with ``_format`` without copying its storage.

    A vTensor is re-tagged in place and returned; anything else is converted
    with ``torch.as_tensor`` first.
    """
    if isinstance(x, vTensor):
        x._format = _format
        return x
    if not isinstance(x, torch.Tensor):
        x = torch.as_tensor(x)
    return vTensor._wrap(x, _format)
