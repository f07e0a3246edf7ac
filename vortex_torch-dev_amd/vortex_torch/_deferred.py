"""Deferred execution inside a flow's ``forward_indexer``.

A flow such as ``block_sparse_attention`` runs, per layer,
``q.mean(1, keepdim=True)`` -> ``GeMV`` -> ``topK``.  Launched one by one,
each of these costs a kernel launch plus a chain of dependent memory round
trips, which at decode batch sizes is most of the layer's time.  Inside an
execute-mode ``forward_indexer`` (a *scope*) the first two are recorded
instead of launched:

* ``q.mean(dim=1, keepdim=True)`` on a BATCHED bf16 GPU vTensor returns a
  :class:`DeferredTensor` whose storage is allocated but not yet written;
* ``GeMV`` returns its output buffer as a DeferredTensor;
* ``topK`` on a deferred GeMV result launches one fused kernel that computes
  the mean, the scores and the selection, writing all three results.

The GQA flow's ``GeMM`` -> ``Softmax`` -> ``Max(dim=2)`` -> ``topK`` chain is
recorded the same way: GeMM returns its output as a DeferredTensor, Softmax
and Max join its record while it is the newest one in the scope, and topK on
the maximum launches the fused GQA kernel.

The Quest flow's two ``Multiply`` -> ``Maximum`` -> ``Sum(dim=2)`` ->
``Max(dim=1)`` -> ``topK`` chain is recorded op by op (:class:`PendingOp`,
each naming the recorded work it reads); topK on the maximum launches the
fused Quest kernel, which writes the row sums, the maximum and the block
table.  The [pages, G, D] products and their elementwise maximum are then
*elided*: they are computed only if something reads them — a torch op or
an indexer op inside the scope, or a tensor still referring to them when
the scope ends.  An op's ``output_buffer`` read directly is not such a read.

Anything else materialises first: a torch operation on any vTensor inside the
scope flushes all pending work (so no input can change under a recorded
computation), a DeferredTensor used after the scope is already materialised,
and leaving the scope flushes whatever is still pending.  Metadata queries
(shape, dtype, device, ...) do not flush.  The results are the ones the
separate ops produce; set ``VORTEX_FUSE=0`` to launch every op on its own.
"""
from __future__ import annotations

import contextlib
import os
import threading
import weakref
from typing import Callable, List, Optional

import torch

_tls = threading.local()

# Tensor queries that never read the data.
_METADATA = {
    torch.Tensor.dim,
    torch.Tensor.size,
    torch.Tensor.numel,
    torch.Tensor.nelement,
    torch.Tensor.is_contiguous,
    torch.Tensor.element_size,
    torch.Tensor.stride,
    torch.Tensor.storage_offset,
    torch.Tensor.get_device,
    torch.Tensor.__len__,
    torch.Tensor.shape.__get__,
    torch.Tensor.dtype.__get__,
    torch.Tensor.device.__get__,
    torch.Tensor.ndim.__get__,
    torch.Tensor.is_cuda.__get__,
    torch.Tensor.layout.__get__,
    torch.Tensor.requires_grad.__get__,
}


# Python switches beside the environment variables: None leaves the decision
# to VORTEX_FUSE / VORTEX_FUSE_CMEAN, True / False override them (set_fusion).
_switch = {"fuse": None, "carry": None}


def fusion_enabled() -> bool:
    if _switch["fuse"] is not None:
        return _switch["fuse"]
    return os.environ.get("VORTEX_FUSE", "1") != "0"


def set_fusion(fuse: Optional[bool] = None, carry_cmean: Optional[bool] = None) -> None:
    """Switches of the fused paths, beside VORTEX_FUSE and VORTEX_FUSE_CMEAN:
    True or False overrides the environment variable, None hands the choice
    back to it.  ``fuse``: one launch per forward_indexer chain (False: every
    op launched when called, as the reference does).  ``carry_cmean``: the
    page-finish mean that forward_cache records is left for the next fused
    indexer launch (False: it runs when forward_cache returns).  Turning the
    carry off launches a pending one and removes the graph-capture hooks."""
    _switch["fuse"] = fuse
    _switch["carry"] = carry_cmean
    if not _carry_enabled():
        flush_carry()
        remove_capture_hooks()


_LAYOUTS = {"auto": 0, "segment": 1, "split": 2}


def fused_layout() -> int:
    """Work layout of the fused indexer kernel (VORTEX_FUSED_LAYOUT = auto,
    segment or split; the outputs are the same in every layout)."""
    name = os.environ.get("VORTEX_FUSED_LAYOUT", "auto")
    if name not in _LAYOUTS:
        raise RuntimeError(f"VORTEX_FUSED_LAYOUT must be one of {sorted(_LAYOUTS)}, got {name!r}")
    return _LAYOUTS[name]


class Pending:
    """A recorded computation that writes a tensor's storage when flushed.

    ``elided`` marks work a fused launch made unnecessary for the flow's
    results (an intermediate of the fused chain): it still runs when its
    result is read, and when the scope ends while a tensor still refers to
    that result; otherwise it is dropped."""

    def __init__(self):
        self.done = False
        self.elided = False
        self._outs: List[weakref.ref] = []  # the DeferredTensors it produces

    def flush(self) -> None:
        if not self.done:
            self.done = True
            self._run()

    def observed(self) -> bool:
        return any(r() is not None for r in self._outs)

    def _run(self) -> None:  # pragma: no cover - subclasses
        raise NotImplementedError


class PendingOp(Pending):
    """A recorded launch of one indexer op (``kind`` names the op and its
    role, ``info`` holds its plain operands).  The recorded work of its
    inputs (``deps``) runs first."""

    def __init__(self, kind: str, launch: Callable[[], None], deps: List[Pending], **info):
        super().__init__()
        self.kind, self._launch, self.deps, self.info = kind, launch, deps, info

    def _run(self) -> None:
        for d in self.deps:
            d.flush()
        self._launch()


class PendingMean(Pending):
    """``out = q.mean(dim=1, keepdim=True)`` (q: [S, G, D] bf16)."""

    def __init__(self, q: torch.Tensor, out: torch.Tensor):
        super().__init__()
        self.q = q
        self.out = out

    def _run(self) -> None:
        torch.mean(self.q, dim=1, keepdim=True, out=self.out)


class Scope:
    def __init__(self):
        self.pending: List[Pending] = []

    def add(self, p: Pending) -> None:
        self.pending.append(p)

    def flush(self) -> None:
        while self.pending:
            p = self.pending.pop(0)
            if p.elided and not p.observed():
                continue  # superseded by a fused launch and never read
            p.flush()


def current_scope() -> Optional[Scope]:
    return getattr(_tls, "scope", None)


# ---------------------------------------------------------------- the carry
# forward_cache's page-finish mean (or CMax + CMin) may be left unlaunched
# when the method returns (the *carry*), for the next forward_indexer to run
# inside its fused launch (vtx_indexer_fused_cmean and its GQA / Quest forms).  It is launched on its own, on the stream
# it was recorded on, as soon as anything else could observe it:
#   * any other kernel launch of this package (every _hip wrapper checks);
#   * any torch operation on a layout-tagged tensor (vTensor) that shares
#     storage with the K pool, the centroid pool or loc;
#   * the start of the next forward_cache;
#   * the end of the forward_indexer that did not consume it.
# So a carried mean is never read or overwritten before it is computed,
# provided the centroid pool and the K pool are only touched through this
# package or through torch on their vTensors between the two calls — as in
# a decode layer, where forward_indexer follows forward_cache.
#
# Graph capture.  A carry belongs to the capture it was recorded in (or to
# none): it is launched into that capture or, recorded outside any, before a
# capture starts.  Once a mean has been carried, torch.cuda.CUDAGraph's
# capture_begin and capture_end (which torch.cuda.graph and
# make_graphed_callables call) launch the carry first, so a capture never
# ends with a carried mean outside the graph, whatever the order of the
# flow's calls within it (forward_indexer may precede forward_cache: the last
# layer's carry then lands at the end of the graph).  These two hooks are
# installed with the first carry and removed by remove_capture_hooks() or by
# switching the carry off (set_fusion(carry_cmean=False)); a process that
# never carries keeps torch's own methods.  A carry found on a stream whose
# capture state has changed by other means (a capture begun or ended outside
# these two methods) is an error, raised instead of launching the mean
# outside the work it belongs to; the carry then stays recorded
# (discard_carry() drops it).


def _carry_enabled() -> bool:
    if not fusion_enabled():
        return False
    if _switch["carry"] is not None:
        return _switch["carry"]
    return os.environ.get("VORTEX_FUSE_CMEAN", "1") != "0"


def current_carry():
    return getattr(_tls, "carry", None)


def _stream_of(dev: torch.device):
    return torch.cuda.current_stream(dev) if dev.type == "cuda" else None


def _capture_of(stream) -> int:
    """Id of the graph capture `stream` takes part in (0: none)."""
    if stream is None:
        return 0
    from . import _hip

    return _hip.stream_capture_id(stream)


def _check_capture(carry) -> None:
    pending, stream, cap = carry
    now = _capture_of(stream)
    if now != cap:
        where = {True: "during a graph capture", False: "outside any graph capture"}
        raise RuntimeError(
            "vortex_torch: a page-finish mean that forward_cache left for the next forward_indexer was "
            f"recorded {where[cap != 0]} and would now be launched "
            f"{'in another capture' if cap and now else where[now != 0]}; begin and end captures with "
            "torch.cuda.graph / torch.cuda.CUDAGraph (which launch it first), or set VORTEX_FUSE_CMEAN=0")


def flush_carry() -> None:
    """Launches the carried page-finish mean, if any, on its own stream.
    When the stream's capture state is no longer the one it was recorded in,
    this raises and the mean stays recorded: it can still be launched once
    that state is back, or dropped with discard_carry()."""
    c = current_carry()
    if c is None:
        return
    _check_capture(c)
    _tls.carry = None
    pending, stream, _ = c
    with (torch.cuda.stream(stream) if stream is not None else contextlib.nullcontext()):
        pending.flush()


def discard_carry() -> None:
    """Drops the carried page-finish mean without launching it (after
    flush_carry raised for a capture that will not come back).  The centroid
    or envelope rows of the pages it would have closed then keep their old
    values until a page-finish reduction over those pages runs again."""
    _tls.carry = None


def _storages(obj, out):
    if isinstance(obj, torch.Tensor):
        with torch._C.DisableTorchFunctionSubclass():
            out.add(obj.untyped_storage().data_ptr())
    elif isinstance(obj, (list, tuple)):
        for x in obj:
            _storages(x, out)
    elif isinstance(obj, dict):
        for x in obj.values():
            _storages(x, out)
    return out


def carry_touched_by(args, kwargs) -> bool:
    """Whether a torch call with these arguments uses the storage of the
    carried mean's pool, output or loc."""
    c = current_carry()
    if c is None:
        return False
    mine = _storages([c[0].x, c[0].outs, c[0].loc], set())
    return bool(mine & _storages([args, kwargs or {}], set()))


def _same(a: torch.Tensor, b: torch.Tensor) -> bool:
    with torch._C.DisableTorchFunctionSubclass():
        return a.data_ptr() == b.data_ptr() and a.shape == b.shape


def _take_if(ok) -> Optional[Pending]:
    c = current_carry()
    if c is None:
        return None
    pending, stream, cap = c
    if not ok(pending) or _stream_of(pending.x.device) != stream or _capture_of(stream) != cap:
        flush_carry()
        return None
    _tls.carry = None
    return pending


def take_carry(y: torch.Tensor):
    """The carried page-finish mean if it writes the centroid pool `y` and
    was recorded on the current stream (the caller then runs it); None
    otherwise (anything carried is launched first)."""
    return _take_if(lambda p: p.carry_kind() == "mean" and _same(p.outs[0], y))


def take_carry_envelope(ya: torch.Tensor, yb: torch.Tensor):
    """The carried CMax + CMin if their outputs are the pools ya and yb (in
    either role), as (record, max pool, min pool); None otherwise (anything
    carried is launched first)."""
    from . import _hip

    def ok(p):
        if p.carry_kind() != "envelope":
            return False
        mx, mn = p.output_of(_hip.REDUCE_MAX), p.output_of(_hip.REDUCE_MIN)
        return (_same(mx, ya) and _same(mn, yb)) or (_same(mx, yb) and _same(mn, ya))

    p = _take_if(ok)
    if p is None:
        return None
    return p, p.output_of(_hip.REDUCE_MAX), p.output_of(_hip.REDUCE_MIN)


@contextlib.contextmanager
def scope(active: bool, kind: str = "indexer"):
    """Deferral scope; flushes everything still pending on exit.  kind
    "cache" (forward_cache) may leave a page-finish mean as the carry;
    kind "indexer" (forward_indexer) may consume it and launches it at exit
    if it did not."""
    if active and kind == "cache":
        flush_carry()
    prev = current_scope()
    sc = Scope() if active else None
    _tls.scope = sc
    try:
        yield sc
    finally:
        _tls.scope = prev
        if sc is not None:
            if (kind == "cache" and _carry_enabled() and len(sc.pending) == 1
                    and getattr(sc.pending[0], "carryable", lambda: False)()):
                p = sc.pending.pop()
                st = _stream_of(p.x.device)
                _install_capture_hooks()  # (only while something is carried)
                _tls.carry = (p, st, _capture_of(st))
            sc.flush()
            if kind == "indexer":
                flush_carry()


def flush_all() -> None:
    sc = current_scope()
    if sc is not None:
        sc.flush()


def is_metadata(func) -> bool:
    return func in _METADATA


def _mean_dim_args(args, kwargs):
    """(dim, keepdim) of a mean call, or None if it has other arguments."""
    rest = list(args[1:])
    kw = dict(kwargs)
    dim = kw.pop("dim", rest.pop(0) if rest else None)
    keepdim = kw.pop("keepdim", rest.pop(0) if rest else False)
    if rest or kw:
        return None
    if isinstance(dim, (tuple, list)):
        if len(dim) != 1:
            return None
        dim = dim[0]
    return dim, keepdim


def try_defer_mean(func, args, kwargs):
    """Records ``q.mean(dim=1, keepdim=True)`` of a BATCHED bf16 GPU vTensor
    and returns the DeferredTensor, or None if the call is anything else."""
    from .abs.tensor import FORMAT, vTensor

    if func not in (torch.Tensor.mean, torch.mean) or not args:
        return None
    q = args[0]
    if type(q) is not vTensor or q._format != FORMAT.BATCHED:
        return None
    parsed = _mean_dim_args(args, kwargs)
    if parsed is None:
        return None
    dim, keepdim = parsed
    with torch._C.DisableTorchFunctionSubclass():
        if not (q.is_cuda and q.dtype == torch.bfloat16 and q.dim() == 3 and q.is_contiguous()):
            return None
        if dim not in (1, -2) or keepdim is not True:
            return None
        qp = q.as_subclass(torch.Tensor)
        out = torch.empty((qp.shape[0], 1, qp.shape[2]), dtype=qp.dtype, device=qp.device)
    p = PendingMean(qp, out)
    current_scope().add(p)
    return DeferredTensor.make(out, FORMAT.BATCHED, p)


def _make_deferred_class():
    from .abs.tensor import vTensor

    class DeferredTensor(vTensor):
        """A vTensor whose contents are produced by a recorded computation."""

        _pending: Pending

        @classmethod
        def make(cls, base: torch.Tensor, fmt, pending: Pending) -> "DeferredTensor":
            out = torch.Tensor._make_subclass(cls, base, require_grad=False)
            out._format = fmt
            out._pending = pending
            pending._outs.append(weakref.ref(out))
            return out

        def materialize(self) -> None:
            self._pending.flush()

        @property
        def is_pending(self) -> bool:
            return not self._pending.done

        @classmethod
        def __torch_function__(cls, func, types, args=(), kwargs=None):
            if not is_metadata(func):
                flush_all()
                for t in _iter_deferred((args, kwargs or {})):
                    t._pending.flush()
            return vTensor.__torch_function__.__func__(vTensor, func, types, args, kwargs)

    return DeferredTensor


def _iter_deferred(obj):
    if isinstance(obj, DeferredTensor):
        yield obj
    elif isinstance(obj, (list, tuple)):
        for x in obj:
            yield from _iter_deferred(x)
    elif isinstance(obj, dict):
        for x in obj.values():
            yield from _iter_deferred(x)


DeferredTensor = _make_deferred_class()


def pending_of(t) -> Optional[Pending]:
    """The unflushed computation behind `t`, if any."""
    if isinstance(t, DeferredTensor) and not t._pending.done:
        return t._pending
    return None


def materialize(t):
    """Flushes `t`'s computation (if deferred) and returns `t`."""
    p = pending_of(t)
    if p is not None:
        p.flush()
    return t


def plain(t: torch.Tensor) -> torch.Tensor:
    """`t` as a plain torch.Tensor over the same storage, without running its
    subclass hooks (a recorded launch must not flush the scope it runs in).
    The result does not keep `t`'s Python object alive (``as_subclass`` would:
    its view refers back to `t`), so a recorded launch holding it does not
    make an elided result look observed."""
    with torch._C.DisableTorchFunctionSubclass():
        return torch.Tensor._make_subclass(torch.Tensor, t, require_grad=False)


def _install_launch_hook() -> None:
    from . import _hip

    _hip.set_pre_launch_hook(flush_carry)


_hooked = None  # (CUDAGraph class, original capture_begin, original capture_end) while the hooks are in


def _install_capture_hooks() -> None:
    """Makes torch.cuda.CUDAGraph.capture_begin / capture_end launch the carry
    first (see "Graph capture" above).  Installed when a mean is first
    carried, so a process that never carries one (VORTEX_FUSE_CMEAN=0,
    set_fusion(carry_cmean=False) or no forward_cache) keeps torch's own
    methods; remove_capture_hooks() puts those back."""
    global _hooked
    import functools

    graph = getattr(torch.cuda, "CUDAGraph", None)
    if graph is None or _hooked is not None:
        return
    begin, end = graph.capture_begin, graph.capture_end

    @functools.wraps(begin)
    def capture_begin(self, *args, **kwargs):
        flush_carry()
        return begin(self, *args, **kwargs)

    @functools.wraps(end)
    def capture_end(self, *args, **kwargs):
        flush_carry()
        return end(self, *args, **kwargs)

    graph.capture_begin, graph.capture_end = capture_begin, capture_end
    _hooked = (graph, begin, end)


def remove_capture_hooks() -> None:
    """Restores torch.cuda.CUDAGraph's own capture_begin / capture_end (a
    pending carry is launched first)."""
    global _hooked
    if _hooked is None:
        return
    flush_carry()
    graph, begin, end = _hooked
    graph.capture_begin, graph.capture_end = begin, end
    _hooked = None


def capture_hooks_installed() -> bool:
    return _hooked is not None


_install_launch_hook()
