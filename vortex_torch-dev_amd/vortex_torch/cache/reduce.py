"""Cache-side page-finish reductions: ``Mean`` (CMean), ``Max`` (CMax),
``Min`` (CMin), ``L2Norm`` (CL2Norm).

``CMean(dim=1)(x, out, loc=loc, ctx=ctx)`` reduces, for every token in
``loc`` that closes a page ((loc+1) % page_size == 0), each of that page's
``head_num`` tiles of the PAGED pool ``x [rows, R, C]`` (row = page*H + h):
``dim=1`` over its R axis into ``out[row, 0, :]``, ``dim=2`` over its C axis
into ``out[row, :, 0]``.  Mean is the fp32 mean, L2Norm the plain L2 norm
(no 1/n), both rounded to bf16 on store.  Other rows are untouched.

Profile / execute contract follows the reference
(vortex_torch/cache/reduce.py:10-350).  The implemented layout pair is
(PAGED, PAGED) — the one flows use on the cache path; it runs the gfx950
kernel ``vtx_page_reduce``.  :class:`MultiReduce` is an addition: several
reductions of the same pool in one pass over it.

Inside a flow's execute-mode ``forward_cache`` the reductions are recorded
and consecutive ones over the same pool and ``loc`` (the Quest flow's CMax
and CMin) run as one such pass when the method returns, or earlier when
torch reads one of their outputs; ``VORTEX_FUSE=0`` launches each at once.
"""
from __future__ import annotations

from typing import Callable, Dict, Optional, Sequence, Tuple

import torch

from .. import _deferred, _hip
from ..abs import FORMAT, as_vtensor, vOp, vTensor
from ..utils import ReduceType
from .context import Context

_KERNEL_TYPES = {
    ReduceType.Mean: _hip.REDUCE_MEAN,
    ReduceType.Max: _hip.REDUCE_MAX,
    ReduceType.Min: _hip.REDUCE_MIN,
    ReduceType.L2Norm: _hip.REDUCE_L2NORM,
}


def _kernel_type(rt: ReduceType) -> int:
    if rt not in _KERNEL_TYPES:
        raise RuntimeError(f"page reduce: {rt} is not a cache-side reduction")
    return _KERNEL_TYPES[rt]


def reduce_pp(x: torch.Tensor, output: torch.Tensor, loc: torch.Tensor, ctx: Context, dim: int,
              reduce_type: ReduceType) -> None:
    """(PAGED x, PAGED output): page-finish reduction triggered by loc."""
    _hip.page_reduce(x, output, loc, ctx.head_num, ctx.page_size, dim, _kernel_type(reduce_type))


class _PendingPageReduce(_deferred.Pending):
    """Page-finish reductions of one pool for one loc, recorded inside a
    flow's forward_cache: consecutive ones (up to four) run as one pass over
    the finished tiles (``vtx_page_reduce_multi``), whose outputs equal the
    separate launches' bit for bit."""

    MAX_OUTPUTS = 4

    def __init__(self, x: torch.Tensor, loc: torch.Tensor, ctx: Context, dim: int):
        super().__init__()
        self.x, self.loc, self.ctx, self.dim = x, loc, ctx, dim
        self.outs, self.types = [], []

    def accepts(self, x: torch.Tensor, out: torch.Tensor, loc: torch.Tensor, ctx: Context, dim: int) -> bool:
        if self.done or ctx is not self.ctx or dim != self.dim or len(self.outs) >= self.MAX_OUTPUTS:
            return False
        ptr = out.data_ptr()
        return (x.data_ptr() == self.x.data_ptr() and x.shape == self.x.shape and loc.data_ptr() == self.loc.data_ptr()
                and loc.numel() == self.loc.numel() and all(o.data_ptr() != ptr for o in self.outs))

    def add(self, out: torch.Tensor, kernel_type: int) -> None:
        self.outs.append(out)
        self.types.append(kernel_type)

    #: loc entries the fused indexer launch scans for a carried mean
    CARRY_MAX_LOC = 256

    def carry_kind(self):
        """"mean" (one CMean) or "envelope" (a CMax and a CMin), the page
        reduces a fused indexer launch can run; None for anything else."""
        kinds = sorted(self.types)
        if kinds == [_hip.REDUCE_MEAN]:
            return "mean"
        if kinds == sorted([_hip.REDUCE_MAX, _hip.REDUCE_MIN]):
            return "envelope"
        return None

    def output_of(self, kernel_type: int) -> torch.Tensor:
        return self.outs[self.types.index(kernel_type)]

    def carryable(self) -> bool:
        """Whether the next forward_indexer's fused launch may run this record
        (vtx_indexer_fused_cmean and its GQA / Quest forms): a decode-sized
        CMean, or CMax + CMin, (dim 1) of [page_size, D] tiles into bf16
        [rows, 1, D] pools."""
        if self.done or self.dim != 1 or self.carry_kind() is None:
            return False
        x = self.x
        for out in self.outs:
            if not _recordable_operands(x, out, self.loc):
                return False
            with torch._C.DisableTorchFunctionSubclass():
                if not (out.dtype == torch.bfloat16 and out.dim() == 3 and x.dim() == 3 and int(out.shape[1]) == 1
                        and int(x.shape[2]) == int(out.shape[2])):
                    return False
        with torch._C.DisableTorchFunctionSubclass():
            return int(x.shape[1]) == int(self.ctx.page_size) and self.loc.numel() <= self.CARRY_MAX_LOC

    def _run(self) -> None:
        c = self.ctx
        if len(self.outs) == 1:
            _hip.page_reduce(self.x, self.outs[0], self.loc, c.head_num, c.page_size, self.dim, self.types[0])
        else:
            _hip.page_reduce_multi(self.x, self.outs, self.types, self.loc, c.head_num, c.page_size, self.dim)


def _record_page_reduce(x, output, loc, ctx: Context, dim: int, reduce_type: ReduceType) -> bool:
    """Records a page-finish reduction in the current forward_cache scope
    (joining the newest record when it reduces the same pool for the same
    loc); False if it must run now.  Only a layout-tagged output is recorded,
    so reading it through torch runs the record first."""
    sc = _deferred.current_scope()
    if sc is None or not _deferred.fusion_enabled() or not isinstance(output, vTensor) or not isinstance(x, vTensor):
        return False
    if not _recordable_operands(x, output, loc):
        return False
    xp, op, lp = _deferred.plain(x), _deferred.plain(output), _deferred.plain(loc)
    last = sc.pending[-1] if sc.pending else None
    if not (isinstance(last, _PendingPageReduce) and last.accepts(xp, op, lp, ctx, dim)):
        last = _PendingPageReduce(xp, lp, ctx, dim)
        sc.add(last)
    last.add(op, _kernel_type(reduce_type))
    return True


def _recordable_operands(x, output, loc) -> bool:
    """GPU tensors, the output distinct from the pool."""
    with torch._C.DisableTorchFunctionSubclass():
        return x.is_cuda and output.is_cuda and loc.is_cuda and output.data_ptr() != x.data_ptr()


class Reduce(vOp):
    _impl_map: Dict[Tuple[FORMAT, FORMAT], Tuple[Callable, FORMAT]] = {
        (FORMAT.PAGED, FORMAT.PAGED): (reduce_pp, FORMAT.PAGED),
    }

    def __init__(self, dim: int = 1):
        super().__init__()
        self.dim = dim
        self.reduce_type: Optional[ReduceType] = None
        self.impl: Optional[Callable] = None
        self.output_format: Optional[FORMAT] = None
        self.output_buffer: Optional[torch.Tensor] = None
        assert self.dim in (1, 2), f"{type(self).__name__}.__init__: dim must be 1 or 2, got dim={self.dim}"

    def _infer_impl_ragged(self, x_fmt: FORMAT) -> Tuple[Callable, FORMAT]:
        key = (x_fmt, FORMAT.RAGGED)
        assert key in self._impl_map, (
            f"{self._prefix()}no RAGGED-output implementation for x_fmt={x_fmt}. "
            f"Available keys: {list(self._impl_map.keys())}")
        return self._impl_map[key]

    def profile(self, x: vTensor, output: Optional[vTensor], loc: torch.Tensor, ctx: Context) -> vTensor:
        p = self._prefix()
        assert isinstance(x, vTensor), f"{p}x must be vTensor, got {type(x)}"
        assert isinstance(loc, torch.Tensor), f"{p}loc must be torch.Tensor, got {type(loc)}"
        assert x.dim() == 3, f"{p}x must be 3D, got ndim={x.dim()} shape={tuple(x.shape)}"
        exp_n = 1 if self.dim == 1 else x.shape[1]
        exp_d = 1 if self.dim == 2 else x.shape[2]

        if output is None:
            self.impl, self.output_format = self._infer_impl_ragged(x._format)
            rows = ctx.max_new_tokens_per_batch * ctx.head_num
            self.output_buffer = torch.empty((rows, exp_n, exp_d), device=x.device, dtype=x.dtype)
            ctx.add_aux_memory(self.output_buffer)
            return as_vtensor(self.output_buffer, self.output_format)

        assert isinstance(output, vTensor), f"{p}output must be vTensor, got {type(output)}"
        assert output.dim() == 3, f"{p}output must be 3D, got ndim={output.dim()} shape={tuple(output.shape)}"
        key = (x._format, output._format)
        assert key in self._impl_map, (
            f"{p}no implementation for (x_fmt={key[0]}, o_fmt={key[1]}). "
            f"Available keys: {list(self._impl_map.keys())}")
        self.impl, self.output_format = self._impl_map[key]
        if self.dim == 1:
            assert output.shape[1] == 1, (
                f"{p}profile(dim=1): expected output.shape[1] == 1, got {tuple(output.shape)}")
            assert output.shape[2] == x.shape[2], (
                f"{p}profile(dim=1): expected output.shape[2] == x.shape[2], "
                f"got {output.shape[2]} vs {x.shape[2]}")
        else:
            assert output.shape[2] == 1, (
                f"{p}profile(dim=2): expected output.shape[2] == 1, got {tuple(output.shape)}")
            assert output.shape[1] == x.shape[1], (
                f"{p}profile(dim=2): expected output.shape[1] == x.shape[1], "
                f"got {output.shape[1]} vs {x.shape[1]}")
        assert x.device == output.device, (
            f"{p}x and output must be on the same device (x.device={x.device}, output.device={output.device})")
        return output

    def execute(self, x: torch.Tensor, output: Optional[torch.Tensor], loc: torch.Tensor,
                ctx: Context) -> torch.Tensor:
        p = self._prefix()
        assert self.impl is not None, f"{p}called before profile() (impl is None)"
        if output is None:
            assert self.output_buffer is not None, f"{p}internal output buffer is None; did profile() run?"
            output = self.output_buffer
        if self.impl is reduce_pp and _record_page_reduce(x, output, loc, ctx, self.dim, self.reduce_type):
            return output
        _deferred.flush_all()  # recorded reductions first, in program order
        self.impl(x, output, loc, ctx, self.dim, self.reduce_type)
        return output


class Mean(Reduce):
    """Arithmetic mean over one inner axis (CMean)."""

    def __init__(self, dim: int = 1):
        super().__init__(dim)
        self.reduce_type = ReduceType.Mean


class Max(Reduce):
    """Maximum over one inner axis (CMax)."""

    def __init__(self, dim: int = 1):
        super().__init__(dim)
        self.reduce_type = ReduceType.Max


class Min(Reduce):
    """Minimum over one inner axis (CMin)."""

    def __init__(self, dim: int = 1):
        super().__init__(dim)
        self.reduce_type = ReduceType.Min


class L2Norm(Reduce):
    """L2 norm (sqrt of the sum of squares, not RMS) over one inner axis."""

    def __init__(self, dim: int = 1):
        super().__init__(dim)
        self.reduce_type = ReduceType.L2Norm


class MultiReduce(vOp):
    """Several page-finish reductions of one PAGED pool in a single pass.

    ``MultiReduce([ReduceType.Mean, ReduceType.Max])(x, [out_mean, out_max],
    loc=loc, ctx=ctx)`` gives the same outputs as ``CMean`` then ``CMax`` while
    reading each finished tile of ``x`` once.  Not present in the reference.
    """

    def __init__(self, reduce_types: Sequence[ReduceType], dim: int = 1):
        super().__init__()
        self.reduce_types = list(reduce_types)
        assert 1 <= len(self.reduce_types) <= 4, "MultiReduce: 1..4 reductions"
        for rt in self.reduce_types:
            _kernel_type(rt)
        assert dim in (1, 2), f"MultiReduce: dim must be 1 or 2, got {dim}"
        self.dim = dim
        self._ready = False

    def profile(self, x: vTensor, outputs: Sequence[vTensor], loc: torch.Tensor, ctx: Context):
        p = self._prefix()
        assert isinstance(x, vTensor) and x._format == FORMAT.PAGED, f"{p}x must be a PAGED vTensor"
        assert len(outputs) == len(self.reduce_types), f"{p}one output per reduction"
        for o in outputs:
            assert isinstance(o, vTensor) and o._format == FORMAT.PAGED, f"{p}outputs must be PAGED vTensors"
            assert o.dim() == 3 and o.device == x.device, f"{p}bad output {tuple(o.shape)} on {o.device}"
            if self.dim == 1:
                assert o.shape[1] == 1 and o.shape[2] == x.shape[2], f"{p}dim=1 output must be [*, 1, {x.shape[2]}]"
            else:
                assert o.shape[2] == 1 and o.shape[1] == x.shape[1], f"{p}dim=2 output must be [*, {x.shape[1]}, 1]"
        self._ready = True
        return list(outputs)

    def execute(self, x: torch.Tensor, outputs: Sequence[torch.Tensor], loc: torch.Tensor, ctx: Context):
        assert self._ready, f"{self._prefix()}called before profile()"
        _deferred.flush_all()  # recorded reductions first, in program order
        _hip.page_reduce_multi(x, outputs, [_kernel_type(t) for t in self.reduce_types], loc,
                               ctx.head_num, ctx.page_size, self.dim)
        return list(outputs)


__all__ = ["Reduce", "Mean", "Max", "Min", "L2Norm", "MultiReduce", "reduce_pp"]
