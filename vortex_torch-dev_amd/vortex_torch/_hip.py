"""ctypes binding of the gfx950 kernel library (C ABI in ``include/vortex_hip.h``).

Every wrapper validates dtypes, devices, contiguity and sizes of its torch
tensors, then launches on torch's current HIP stream of the tensors' device.
Nothing here synchronises, reads device memory or allocates, so the wrappers
can be recorded into a HIP graph (``torch.cuda.graph``).

There is no CPU fallback: a tensor that is not on a GPU, or a missing
library, raises ``RuntimeError``.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch

_LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libvortex_hip.so"
_lock = threading.Lock()
_lib = None

_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_vp = ctypes.c_void_p

# Exported symbol -> argument types (order of include/vortex_hip.h).
_SIGNATURES = {
    "vtx_last_error": ([], ctypes.c_char_p),
    "vtx_version": ([], ctypes.c_char_p),
    "vtx_plan_decode": (
        [_vp, _i32, _vp, _vp, _i64, _vp, _vp, _i64, _vp, _vp, _i64, _i64, _vp, _vp, _vp, _vp,
         _i64, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _vp, _i64, _i32, _vp],
        ctypes.c_int,
    ),
    "vtx_plan_decode_fa3": (
        [_vp, _i32, _vp, _vp, _i64, _vp, _vp, _i64, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _vp,
         _vp, _vp, _vp, _i64, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _vp],
        ctypes.c_int,
    ),
    "vtx_gemv_paged": (
        [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _i32, _i32, _vp],
        ctypes.c_int,
    ),
    "vtx_topk_select": (
        [_vp, _i64, _vp, _vp, _vp, _i64, _vp, _i64, _i32, _i32, _i32, _i32, _i32, _vp],
        ctypes.c_int,
    ),
    "vtx_page_reduce": (
        [_vp, _i64, _i32, _i32, _vp, _i32, _i64, _vp, _i64, _i32, _i32, _i32, _i32, _vp],
        ctypes.c_int,
    ),
    "vtx_page_reduce_multi": (
        [_vp, _i64, _i32, _i32, _i32, _vp, _vp, _vp, _i64, _vp, _i64, _i32, _i32, _i32, _vp],
        ctypes.c_int,
    ),
    "vtx_indexer_fused": (
        [_vp, _i64, _i32, _vp, _vp, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _i64,
         _i32, _i32, _i32, _i32, _i32, _i32, _vp, _i64, _i32, _vp, _i64, _vp],
        ctypes.c_int,
    ),
    "vtx_indexer_fused_noalloc": (
        [_vp, _i64, _i32, _vp, _vp, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _i64,
         _i32, _i32, _i32, _i32, _i32, _i32, _i32, _vp, _i64, _vp],
        ctypes.c_int,
    ),
    "vtx_indexer_fused_workspace_len": ([_i32], ctypes.c_int64),
    "vtx_indexer_fused_noalloc_reset": ([_vp], ctypes.c_int),
    "vtx_indexer_fused_supported": ([_i32], ctypes.c_int),
    "vtx_indexer_fused_cmean": (
        [_vp, _i64, _i32, _vp, _vp, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _i64,
         _i32, _i32, _i32, _i32, _i32, _i32, _vp, _i64, _i32, _vp, _i64, _i32, _i32, _vp, _i64, _vp, _i64, _vp],
        ctypes.c_int,
    ),
    "vtx_indexer_gqa_fused": (
        [_vp, _i64, _i32, _vp, _i64, _i32, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _i64,
         _i32, _i32, _i32, _i32, _i32, _i32, ctypes.c_float, _vp, _i64, _vp],
        ctypes.c_int,
    ),
    "vtx_indexer_gqa_fused_supported": ([_i32, _i32], ctypes.c_int),
    "vtx_indexer_gqa_fused_cmean": (
        [_vp, _i64, _i32, _vp, _i64, _i32, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _i64,
         _i32, _i32, _i32, _i32, _i32, _i32, ctypes.c_float, _vp, _i64, _i32, _i32, _vp, _i64, _vp, _i64, _vp],
        ctypes.c_int,
    ),
    "vtx_indexer_quest_fused": (
        [_vp, _i64, _i32, _vp, _vp, _i64, _i32, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _i64,
         _i32, _i32, _i32, _i32, _i32, _vp, _i64, _vp],
        ctypes.c_int,
    ),
    "vtx_indexer_quest_fused_supported": ([_i32, _i32], ctypes.c_int),
    "vtx_indexer_quest_fused_cmean": (
        [_vp, _i64, _i32, _vp, _vp, _i64, _i32, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _i64,
         _i32, _i32, _i32, _i32, _i32, _vp, _i64, _i32, _i32, _vp, _i64, _vp, _i64, _vp],
        ctypes.c_int,
    ),
    "vtx_ragged_gemm": (
        [_vp, _i64, _i32, _i32, _vp, _i64, _i32, _i32, _i32, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _i64,
         _vp, _vp],
        ctypes.c_int,
    ),
    "vtx_ragged_binary": (
        [_i32, ctypes.c_float, ctypes.c_float, _vp, _i64, _i32, _i32, _i32, _vp, _i64, _i32, _i32, _i32,
         _vp, _i64, _i32, _i32, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _vp],
        ctypes.c_int,
    ),
    "vtx_ragged_unary": (
        [_i32, ctypes.c_float, ctypes.c_float, _vp, _i64, _i32, _i32, _vp, _i64, _vp, _vp, _i64, _vp, _vp],
        ctypes.c_int,
    ),
    "vtx_ragged_reduce": (
        [_vp, _i64, _i32, _i32, _vp, _i64, _i32, _i32, _vp, _vp, _i64, _vp, _vp],
        ctypes.c_int,
    ),
    "vtx_set_kv_buffer": (
        [_vp, _vp, _i64, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _i32, _vp],
        ctypes.c_int,
    ),
    "vtx_paged_decode_attention": (
        [_vp, _vp, _vp, _vp, _i64, _vp, _vp, _i64, _vp, _i32, _i32, _i32, _i32, _i32, ctypes.c_float, _vp],
        ctypes.c_int,
    ),
    "vtx_paged_decode_attention_supported": ([_i32, _i32], ctypes.c_int),
    "vtx_bf16_rounding_check": ([_vp, _vp], ctypes.c_int),
    "vtx_stream_capture_id": ([_vp, ctypes.POINTER(ctypes.c_ulonglong)], ctypes.c_int),
    "vtx_probe_read": ([_vp, _i64, _vp, _i64, ctypes.c_uint32, _vp], ctypes.c_int),
    "vtx_probe_gather": ([_vp, _i64, _i32, _vp, _i64, _vp, _i32, _vp, _i64, ctypes.c_uint32, _vp], ctypes.c_int),
    "vtx_segment_scan": (
        [_i32, ctypes.c_float, _vp, _i64, _i32, _vp, _i32, _i32, _i32, _i32, _vp],
        ctypes.c_int,
    ),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)

REDUCE_MEAN, REDUCE_MAX, REDUCE_MIN, REDUCE_L2NORM, REDUCE_SUM = 0, 1, 2, 3, 4
ROWS_BATCHED, ROWS_PAGED, ROWS_RAGGED = 0, 1, 2
SEGMENT_SOFTMAX, SEGMENT_NORMALIZE = 0, 1
DTYPE_BF16, DTYPE_F32 = 0, 1
FUSED_AUTO, FUSED_SEGMENT, FUSED_SPLIT = 0, 1, 2


def library_path() -> Path:
    return _LIB_PATH


def load_library(path: os.PathLike | str | None = None) -> ctypes.CDLL:
    """Loads (once) and returns the kernel library; raises if it is missing."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = Path(path) if path is not None else _LIB_PATH
        if not p.exists():
            raise RuntimeError(
                f"vortex_torch: kernel library not found at {p}; build it with "
                "`python vortex_torch-dev_amd/build_native.py` (or __graft_entry__.build())"
            )
        lib = ctypes.CDLL(str(p), mode=ctypes.RTLD_LOCAL)
        for name, (argtypes, restype) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = restype
        if path is None:
            _lib = lib
        return lib


def _plain(t):
    """The same tensor without its subclass: layout-tagged and deferred tensors
    are passed to the kernels by pointer, without running their torch hooks."""
    if isinstance(t, torch.Tensor) and type(t) is not torch.Tensor:
        with torch._C.DisableTorchFunctionSubclass():
            return t.as_subclass(torch.Tensor)
    if isinstance(t, (list, tuple)):
        return type(t)(_plain(x) for x in t)
    return t


def _plain_args(fn):
    import functools

    @functools.wraps(fn)
    def wrapper(*args, **kwargs):
        return fn(*[_plain(a) for a in args], **{k: _plain(v) for k, v in kwargs.items()})

    return wrapper


def _check(rc: int, what: str) -> None:
    if rc != 0:
        msg = _lib.vtx_last_error().decode(errors="replace") if _lib is not None else ""
        raise RuntimeError(f"vortex_torch HIP {what} failed (code {rc}): {msg}")


_pre_launch = None


def set_pre_launch_hook(fn) -> None:
    """fn() runs before every launch of this module (the deferral layer uses
    it to launch recorded work that a new launch could observe)."""
    global _pre_launch
    _pre_launch = fn


def _require_gpu(*tensors: torch.Tensor) -> torch.device:
    if _pre_launch is not None:
        _pre_launch()
    dev = None
    for t in tensors:
        if t.device.type != "cuda":
            raise RuntimeError(
                f"vortex_torch: HIP kernels need GPU tensors, got a tensor on {t.device} "
                "(there is no CPU implementation)"
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"vortex_torch: tensors on different devices ({dev} vs {t.device})")
    return dev


def _req(t: torch.Tensor, dtype: torch.dtype, name: str) -> torch.Tensor:
    if t.dtype != dtype:
        raise RuntimeError(f"vortex_torch: {name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise RuntimeError(f"vortex_torch: {name} must be contiguous")
    return t


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def stream_capture_id(stream) -> int:
    """0 if the torch stream `stream` is not being captured into a graph, else
    an id of the capture in progress (host-side query, no launch)."""
    lib = load_library()
    out = ctypes.c_ulonglong(0)
    _check(lib.vtx_stream_capture_id(stream.cuda_stream, ctypes.byref(out)), "stream_capture_id")
    return int(out.value)


_cu_counts: dict = {}


def device_cu_count(dev: torch.device) -> int:
    """Compute units of `dev` (cached)."""
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    if idx not in _cu_counts:
        _cu_counts[idx] = int(torch.cuda.get_device_properties(idx).multi_processor_count)
    return _cu_counts[idx]


class _on_device:
    """Makes `dev` current for the duration of a launch (no-op if it already is)."""

    def __init__(self, dev: torch.device):
        self.dev = dev
        self.prev = None

    def __enter__(self):
        cur = torch.cuda.current_device()
        idx = self.dev.index if self.dev.index is not None else cur
        if idx != cur:
            self.prev = cur
            torch.cuda.set_device(idx)
        return self

    def __exit__(self, *exc):
        if self.prev is not None:
            torch.cuda.set_device(self.prev)
        return False


# ----------------------------------------------------------------------------
# entry points
# ----------------------------------------------------------------------------
@_plain_args
def plan_decode(
    cached_seq_lens: torch.Tensor,
    dense_kv_indptr: torch.Tensor,
    dense_kv_indices: torch.Tensor,
    sparse_kv_indptr: torch.Tensor,
    sparse_kv_indices: torch.Tensor,
    kv_last_page_len: torch.Tensor,
    req_to_token: torch.Tensor,
    req_indices: torch.Tensor,
    winfo_q_indices: torch.Tensor,
    winfo_kv_offsets: torch.Tensor,
    winfo_kv_lens: torch.Tensor,
    winfo_num_workloads: torch.Tensor,
    winfo_chunk_size: torch.Tensor,
    page_size: int,
    num_kv_heads: int,
    topk_val: int,
    page_reserved_bos: int,
    page_reserved_eos: int,
    max_chunk_size: int,
    min_chunk_size: int,
    fused_schedule=None,
    schedule_round: int = 0,
) -> None:
    """Decode planner (vtx_plan_decode).  fused_schedule (optional int32
    buffer of at least 4 + 4 * B * H entries): also write the fused indexer's
    workgroup order for this block table, dealt in rounds of schedule_round
    workgroups (the device's compute-unit count; 0 = this device's)."""
    lib = load_library()
    i32 = torch.int32
    dev = _require_gpu(cached_seq_lens, dense_kv_indptr, dense_kv_indices, sparse_kv_indptr,
                       sparse_kv_indices, kv_last_page_len, req_to_token, req_indices,
                       winfo_q_indices, winfo_kv_offsets, winfo_kv_lens, winfo_num_workloads,
                       winfo_chunk_size, *([fused_schedule] if fused_schedule is not None else []))
    for t, n in ((cached_seq_lens, "cached_seq_lens"), (dense_kv_indptr, "dense_kv_indptr"),
                 (dense_kv_indices, "dense_kv_indices"), (sparse_kv_indptr, "sparse_kv_indptr"),
                 (sparse_kv_indices, "sparse_kv_indices"), (kv_last_page_len, "kv_last_page_len"),
                 (req_to_token, "req_to_token"), (winfo_q_indices, "winfo_q_indices"),
                 (winfo_kv_offsets, "winfo_kv_offsets"), (winfo_kv_lens, "winfo_kv_lens"),
                 (winfo_num_workloads, "winfo_num_workloads"), (winfo_chunk_size, "winfo_chunk_size")):
        _req(t, i32, n)
    _req(req_indices, torch.int64, "req_indices")
    B = int(cached_seq_lens.shape[0])
    H = int(num_kv_heads)
    if req_to_token.dim() != 2:
        raise RuntimeError("vortex_torch: req_to_token must be 2-D [rows, max_tokens]")
    if req_indices.numel() < B:
        raise RuntimeError("vortex_torch: req_indices shorter than cached_seq_lens")
    if dense_kv_indptr.numel() < B * H + 1 or sparse_kv_indptr.numel() < B * H + 1:
        raise RuntimeError(f"vortex_torch: indptr buffers need {B * H + 1} entries")
    if kv_last_page_len.numel() < B * H:
        raise RuntimeError(f"vortex_torch: kv_last_page_len needs {B * H} entries")
    if winfo_num_workloads.numel() < 1 or winfo_chunk_size.numel() < 1:
        raise RuntimeError("vortex_torch: winfo_num_workloads / winfo_chunk_size need 1 entry")
    wcap = min(winfo_q_indices.numel(), winfo_kv_offsets.numel(), winfo_kv_lens.numel())
    sched_ptr, sched_len, sched_round = None, 0, 0
    if fused_schedule is not None:
        _req(fused_schedule, i32, "fused_schedule")
        if fused_schedule.numel() >= 4 + 4 * B * H:  # (too small: no schedule)
            sched_ptr, sched_len = fused_schedule.data_ptr(), fused_schedule.numel()
            sched_round = int(schedule_round) if schedule_round else device_cu_count(dev)
    with _on_device(dev):
        rc = lib.vtx_plan_decode(
            cached_seq_lens.data_ptr(), B,
            dense_kv_indptr.data_ptr(), dense_kv_indices.data_ptr(), dense_kv_indices.numel(),
            sparse_kv_indptr.data_ptr(), sparse_kv_indices.data_ptr(), sparse_kv_indices.numel(),
            kv_last_page_len.data_ptr(),
            req_to_token.data_ptr(), int(req_to_token.shape[0]), int(req_to_token.shape[1]),
            req_indices.data_ptr(),
            winfo_q_indices.data_ptr(), winfo_kv_offsets.data_ptr(), winfo_kv_lens.data_ptr(), wcap,
            winfo_num_workloads.data_ptr(), winfo_chunk_size.data_ptr(),
            int(page_size), H, int(topk_val), int(page_reserved_bos), int(page_reserved_eos),
            int(max_chunk_size), int(min_chunk_size), sched_ptr, sched_len, sched_round, _stream(dev))
    _check(rc, "plan_decode")


@_plain_args
def plan_decode_fa3(
    cached_seq_lens: torch.Tensor,
    dense_kv_indptr: torch.Tensor,
    dense_kv_indices: torch.Tensor,
    sparse_kv_indptr: torch.Tensor,
    sparse_kv_indices: torch.Tensor,
    dense_page_table: torch.Tensor,
    dense_cache_seqlens: torch.Tensor,
    sparse_page_table: torch.Tensor,
    sparse_cache_seqlens: torch.Tensor,
    req_to_token: torch.Tensor,
    req_indices: torch.Tensor,
    winfo_q_indices: torch.Tensor,
    winfo_kv_offsets: torch.Tensor,
    winfo_kv_lens: torch.Tensor,
    winfo_num_workloads: torch.Tensor,
    winfo_chunk_size: torch.Tensor,
    page_size: int,
    num_kv_heads: int,
    topk_val: int,
    page_reserved_bos: int,
    page_reserved_eos: int,
    max_chunk_size: int,
    min_chunk_size: int,
) -> None:
    """FA3 decode planner: the block tables and workload list of plan_decode
    plus per-segment padded page tables and cache sequence lengths."""
    lib = load_library()
    i32 = torch.int32
    tensors = (cached_seq_lens, dense_kv_indptr, dense_kv_indices, sparse_kv_indptr, sparse_kv_indices,
               dense_page_table, dense_cache_seqlens, sparse_page_table, sparse_cache_seqlens, req_to_token,
               winfo_q_indices, winfo_kv_offsets, winfo_kv_lens, winfo_num_workloads, winfo_chunk_size)
    dev = _require_gpu(req_indices, *tensors)
    for t in tensors:
        _req(t, i32, "FA3 planner int32 buffer")
    _req(req_indices, torch.int64, "req_indices")
    B = int(cached_seq_lens.shape[0])
    H = int(num_kv_heads)
    if req_to_token.dim() != 2:
        raise RuntimeError("vortex_torch: req_to_token must be 2-D [rows, max_tokens]")
    if dense_page_table.dim() != 2 or sparse_page_table.shape != dense_page_table.shape:
        raise RuntimeError("vortex_torch: dense and sparse page tables must be 2-D and of one shape")
    if req_indices.numel() < B:
        raise RuntimeError("vortex_torch: req_indices shorter than cached_seq_lens")
    if dense_kv_indptr.numel() < B * H + 1 or sparse_kv_indptr.numel() < B * H + 1:
        raise RuntimeError(f"vortex_torch: indptr buffers need {B * H + 1} entries")
    if winfo_num_workloads.numel() < 1 or winfo_chunk_size.numel() < 1:
        raise RuntimeError("vortex_torch: winfo_num_workloads / winfo_chunk_size need 1 entry")
    wcap = min(winfo_q_indices.numel(), winfo_kv_offsets.numel(), winfo_kv_lens.numel())
    cs_len = min(dense_cache_seqlens.numel(), sparse_cache_seqlens.numel())
    with _on_device(dev):
        rc = lib.vtx_plan_decode_fa3(
            cached_seq_lens.data_ptr(), B,
            dense_kv_indptr.data_ptr(), dense_kv_indices.data_ptr(), dense_kv_indices.numel(),
            sparse_kv_indptr.data_ptr(), sparse_kv_indices.data_ptr(), sparse_kv_indices.numel(),
            dense_page_table.data_ptr(), dense_cache_seqlens.data_ptr(), sparse_page_table.data_ptr(),
            sparse_cache_seqlens.data_ptr(), int(dense_page_table.shape[0]), int(dense_page_table.shape[1]), cs_len,
            req_to_token.data_ptr(), int(req_to_token.shape[0]), int(req_to_token.shape[1]), req_indices.data_ptr(),
            winfo_q_indices.data_ptr(), winfo_kv_offsets.data_ptr(), winfo_kv_lens.data_ptr(), wcap,
            winfo_num_workloads.data_ptr(), winfo_chunk_size.data_ptr(),
            int(page_size), H, int(topk_val), int(page_reserved_bos), int(page_reserved_eos),
            int(max_chunk_size), int(min_chunk_size), _stream(dev))
    _check(rc, "plan_decode_fa3")


@_plain_args
def gemv_paged(
    x: torch.Tensor,
    y: torch.Tensor,
    o: torch.Tensor,
    dense_kv_indices: torch.Tensor,
    winfo_q_indices: torch.Tensor,
    winfo_kv_offsets: torch.Tensor,
    winfo_kv_lens: torch.Tensor,
    winfo_num_workloads: torch.Tensor,
    max_chunk_size: int,
) -> None:
    lib = load_library()
    dev = _require_gpu(x, y, o, dense_kv_indices, winfo_q_indices, winfo_kv_offsets,
                       winfo_kv_lens, winfo_num_workloads)
    _req(x, torch.bfloat16, "x")
    _req(y, torch.bfloat16, "y")
    _req(o, torch.bfloat16, "o")
    for t, n in ((dense_kv_indices, "dense_kv_indices"), (winfo_q_indices, "winfo_q_indices"),
                 (winfo_kv_offsets, "winfo_kv_offsets"), (winfo_kv_lens, "winfo_kv_lens"),
                 (winfo_num_workloads, "winfo_num_workloads")):
        _req(t, torch.int32, n)
    D = int(x.shape[-1])
    if int(y.shape[-1]) != D:
        raise RuntimeError(f"vortex_torch: GeMV head_dim mismatch ({D} vs {int(y.shape[-1])})")
    wcap = min(winfo_q_indices.numel(), winfo_kv_offsets.numel(), winfo_kv_lens.numel())
    with _on_device(dev):
        rc = lib.vtx_gemv_paged(
            x.data_ptr(), x.numel() // D, y.data_ptr(), y.numel() // D, o.data_ptr(), o.numel(),
            dense_kv_indices.data_ptr(), dense_kv_indices.numel(),
            winfo_q_indices.data_ptr(), winfo_kv_offsets.data_ptr(), winfo_kv_lens.data_ptr(), wcap,
            winfo_num_workloads.data_ptr(), D, int(max_chunk_size), _stream(dev))
    _check(rc, "gemv_paged")


@_plain_args
def topk_select(
    x: torch.Tensor,
    dense_kv_indptr: torch.Tensor,
    sparse_kv_indptr: torch.Tensor,
    dense_kv_indices: torch.Tensor,
    sparse_kv_indices: torch.Tensor,
    eff_batch_size: int,
    topk_val: int,
    reserved_bos: int,
    reserved_eos: int,
    max_num_pages: int,
) -> None:
    lib = load_library()
    dev = _require_gpu(x, dense_kv_indptr, sparse_kv_indptr, dense_kv_indices, sparse_kv_indices)
    _req(x, torch.bfloat16, "x (scores)")
    for t, n in ((dense_kv_indptr, "dense_kv_indptr"), (sparse_kv_indptr, "sparse_kv_indptr"),
                 (dense_kv_indices, "dense_kv_indices"), (sparse_kv_indices, "sparse_kv_indices")):
        _req(t, torch.int32, n)
    eff = int(eff_batch_size)
    if eff < 0:
        raise RuntimeError("vortex_torch: eff_batch_size must be >= 0")
    if dense_kv_indptr.numel() < eff + 1 or sparse_kv_indptr.numel() < eff + 1:
        raise RuntimeError(f"vortex_torch: indptr buffers need {eff + 1} entries")
    with _on_device(dev):
        rc = lib.vtx_topk_select(
            x.data_ptr(), x.numel(), dense_kv_indptr.data_ptr(), sparse_kv_indptr.data_ptr(),
            dense_kv_indices.data_ptr(), dense_kv_indices.numel(),
            sparse_kv_indices.data_ptr(), sparse_kv_indices.numel(),
            eff, int(topk_val), int(reserved_bos), int(reserved_eos), int(max_num_pages),
            _stream(dev))
    _check(rc, "topk_select")


_OUT_DTYPES = {torch.bfloat16: DTYPE_BF16, torch.float32: DTYPE_F32}


def _reduce_geometry(x: torch.Tensor, out: torch.Tensor, dim: int):
    if x.dim() != 3:
        raise RuntimeError("vortex_torch: page reduce expects x of rank 3 [rows, R, C]")
    rows, R, C = (int(s) for s in x.shape)
    if dim == 1:
        per_row = C
    elif dim == 2:
        per_row = R
    else:
        raise RuntimeError(f"vortex_torch: dim must be 1 or 2, got {dim}")
    if out.numel() % max(per_row, 1) != 0:
        raise RuntimeError("vortex_torch: page reduce output size is not a multiple of its row")
    return rows, R, C, out.numel() // max(per_row, 1)


@_plain_args
def page_reduce(x: torch.Tensor, out: torch.Tensor, loc: torch.Tensor, num_kv_heads: int,
                page_size: int, dim: int, reduce_type: int) -> None:
    lib = load_library()
    dev = _require_gpu(x, out, loc)
    _req(x, torch.bfloat16, "x")
    _req(loc, torch.int64, "loc")
    if out.dtype not in _OUT_DTYPES:
        raise RuntimeError(f"vortex_torch: reduce output must be bf16 or fp32, got {out.dtype}")
    _req(out, out.dtype, "output")
    rows, R, C, out_rows = _reduce_geometry(x, out, dim)
    with _on_device(dev):
        rc = lib.vtx_page_reduce(
            x.data_ptr(), rows, R, C, out.data_ptr(), _OUT_DTYPES[out.dtype], out_rows,
            loc.data_ptr(), loc.numel(), int(num_kv_heads), int(page_size), int(dim),
            int(reduce_type), _stream(dev))
    _check(rc, "page_reduce")


@_plain_args
def page_reduce_multi(x: torch.Tensor, outs, reduce_types, loc: torch.Tensor, num_kv_heads: int,
                      page_size: int, dim: int = 1) -> None:
    """One pass over every finished tile of x feeding up to four reductions."""
    lib = load_library()
    outs = list(outs)
    reduce_types = [int(t) for t in reduce_types]
    if not 1 <= len(outs) <= 4 or len(outs) != len(reduce_types):
        raise RuntimeError("vortex_torch: page_reduce_multi needs 1..4 outputs, one type each")
    dev = _require_gpu(x, loc, *outs)
    _req(x, torch.bfloat16, "x")
    _req(loc, torch.int64, "loc")
    out_rows = None
    for o in outs:
        if o.dtype not in _OUT_DTYPES:
            raise RuntimeError(f"vortex_torch: reduce output must be bf16 or fp32, got {o.dtype}")
        _req(o, o.dtype, "output")
        rows, R, C, r = _reduce_geometry(x, o, dim)
        out_rows = r if out_rows is None else min(out_rows, r)
    n = len(outs)
    ptrs = (ctypes.c_void_p * n)(*[o.data_ptr() for o in outs])
    dts = (ctypes.c_int32 * n)(*[_OUT_DTYPES[o.dtype] for o in outs])
    tys = (ctypes.c_int32 * n)(*reduce_types)
    with _on_device(dev):
        rc = lib.vtx_page_reduce_multi(
            x.data_ptr(), rows, R, C, n, ptrs, dts, tys, out_rows, loc.data_ptr(), loc.numel(),
            int(num_kv_heads), int(page_size), int(dim), _stream(dev))
    _check(rc, "page_reduce_multi")


def indexer_fused_supported(head_dim: int) -> bool:
    return bool(load_library().vtx_indexer_fused_supported(int(head_dim)))


def indexer_fused_workspace_len(segments: int) -> int:
    """int32 entries of a fused-indexer workspace (arrival counters and the
    staging zone of the split layout's pre-selection) that serves every call
    with up to `segments` segments; allocate it zeroed."""
    n = int(load_library().vtx_indexer_fused_workspace_len(int(segments)))
    if n < 0:
        raise RuntimeError(f"vortex_torch: no fused-indexer workspace for {segments} segments")
    return n


def indexer_fused_noalloc_reset(device=None) -> None:
    """Clears the arrival counters of the no-allocation entry point's
    workspace on `device` (a fill kernel on its current stream)."""
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    lib = load_library()
    with _on_device(dev):
        rc = lib.vtx_indexer_fused_noalloc_reset(_stream(dev))
    _check(rc, "indexer_fused_noalloc_reset")


def _schedule_args(schedule):
    """(pointer, length) of a planner-written fused schedule, or (None, 0)."""
    if schedule is None:
        return (None, 0)
    _req(schedule, torch.int32, "schedule")
    return (schedule.data_ptr(), schedule.numel())


@_plain_args
def indexer_fused(
    q: torch.Tensor,
    x_out,
    y: torch.Tensor,
    score: torch.Tensor,
    dense_kv_indptr: torch.Tensor,
    sparse_kv_indptr: torch.Tensor,
    dense_kv_indices: torch.Tensor,
    sparse_kv_indices: torch.Tensor,
    eff_batch_size: int,
    topk_val: int,
    reserved_bos: int,
    reserved_eos: int,
    max_num_pages: int,
    seg_counters=None,
    mode: int = FUSED_AUTO,
    cmean=None,
    schedule=None,
    noalloc: bool = False,
) -> None:
    """q-mean + GeMV + topK of one layer in one launch.

    q: bf16 [S, G, D] (the head-group mean is taken in the kernel and written
    to x_out if given) or [S, 1, D] / [S, D] already-averaged rows (G taken as
    0: rows used as they are).  y: centroid pool [rows, 1, D]; score: the GeMV
    output buffer; the block tables come from the planner.  seg_counters: the
    split layout's int32 workspace, zeroed once (``indexer_fused_workspace_len``
    entries for up to S segments, or at least S for counters only), that
    lets long segments be split over several workgroups (the kernel leaves
    its counters at zero); mode: FUSED_AUTO,
    FUSED_SEGMENT or FUSED_SPLIT.  cmean: (k_cache [rows, P, D] bf16, loc
    int64, num_kv_heads) — the layer's page-finish mean into y, run first in
    the same launch (``vtx_indexer_fused_cmean``), with the results of a
    separate ``page_reduce`` launch before this one.  schedule: the
    fused_schedule plan_decode wrote for this block table (the workgroup
    order of the one-workgroup-per-segment layout; speed only).  noalloc:
    launch through ``vtx_indexer_fused_noalloc`` (the library's own
    workspace; no seg_counters, no cmean).
    """
    lib = load_library()
    tensors = [q, y, score, dense_kv_indptr, sparse_kv_indptr, dense_kv_indices, sparse_kv_indices]
    if schedule is not None:
        tensors.append(schedule)
    if cmean is not None:
        tensors += [cmean[0], cmean[1]]
    if x_out is not None:
        tensors.append(x_out)
    if seg_counters is not None:
        tensors.append(seg_counters)
    dev = _require_gpu(*tensors)
    if seg_counters is not None:
        _req(seg_counters, torch.int32, "seg_counters")
    _req(q, torch.bfloat16, "q")
    _req(y, torch.bfloat16, "y (centroids)")
    _req(score, torch.bfloat16, "score")
    for t, n in ((dense_kv_indptr, "dense_kv_indptr"), (sparse_kv_indptr, "sparse_kv_indptr"),
                 (dense_kv_indices, "dense_kv_indices"), (sparse_kv_indices, "sparse_kv_indices")):
        _req(t, torch.int32, n)
    D = int(q.shape[-1])
    if int(y.shape[-1]) != D:
        raise RuntimeError(f"vortex_torch: fused indexer head_dim mismatch ({D} vs {int(y.shape[-1])})")
    eff = int(eff_batch_size)
    G = int(q.shape[1]) if q.dim() == 3 else 1
    S = q.numel() // (G * D)
    if S < eff:
        raise RuntimeError(f"vortex_torch: {S} query rows for {eff} segments")
    if dense_kv_indptr.numel() < eff + 1 or sparse_kv_indptr.numel() < eff + 1:
        raise RuntimeError(f"vortex_torch: indptr buffers need {eff + 1} entries")
    if x_out is not None:
        _req(x_out, torch.bfloat16, "x_out (q_mean)")
        if x_out.numel() < S * D:
            raise RuntimeError("vortex_torch: q_mean output too small")
    averaged = G == 1 and x_out is None
    args = (None if averaged else q.data_ptr(), S, 0 if averaged else G,
            q.data_ptr() if averaged else None,
            x_out.data_ptr() if x_out is not None else None,
            y.data_ptr(), y.numel() // D, score.data_ptr(), score.numel(),
            dense_kv_indptr.data_ptr(), sparse_kv_indptr.data_ptr(),
            dense_kv_indices.data_ptr(), dense_kv_indices.numel(),
            sparse_kv_indices.data_ptr(), sparse_kv_indices.numel(),
            eff, int(topk_val), int(reserved_bos), int(reserved_eos), int(max_num_pages), D,
            seg_counters.data_ptr() if seg_counters is not None else None,
            seg_counters.numel() if seg_counters is not None else 0, int(mode))
    sched = _schedule_args(schedule)
    if noalloc:
        if seg_counters is not None or cmean is not None:
            raise RuntimeError("vortex_torch: the no-allocation entry point takes no seg_counters and no cmean")
        with _on_device(dev):
            rc = lib.vtx_indexer_fused_noalloc(*args[:-3], int(mode), *sched, _stream(dev))
        _check(rc, "indexer_fused_noalloc")
        return
    if cmean is not None:
        k, loc, heads = cmean
        _req(k, torch.bfloat16, "k_cache")
        _req(loc, torch.int64, "loc")
        if k.dim() != 3 or int(k.shape[2]) != D or int(y.shape[1]) != 1:
            raise RuntimeError(f"vortex_torch: CMean pool {tuple(k.shape)} / centroids {tuple(y.shape)} "
                               f"do not match head_dim {D}")
        with _on_device(dev):
            rc = lib.vtx_indexer_fused_cmean(*args, k.data_ptr(), int(k.shape[0]), int(k.shape[1]), int(heads),
                                             loc.data_ptr(), loc.numel(), *sched, _stream(dev))
        _check(rc, "indexer_fused_cmean")
        return
    with _on_device(dev):
        rc = lib.vtx_indexer_fused(*args, *sched, _stream(dev))
    _check(rc, "indexer_fused")


def indexer_gqa_fused_supported(head_dim: int, group_size: int) -> bool:
    return bool(load_library().vtx_indexer_gqa_fused_supported(int(head_dim), int(group_size)))


@_plain_args
def indexer_gqa_fused(
    q: torch.Tensor,
    y: torch.Tensor,
    score: torch.Tensor,
    aggr: torch.Tensor,
    dense_kv_indptr: torch.Tensor,
    sparse_kv_indptr: torch.Tensor,
    dense_kv_indices: torch.Tensor,
    sparse_kv_indices: torch.Tensor,
    eff_batch_size: int,
    topk_val: int,
    reserved_bos: int,
    reserved_eos: int,
    max_num_pages: int,
    softmax_scale=None,
    cmean=None,
    schedule=None,
) -> None:
    """GeMM + segment softmax (unless softmax_scale is None) + max over the
    query heads + topK of one GQA layer in one launch.

    q: bf16 [S, G, D]; y: centroid pool [rows, 1, D]; score: the GeMM output
    buffer [pages, 1, G]; aggr: the Max output buffer [pages, 1, 1]; the
    block tables come from the planner.  cmean: (k_cache [rows, P, D] bf16,
    loc int64, num_kv_heads) — the layer's page-finish mean into y, run first
    in the same launch (``vtx_indexer_gqa_fused_cmean``).  schedule: the
    fused_schedule plan_decode wrote for this block table (workgroup order;
    speed only).
    """
    lib = load_library()
    tensors = [q, y, score, aggr, dense_kv_indptr, sparse_kv_indptr, dense_kv_indices, sparse_kv_indices]
    if schedule is not None:
        tensors.append(schedule)
    if cmean is not None:
        tensors += [cmean[0], cmean[1]]
    dev = _require_gpu(*tensors)
    for t, n in ((q, "q"), (y, "y (centroids)"), (score, "score"), (aggr, "aggr")):
        _req(t, torch.bfloat16, n)
    for t, n in ((dense_kv_indptr, "dense_kv_indptr"), (sparse_kv_indptr, "sparse_kv_indptr"),
                 (dense_kv_indices, "dense_kv_indices"), (sparse_kv_indices, "sparse_kv_indices")):
        _req(t, torch.int32, n)
    if q.dim() != 3:
        raise RuntimeError(f"vortex_torch: GQA indexer expects q [S, G, D], got {tuple(q.shape)}")
    S, G, D = (int(v) for v in q.shape)
    if int(y.shape[-1]) != D:
        raise RuntimeError(f"vortex_torch: GQA indexer head_dim mismatch ({D} vs {int(y.shape[-1])})")
    if score.numel() % G:
        raise RuntimeError(f"vortex_torch: GQA score buffer {tuple(score.shape)} is not [pages, 1, {G}]")
    eff = int(eff_batch_size)
    if dense_kv_indptr.numel() < eff + 1 or sparse_kv_indptr.numel() < eff + 1:
        raise RuntimeError(f"vortex_torch: indptr buffers need {eff + 1} entries")
    args = (q.data_ptr(), S * G, G, y.data_ptr(), y.numel() // D, D,
            score.data_ptr(), score.numel() // G, aggr.data_ptr(), aggr.numel(),
            dense_kv_indptr.data_ptr(), sparse_kv_indptr.data_ptr(),
            dense_kv_indices.data_ptr(), dense_kv_indices.numel(),
            sparse_kv_indices.data_ptr(), sparse_kv_indices.numel(),
            eff, int(topk_val), int(reserved_bos), int(reserved_eos), int(max_num_pages),
            0 if softmax_scale is None else 1, float(softmax_scale or 0.0))
    sched = _schedule_args(schedule)
    if cmean is not None:
        k, loc, heads = cmean
        _req(k, torch.bfloat16, "k_cache")
        _req(loc, torch.int64, "loc")
        if k.dim() != 3 or int(k.shape[2]) != D:
            raise RuntimeError(f"vortex_torch: CMean pool {tuple(k.shape)} does not match head_dim {D}")
        with _on_device(dev):
            rc = lib.vtx_indexer_gqa_fused_cmean(*args, k.data_ptr(), int(k.shape[0]), int(k.shape[1]), int(heads),
                                                 loc.data_ptr(), loc.numel(), *sched, _stream(dev))
        _check(rc, "indexer_gqa_fused_cmean")
        return
    with _on_device(dev):
        rc = lib.vtx_indexer_gqa_fused(*args, *sched, _stream(dev))
    _check(rc, "indexer_gqa_fused")


def indexer_quest_fused_supported(head_dim: int, group_size: int) -> bool:
    return bool(load_library().vtx_indexer_quest_fused_supported(int(head_dim), int(group_size)))


@_plain_args
def indexer_quest_fused(
    q: torch.Tensor,
    ymax: torch.Tensor,
    ymin: torch.Tensor,
    score: torch.Tensor,
    aggr: torch.Tensor,
    dense_kv_indptr: torch.Tensor,
    sparse_kv_indptr: torch.Tensor,
    dense_kv_indices: torch.Tensor,
    sparse_kv_indices: torch.Tensor,
    eff_batch_size: int,
    topk_val: int,
    reserved_bos: int,
    reserved_eos: int,
    max_num_pages: int,
    envelope=None,
    schedule=None,
) -> None:
    """Quest envelope scores + max over the query heads + topK of one layer
    in one launch.  envelope: (k_cache [rows, P, D] bf16, loc int64,
    num_kv_heads) — the layer's CMax into ymax and CMin into ymin, run first in
    the same launch (``vtx_indexer_quest_fused_cmean``).

    q: bf16 [S, G, D]; ymax, ymin: the envelope pools [rows, 1, D]; score:
    the Sum(dim=2) output buffer [pages, G, 1]; aggr: the Max(dim=1) output
    buffer [pages, 1, 1]; the block tables come from the planner.  schedule:
    the fused_schedule plan_decode wrote for this block table (workgroup
    order; speed only).
    """
    lib = load_library()
    tensors = [q, ymax, ymin, score, aggr, dense_kv_indptr, sparse_kv_indptr, dense_kv_indices,
               sparse_kv_indices]
    if schedule is not None:
        tensors.append(schedule)
    dev = _require_gpu(*tensors)
    for t, n in ((q, "q"), (ymax, "ymax"), (ymin, "ymin"), (score, "score"), (aggr, "aggr")):
        _req(t, torch.bfloat16, n)
    for t, n in ((dense_kv_indptr, "dense_kv_indptr"), (sparse_kv_indptr, "sparse_kv_indptr"),
                 (dense_kv_indices, "dense_kv_indices"), (sparse_kv_indices, "sparse_kv_indices")):
        _req(t, torch.int32, n)
    if q.dim() != 3:
        raise RuntimeError(f"vortex_torch: Quest indexer expects q [S, G, D], got {tuple(q.shape)}")
    S, G, D = (int(v) for v in q.shape)
    if int(ymax.shape[-1]) != D or tuple(ymax.shape) != tuple(ymin.shape):
        raise RuntimeError(f"vortex_torch: Quest envelope pools {tuple(ymax.shape)} / {tuple(ymin.shape)} "
                           f"do not match head_dim {D}")
    if score.numel() % G:
        raise RuntimeError(f"vortex_torch: Quest score buffer {tuple(score.shape)} is not [pages, {G}, 1]")
    eff = int(eff_batch_size)
    if dense_kv_indptr.numel() < eff + 1 or sparse_kv_indptr.numel() < eff + 1:
        raise RuntimeError(f"vortex_torch: indptr buffers need {eff + 1} entries")
    args = (q.data_ptr(), S * G, G, ymax.data_ptr(), ymin.data_ptr(), ymax.numel() // D, D,
            score.data_ptr(), score.numel() // G, aggr.data_ptr(), aggr.numel(),
            dense_kv_indptr.data_ptr(), sparse_kv_indptr.data_ptr(),
            dense_kv_indices.data_ptr(), dense_kv_indices.numel(),
            sparse_kv_indices.data_ptr(), sparse_kv_indices.numel(),
            eff, int(topk_val), int(reserved_bos), int(reserved_eos), int(max_num_pages))
    sched = _schedule_args(schedule)
    if envelope is not None:
        k, loc, heads = envelope
        _require_gpu(k, loc)
        _req(k, torch.bfloat16, "k_cache")
        _req(loc, torch.int64, "loc")
        if k.dim() != 3 or int(k.shape[2]) != D:
            raise RuntimeError(f"vortex_torch: envelope pool {tuple(k.shape)} does not match head_dim {D}")
        with _on_device(dev):
            rc = lib.vtx_indexer_quest_fused_cmean(*args, k.data_ptr(), int(k.shape[0]), int(k.shape[1]),
                                                   int(heads), loc.data_ptr(), loc.numel(), *sched, _stream(dev))
        _check(rc, "indexer_quest_fused_cmean")
        return
    with _on_device(dev):
        rc = lib.vtx_indexer_quest_fused(*args, *sched, _stream(dev))
    _check(rc, "indexer_quest_fused")


# ----------------------------------------------------------------------------
# workload-walking indexer ops (GQA / Quest flows)
# ----------------------------------------------------------------------------
def _tile(t: torch.Tensor, name: str):
    """(rows, d0, d1) of a rank-3 (or rank-2 as [rows, 1, d1]) bf16 tensor."""
    _req(t, torch.bfloat16, name)
    if t.dim() == 3:
        return int(t.shape[0]), int(t.shape[1]), int(t.shape[2])
    if t.dim() == 2:
        return int(t.shape[0]), 1, int(t.shape[1])
    raise RuntimeError(f"vortex_torch: {name} must be rank 3 [rows, d0, d1]")


def _walk_args(winfo, dense=None):
    """Device pointers and capacity of a workload list (q, off, len, num)."""
    wq, woff, wlen, wnum = winfo
    for t, n in ((woff, "winfo_kv_offsets"), (wlen, "winfo_kv_lens"), (wnum, "winfo_num_workloads")):
        _req(t, torch.int32, n)
    if wq is not None:
        _req(wq, torch.int32, "winfo_q_indices")
    if dense is not None:
        _req(dense, torch.int32, "dense_kv_indices")
    cap = min(woff.numel(), wlen.numel(), *( [wq.numel()] if wq is not None else []))
    return (wq.data_ptr() if wq is not None else None, woff.data_ptr(), wlen.data_ptr(), cap, wnum.data_ptr())


@_plain_args
def ragged_gemm(x, x_mode: int, y, y_mode: int, o, dense_kv_indices, winfo) -> None:
    """o[p, c, g] = sum_k x[rx, g, k] * y[ry, c, k] over the workload list
    winfo = (winfo_q_indices, winfo_kv_offsets, winfo_kv_lens, winfo_num_workloads)."""
    lib = load_library()
    dev = _require_gpu(x, y, o, dense_kv_indices, *[t for t in winfo if t is not None])
    xr, G, K = _tile(x, "x")
    yr, C, Ky = _tile(y, "y")
    orows, oc, og = _tile(o, "o")
    if K != Ky:
        raise RuntimeError(f"vortex_torch: GeMM inner dimension mismatch ({K} vs {Ky})")
    if oc * og != C * G:
        raise RuntimeError(f"vortex_torch: GeMM output tile must be [{C}, {G}], got [{oc}, {og}]")
    wq, woff, wlen, cap, wnum = _walk_args(winfo, dense_kv_indices)
    with _on_device(dev):
        rc = lib.vtx_ragged_gemm(x.data_ptr(), xr, int(x_mode), G, y.data_ptr(), yr, int(y_mode), C, K,
                                 o.data_ptr(), orows, dense_kv_indices.data_ptr(), dense_kv_indices.numel(),
                                 wq, woff, wlen, cap, wnum, _stream(dev))
    _check(rc, "ragged_gemm")


@_plain_args
def ragged_binary(op: int, alpha: float, beta: float, x, x_mode: int, y, y_mode: int, o,
                  dense_kv_indices, winfo) -> None:
    """o[p] = op(x[rx], y[ry]) with broadcasting over size-1 tile axes."""
    lib = load_library()
    dev = _require_gpu(x, y, o, dense_kv_indices, *[t for t in winfo if t is not None])
    xr, x0, x1 = _tile(x, "x")
    yr, y0, y1 = _tile(y, "y")
    orows, o0, o1 = _tile(o, "o")
    wq, woff, wlen, cap, wnum = _walk_args(winfo, dense_kv_indices)
    with _on_device(dev):
        rc = lib.vtx_ragged_binary(int(op), float(alpha), float(beta), x.data_ptr(), xr, int(x_mode), x0, x1,
                                   y.data_ptr(), yr, int(y_mode), y0, y1, o.data_ptr(), orows, o0, o1,
                                   dense_kv_indices.data_ptr(), dense_kv_indices.numel(), wq, woff, wlen, cap,
                                   wnum, _stream(dev))
    _check(rc, "ragged_binary")


@_plain_args
def ragged_unary(op: int, alpha: float, beta: float, x, o, winfo) -> None:
    lib = load_library()
    dev = _require_gpu(x, o, *[t for t in winfo if t is not None])
    xr, d0, d1 = _tile(x, "x")
    orows, o0, o1 = _tile(o, "o")
    if (o0, o1) != (d0, d1):
        raise RuntimeError("vortex_torch: elementwise output tile must equal the input tile")
    _, woff, wlen, cap, wnum = _walk_args((None,) + tuple(winfo[1:]))
    with _on_device(dev):
        rc = lib.vtx_ragged_unary(int(op), float(alpha), float(beta), x.data_ptr(), xr, d0, d1, o.data_ptr(), orows,
                                  woff, wlen, cap, wnum, _stream(dev))
    _check(rc, "ragged_unary")


@_plain_args
def ragged_reduce(x, o, dim: int, reduce_type: int, winfo) -> None:
    lib = load_library()
    dev = _require_gpu(x, o, *[t for t in winfo if t is not None])
    xr, d0, d1 = _tile(x, "x")
    _req(o, torch.bfloat16, "o")
    per = d1 if int(dim) == 1 else d0
    _, woff, wlen, cap, wnum = _walk_args((None,) + tuple(winfo[1:]))
    with _on_device(dev):
        rc = lib.vtx_ragged_reduce(x.data_ptr(), xr, d0, d1, o.data_ptr(), o.numel() // max(per, 1), int(dim),
                                   int(reduce_type), woff, wlen, cap, wnum, _stream(dev))
    _check(rc, "ragged_reduce")


@_plain_args
def segment_scan(op: int, scale: float, x, dense_kv_indptr, eff_batch_size: int, topk_val: int,
                 reserved_bos: int, reserved_eos: int) -> None:
    """In-place segment softmax (op SEGMENT_SOFTMAX) or L2 normalize over each
    segment's middle positions, per tile column."""
    lib = load_library()
    dev = _require_gpu(x, dense_kv_indptr)
    xr, d0, d1 = _tile(x, "x")
    _req(dense_kv_indptr, torch.int32, "dense_kv_indptr")
    eff = int(eff_batch_size)
    if dense_kv_indptr.numel() < eff + 1:
        raise RuntimeError(f"vortex_torch: dense_kv_indptr needs {eff + 1} entries")
    with _on_device(dev):
        rc = lib.vtx_segment_scan(int(op), float(scale), x.data_ptr(), xr, d0 * d1, dense_kv_indptr.data_ptr(), eff,
                                  int(topk_val), int(reserved_bos), int(reserved_eos), _stream(dev))
    _check(rc, "segment_scan")


@_plain_args
def set_kv_buffer(k_cache, v_cache, new_k, new_v, loc, page_size: int) -> None:
    """Writes new_k / new_v [nnz, H, D] into the paged pools at the token
    slots loc (int64 [nnz]); pools [pages * H, page_size, D] of the same dtype."""
    lib = load_library()
    dev = _require_gpu(k_cache, v_cache, new_k, new_v, loc)
    _req(loc, torch.int64, "loc")
    if new_k.dim() != 3 or new_v.shape != new_k.shape:
        raise RuntimeError("vortex_torch: new_k and new_v must both be [nnz, num_kv_heads, head_dim]")
    for t, n in ((k_cache, "k_cache"), (v_cache, "v_cache"), (new_k, "new_k"), (new_v, "new_v")):
        if t.dtype != new_k.dtype:
            raise RuntimeError(f"vortex_torch: {n} is {t.dtype}, the new tokens are {new_k.dtype}")
        if not t.is_contiguous():
            raise RuntimeError(f"vortex_torch: {n} must be contiguous")
    nnz, H, D = (int(s) for s in new_k.shape)
    if loc.numel() < nnz:
        raise RuntimeError("vortex_torch: loc shorter than the new tokens")
    if k_cache.shape != v_cache.shape or int(k_cache.shape[-1]) != D:
        raise RuntimeError("vortex_torch: k_cache and v_cache must be [pages * H, page_size, head_dim]")
    with _on_device(dev):
        rc = lib.vtx_set_kv_buffer(k_cache.data_ptr(), v_cache.data_ptr(), k_cache.numel() // D, new_k.data_ptr(),
                                   new_v.data_ptr(), loc.data_ptr(), nnz, H, D, new_k.element_size(),
                                   int(page_size), _stream(dev))
    _check(rc, "set_kv_buffer")


@_plain_args
def paged_decode_attention(q, o, k_cache, v_cache, kv_indptr, kv_indices, kv_last_page_len, batch_size: int,
                           num_kv_heads: int, sm_scale: float) -> None:
    """o[s*G + g] = softmax(sm_scale * q K^T) V over segment s's pages of the
    block table; q / o [B*H*G, D] (or [B, H*G, D]) bf16, pools [rows, P, D]."""
    lib = load_library()
    dev = _require_gpu(q, o, k_cache, v_cache, kv_indptr, kv_indices, kv_last_page_len)
    for t, n in ((q, "q"), (o, "o"), (k_cache, "k_cache"), (v_cache, "v_cache")):
        _req(t, torch.bfloat16, n)
    for t, n in ((kv_indptr, "kv_indptr"), (kv_indices, "kv_indices"), (kv_last_page_len, "kv_last_page_len")):
        _req(t, torch.int32, n)
    if k_cache.dim() != 3 or v_cache.shape != k_cache.shape:
        raise RuntimeError("vortex_torch: k_cache and v_cache must both be [pages * H, page_size, head_dim]")
    rows, P, D = (int(x) for x in k_cache.shape)
    B, H = int(batch_size), int(num_kv_heads)
    if q.numel() % max(B * H * D, 1) != 0 or o.numel() != q.numel():
        raise RuntimeError("vortex_torch: q and o must hold B * H * G rows of head_dim")
    G = q.numel() // max(B * H * D, 1)
    if kv_indptr.numel() < B * H + 1 or kv_last_page_len.numel() < B * H:
        raise RuntimeError(f"vortex_torch: kv_indptr needs {B * H + 1} and kv_last_page_len {B * H} entries")
    with _on_device(dev):
        rc = lib.vtx_paged_decode_attention(q.data_ptr(), o.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), rows,
                                            kv_indptr.data_ptr(), kv_indices.data_ptr(), kv_indices.numel(),
                                            kv_last_page_len.data_ptr(), B, H, G, D, P, float(sm_scale), _stream(dev))
    _check(rc, "paged_decode_attention")


def bf16_rounding_check(device="cuda") -> tuple:
    """(non-NaN mismatches, NaN mismatches) of the device's bf16 rounding
    against the integer round-to-nearest-even formulation, over all fp32
    inputs; both are 0 on a conforming device.  Synchronises (a test helper)."""
    lib = load_library()
    counts = torch.zeros(2, dtype=torch.int64, device=device)
    dev = _require_gpu(counts)
    with _on_device(dev):
        _check(lib.vtx_bf16_rounding_check(counts.data_ptr(), _stream(dev)), "bf16_rounding_check")
    c = counts.cpu()
    return int(c[0]), int(c[1])


def probe_read(src: torch.Tensor, sink: torch.Tensor, magic: int = 0x5a17c0de) -> None:
    """Sequential read of every byte of `src` (bandwidth probe; see
    include/vortex_hip.h); sink: int32 scratch, left as it was."""
    dev = _require_gpu(src, sink)
    lib = load_library()
    with _on_device(dev):
        rc = lib.vtx_probe_read(src.data_ptr(), src.numel() * src.element_size(), sink.data_ptr(), sink.numel(),
                                magic, _stream(dev))
    _check(rc, "probe_read")


def probe_gather(pool: torch.Tensor, rows: torch.Tensor, sink: torch.Tensor, indptr=None,
                 magic: int = 0x5a17c0de) -> None:
    """Reads the rows `rows` (int32) of `pool` ([R, ..] bf16, 256- or
    1152-byte rows) in the indexer's scoring passes (bandwidth probe); with
    `indptr` every workgroup first waits for one load of it."""
    dev = _require_gpu(pool, rows, sink)
    _req(rows, torch.int32, "rows")
    row_bytes = pool[0].numel() * pool.element_size()
    lib = load_library()
    with _on_device(dev):
        rc = lib.vtx_probe_gather(pool.data_ptr(), pool.shape[0], row_bytes, rows.data_ptr(), rows.numel(),
                                  indptr.data_ptr() if indptr is not None else None,
                                  (indptr.numel() - 1) if indptr is not None else 0, sink.data_ptr(), sink.numel(),
                                  magic, _stream(dev))
    _check(rc, "probe_gather")
