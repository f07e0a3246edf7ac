"""Indexer runtime context: the per-step block tables, the GeMV workload list
and the shape / top-k configuration the indexer ops read.

Field names, the sizing model of :meth:`Context.create` and the module-level
singleton follow the reference (vortex_torch/indexer/context.py:8-170), so a
serving runtime that populates the reference context populates this one.
"""
from __future__ import annotations

import os
from typing import Any

import torch

from ..abs import ContextBase
from ..utils import UNSET, Mode

_FIELDS = (
    # block tables (owned by the serving runtime)
    "dense_kv_indices", "sparse_kv_indices", "dense_kv_indptr", "sparse_kv_indptr",
    "kv_last_page_len", "batch_size",
    # GeMV workload list
    "winfo_q_indices", "winfo_kv_offsets", "winfo_kv_lens", "winfo_num_workloads",
    "winfo_chunk_size", "max_num_workloads",
    # chunking of long segments
    "max_chunk_size", "min_chunk_size",
    # heads / shapes
    "group_size", "num_kv_heads", "num_qo_heads", "head_dim",
    # device / paging capacity
    "num_sms", "page_size", "max_num_pages", "max_num_pages_per_request",
    # selection
    "indexer_dtype", "topk_val", "page_reserved_bos", "page_reserved_eos",
)


def _compute_units() -> int:
    if torch.cuda.is_available():
        return int(torch.cuda.get_device_properties(torch.cuda.current_device()).multi_processor_count)
    return os.cpu_count() or 1


class Context(ContextBase):
    """Mutable single-instance context, populated by :meth:`create`."""

    # _fused_schedule: int32 buffer the decode planner fills with the fused
    # indexer's workgroup order (speed only; not a reference field)
    __slots__ = ContextBase.__slots__ + _FIELDS + ("_aux_total_bytes", "_aux_total_flops", "_fused_schedule")

    def __init__(self) -> None:
        for n in self.__slots__:
            object.__setattr__(self, n, UNSET)
        self.name = "Indexer"
        self.mode = Mode.profile
        self._created = False
        self.batch_size = 0
        self._aux_total_bytes = 0
        self._aux_total_flops = 0
        self._fused_schedule = None

    def set_batch_size(self, n: int) -> None:
        self.batch_size = n

    def create(self, parent: Any, model_runner: Any, *, overwrite: bool = False) -> "Context":
        """Populates the context from the attention backend (`parent`) and the
        model runner.  Not thread-safe: call once, from one thread.

        Capacity model (reference vortex_torch/indexer/context.py:108-157):
        pages per request = ceil(max_seq_len / page_size), with max_seq_len
        = server_args.vortex_max_seq_lens, or the model context length when
        that is negative; max_num_pages = pages per request * max batch * H_kv;
        max_num_workloads = max_num_pages // min_chunk + max batch * H_kv.
        """
        if self._created and not overwrite:
            raise RuntimeError("Context.create() already called; pass overwrite=True to reinitialize.")
        sa = model_runner.server_args
        page = sa.page_size
        max_len = model_runner.model_config.context_len if sa.vortex_max_seq_lens < 0 else sa.vortex_max_seq_lens
        pages_per_req = (max_len + page - 1) // page
        max_bs = int(model_runner.req_to_token_pool.size)

        self.dense_kv_indices = parent.kv_indices_decode[0]
        self.sparse_kv_indices = parent.kv_indices_decode[1]
        self.dense_kv_indptr = parent.kv_indptr_decode[0]
        self.sparse_kv_indptr = parent.kv_indptr_decode[1]
        self.kv_last_page_len = parent.kv_last_page_len_decode

        self.max_chunk_size = sa.vortex_lb_max_chunk_size
        self.min_chunk_size = sa.vortex_lb_min_chunk_size

        self.group_size = parent.group_size
        self.num_kv_heads = parent.num_kv_heads
        self.num_qo_heads = parent.num_qo_heads
        self.head_dim = parent.head_dim

        self.num_sms = _compute_units()
        self.page_size = page
        self.max_num_pages = pages_per_req * max_bs * self.num_kv_heads
        self.max_num_pages_per_request = pages_per_req

        self.topk_val = sa.vortex_topk_val
        dt = getattr(sa, "vortex_indexer_dtype", "float32")
        self.indexer_dtype = getattr(torch, dt, torch.float32) if isinstance(dt, str) else dt
        self.page_reserved_bos = sa.vortex_page_reserved_bos
        self.page_reserved_eos = sa.vortex_page_reserved_eos

        self.max_num_workloads = self.max_num_pages // max(1, sa.vortex_lb_min_chunk_size) + max_bs * self.num_kv_heads
        device = getattr(model_runner, "device", "cpu")
        n = self.max_num_workloads
        self.winfo_q_indices = torch.zeros((n,), dtype=torch.int32, device=device)
        self.winfo_kv_offsets = torch.zeros((n,), dtype=torch.int32, device=device)
        self.winfo_kv_lens = torch.zeros((n,), dtype=torch.int32, device=device)
        self.winfo_num_workloads = torch.zeros((1,), dtype=torch.int32, device=device)
        self.winfo_chunk_size = torch.zeros((1,), dtype=torch.int32, device=device)
        self._fused_schedule = torch.zeros((4 + 4 * max_bs * self.num_kv_heads,), dtype=torch.int32, device=device)

        self._created = True
        return self


#: Process-wide indexer context (part of the public API).
ctx: Context = Context()


def get_ctx() -> Context:
    return ctx


__all__ = ["Context", "ctx", "get_ctx"]
