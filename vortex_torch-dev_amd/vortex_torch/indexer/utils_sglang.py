"""Serving-runtime helpers of the indexer.

``plan_decode`` is called once per decode step by the attention backend,
before any layer runs: it fills the context's block tables and workload list
(reference vortex_torch/indexer/utils_sglang.py:15-44); ``plan_decode_fa3``
does the same for the FA3 attention backend and also fills its padded page
tables (utils_sglang.py:135-168).  The prefill and transpose helpers of the
reference serve other attention paths; they exist here under the same names
and raise ``NotImplementedError``.
"""
from __future__ import annotations

import torch

from .. import _C, _hip
from .context import Context


def plan_decode(
    cached_seq_lens: torch.Tensor,
    req_to_token: torch.Tensor,
    req_indices: torch.Tensor,
    ctx: Context,
) -> None:
    """Reference: vortex_torch/indexer/utils_sglang.py:15-44.  The same
    launch also writes the context's fused-indexer schedule (the workgroup
    order that pairs long with short segments on each compute unit), which the
    fused indexer launches of this step read."""
    sched = getattr(ctx, "_fused_schedule", None)
    _hip.plan_decode(
        cached_seq_lens,
        ctx.dense_kv_indptr,
        ctx.dense_kv_indices,
        ctx.sparse_kv_indptr,
        ctx.sparse_kv_indices,
        ctx.kv_last_page_len,
        req_to_token,
        req_indices,
        ctx.winfo_q_indices,
        ctx.winfo_kv_offsets,
        ctx.winfo_kv_lens,
        ctx.winfo_num_workloads,
        ctx.winfo_chunk_size,
        ctx.page_size,
        ctx.num_kv_heads,
        ctx.topk_val,
        ctx.page_reserved_bos,
        ctx.page_reserved_eos,
        ctx.max_chunk_size,
        ctx.min_chunk_size,
        fused_schedule=sched if isinstance(sched, torch.Tensor) else None,
    )
    ctx.set_batch_size(cached_seq_lens.shape[0])


def plan_prefill(*args, **kwargs):
    return _C.sglang_plan_prefill(*args, **kwargs)


def plan_prefill_fa3(*args, **kwargs):
    return _C.sglang_plan_prefill_fa3(*args, **kwargs)


def plan_decode_fa3(
    cached_seq_lens: torch.Tensor,
    req_to_token: torch.Tensor,
    req_indices: torch.Tensor,
    dense_page_table: torch.Tensor,
    dense_cache_seqlens: torch.Tensor,
    sparse_page_table: torch.Tensor,
    sparse_cache_seqlens: torch.Tensor,
    ctx: Context,
) -> None:
    """FA3 decode planner (reference utils_sglang.py:135-168): ctx's block
    tables and workload list plus the caller's per-segment page tables and
    cache sequence lengths."""
    _C.sglang_plan_decode_fa3(
        cached_seq_lens,
        ctx.dense_kv_indptr,
        ctx.dense_kv_indices,
        ctx.sparse_kv_indptr,
        ctx.sparse_kv_indices,
        dense_page_table,
        dense_cache_seqlens,
        sparse_page_table,
        sparse_cache_seqlens,
        req_to_token,
        req_indices,
        ctx.winfo_q_indices,
        ctx.winfo_kv_offsets,
        ctx.winfo_kv_lens,
        ctx.winfo_num_workloads,
        ctx.winfo_chunk_size,
        ctx.page_size,
        ctx.num_kv_heads,
        ctx.topk_val,
        ctx.page_reserved_bos,
        ctx.page_reserved_eos,
        ctx.max_chunk_size,
        ctx.min_chunk_size,
    )
    ctx.set_batch_size(cached_seq_lens.shape[0])


def chunkwise_nh2hn_transpose(*args, **kwargs):
    return _C.Chunkwise_NH2HN_Transpose(*args, **kwargs)


def chunkwise_hn2nh_transpose(*args, **kwargs):
    return _C.Chunkwise_HN2NH_Transpose(*args, **kwargs)


def chunkwise_hn2nh_transpose_fa3(*args, **kwargs):
    return _C.Chunkwise_HN2NH_Transpose_FA3(*args, **kwargs)


def indices_to_page_table(page_table: torch.Tensor, ctx: Context) -> None:
    """No-op, as in the reference (utils_sglang.py:190-193)."""
    return None
