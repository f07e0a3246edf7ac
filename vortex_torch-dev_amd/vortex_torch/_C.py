"""Native entry points under the reference extension's names and signatures.

The reference binds these from its CUDA extension ``vortex_torch_C``
(csrc/register.cc:5-13); here they are thin wrappers over the gfx950 C ABI
(``include/vortex_hip.h``).  Arguments, argument order and in-place semantics
are unchanged, so a serving runtime written against the reference calls them
as before.  The top-level module ``vortex_torch_C`` re-exports this module.
"""
from __future__ import annotations

import torch

from . import _hip


def topk_output(
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
    """Writes each segment's top-k pages into ``sparse_kv_indices`` in place.

    Reference: csrc/topk.cu:117-203 (argument order of topk.cu:117-128).  The
    reference rejects ``max_num_pages > 4096``; this implementation has no
    page cap (``topk_val`` up to 4096).
    """
    _hip.topk_select(x, dense_kv_indptr, sparse_kv_indptr, dense_kv_indices, sparse_kv_indices,
                     eff_batch_size, topk_val, reserved_bos, reserved_eos, max_num_pages)


def sglang_plan_decode(
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
) -> None:
    """Builds the decode block tables and GeMV workload list in place.

    Reference: csrc/utils_sglang.cu:313-460.  One launch instead of three;
    no batch-size limit (the reference scans at most 1024 requests and
    8192 segments).
    """
    _hip.plan_decode(cached_seq_lens, dense_kv_indptr, dense_kv_indices, sparse_kv_indptr,
                     sparse_kv_indices, kv_last_page_len, req_to_token, req_indices,
                     winfo_q_indices, winfo_kv_offsets, winfo_kv_lens, winfo_num_workloads,
                     winfo_chunk_size, page_size, num_kv_heads, topk_val, page_reserved_bos,
                     page_reserved_eos, max_chunk_size, min_chunk_size)


def sglang_plan_decode_fa3(
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
    """FA3 decode planner: block tables, workload list, per-segment padded
    page tables and cache sequence lengths, in place.

    Reference: csrc/utils_sglang.cu:1085-1239 (argument order), kernels
    950-1082.  One launch instead of three; no batch-size limit.
    """
    _hip.plan_decode_fa3(cached_seq_lens, dense_kv_indptr, dense_kv_indices, sparse_kv_indptr,
                         sparse_kv_indices, dense_page_table, dense_cache_seqlens, sparse_page_table,
                         sparse_cache_seqlens, req_to_token, req_indices, winfo_q_indices, winfo_kv_offsets,
                         winfo_kv_lens, winfo_num_workloads, winfo_chunk_size, page_size, num_kv_heads,
                         topk_val, page_reserved_bos, page_reserved_eos, max_chunk_size, min_chunk_size)


def _out_of_scope(name: str):
    def fn(*args, **kwargs):
        raise NotImplementedError(
            f"{name} belongs to the prefill paths, which this MI355X build of the "
            "decode indexer does not implement")
    fn.__name__ = name
    return fn


sglang_plan_prefill = _out_of_scope("sglang_plan_prefill")
sglang_plan_prefill_fa3 = _out_of_scope("sglang_plan_prefill_fa3")
Chunkwise_NH2HN_Transpose = _out_of_scope("Chunkwise_NH2HN_Transpose")
Chunkwise_HN2NH_Transpose = _out_of_scope("Chunkwise_HN2NH_Transpose")
Chunkwise_HN2NH_Transpose_FA3 = _out_of_scope("Chunkwise_HN2NH_Transpose_FA3")
