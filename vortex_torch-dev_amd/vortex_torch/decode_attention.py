"""Paged decode attention over the indexer's block tables.

The reference hands its sparse block table — ``sparse_kv_indptr``,
``sparse_kv_indices`` (entries ``page * H + h``) and ``kv_last_page_len``,
as written by the planner (csrc/utils_sglang.cu:123-184) and top-k
(csrc/topk.cu:56-113) — to FlashInfer's paged decode attention inside its
SGLang fork.  This module is that consumer on gfx950
(``vtx_paged_decode_attention``): one decode token per request, grouped
query heads, the last page of each segment partial.

``sparse_decode_attention`` reads the sparse table from an indexer context,
``dense_decode_attention`` the dense one (full attention over every page).
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from . import _hip


def paged_decode_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, kv_indptr: torch.Tensor,
                           kv_indices: torch.Tensor, kv_last_page_len: torch.Tensor, batch_size: int,
                           num_kv_heads: int, sm_scale: Optional[float] = None,
                           out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Attention of q ([B, H_q, D] or [B*H_kv, G, D], bf16) over the pages of
    each (request, kv head) segment of the table; returns [*q.shape] bf16."""
    D = int(q.shape[-1])
    scale = 1.0 / math.sqrt(D) if sm_scale is None else float(sm_scale)
    o = torch.empty_like(q) if out is None else out
    _hip.paged_decode_attention(q, o, k_cache, v_cache, kv_indptr, kv_indices, kv_last_page_len, batch_size,
                                num_kv_heads, scale)
    return o


def sparse_decode_attention(q, k_cache, v_cache, ctx, sm_scale: Optional[float] = None, out=None):
    """Attention over the pages the indexer selected (ctx's sparse table)."""
    return paged_decode_attention(q, k_cache, v_cache, ctx.sparse_kv_indptr, ctx.sparse_kv_indices,
                                  ctx.kv_last_page_len, ctx.batch_size, ctx.num_kv_heads, sm_scale, out)


def dense_decode_attention(q, k_cache, v_cache, ctx, sm_scale: Optional[float] = None, out=None):
    """Full attention over every page of each request (ctx's dense table)."""
    return paged_decode_attention(q, k_cache, v_cache, ctx.dense_kv_indptr, ctx.dense_kv_indices,
                                  ctx.kv_last_page_len, ctx.batch_size, ctx.num_kv_heads, sm_scale, out)


__all__ = ["paged_decode_attention", "sparse_decode_attention", "dense_decode_attention"]
