"""Registered flows.

``block_sparse_attention`` (reference vortex_torch/flow/algorithms.py:20-235):
the cache keeps one centroid (CMean of the page's keys) per (page, kv head);
the indexer averages the G query heads of each kv head, scores every page
centroid with GeMV and keeps the top-k pages besides the reserved BOS/EOS
pages.

Op instances own their output buffers, so every call site gets its own op.
"""
from __future__ import annotations

from typing import Dict

import torch

from ..abs import ContextBase
from ..cache import Mean as CMean
from ..indexer import GeMV, topK
from .flow import vFlow
from .registry import register


@register("block_sparse_attention")
class BlockSparseAttention(vFlow):
    """Centroid-routed block-sparse attention (block top-k routing in the
    style of Kinetics, arXiv:2506.05333)."""

    def __init__(self):
        super().__init__()
        self.gemv = GeMV()
        self.output_func = topK()
        self.reduction = CMean(dim=1)

    def forward_indexer(self, q: torch.Tensor, o: torch.Tensor, cache: Dict[str, torch.Tensor],
                        ctx: ContextBase):
        q_mean = q.mean(dim=1, keepdim=True)
        score = self.gemv(q_mean, cache["centroids"], ctx=ctx)
        self.output_func(score, o, ctx=ctx)

    def forward_cache(self, cache: Dict[str, torch.Tensor], loc: torch.Tensor, ctx: ContextBase):
        self.reduction(cache["k"], cache["centroids"], loc=loc, ctx=ctx)

    def create_cache(self, page_size: int, head_dim: int):
        return {"centroids": (1, head_dim)}
