"""Registered flows.

``block_sparse_attention`` (reference vortex_torch/flow/algorithms.py:20-235):
the cache keeps one centroid (CMean of the page's keys) per (page, kv head);
the indexer averages the G query heads of each kv head, scores every page
centroid with GeMV and keeps the top-k pages besides the reserved BOS/EOS
pages.

``gqa_block_sparse_attention`` (reference algorithms.py:238-352): every query
head scores every centroid (GeMM), the scores are softmax-normalised over
each segment's pages per query head (scale 0.09), the per-page maximum over
the query heads is the page score for topK.

``gqa_quest_sparse_attention`` (reference algorithms.py:356-496): the cache
keeps per-page key envelopes (CMax, CMin); a page scores
max_g sum_d max(q_gd * max_d, q_gd * min_d), an upper bound of q . k over
the page's keys (Quest, arXiv:2406.10774).

Op instances own their output buffers, so every call site gets its own op.
"""
from __future__ import annotations

from typing import Dict

import torch

from ..abs import ContextBase
from ..cache import Max as CMax
from ..cache import Mean as CMean
from ..cache import Min as CMin
from ..indexer import GeMM, GeMV, Max, Maximum, Multiply, Softmax, Sum, topK
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


@register("gqa_block_sparse_attention")
class GQABlockSparseAttention(vFlow):
    """Grouped-query block-sparse routing (in the spirit of arXiv:2502.11089)."""

    def __init__(self):
        super().__init__()
        self.gemm = GeMM()
        self.softmax = Softmax(dim=0, scale=0.09)
        self.max_op = Max(dim=2)
        self.output_func = topK()
        self.reduction = CMean(dim=1)

    def forward_indexer(self, q: torch.Tensor, o: torch.Tensor, cache: Dict[str, torch.Tensor],
                        ctx: ContextBase):
        score = self.gemm(q, cache["centroids"], ctx=ctx)
        self.softmax(score, ctx=ctx)
        aggr_score = self.max_op(score, ctx=ctx)
        self.output_func(aggr_score, o, ctx=ctx)

    def forward_cache(self, cache: Dict[str, torch.Tensor], loc: torch.Tensor, ctx: ContextBase):
        self.reduction(cache["k"], cache["centroids"], loc=loc, ctx=ctx)

    def create_cache(self, page_size: int, head_dim: int):
        return {"centroids": (1, head_dim)}


@register("gqa_quest_sparse_attention")
class GQAQuestSparseAttention(vFlow):
    """Query-envelope matching over per-page key maxima and minima."""

    def __init__(self):
        super().__init__()
        self.mul_max = Multiply()
        self.mul_min = Multiply()
        self.maximum_op = Maximum()
        self.sum = Sum(dim=2)
        self.max_op = Max(dim=1)
        self.output_func = topK()
        self.reduction_max = CMax(dim=1)
        self.reduction_min = CMin(dim=1)

    def forward_indexer(self, q: torch.Tensor, o: torch.Tensor, cache: Dict[str, torch.Tensor],
                        ctx: ContextBase):
        s_max = self.mul_max(q, cache["max"], ctx=ctx)
        s_min = self.mul_min(q, cache["min"], ctx=ctx)
        s = self.maximum_op(s_max, s_min, ctx=ctx)
        score = self.sum(s, ctx=ctx)
        aggr_score = self.max_op(score, ctx=ctx)
        self.output_func(aggr_score, o, ctx=ctx)

    def forward_cache(self, cache: Dict[str, torch.Tensor], loc: torch.Tensor, ctx: ContextBase):
        self.reduction_max(cache["k"], cache["max"], loc=loc, ctx=ctx)
        self.reduction_min(cache["k"], cache["min"], loc=loc, ctx=ctx)

    def create_cache(self, page_size: int, head_dim: int):
        return {"max": (1, head_dim), "min": (1, head_dim)}
