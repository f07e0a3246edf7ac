"""Writes new keys and values into the paged K / V pools.

``set_kv_buffer_launcher`` keeps the reference's name and arguments
(vortex_torch/cache/triton_kernels/set_kv.py:45-63): token i's row for kv
head h goes to pool row ``(loc[i] // P) * (P * H) + h * P + loc[i] % P`` of
``k_cache`` / ``v_cache`` ([pages * H, P, D]), the layout the page-finish
reductions and the indexer read.  Kernel: ``vtx_set_kv_buffer``.
"""
from __future__ import annotations

import torch

from .. import _hip


def set_kv_buffer_launcher(k_cache: torch.Tensor, v_cache: torch.Tensor, new_k: torch.Tensor,
                           new_v: torch.Tensor, loc: torch.Tensor, page_size: int) -> None:
    _hip.set_kv_buffer(k_cache, v_cache, new_k, new_v, loc, page_size)


__all__ = ["set_kv_buffer_launcher"]
