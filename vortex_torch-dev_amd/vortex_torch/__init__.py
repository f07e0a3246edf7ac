"""vortex_torch for MI355X (gfx950).

Same import surface as the reference package for the sparse-attention
indexer + cache path: ``vortex_torch.flow`` (vFlow, register, build_vflow,
algorithms), ``vortex_torch.indexer`` (GeMV, topK, Context, utils_sglang),
``vortex_torch.cache`` (Mean, Max, Min, L2Norm, Context), ``vortex_torch.abs``.
The numeric work runs in hand-written HIP kernels (``_lib/libvortex_hip.so``).
``set_fusion`` switches the fused launches (beside VORTEX_FUSE and
VORTEX_FUSE_CMEAN).
"""
from . import abs as abs
from . import cache as cache
from ._deferred import set_fusion
from . import flow as flow
from . import indexer as indexer
from .version import __version__

__all__ = ["indexer", "cache", "flow", "abs", "set_fusion", "__version__"]
