"""Drop-in for the reference's native extension module ``vortex_torch_C``.

Code written against the reference (``from vortex_torch_C import
topk_output, sglang_plan_decode``) gets the gfx950 implementations.
"""
from vortex_torch._C import (  # noqa: F401
    Chunkwise_HN2NH_Transpose,
    Chunkwise_HN2NH_Transpose_FA3,
    Chunkwise_NH2HN_Transpose,
    sglang_plan_decode,
    sglang_plan_decode_fa3,
    sglang_plan_prefill,
    sglang_plan_prefill_fa3,
    topk_output,
)
