"""GPU test of vtx_indexer_fused_noalloc, the entry point that allocates
nothing: the split layout's workspace (per-segment arrival counters and the
staging zone of its pre-selection) lives in a device array of the library
instead of a caller workspace.

Through the C-ABI (ctypes), calls in a row — a layout of 64 segments split
over many workgroups, then a smaller one, then MLA rows (whose selecting
workgroups read the staged lists as they arrive) — each compared bit for
bit with vtx_indexer_fused given zeroed counters only (so also the staged
pre-selection against the unstaged path): q-mean, scores and block table.
A last call repeats the first layout, which only gives the same result if
the earlier calls left every counter and staged list place at zero.
"""
import numpy as np
import pytest
import torch

import workloads as W
from vortex_torch import _hip

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.detach().view(torch.int16).cpu().numpy() if t.dtype == torch.bfloat16 else t.detach().cpu().numpy()


def _case(batch, dev, seed):
    from vortex_torch.indexer.utils_sglang import plan_decode

    ic, _ = W.make_contexts(batch, dev)
    b = batch.to(dev)
    plan_decode(b.seq_lens, b.req_to_token, b.req_indices, ic)
    H, G, D = batch.num_kv_heads, batch.group_size, batch.head_dim
    S = batch.batch * H
    q = W.randn_bf16((S, G, D), seed, dev)
    y = W.randn_bf16((batch.pool_pages * H, 1, D), seed + 1, dev, std=0.25)
    return ic, q, y, S


def _run(batch, ic, q, y, S, mode, noalloc):
    dev = q.device
    D = batch.head_dim
    qm = torch.full((S, 1, D), 3.0, device=dev, dtype=torch.bfloat16)
    sc = torch.full((ic.dense_kv_indices.numel(), 1, 1), -5.0, device=dev, dtype=torch.bfloat16)
    sp = ic.sparse_kv_indices.clone()
    counters = None if noalloc else torch.zeros(S, dtype=torch.int32, device=dev)
    _hip.indexer_fused(q, qm, y, sc, ic.dense_kv_indptr, ic.sparse_kv_indptr, ic.dense_kv_indices, sp, S,
                       batch.topk, batch.bos, batch.eos, batch.max_pages_per_request, seg_counters=counters,
                       mode=mode, noalloc=noalloc)
    torch.cuda.synchronize()
    return [_bits(qm), _bits(sc), _bits(sp)]


@pytest.mark.parametrize("mode", [_hip.FUSED_SPLIT, _hip.FUSED_AUTO])
def test_noalloc_entry_point_equals_workspace_entry_point(gpu, mode):
    first = (W.c3(), 1)
    second = (W.make_batch([3000, 9000, 700], pool_pages=900, seed=51, num_kv_heads=2, group_size=2,
                           head_dim=128, topk=20, bos=1, eos=1), 2)
    wide = (W.make_batch([5000, 7000, 9000], pool_pages=2000, seed=53, num_kv_heads=1, group_size=16,
                         head_dim=576, topk=32, bos=1, eos=1), 3)
    for batch, seed in (first, second, wide, first):
        ic, q, y, S = _case(batch, gpu, seed)
        got = _run(batch, ic, q, y, S, mode, noalloc=True)
        exp = _run(batch, ic, q, y, S, mode, noalloc=False)
        for a, b in zip(got, exp):
            np.testing.assert_array_equal(a, b)


def test_noalloc_reset_then_calls_equal_workspace_entry_point(gpu):
    """vtx_indexer_fused_noalloc_reset clears the library's counters; calls
    after it (a larger batch after a smaller one) still equal the workspace
    entry point bit for bit."""
    _hip.indexer_fused_noalloc_reset(gpu)
    small = (W.make_batch([3000, 9000, 700], pool_pages=900, seed=51, num_kv_heads=2, group_size=2,
                          head_dim=128, topk=20, bos=1, eos=1), 2)
    for batch, seed in (small, (W.c3(), 1)):
        ic, q, y, S = _case(batch, gpu, seed)
        got = _run(batch, ic, q, y, S, _hip.FUSED_SPLIT, noalloc=True)
        exp = _run(batch, ic, q, y, S, _hip.FUSED_SPLIT, noalloc=False)
        for a, b in zip(got, exp):
            np.testing.assert_array_equal(a, b)


def test_noalloc_entry_point_rejects_too_many_segments(gpu):
    lib = _hip.load_library()
    rc = lib.vtx_indexer_fused_noalloc(None, 70000, 1, None, None, None, 1, None, 0, None, None, None, 0, None, 0,
                                       70000, 8, 1, 1, 64, 128, _hip.FUSED_SPLIT, None, 0, None)
    assert rc == -1
    assert b"65536" in lib.vtx_last_error()
