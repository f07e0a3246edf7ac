"""GPU tests of the fused indexer's workgroup schedule.

The decode planner can also write the order in which the fused indexer's
one-workgroup-per-segment launch takes the segments: sorted by page count
(fewer pages first, ties by request index, the H heads of a request
consecutive) and dealt in snake order over rounds of `round` workgroups
(vtx_fused_schedule.h).  The schedule only steers speed: with it the fused
kernel must give exactly the outputs it gives without it — also when the
schedule is stale (written for another block table with the same segment
count) or has no valid header.
"""
import numpy as np
import pytest
import torch

import workloads as W
from vortex_torch import _hip

pytestmark = pytest.mark.gpu

MAGIC = 0x56545853


def _np(t):
    return t.detach().cpu().numpy()


def _plan(batch, dev, schedule=None, schedule_round=0):
    ic, _ = W.make_contexts(batch, dev)
    b = batch.to(dev)
    _hip.plan_decode(b.seq_lens, ic.dense_kv_indptr, ic.dense_kv_indices, ic.sparse_kv_indptr,
                     ic.sparse_kv_indices, ic.kv_last_page_len, b.req_to_token, b.req_indices,
                     ic.winfo_q_indices, ic.winfo_kv_offsets, ic.winfo_kv_lens, ic.winfo_num_workloads,
                     ic.winfo_chunk_size, batch.page_size, batch.num_kv_heads, batch.topk, batch.bos,
                     batch.eos, batch.max_chunk, batch.min_chunk, fused_schedule=schedule,
                     schedule_round=schedule_round)
    return ic


def expected_schedule(batch, dense_indptr, sparse_indptr, rnd):
    """The documented rule, restated on the host."""
    B, H, P = batch.batch, batch.num_kv_heads, batch.page_size
    pages = [(int(L) + P - 1) // P for L in batch.seq_lens.tolist()]
    order = sorted(range(B), key=lambda r: (pages[r], r))
    S = B * H
    out = np.zeros((S, 4), dtype=np.int64)
    for i in range(S):
        seg = order[i // H] * H + i % H
        r = i // rnd
        slot = i if r % 2 == 0 else min(S, (r + 1) * rnd) - 1 - (i - r * rnd)
        out[slot] = (seg, dense_indptr[seg], dense_indptr[seg + 1], sparse_indptr[seg])
    return out


def _batches():
    return {"c1": W.c1, "c2": W.c2, "c3": W.c3, "c5": W.c5,
            "r0": lambda: W.random_small(0), "r3": lambda: W.random_small(3),
            "r5": lambda: W.random_small(5), "r9": lambda: W.random_small(9)}


@pytest.mark.parametrize("rnd", [0, 1, 7, 256])
@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c5", "r0", "r3", "r5", "r9"])
def test_planner_schedule_matches_rule(gpu, name, rnd):
    dev = gpu
    batch = _batches()[name]()
    S = batch.batch * batch.num_kv_heads
    sched = torch.full((4 + 4 * S + 8,), -3, dtype=torch.int32, device=dev)
    ic = _plan(batch, dev, sched, rnd)
    torch.cuda.synchronize()
    s = _np(sched)
    used_round = rnd if rnd else torch.cuda.get_device_properties(dev).multi_processor_count
    assert s[0] == MAGIC and s[1] == S and s[2] == used_round
    used_round = rnd if rnd else torch.cuda.get_device_properties(dev).multi_processor_count
    exp = expected_schedule(batch, _np(ic.dense_kv_indptr), _np(ic.sparse_kv_indptr), used_round)
    np.testing.assert_array_equal(s[4:4 + 4 * S].reshape(S, 4), exp)
    assert (s[4 + 4 * S:] == -3).all(), "planner wrote past the schedule"
    assert sorted(s[4:4 + 4 * S:4].tolist()) == list(range(S)), "not a permutation of the segments"


def test_planner_schedule_too_small_is_not_written(gpu):
    dev = gpu
    batch = W.c1()
    sched = torch.full((8,), -3, dtype=torch.int32, device=dev)
    _plan(batch, dev, sched)
    torch.cuda.synchronize()
    assert (_np(sched) == -3).all()


def _fused(batch, ic, dev, schedule, cmean=False, seed=1):
    H, G, D = batch.num_kv_heads, batch.group_size, batch.head_dim
    S = batch.batch * H
    q = W.randn_bf16((S, G, D), seed, dev)
    rows = batch.pool_pages * H
    y = W.randn_bf16((rows, 1, D), seed + 1, dev, std=0.25)
    qm = torch.zeros((S, 1, D), device=dev, dtype=torch.bfloat16)  # (not written when G > 2)
    sc = torch.full((ic.dense_kv_indices.numel(), 1, 1), -5.0, device=dev, dtype=torch.bfloat16)
    sp = ic.sparse_kv_indices.clone()
    cm = None
    if cmean:
        k = W.randn_bf16((rows, batch.page_size, D), seed + 2, dev)
        cm = (k, W.decode_loc(batch).to(dev), H)
    _hip.indexer_fused(q if G <= 2 else q.mean(dim=1, keepdim=True), qm if G <= 2 else None, y, sc,
                       ic.dense_kv_indptr, ic.sparse_kv_indptr, ic.dense_kv_indices, sp, S, batch.topk,
                       batch.bos, batch.eos, batch.max_pages_per_request, mode=_hip.FUSED_SEGMENT,
                       cmean=cm, schedule=schedule)
    torch.cuda.synchronize()
    return [qm, sc, sp, y]


def _equal(a, b):
    for x, y in zip(a, b):
        assert torch.equal(x.view(torch.int16) if x.dtype == torch.bfloat16 else x,
                           y.view(torch.int16) if y.dtype == torch.bfloat16 else y)


@pytest.mark.parametrize("cmean", [False, True])
@pytest.mark.parametrize("name", ["c1", "c2", "c5", "r3", "r5", "r9"])
def test_fused_with_schedule_equals_without(gpu, name, cmean):
    dev = gpu
    batch = _batches()[name]()
    if cmean and batch.head_dim not in (64, 128):
        pytest.skip("the in-launch CMean serves head_dim 64 / 128")
    S = batch.batch * batch.num_kv_heads
    sched = torch.zeros((4 + 4 * S,), dtype=torch.int32, device=dev)
    ic = _plan(batch, dev, sched, 7)
    _equal(_fused(batch, ic, dev, sched, cmean), _fused(batch, ic, dev, None, cmean))


@pytest.mark.parametrize("cmean", [False, True])
def test_fused_with_stale_schedule_is_still_exact(gpu, cmean):
    """A schedule written for another block table with the same segment
    count: every workgroup's predicted bounds are wrong, and the kernel must
    notice and use the block tables' own."""
    dev = gpu
    a, b = W.c2(seed=1), W.c2(seed=5)
    S = a.batch * a.num_kv_heads
    sched = torch.zeros((4 + 4 * S,), dtype=torch.int32, device=dev)
    _plan(a, dev, sched)            # schedule of layout a
    ic_b = _plan(b, dev, None)      # block tables of layout b, schedule untouched
    assert int(sched[0]) == MAGIC
    _equal(_fused(b, ic_b, dev, sched, cmean), _fused(b, ic_b, dev, None, cmean))


def test_fused_schedule_without_header_is_ignored(gpu):
    dev = gpu
    batch = W.c2()
    S = batch.batch * batch.num_kv_heads
    ic = _plan(batch, dev)
    junk = torch.randint(0, S, (4 + 4 * S,), dtype=torch.int32, generator=torch.Generator().manual_seed(3)).to(dev)
    junk[0] = 0  # no header
    _equal(_fused(batch, ic, dev, junk), _fused(batch, ic, dev, None))


def _gqa(batch, ic, dev, schedule, cmean=False, softmax=True, seed=1):
    """The fused GQA indexer step (GeMM, softmax, max, topK) on one layer."""
    H, G, D = batch.num_kv_heads, batch.group_size, batch.head_dim
    S = batch.batch * H
    q = W.randn_bf16((S, G, D), seed, dev)
    rows = batch.pool_pages * H
    y = W.randn_bf16((rows, 1, D), seed + 1, dev, std=0.25)
    pages = ic.dense_kv_indices.numel()
    sc = torch.full((pages, 1, G), -5.0, device=dev, dtype=torch.bfloat16)
    ag = torch.full((pages, 1, 1), -5.0, device=dev, dtype=torch.bfloat16)
    sp = ic.sparse_kv_indices.clone()
    cm = None
    if cmean:
        k = W.randn_bf16((rows, batch.page_size, D), seed + 2, dev)
        cm = (k, W.decode_loc(batch).to(dev), H)
    _hip.indexer_gqa_fused(q, y, sc, ag, ic.dense_kv_indptr, ic.sparse_kv_indptr, ic.dense_kv_indices, sp, S,
                           batch.topk, batch.bos, batch.eos, batch.max_pages_per_request,
                           softmax_scale=D ** -0.5 if softmax else None, cmean=cm, schedule=schedule)
    torch.cuda.synchronize()
    return [sc, ag, sp, y]


def _gqa_batch(name):
    batch = _batches()[name]()
    if not _hip.indexer_gqa_fused_supported(batch.head_dim, batch.group_size):
        pytest.skip(f"the fused GQA kernel does not serve D {batch.head_dim}, G {batch.group_size}")
    return batch


@pytest.mark.parametrize("softmax", [False, True])
@pytest.mark.parametrize("cmean", [False, True])
@pytest.mark.parametrize("name", ["c1", "c2", "r3", "r5", "r9"])
def test_gqa_fused_with_schedule_equals_without(gpu, name, cmean, softmax):
    dev = gpu
    batch = _gqa_batch(name)
    if cmean and batch.head_dim not in (64, 128):
        pytest.skip("the in-launch CMean serves head_dim 64 / 128")
    S = batch.batch * batch.num_kv_heads
    sched = torch.zeros((4 + 4 * S,), dtype=torch.int32, device=dev)
    ic = _plan(batch, dev, sched, 7)
    _equal(_gqa(batch, ic, dev, sched, cmean, softmax), _gqa(batch, ic, dev, None, cmean, softmax))


@pytest.mark.parametrize("cmean", [False, True])
def test_gqa_fused_with_stale_schedule_is_still_exact(gpu, cmean):
    dev = gpu
    a, b = W.c2(seed=1), W.c2(seed=5)
    S = a.batch * a.num_kv_heads
    sched = torch.zeros((4 + 4 * S,), dtype=torch.int32, device=dev)
    _plan(a, dev, sched)
    ic_b = _plan(b, dev, None)
    assert int(sched[0]) == MAGIC
    _equal(_gqa(b, ic_b, dev, sched, cmean), _gqa(b, ic_b, dev, None, cmean))


def test_gqa_fused_schedule_without_header_is_ignored(gpu):
    dev = gpu
    batch = W.c2()
    S = batch.batch * batch.num_kv_heads
    ic = _plan(batch, dev)
    junk = torch.randint(0, S, (4 + 4 * S,), dtype=torch.int32, generator=torch.Generator().manual_seed(3)).to(dev)
    junk[0] = 0
    _equal(_gqa(batch, ic, dev, junk), _gqa(batch, ic, dev, None))


def _quest(batch, ic, dev, schedule, envelope=False, seed=1):
    """The fused Quest indexer step (envelope scores, max, topK) on one layer."""
    H, G, D = batch.num_kv_heads, batch.group_size, batch.head_dim
    S = batch.batch * H
    q = W.randn_bf16((S, G, D), seed, dev)
    rows = batch.pool_pages * H
    ymax = W.randn_bf16((rows, 1, D), seed + 1, dev, std=0.25)
    ymin = W.randn_bf16((rows, 1, D), seed + 3, dev, std=0.25)
    pages = ic.dense_kv_indices.numel()
    sm = torch.full((pages, G, 1), -5.0, device=dev, dtype=torch.bfloat16)
    ag = torch.full((pages, 1, 1), -5.0, device=dev, dtype=torch.bfloat16)
    sp = ic.sparse_kv_indices.clone()
    env = None
    if envelope:
        k = W.randn_bf16((rows, batch.page_size, D), seed + 2, dev)
        env = (k, W.decode_loc(batch).to(dev), H)
    _hip.indexer_quest_fused(q, ymax, ymin, sm, ag, ic.dense_kv_indptr, ic.sparse_kv_indptr, ic.dense_kv_indices,
                             sp, S, batch.topk, batch.bos, batch.eos, batch.max_pages_per_request, envelope=env,
                             schedule=schedule)
    torch.cuda.synchronize()
    return [sm, ag, sp, ymax, ymin]


def _quest_batch(name):
    batch = _batches()[name]()
    if not _hip.indexer_quest_fused_supported(batch.head_dim, batch.group_size):
        pytest.skip(f"the fused Quest kernel does not serve D {batch.head_dim}, G {batch.group_size}")
    return batch


@pytest.mark.parametrize("envelope", [False, True])
@pytest.mark.parametrize("name", ["c1", "c2", "r3", "r5", "r9"])
def test_quest_fused_with_schedule_equals_without(gpu, name, envelope):
    dev = gpu
    batch = _quest_batch(name)
    if envelope and batch.head_dim not in (64, 128):
        pytest.skip("the in-launch page reduce serves head_dim 64 / 128")
    S = batch.batch * batch.num_kv_heads
    sched = torch.zeros((4 + 4 * S,), dtype=torch.int32, device=dev)
    ic = _plan(batch, dev, sched, 7)
    _equal(_quest(batch, ic, dev, sched, envelope), _quest(batch, ic, dev, None, envelope))


@pytest.mark.parametrize("envelope", [False, True])
def test_quest_fused_with_stale_schedule_is_still_exact(gpu, envelope):
    dev = gpu
    a, b = W.c2(seed=1), W.c2(seed=5)
    S = a.batch * a.num_kv_heads
    sched = torch.zeros((4 + 4 * S,), dtype=torch.int32, device=dev)
    _plan(a, dev, sched)
    ic_b = _plan(b, dev, None)
    assert int(sched[0]) == MAGIC
    _equal(_quest(b, ic_b, dev, sched, envelope), _quest(b, ic_b, dev, None, envelope))
