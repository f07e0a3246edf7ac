"""The decode planner's int16 rule on the GPU.

The reference planner keeps a segment's middle-page count in an int16
(csrc/utils_sglang.cu:221-225): a segment with 32,768 or more middle pages
wraps to a negative count and gets no GeMV workload.  With page size 1 a
request of 32,772 tokens has 32,770 middle pages (bos 1, eos 1).

* vtx_plan_decode must write the oracle's tables bit for bit for such a
  batch, including the missing workloads of the long request's segments.
* A flow step on that batch must not take the fused indexer (its scoring
  would cover the pages the reference leaves unscored) and must write the
  same block table and scores as the step with every op launched on its own.
"""
import numpy as np
import pytest
import torch

import workloads as W
from oracle import vortex_oracle as O
from test_gpu_parity import assert_plan_equal, plan_on_gpu, plan_oracle
from vortex_torch import _hip
from vortex_torch.abs import FORMAT, as_vtensor

pytestmark = pytest.mark.gpu


def _batch():
    return W.make_batch([32772, 100, 5000], pool_pages=38000, seed=61, page_size=1, num_kv_heads=2, group_size=2,
                        head_dim=128, topk=30, bos=1, eos=1)


def test_planner_int16_rule_on_gpu(gpu):
    batch = _batch()
    ref = plan_oracle(batch)
    # the long request's segments (request 0, heads 0 and 1) wrap and get no workload
    long_segs = [s for s in range(batch.batch * batch.num_kv_heads)
                 if int(ref["dense_indptr"][s + 1] - ref["dense_indptr"][s]) - batch.bos - batch.eos >= 32768]
    assert len(long_segs) == batch.num_kv_heads
    assert not set(long_segs) & set(ref["winfo_q"].tolist())
    g = plan_on_gpu(batch, gpu)
    assert_plan_equal(g, ref)


def test_flow_with_a_wrapped_segment_runs_unfused(gpu, monkeypatch):
    from vortex_torch import flow as vflow
    from vortex_torch.indexer.utils_sglang import plan_decode

    batch = _batch()
    H, G, D, P = batch.num_kv_heads, batch.group_size, batch.head_dim, batch.page_size
    calls = {"fused": 0, "gemv": 0}
    real_fused, real_gemv = _hip.indexer_fused, _hip.gemv_paged

    def fused(*a, **k):
        calls["fused"] += 1
        return real_fused(*a, **k)

    def gemv(*a, **k):
        calls["gemv"] += 1
        return real_gemv(*a, **k)

    monkeypatch.setattr(_hip, "indexer_fused", fused)
    monkeypatch.setattr(_hip, "gemv_paged", gemv)
    out = {}
    for fuse in ("1", "0"):
        monkeypatch.setenv("VORTEX_FUSE", fuse)
        ic, cc = W.make_contexts(batch, gpu)
        f = vflow.build_vflow("block_sparse_attention")
        rows = batch.pool_pages * H
        cache = {"k": as_vtensor(W.randn_bf16((rows, P, D), 1, gpu), FORMAT.PAGED),
                 "centroids": as_vtensor(W.randn_bf16((rows, 1, D), 2, gpu, std=0.25), FORMAT.PAGED)}
        q = as_vtensor(W.randn_bf16((batch.batch * H, G, D), 3, gpu), FORMAT.BATCHED)
        o = as_vtensor(ic.sparse_kv_indices.view(-1, 1, 1), FORMAT.RAGGED)
        loc = W.decode_loc(batch).to(gpu)
        ic.profile()
        cc.profile()
        f.forward_cache(cache, loc, cc)
        f.forward_indexer(q, o, cache, ic)
        ic.execute()
        cc.execute()
        b = batch.to(gpu)
        plan_decode(b.seq_lens, b.req_to_token, b.req_indices, ic)
        with torch._C.DisableTorchFunctionSubclass():
            f.gemv.output_buffer.fill_(0.25)  # the scores the wrapped segments keep
        calls["fused"] = calls["gemv"] = 0
        f.forward_cache(cache, loc, cc)
        f.forward_indexer(q, o, cache, ic)
        torch.cuda.synchronize()
        assert calls["fused"] == 0 and calls["gemv"] == 1, f"VORTEX_FUSE={fuse}: {calls}"
        with torch._C.DisableTorchFunctionSubclass():
            out[fuse] = (ic.sparse_kv_indices.cpu().numpy(),
                         f.gemv.output_buffer.view(torch.int16).cpu().numpy(),
                         cache["centroids"].view(torch.int16).cpu().numpy())
        # the selection is the oracle's top-k of the step's own scores
        ref = plan_oracle(batch)
        sel, _ = O.topk(out[fuse][1].reshape(-1).view(np.uint16), ref["dense_indptr"], ref["sparse_indptr"],
                        ref["dense_indices"], ref["sparse_indices"], batch.batch * H, batch.topk, batch.bos,
                        batch.eos)
        np.testing.assert_array_equal(out[fuse][0][:sel.shape[0]], sel)
    for a, b in zip(out["1"], out["0"]):
        np.testing.assert_array_equal(a, b)
