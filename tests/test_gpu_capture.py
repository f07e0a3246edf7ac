"""Graph capture of a multi-layer decode step whose forward_cache leaves its
page-finish mean (or CMax + CMin) for the next forward_indexer.

For each of the three registered flows and both per-layer call orders
(cache then indexer, indexer then cache), a step of three layers is
captured with fusion on and replayed several times.  Before every replay the
K pools and the centroid / envelope pools are refilled with new values, so a
page-finish reduction missing from the graph (or one launched outside it)
leaves the old pool rows behind.  Each replay is checked bit for bit against
the same step run eagerly with every op launched on its own
(VORTEX_FUSE=0) from the same state: every layer's block table and every
pool.  In the indexer-then-cache order the last layer's reduction is still
carried when the capture ends, and it must land inside the graph.
"""
import pytest
import torch

import workloads as W
from vortex_torch import _deferred
from vortex_torch.abs import FORMAT, as_vtensor

pytestmark = pytest.mark.gpu

FLOWS = ["block_sparse_attention", "gqa_block_sparse_attention", "gqa_quest_sparse_attention"]
LAYERS = 3


def _batch(name):
    if name == "eos0":  # every request's last page closes and is scored (eos 0)
        return W.cmean_case("eos0")[0]
    # four query heads per kv head
    return W.make_batch([1024, 2048, 640, 4096, 512], pool_pages=900, seed=31, eos=0, topk=12, num_kv_heads=2,
                        group_size=4, head_dim=128, bos=1)


def _plain(t):
    with torch._C.DisableTorchFunctionSubclass():
        return torch.Tensor._make_subclass(torch.Tensor, t, require_grad=False)


class _Model:
    """LAYERS layers of one flow over a shared decode batch."""

    def __init__(self, flow_name, batch, dev):
        from vortex_torch import flow as vflow

        self.batch, self.dev = batch, dev
        H, G, D, P, B = batch.num_kv_heads, batch.group_size, batch.head_dim, batch.page_size, batch.batch
        self.ic, self.cc = W.make_contexts(batch, dev)
        self.dev_batch = batch.to(dev)
        self.loc = W.decode_loc(batch).to(dev)
        rows = batch.pool_pages * H
        self.flows, self.caches, self.qs = [], [], []
        for layer in range(LAYERS):
            f = vflow.build_vflow(flow_name)
            cache = {"k": as_vtensor(W.randn_bf16((rows, P, D), 10 * layer, dev), FORMAT.PAGED)}
            for j, (name, (r, c)) in enumerate(f.create_cache(P, D).items()):
                cache[name] = as_vtensor(W.randn_bf16((rows, r, c), 10 * layer + 1 + j, dev, std=0.25),
                                         FORMAT.PAGED)
            self.flows.append(f)
            self.caches.append(cache)
            self.qs.append(as_vtensor(W.randn_bf16((B * H, G, D), 10 * layer + 5, dev), FORMAT.BATCHED))
        self.o = as_vtensor(self.ic.sparse_kv_indices.view(-1, 1, 1), FORMAT.RAGGED)
        self.tables = [torch.empty_like(self.ic.sparse_kv_indices) for _ in range(LAYERS)]
        self.ic.profile()
        self.cc.profile()
        for f, cache, q in zip(self.flows, self.caches, self.qs):
            f.forward_cache(cache, self.loc, self.cc)
            f.forward_indexer(q, self.o, cache, self.ic)
        self.ic.execute()
        self.cc.execute()

    def step(self, order):
        from vortex_torch.indexer.utils_sglang import plan_decode

        b = self.dev_batch
        plan_decode(b.seq_lens, b.req_to_token, b.req_indices, self.ic)
        for layer, (f, cache, q) in enumerate(zip(self.flows, self.caches, self.qs)):
            if order == "cache_first":
                f.forward_cache(cache, self.loc, self.cc)
                f.forward_indexer(q, self.o, cache, self.ic)
            else:
                f.forward_indexer(q, self.o, cache, self.ic)
                f.forward_cache(cache, self.loc, self.cc)
            with torch._C.DisableTorchFunctionSubclass():
                self.tables[layer].copy_(self.ic.sparse_kv_indices)

    def pools(self):
        return [_plain(t) for cache in self.caches for t in cache.values()]

    def refill(self, seed):
        g = torch.Generator(device=self.dev).manual_seed(seed)
        for t in self.pools():
            t.copy_(torch.randn(t.shape, generator=g, device=self.dev, dtype=torch.float32).mul_(0.5))
        for t in self.tables + [self.ic.sparse_kv_indices]:
            t.fill_(-7)

    def snapshot(self):
        return [t.clone() for t in self.pools() + self.tables]


def _bits(t):
    return t.view(torch.int16) if t.dtype == torch.bfloat16 else t


@pytest.mark.parametrize("order", ["cache_first", "indexer_first"])
@pytest.mark.parametrize("flow_name", FLOWS)
@pytest.mark.parametrize("name", ["eos0", "g4"])
def test_captured_step_replays_equal_unfused_eager(gpu, monkeypatch, name, flow_name, order):
    monkeypatch.setenv("VORTEX_FUSE", "1")
    monkeypatch.delenv("VORTEX_FUSE_CMEAN", raising=False)
    model = _Model(flow_name, _batch(name), gpu)
    side = torch.cuda.Stream(gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(side):
        model.step(order)  # warm-up; in indexer_first order it ends with a carry pending
    torch.cuda.current_stream(gpu).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        model.step(order)
    assert _deferred.current_carry() is None, "a carry outlived the capture"
    torch.cuda.synchronize()
    closed = int(((model.loc + 1) % model.batch.page_size == 0).sum())
    assert closed > 0
    for rep in range(3):
        model.refill(100 + rep)
        before = model.snapshot()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = model.snapshot()
        assert any(not torch.equal(_bits(a), _bits(b)) for a, b in zip(got[:len(before) - LAYERS],
                                                                          before[:len(before) - LAYERS])), \
            "the replay changed no pool"
        # the same step from the same state, every op launched on its own
        for t, v in zip(model.pools() + model.tables, before):
            t.copy_(v)
        monkeypatch.setenv("VORTEX_FUSE", "0")
        model.step(order)
        torch.cuda.synchronize()
        monkeypatch.setenv("VORTEX_FUSE", "1")
        exp = model.snapshot()
        for i, (a, b) in enumerate(zip(got, exp)):
            assert torch.equal(_bits(a), _bits(b)), f"replay {rep}: tensor {i} differs from the unfused step"
