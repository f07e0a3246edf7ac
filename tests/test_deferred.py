"""Host logic of the fused Quest chain (no GPU needed): which launches the
deferral scope issues for the Quest flow, with the kernels replaced by
recorders.  The GPU tests check the numbers; these check the bookkeeping —
one fused launch when the intermediates are not read, the intermediates
computed when something still refers to them, and every op launched on its
own under VORTEX_FUSE=0."""
import pytest
import torch

import workloads as W
from vortex_torch import _deferred, _hip
from vortex_torch.abs import FORMAT, as_vtensor
from vortex_torch.flow import algorithms, build_vflow, registry
from vortex_torch.cache import reduce as CR
from vortex_torch.indexer import elementwise_binary as EB


@pytest.fixture
def launches(monkeypatch):
    log = []

    def rec(name):
        return lambda *a, **k: log.append(name)

    monkeypatch.setattr(EB, "_quest_operands", lambda x, y, ctx: True)  # CPU tensors stand in
    monkeypatch.setattr(CR, "_recordable_operands", lambda x, out, loc: True)
    monkeypatch.setattr(_hip, "ragged_binary", rec("binary"))
    monkeypatch.setattr(_hip, "ragged_reduce", rec("reduce"))
    monkeypatch.setattr(_hip, "indexer_quest_fused",
                        lambda *a, **k: log.append("fused" + ("+envelope" if k.get("envelope") else "")))
    monkeypatch.setattr(_hip, "topk_select", rec("topk"))
    monkeypatch.setattr(_hip, "page_reduce", rec("page_reduce"))
    monkeypatch.setattr(_hip, "page_reduce_multi", lambda x, outs, *a, **k: log.append(f"page_reduce_multi{len(outs)}"))
    yield log
    _deferred._tls.carry = None


def _run(flow_name, cache_step=False, indexer=True):
    batch = W.c1()
    ic, cc = W.make_contexts(batch, "cpu")
    flow = build_vflow(flow_name)
    H, G, D, P = batch.num_kv_heads, batch.group_size, batch.head_dim, batch.page_size
    rows = batch.pool_pages * H
    cache = {"k": as_vtensor(torch.zeros((rows, P, D), dtype=torch.bfloat16), FORMAT.PAGED)}
    for name, (r, c) in flow.create_cache(P, D).items():
        cache[name] = as_vtensor(torch.zeros((rows, r, c), dtype=torch.bfloat16), FORMAT.PAGED)
    q = as_vtensor(torch.zeros((batch.batch * H, G, D), dtype=torch.bfloat16), FORMAT.BATCHED)
    o = as_vtensor(ic.sparse_kv_indices.view(-1, 1, 1), FORMAT.RAGGED)
    loc = torch.arange(batch.batch, dtype=torch.int64) * P + P - 1
    ic.profile()
    cc.profile()
    flow.forward_cache(cache, loc, cc)
    flow.forward_indexer(q, o, cache, ic)
    ic.execute()
    cc.execute()
    if cache_step:
        flow.forward_cache(cache, loc, cc)
    if indexer:
        flow.forward_indexer(q, o, cache, ic)
    return flow


def _keep_flow():
    name = "test_quest_keep_cpu"
    if not registry.has(name):
        @registry.register(name)
        class _Keep(algorithms.GQAQuestSparseAttention):
            def forward_indexer(self, q, o, cache, ctx):
                s_max = self.mul_max(q, cache["max"], ctx=ctx)
                s_min = self.mul_min(q, cache["min"], ctx=ctx)
                self.kept = self.maximum_op(s_max, s_min, ctx=ctx)
                self.output_func(self.max_op(self.sum(self.kept, ctx=ctx), ctx=ctx), o, ctx=ctx)
    return name


def test_quest_chain_is_one_launch(launches):
    _run("gqa_quest_sparse_attention")
    assert launches == ["fused"]


def test_quest_chain_computes_observed_intermediates(launches):
    flow = _run(_keep_flow())
    # the fused kernel first, then the kept maximum (its two products, then itself)
    assert launches == ["fused", "binary", "binary", "binary"]
    assert not flow.kept.is_pending


def test_quest_chain_unfused(launches, monkeypatch):
    monkeypatch.setenv("VORTEX_FUSE", "0")
    _run("gqa_quest_sparse_attention")
    assert launches == ["binary", "binary", "binary", "reduce", "reduce", "topk"]


def test_quest_chain_broken_by_a_read(launches, monkeypatch):
    """A torch op on an intermediate inside forward_indexer runs the recorded
    work first; the chain then launches op by op."""
    name = "test_quest_read_cpu"
    if not registry.has(name):
        @registry.register(name)
        class _Read(algorithms.GQAQuestSparseAttention):
            def forward_indexer(self, q, o, cache, ctx):
                s_max = self.mul_max(q, cache["max"], ctx=ctx)
                s_min = self.mul_min(q, cache["min"], ctx=ctx)
                s = self.maximum_op(s_max, s_min, ctx=ctx)
                self.peek = float(s.sum())  # a read
                self.output_func(self.max_op(self.sum(s, ctx=ctx), ctx=ctx), o, ctx=ctx)
    _run(name)
    assert launches == ["binary", "binary", "binary", "reduce", "reduce", "topk"]


def test_quest_cache_reductions_are_one_pass(launches):
    """forward_cache's CMax and CMin of the same pool and loc: one pass,
    carried into the Quest chain's fused launch."""
    _run("gqa_quest_sparse_attention", cache_step=True)
    assert launches == ["fused+envelope"]


def test_quest_cache_reductions_one_pass_when_not_carried(launches, monkeypatch):
    monkeypatch.setenv("VORTEX_FUSE_CMEAN", "0")
    _run("gqa_quest_sparse_attention", cache_step=True)
    assert launches == ["page_reduce_multi2", "fused"]


def test_quest_cache_reductions_unfused(launches, monkeypatch):
    monkeypatch.setenv("VORTEX_FUSE", "0")
    _run("gqa_quest_sparse_attention", cache_step=True)
    assert launches[:2] == ["page_reduce", "page_reduce"]


def test_single_cache_reduction_stays_single(launches):
    _run("gqa_block_sparse_attention", cache_step=True, indexer=False)
    assert launches == []  # carried for the next forward_indexer
    _deferred.flush_carry()
    assert launches == ["page_reduce"]



# ------------------------------------------------ the carried page-finish mean
@pytest.fixture
def carry_launches(monkeypatch):
    """Kernel wrappers replaced by recorders that, like the real ones, first
    run the deferral layer's pre-launch hook."""
    from vortex_torch.indexer import matmul as MM

    log = []

    def rec(name):
        def f(*a, **k):
            _hip._pre_launch()
            log.append(name + ("+cmean" if k.get("cmean") is not None else ""))
        return f

    monkeypatch.setattr(CR, "_recordable_operands", lambda x, out, loc: True)
    monkeypatch.setattr(MM, "_fusable", lambda x, y, ctx: True)
    for name in ("page_reduce", "page_reduce_multi", "indexer_fused", "gemv_paged", "topk_select"):
        monkeypatch.setattr(_hip, name, rec(name))
    yield log
    _deferred._tls.carry = None


class _Layer:
    """block_sparse_attention on C1-shaped CPU tensors, execute mode."""

    def __init__(self, flow_name="block_sparse_attention"):
        batch = W.c1()
        self.ic, self.cc = W.make_contexts(batch, "cpu")
        self.flow = build_vflow(flow_name)
        H, G, D, P = batch.num_kv_heads, batch.group_size, batch.head_dim, batch.page_size
        rows = batch.pool_pages * H
        self.cache = {"k": as_vtensor(torch.zeros((rows, P, D), dtype=torch.bfloat16), FORMAT.PAGED)}
        for name, (r, c) in self.flow.create_cache(P, D).items():
            self.cache[name] = as_vtensor(torch.zeros((rows, r, c), dtype=torch.bfloat16), FORMAT.PAGED)
        self.q = as_vtensor(torch.zeros((batch.batch * H, G, D), dtype=torch.bfloat16), FORMAT.BATCHED)
        self.o = as_vtensor(self.ic.sparse_kv_indices.view(-1, 1, 1), FORMAT.RAGGED)
        self.loc = torch.arange(batch.batch, dtype=torch.int64) * P + P - 1
        self.ic.profile()
        self.cc.profile()
        self.flow.forward_cache(self.cache, self.loc, self.cc)
        self.flow.forward_indexer(self.q, self.o, self.cache, self.ic)
        self.ic.execute()
        self.cc.execute()

    def cache_step(self):
        self.flow.forward_cache(self.cache, self.loc, self.cc)

    def indexer_step(self):
        self.flow.forward_indexer(self.q, self.o, self.cache, self.ic)


def test_cmean_runs_inside_the_next_indexer_launch(carry_launches):
    layer = _Layer()
    layer.cache_step()
    assert carry_launches == []  # carried
    layer.indexer_step()
    assert carry_launches == ["indexer_fused+cmean"]


def test_carried_cmean_runs_before_a_torch_read(carry_launches):
    layer = _Layer()
    layer.cache_step()
    float(layer.cache["centroids"].sum())
    assert carry_launches == ["page_reduce"]
    layer.indexer_step()
    assert carry_launches == ["page_reduce", "indexer_fused"]


def test_carried_cmean_runs_before_the_next_cache_step(carry_launches):
    a, b = _Layer(), _Layer()
    a.cache_step()
    b.cache_step()
    assert carry_launches == ["page_reduce"]  # a's, at b's forward_cache
    b.indexer_step()
    assert carry_launches == ["page_reduce", "indexer_fused+cmean"]


def test_carried_cmean_runs_before_any_other_launch(carry_launches, monkeypatch):
    layer = _Layer()
    layer.cache_step()
    _hip.topk_select(None)  # any other kernel of the package
    assert carry_launches == ["page_reduce", "topk_select"]


def test_carried_cmean_for_other_centroids_is_not_consumed(carry_launches):
    a, b = _Layer(), _Layer()
    a.cache_step()
    b.indexer_step()  # scores b's centroids: a's mean runs first, on its own
    assert carry_launches == ["page_reduce", "indexer_fused"]


def test_unconsumed_carry_runs_at_indexer_exit(carry_launches):
    name = "test_cmean_no_indexer"
    if not registry.has(name):
        @registry.register(name)
        class _NoIndexer(algorithms.BlockSparseAttention):
            def forward_indexer(self, q, o, cache, ctx):
                pass
    layer = _Layer(name)
    layer.cache_step()
    assert carry_launches == []
    layer.indexer_step()
    assert carry_launches == ["page_reduce"]


def test_carry_off(carry_launches, monkeypatch):
    monkeypatch.setenv("VORTEX_FUSE_CMEAN", "0")
    layer = _Layer()
    layer.cache_step()
    assert carry_launches == ["page_reduce"]
    layer.indexer_step()
    assert carry_launches == ["page_reduce", "indexer_fused"]


# ------------------------------------------------------------ graph capture
def test_capture_boundaries_launch_the_carry(carry_launches):
    """torch.cuda.CUDAGraph.capture_begin / capture_end launch a carried mean
    before torch's own method runs (here it then fails on a non-graph)."""
    layer = _Layer()
    layer.cache_step()
    assert carry_launches == []
    with pytest.raises(TypeError):
        torch.cuda.CUDAGraph.capture_end(object())
    assert carry_launches == ["page_reduce"]
    layer.cache_step()
    with pytest.raises(TypeError):
        torch.cuda.CUDAGraph.capture_begin(object())
    assert carry_launches == ["page_reduce", "page_reduce"]
    assert _deferred.current_carry() is None


def test_carry_across_a_capture_boundary_is_an_error(carry_launches, monkeypatch):
    state = {"id": 0}
    monkeypatch.setattr(_deferred, "_capture_of", lambda stream: state["id"])
    layer = _Layer()
    state["id"] = 5  # recorded during capture 5 ...
    layer.cache_step()
    state["id"] = 0  # ... which ended without launching it
    with pytest.raises(RuntimeError, match="recorded during a graph capture and would now be launched outside"):
        layer.indexer_step()
    assert _deferred.current_carry() is not None  # kept: it can still run where it belongs
    _deferred.discard_carry()
    layer.cache_step()  # recorded outside any capture ...
    state["id"] = 9  # ... found inside one
    with pytest.raises(RuntimeError, match="recorded outside any graph capture and would now be launched during"):
        layer.indexer_step()
    state["id"] = 0  # back outside: the kept carry launches
    _deferred.flush_carry()
    assert carry_launches[-1] == "page_reduce"
    carry_launches.clear()
    state["id"] = 3
    layer.cache_step()
    state["id"] = 4  # another capture
    with pytest.raises(RuntimeError, match="in another capture"):
        _deferred.flush_carry()
    _deferred.discard_carry()
    assert "page_reduce" not in carry_launches  # never launched where it does not belong
    state["id"] = 6
    layer.cache_step()
    carry_launches.clear()
    layer.indexer_step()  # same capture: consumed
    assert carry_launches == ["indexer_fused+cmean"]


def test_capture_hooks_only_while_carrying(carry_launches):
    """torch.cuda.CUDAGraph's capture methods are wrapped only once a mean is
    carried, and switching the carry off launches it and restores them."""
    graph = torch.cuda.CUDAGraph
    _deferred.remove_capture_hooks()  # (earlier tests carried means)
    assert not _deferred.capture_hooks_installed()
    begin, end = graph.capture_begin, graph.capture_end  # torch's own
    layer = _Layer()
    layer.cache_step()
    assert _deferred.capture_hooks_installed() and graph.capture_begin is not begin
    try:
        _deferred.set_fusion(carry_cmean=False)
        assert carry_launches[-1] == "page_reduce" and _deferred.current_carry() is None
        assert not _deferred.capture_hooks_installed()
        assert graph.capture_begin is begin and graph.capture_end is end
        layer.cache_step()  # the carry is off: launched when forward_cache returns
        assert _deferred.current_carry() is None and carry_launches[-1] == "page_reduce"
    finally:
        _deferred.set_fusion()


def test_set_fusion_overrides_environment(monkeypatch):
    monkeypatch.setenv("VORTEX_FUSE", "1")
    monkeypatch.setenv("VORTEX_FUSE_CMEAN", "1")
    try:
        _deferred.set_fusion(fuse=False)
        assert not _deferred.fusion_enabled() and not _deferred._carry_enabled()
        _deferred.set_fusion(fuse=True, carry_cmean=False)
        assert _deferred.fusion_enabled() and not _deferred._carry_enabled()
        monkeypatch.setenv("VORTEX_FUSE", "0")
        assert _deferred.fusion_enabled()  # the switch wins over the variable
    finally:
        _deferred.set_fusion()
    assert not _deferred.fusion_enabled()  # handed back to VORTEX_FUSE=0
