"""Host-side behaviour of the vortex_torch API (no GPU needed): layout tags,
flow registry and loader, contexts, op dispatch and profile-mode checks, the
deferral scope, and the absence of any CPU fallback.  Expected behaviours are
those of the reference (vortex_torch/abs, flow, indexer, cache)."""
import pickle
import textwrap
from types import SimpleNamespace

import pytest
import torch

import workloads as W
import vortex_torch
from vortex_torch import _deferred
from vortex_torch.abs import FORMAT, ContextBase, as_vtensor, vOp, vTensor
from vortex_torch.flow import build_vflow, register, vFlow
from vortex_torch.flow import registry
from vortex_torch.flow.loader import FlowInitError, FlowLoadError
from vortex_torch.utils import UNSET, Mode, ReduceType


# ----------------------------------------------------------------- vTensor
def test_vtensor_format_propagation_and_mixing():
    a = as_vtensor(torch.randn(2, 3), FORMAT.RAGGED)
    b = as_vtensor(torch.ones(2, 3), FORMAT.RAGGED)
    y = a + 2.0
    assert isinstance(y, vTensor) and y._format == FORMAT.RAGGED
    z = a * b
    assert isinstance(z, vTensor) and z._format == FORMAT.RAGGED
    with pytest.raises(RuntimeError, match="plain torch.Tensor"):
        _ = a + torch.randn(2, 3)
    c = as_vtensor(torch.randn(2, 3), FORMAT.PAGED)
    with pytest.raises(RuntimeError, match="mismatch"):
        _ = a + c
    # views share storage; re-tagging a vTensor is in place
    base = torch.zeros(4)
    v = as_vtensor(base, FORMAT.BATCHED)
    v[1] = 5.0
    assert base[1] == 5.0
    assert as_vtensor(v, FORMAT.PAGED) is v and v._format == FORMAT.PAGED
    assert isinstance(v.sum(), vTensor)
    assert "vTensor(format=" in repr(v)


def test_vtensor_pickle_keeps_format():
    v = as_vtensor(torch.arange(6.0).view(2, 3), FORMAT.PAGED)
    w = pickle.loads(pickle.dumps(v))
    assert isinstance(w, vTensor) and w._format == FORMAT.PAGED and torch.equal(w, v)


def test_enums():
    assert [m.value for m in Mode] == [0, 1]
    assert [r.name for r in ReduceType] == ["Mean", "Max", "Min", "L2Norm", "Sum"]
    assert repr(UNSET) == "UNSET"
    assert vortex_torch.__version__ == "1.0.0"


# ----------------------------------------------------------------- registry / loader
def test_registry_and_loader_errors(tmp_path):
    assert "block_sparse_attention" in registry.list_keys()
    with pytest.raises(registry.RegistryError, match="already exists"):
        register("block_sparse_attention")(type("Dup", (vFlow,), {}))
    with pytest.raises(registry.RegistryError, match="must inherit from vFlow"):
        register("not_a_flow")(object)
    with pytest.raises(FlowLoadError, match="available"):
        build_vflow("no_such_flow")
    with pytest.raises(FlowLoadError, match="does not exist"):
        build_vflow("x", user_file=str(tmp_path / "missing.py"))
    bad = tmp_path / "bad.py"
    bad.write_text("raise ValueError('boom')\n")
    with pytest.raises(FlowLoadError, match="boom"):
        build_vflow("x", user_file=str(bad))
    with pytest.raises(FlowInitError, match="mismatch"):
        build_vflow("block_sparse_attention", init_kwargs={"nope": 1})


def test_user_file_registration(tmp_path):
    user = tmp_path / "my_flow.py"
    user.write_text(textwrap.dedent("""
        from vortex_torch.flow import vFlow, register
        from vortex_torch.indexer import GeMV, topK
        from vortex_torch.cache import Max as CMax

        @register("test_user_flow_max")
        class MyFlow(vFlow):
            def __init__(self, scale=1.0):
                super().__init__()
                self.scale = scale
                self.gemv, self.topk, self.red = GeMV(), topK(), CMax(dim=1)
            def forward_indexer(self, q, o, cache, ctx):
                self.topk(self.gemv(q.mean(dim=1, keepdim=True), cache["env"], ctx=ctx), o, ctx=ctx)
            def forward_cache(self, cache, loc, ctx):
                self.red(cache["k"], cache["env"], loc=loc, ctx=ctx)
            def create_cache(self, page_size, head_dim):
                return {"env": (1, head_dim)}

        @register("test_user_flow_raises")
        class Raises(vFlow):
            def __init__(self):
                raise RuntimeError("ctor failed")
            def forward_indexer(self, q, o, cache, ctx): pass
            def forward_cache(self, cache, loc, ctx): pass
            def create_cache(self, page_size, head_dim): return {}
    """))
    f = build_vflow("test_user_flow_max", init_kwargs={"scale": 2.0}, user_file=str(user))
    assert f.scale == 2.0
    assert f.get_cache_meta_info(16, 128) == {"env": (1, 128), "k": (16, 128), "v": (16, 128)}
    assert f.get_token_ratio(16, 128) == pytest.approx(2 + 1 / 16)
    assert f.run_indexer_virtual(2, 16, 128) == 128  # GeMV declares 1*D flops per page
    with pytest.raises(FlowInitError, match="ctor failed"):
        build_vflow("test_user_flow_raises")


def test_cache_meta_rejects_k_v():
    class Bad(vFlow):
        def forward_indexer(self, q, o, cache, ctx): pass
        def forward_cache(self, cache, loc, ctx): pass
        def create_cache(self, page_size, head_dim): return {"k": (1, 1)}

    with pytest.raises(AssertionError):
        Bad().get_cache_meta_info(16, 128)


# ----------------------------------------------------------------- contexts
def _fake_runtime(H=8, G=2, D=128, P=16, max_seq=8192, max_bs=64, min_chunk=16, max_chunk=64):
    sa = SimpleNamespace(page_size=P, vortex_max_seq_lens=max_seq, vortex_lb_max_chunk_size=max_chunk,
                         vortex_lb_min_chunk_size=min_chunk, vortex_topk_val=30, vortex_indexer_dtype="bfloat16",
                         vortex_page_reserved_bos=1, vortex_page_reserved_eos=1, max_prefill_tokens=16384)
    mr = SimpleNamespace(server_args=sa, model_config=SimpleNamespace(context_len=40960),
                         req_to_token_pool=SimpleNamespace(size=max_bs), device="cpu")
    i32 = dict(dtype=torch.int32)
    parent = SimpleNamespace(kv_indices_decode=[torch.zeros(10, **i32), torch.zeros(10, **i32)],
                             kv_indptr_decode=[torch.zeros(3, **i32), torch.zeros(3, **i32)],
                             kv_last_page_len_decode=torch.zeros(2, **i32), group_size=G, num_kv_heads=H,
                             num_qo_heads=G * H, head_dim=D, page_size=P, num_pages=1000, head_num=H)
    return parent, mr


def test_indexer_context_create():
    from vortex_torch.indexer import Context

    parent, mr = _fake_runtime()
    ctx = Context()
    assert ctx.mode == Mode.profile and not ctx.created and "topk_val" in ctx.missing()
    ctx.create(parent, mr)
    assert ctx.created and ctx.missing() == []
    assert ctx.max_num_pages_per_request == 512
    assert ctx.max_num_pages == 512 * 64 * 8
    assert ctx.max_num_workloads == 512 * 64 * 8 // 16 + 64 * 8
    assert ctx.winfo_q_indices.shape == (ctx.max_num_workloads,)
    assert ctx.indexer_dtype == torch.bfloat16
    with pytest.raises(RuntimeError, match="already called"):
        ctx.create(parent, mr)
    ctx.create(parent, mr, overwrite=True)
    mr.server_args.vortex_max_seq_lens = -1  # falls back to the model context length
    ctx.create(parent, mr, overwrite=True)
    assert ctx.max_num_pages_per_request == 40960 // 16
    ctx.set_batch_size(7)
    assert ctx.batch_size == 7


def test_cache_context_create_and_aux_accounting():
    from vortex_torch.cache import Context

    parent, mr = _fake_runtime()
    c = Context()
    c.create(parent, mr)
    assert (c.page_size, c.total_num_pages, c.head_num, c.head_dim) == (16, 1000, 8, 128)
    assert c.max_new_tokens_per_batch == 16384
    with pytest.raises(RuntimeError):
        c.create(parent, mr)
    assert c.add_aux_memory(100) == 100
    assert c.add_aux_memory(torch.zeros(4, dtype=torch.float32)) == 16
    with pytest.raises(TypeError):
        c.add_aux_memory(1.5)
    with pytest.raises(ValueError):
        c.add_aux_memory(-1)
    c.add_aux_flops(7)
    s = c.summary()
    assert s["aux_bytes"] == 116 and s["aux_flops"] == 7
    c.clear_aux_memory()
    c.clear_aux_flops()
    assert c.summary()["aux_bytes"] == 0 and c.summary()["aux_flops"] == 0


def test_vop_mode_dispatch():
    class Probe(vOp):
        def profile(self, *a, ctx=None, **k):
            return "profile"

        def execute(self, *a, ctx=None, **k):
            return "execute"

    op = Probe()
    assert op(ctx=SimpleNamespace(mode=Mode.profile)) == "profile"
    assert op(ctx=SimpleNamespace(mode=Mode.execute)) == "execute"
    assert op(ctx=SimpleNamespace(mode=None)) == "execute"
    with pytest.raises(ValueError, match="Unknown mode"):
        op(ctx=SimpleNamespace(mode="train"))


# ----------------------------------------------------------------- ops in profile mode
def _profiled_flow(batch):
    ic, cc = W.make_contexts(batch, "cpu")
    f = build_vflow("block_sparse_attention")
    H, G, D, P = batch.num_kv_heads, batch.group_size, batch.head_dim, batch.page_size
    cache = {
        "k": as_vtensor(torch.zeros(batch.pool_pages * H, P, D, dtype=torch.bfloat16), FORMAT.PAGED),
        "centroids": as_vtensor(torch.zeros(batch.pool_pages * H, 1, D, dtype=torch.bfloat16), FORMAT.PAGED),
    }
    q = as_vtensor(torch.zeros(batch.batch * H, G, D, dtype=torch.bfloat16), FORMAT.BATCHED)
    o = as_vtensor(ic.sparse_kv_indices.view(-1, 1, 1), FORMAT.RAGGED)
    ic.profile()
    cc.profile()
    f.forward_cache(cache, W.decode_loc(batch), cc)
    f.forward_indexer(q, o, cache, ic)
    return f, ic, cc, cache, q, o


def test_block_sparse_profile_pass():
    batch = W.c1()
    f, ic, cc, cache, q, o = _profiled_flow(batch)
    assert f.gemv.output_buffer.shape == (ic.max_num_pages, 1, 1)
    assert f.gemv.output_buffer.dtype == torch.bfloat16
    assert ic._aux_total_flops == batch.head_dim
    assert ic._aux_total_bytes == ic.max_num_pages * 2
    assert f.output_func.impl is not None and f.reduction.impl is not None


def test_no_cpu_fallback():
    batch = W.c1()
    f, ic, cc, cache, q, o = _profiled_flow(batch)
    ic.execute()
    cc.execute()
    with pytest.raises(RuntimeError, match="no CPU implementation"):
        f.forward_cache(cache, W.decode_loc(batch), cc)
    with pytest.raises(RuntimeError, match="no CPU implementation"):
        f.forward_indexer(q, o, cache, ic)
    from vortex_torch.indexer.utils_sglang import plan_decode

    with pytest.raises(RuntimeError, match="no CPU implementation"):
        plan_decode(batch.seq_lens, batch.req_to_token, batch.req_indices, ic)


def test_op_profile_checks():
    from vortex_torch.cache import Mean as CMean
    from vortex_torch.indexer import GeMV, topK

    ctx = SimpleNamespace(mode=Mode.profile, max_num_pages=8, add_aux_memory=lambda t: 0,
                          add_aux_flops=lambda n: 0)
    g = GeMV()
    x = as_vtensor(torch.zeros(4, 1, 16), FORMAT.BATCHED)
    with pytest.raises(AssertionError, match="last dimension"):
        g(x, as_vtensor(torch.zeros(9, 1, 8), FORMAT.PAGED), ctx=ctx)
    with pytest.raises(AssertionError, match="no implementation"):
        g(x, as_vtensor(torch.zeros(9, 1, 16), FORMAT.RAGGED), ctx=ctx)
    with pytest.raises(AssertionError, match="vTensor"):
        g(torch.zeros(4, 1, 16), as_vtensor(torch.zeros(9, 1, 16), FORMAT.PAGED), ctx=ctx)
    t = topK()
    with pytest.raises(AssertionError, match="x.shape"):
        t(as_vtensor(torch.zeros(8, 2, 1), FORMAT.RAGGED), as_vtensor(torch.zeros(8, 1, 1), FORMAT.RAGGED), ctx=ctx)
    with pytest.raises(AssertionError, match="no implementation"):
        t(as_vtensor(torch.zeros(8, 1, 1), FORMAT.PAGED), as_vtensor(torch.zeros(8, 1, 1), FORMAT.PAGED), ctx=ctx)
    with pytest.raises(AssertionError, match="before profile"):
        topK().execute(torch.zeros(8, 1, 1), torch.zeros(8, 1, 1), ctx=ctx)
    with pytest.raises(AssertionError, match="dim must be 1 or 2"):
        CMean(dim=3)
    m = CMean(dim=1)
    kx = as_vtensor(torch.zeros(6, 16, 8), FORMAT.PAGED)
    with pytest.raises(AssertionError, match="output.shape"):
        m(kx, as_vtensor(torch.zeros(6, 1, 4), FORMAT.PAGED), loc=torch.zeros(1, dtype=torch.int64), ctx=ctx)
    with pytest.raises(AssertionError, match="RAGGED-output"):
        m(kx, None, loc=torch.zeros(1, dtype=torch.int64), ctx=SimpleNamespace(mode=Mode.profile))


def test_out_of_scope_entry_points_say_so():
    import vortex_torch_C
    from vortex_torch.indexer import utils_sglang

    with pytest.raises(NotImplementedError, match="prefill"):
        vortex_torch_C.sglang_plan_prefill()
    with pytest.raises(NotImplementedError):
        utils_sglang.plan_prefill_fa3()
    with pytest.raises(NotImplementedError, match="prefill"):
        vortex_torch_C.Chunkwise_HN2NH_Transpose_FA3()
    assert utils_sglang.indices_to_page_table(None, None) is None


# ----------------------------------------------------------------- deferral scope
def test_deferral_scope_flush_rules():
    log = []

    class P(_deferred.Pending):
        def _run(self):
            log.append("ran")

    with _deferred.scope(True) as sc:
        p = P()
        sc.add(p)
        t = _deferred.DeferredTensor.make(torch.zeros(4, 1, 2), FORMAT.RAGGED, p)
        _ = (t.shape, t.dtype, t.device, t.dim(), t.numel())
        assert log == [] and t.is_pending  # metadata does not flush
        _ = as_vtensor(torch.ones(2), FORMAT.RAGGED) + 1  # any other vTensor op flushes
        assert log == ["ran"] and not t.is_pending
    with _deferred.scope(True) as sc:
        sc.add(P())
    assert log == ["ran", "ran"]  # leaving the scope flushes
    with _deferred.scope(False) as sc:
        assert sc is None and _deferred.current_scope() is None


def test_forward_indexer_runs_in_scope_only_in_execute_mode():
    seen = []

    class Spy(vFlow):
        def forward_indexer(self, q, o, cache, ctx):
            seen.append(_deferred.current_scope() is not None)

        def forward_cache(self, cache, loc, ctx):
            pass

        def create_cache(self, page_size, head_dim):
            return {}

    s = Spy()
    s.forward_indexer(None, None, None, SimpleNamespace(mode=Mode.profile))
    s.forward_indexer(None, None, None, ctx=SimpleNamespace(mode=Mode.execute))
    assert seen == [False, True]
    assert _deferred.current_scope() is None


def test_mean_not_deferred_on_cpu_or_outside_scope():
    q = as_vtensor(torch.randn(4, 2, 8).to(torch.bfloat16), FORMAT.BATCHED)
    with _deferred.scope(True):
        m = q.mean(dim=1, keepdim=True)
    assert type(m) is vTensor
    with torch._C.DisableTorchFunctionSubclass():
        assert torch.equal(m.as_subclass(torch.Tensor), q.as_subclass(torch.Tensor).mean(dim=1, keepdim=True))
