"""GPU tests of the fused indexer kernel and of block_sparse_attention run
through the public flow API (eager, fused and unfused, and replayed from a
HIP graph).  Selections are bit-exact against the oracle's top-k of the same
scores; scores and q-means are bit-exact against the separate kernels."""
import os

import numpy as np
import pytest
import torch

import workloads as W
from oracle import vortex_oracle as O
from vortex_torch import _hip
from vortex_torch.abs import FORMAT, as_vtensor

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().cpu().numpy()


def _bits(t):
    with torch._C.DisableTorchFunctionSubclass():
        return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)


def _plan(batch, ic, dev):
    from vortex_torch.indexer.utils_sglang import plan_decode

    b = batch.to(dev)
    plan_decode(b.seq_lens, b.req_to_token, b.req_indices, ic)


@pytest.mark.parametrize("mode", [_hip.FUSED_SEGMENT, _hip.FUSED_SPLIT])
@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c5"])
def test_fused_kernel_matches_separate_kernels(gpu, name, mode):
    dev = gpu
    batch = getattr(W, name)()
    ic, _ = W.make_contexts(batch, dev)
    _plan(batch, ic, dev)
    H, G, D = batch.num_kv_heads, batch.group_size, batch.head_dim
    S = batch.batch * H
    q = W.randn_bf16((S, G, D), 1, dev)
    y = W.randn_bf16((batch.pool_pages * H, 1, D), 2, dev, std=0.25)
    n_dense = ic.dense_kv_indices.numel()

    # separate kernels: torch mean, GeMV, topK
    qm_ref = q.mean(dim=1, keepdim=True)
    sc_ref = torch.full((n_dense, 1, 1), -5.0, device=dev, dtype=torch.bfloat16)
    _hip.gemv_paged(qm_ref, y, sc_ref, ic.dense_kv_indices, ic.winfo_q_indices, ic.winfo_kv_offsets,
                    ic.winfo_kv_lens, ic.winfo_num_workloads, batch.max_chunk)
    sp_ref = ic.sparse_kv_indices.clone()
    _hip.topk_select(sc_ref, ic.dense_kv_indptr, ic.sparse_kv_indptr, ic.dense_kv_indices, sp_ref,
                     S, batch.topk, batch.bos, batch.eos, batch.max_pages_per_request)

    # fused, twice with the same counters (the first call must leave them zeroed)
    counters = torch.zeros(S, dtype=torch.int32, device=dev)
    for _ in range(2):
        qm = torch.empty_like(qm_ref)
        sc = torch.full_like(sc_ref, -5.0)
        sp = ic.sparse_kv_indices.clone()
        _hip.indexer_fused(q, qm, y, sc, ic.dense_kv_indptr, ic.sparse_kv_indptr, ic.dense_kv_indices, sp,
                           S, batch.topk, batch.bos, batch.eos, batch.max_pages_per_request,
                           seg_counters=counters, mode=mode)
        torch.cuda.synchronize()
        assert int(counters.abs().sum()) == 0, "segment counters not reset"
    assert torch.equal(qm, qm_ref), "q-mean differs from torch.mean"
    # same query -> same scores as the GeMV kernel, written at the same positions
    sc_sep = torch.full_like(sc_ref, -5.0)
    _hip.gemv_paged(qm, y, sc_sep, ic.dense_kv_indices, ic.winfo_q_indices, ic.winfo_kv_offsets,
                    ic.winfo_kv_lens, ic.winfo_num_workloads, batch.max_chunk)
    assert torch.equal(sc, sc_sep), "fused scores differ from the GeMV kernel"
    # selection: oracle top-k of the fused kernel's own scores
    exp, _ = O.topk(_bits(sc), _np(ic.dense_kv_indptr), _np(ic.sparse_kv_indptr), _np(ic.dense_kv_indices),
                    _np(ic.sparse_kv_indices), S, batch.topk, batch.bos, batch.eos)
    np.testing.assert_array_equal(_np(sp), exp)


def _wide_q(shape, seed, dev):
    """bf16 values over 2^-24 .. 2^24: fp32 sums of them round, so a
    different summation order gives different bits."""
    g = torch.Generator(device=dev).manual_seed(seed)
    mag = torch.exp2(torch.randint(-24, 24, shape, generator=g, device=dev).float())
    return (torch.randn(shape, generator=g, device=dev) * mag).to(torch.bfloat16)


@pytest.mark.parametrize("mode", [_hip.FUSED_SEGMENT, _hip.FUSED_SPLIT])
@pytest.mark.parametrize("D", [64, 128, 576])
@pytest.mark.parametrize("G", [1, 2, 3, 4, 5, 6, 8, 12, 16])
def test_fused_query_mean_is_torch_mean(gpu, G, D, mode):
    """The kernel's q-mean (written to x_out, also for query rows past the
    segments) equals torch.mean(dim=1) bit for bit on values whose fp32 sums
    round: it sums in torch's order and scales by torch's factor."""
    dev = gpu
    batch = W.make_batch([4096, 3000, 600], pool_pages=900, seed=40 + G, num_kv_heads=2, group_size=G,
                         head_dim=D, topk=30, bos=1, eos=1)
    ic, _ = W.make_contexts(batch, dev)
    _plan(batch, ic, dev)
    S = batch.batch * batch.num_kv_heads
    q = _wide_q((S + 3, G, D), G * 7 + D, dev)
    y = W.randn_bf16((batch.pool_pages * batch.num_kv_heads, 1, D), 4, dev, std=0.25)
    qm = torch.full((S + 3, 1, D), 3.0, device=dev, dtype=torch.bfloat16)
    sc = torch.zeros((ic.dense_kv_indices.numel(), 1, 1), device=dev, dtype=torch.bfloat16)
    counters = torch.zeros(S, dtype=torch.int32, device=dev)
    _hip.indexer_fused(q, qm, y, sc, ic.dense_kv_indptr, ic.sparse_kv_indptr, ic.dense_kv_indices,
                       ic.sparse_kv_indices.clone(), S, batch.topk, batch.bos, batch.eos,
                       batch.max_pages_per_request, seg_counters=counters, mode=mode)
    torch.cuda.synchronize()
    ref = q.mean(dim=1, keepdim=True)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(qm), _bits(ref))


@pytest.mark.parametrize("cmean", [False, True])
@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c5", "eos0", "d64", "d256", "d576", "d576many", "r3", "r9"])
def test_fused_segment_and_split_layouts_agree(gpu, name, cmean):
    """FUSED_SEGMENT and FUSED_SPLIT write the same bits: q-mean, scores,
    block table and (with the layer's CMean) centroids."""
    dev = gpu
    batch, loc = W.cmean_case(name)
    loc = loc.to(dev)
    ic, _ = W.make_contexts(batch, dev)
    _plan(batch, ic, dev)
    H, G, D, P = batch.num_kv_heads, batch.group_size, batch.head_dim, batch.page_size
    S = batch.batch * H
    rows = batch.pool_pages * H
    q = _wide_q((S, G, D), 11, dev)
    k = W.randn_bf16((rows, P, D), 3, dev)
    y0 = W.randn_bf16((rows, 1, D), 2, dev, std=0.25)
    out = {}
    for mode in (_hip.FUSED_SEGMENT, _hip.FUSED_SPLIT):
        y = y0.clone()
        qm = torch.full((S, 1, D), 3.0, device=dev, dtype=torch.bfloat16)
        sc = torch.full((ic.dense_kv_indices.numel(), 1, 1), -5.0, device=dev, dtype=torch.bfloat16)
        sp = ic.sparse_kv_indices.clone()
        counters = torch.zeros(S, dtype=torch.int32, device=dev)
        _hip.indexer_fused(q, qm, y, sc, ic.dense_kv_indptr, ic.sparse_kv_indptr, ic.dense_kv_indices, sp, S,
                           batch.topk, batch.bos, batch.eos, batch.max_pages_per_request, seg_counters=counters,
                           mode=mode, cmean=(k, loc, H) if cmean else None)
        torch.cuda.synchronize()
        out[mode] = (_bits(y), _bits(qm), _bits(sc), _np(sp))
    for a, b in zip(out[_hip.FUSED_SEGMENT], out[_hip.FUSED_SPLIT]):
        np.testing.assert_array_equal(a, b)
    if cmean:
        assert (out[_hip.FUSED_SPLIT][0] != _bits(y0)).any() or int(((loc + 1) % P == 0).sum()) == 0


@pytest.mark.parametrize("kind", ["ties", "const"])
@pytest.mark.parametrize("mode", [_hip.FUSED_SEGMENT, _hip.FUSED_SPLIT])
@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c5"])
def test_fused_kernel_tie_order(gpu, name, mode, kind):
    """Heavily tied scores: centroid rows drawn from three distinct rows
    ("ties") or all equal ("const", so every segment selects its first k
    middle pages).  The selection must be the oracle's stable order of the
    kernel's own scores: score descending, lower position first."""
    dev = gpu
    batch = getattr(W, name)()
    ic, _ = W.make_contexts(batch, dev)
    _plan(batch, ic, dev)
    H, G, D = batch.num_kv_heads, batch.group_size, batch.head_dim
    S = batch.batch * H
    rows = batch.pool_pages * H
    q = W.randn_bf16((S, G, D), 5, dev)
    base = W.randn_bf16((3, D), 6, dev, std=0.25)
    if kind == "const":
        pick = torch.zeros(rows, dtype=torch.long)
    else:
        pick = torch.randint(0, 3, (rows,), generator=torch.Generator().manual_seed(7))
    y = base[pick.to(dev)].view(rows, 1, D).contiguous()
    qm = torch.empty((S, 1, D), device=dev, dtype=torch.bfloat16)
    sc = torch.zeros((ic.dense_kv_indices.numel(), 1, 1), device=dev, dtype=torch.bfloat16)
    sp = ic.sparse_kv_indices.clone()
    counters = torch.zeros(S, dtype=torch.int32, device=dev)
    _hip.indexer_fused(q, qm, y, sc, ic.dense_kv_indptr, ic.sparse_kv_indptr, ic.dense_kv_indices, sp,
                       S, batch.topk, batch.bos, batch.eos, batch.max_pages_per_request,
                       seg_counters=counters, mode=mode)
    torch.cuda.synchronize()
    exp, _ = O.topk(_bits(sc), _np(ic.dense_kv_indptr), _np(ic.sparse_kv_indptr), _np(ic.dense_kv_indices),
                    _np(ic.sparse_kv_indices), S, batch.topk, batch.bos, batch.eos)
    np.testing.assert_array_equal(_np(sp), exp)


@pytest.mark.parametrize("mode", [_hip.FUSED_SEGMENT, _hip.FUSED_SPLIT])
def test_fused_kernel_extra_query_rows(gpu, mode):
    # more query rows than segments (padded batch): every row gets its mean
    dev = gpu
    batch = W.c1()
    ic, _ = W.make_contexts(batch, dev)
    _plan(batch, ic, dev)
    S = batch.batch * batch.num_kv_heads
    q = W.randn_bf16((S + 5, 2, 128), 3, dev)
    y = W.randn_bf16((batch.pool_pages * batch.num_kv_heads, 1, 128), 4, dev)
    qm = torch.empty((S + 5, 1, 128), device=dev, dtype=torch.bfloat16)
    sc = torch.zeros((ic.dense_kv_indices.numel(), 1, 1), device=dev, dtype=torch.bfloat16)
    counters = torch.zeros(S, dtype=torch.int32, device=dev)
    _hip.indexer_fused(q, qm, y, sc, ic.dense_kv_indptr, ic.sparse_kv_indptr, ic.dense_kv_indices,
                       ic.sparse_kv_indices, S, batch.topk, batch.bos, batch.eos, batch.max_pages_per_request,
                       seg_counters=counters, mode=mode)
    assert torch.equal(qm, q.mean(dim=1, keepdim=True))


class _FlowRun:
    """block_sparse_attention on one layer of `batch` through the public API."""

    def __init__(self, batch, dev, seed=0):
        from vortex_torch import flow as vflow

        self.batch, self.dev = batch, dev
        self.ic, self.cc = W.make_contexts(batch, dev)
        H, G, D = batch.num_kv_heads, batch.group_size, batch.head_dim
        self.flow = vflow.build_vflow("block_sparse_attention")
        self.k = W.randn_bf16((batch.pool_pages * H, batch.page_size, D), seed, dev)
        self.cen = W.randn_bf16((batch.pool_pages * H, 1, D), seed + 1, dev, std=0.25)
        self.cache = {"k": as_vtensor(self.k, FORMAT.PAGED), "centroids": as_vtensor(self.cen, FORMAT.PAGED)}
        self.q = as_vtensor(W.randn_bf16((batch.batch * H, G, D), seed + 2, dev), FORMAT.BATCHED)
        self.o = as_vtensor(self.ic.sparse_kv_indices.view(-1, 1, 1), FORMAT.RAGGED)
        self.loc = W.decode_loc(batch).to(dev)
        self.dev_batch = batch.to(dev)  # no host copies inside a captured step
        self.ic.profile()
        self.cc.profile()
        self.flow.forward_cache(self.cache, self.loc, self.cc)
        self.flow.forward_indexer(self.q, self.o, self.cache, self.ic)
        self.ic.execute()
        self.cc.execute()

    def step(self):
        from vortex_torch.indexer.utils_sglang import plan_decode

        b = self.dev_batch
        plan_decode(b.seq_lens, b.req_to_token, b.req_indices, self.ic)
        self.flow.forward_cache(self.cache, self.loc, self.cc)
        self.flow.forward_indexer(self.q, self.o, self.cache, self.ic)


@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c5", "eos0"])
def test_flow_fused_equals_unfused(gpu, name, monkeypatch):
    batch = _cmean_case(name)[0] if name == "eos0" else getattr(W, name)()
    results = {}
    for fuse in ("1", "0"):
        monkeypatch.setenv("VORTEX_FUSE", fuse)
        run = _FlowRun(batch, gpu)
        run.step()
        torch.cuda.synchronize()
        with torch._C.DisableTorchFunctionSubclass():
            results[fuse] = (run.ic.sparse_kv_indices.clone(), run.flow.gemv.output_buffer.clone(),
                             run.cen.clone())
    assert torch.equal(results["1"][2], results["0"][2]), "centroids differ"
    assert torch.equal(results["1"][0], results["0"][0]), "sparse indices differ"
    # scores: compare the positions the GeMV covers (the planner's workloads)
    ref = O.plan_decode(_np(batch.seq_lens), _np(batch.req_to_token), _np(batch.req_indices), batch.page_size,
                        batch.num_kv_heads, batch.topk, batch.bos, batch.eos, batch.max_chunk)
    cov = np.zeros(results["1"][1].numel(), dtype=bool)
    for off, ln in zip(ref["winfo_off"], ref["winfo_len"]):
        cov[off:off + ln] = True
    np.testing.assert_array_equal(_bits(results["1"][1])[cov], _bits(results["0"][1])[cov])


def test_flow_end_to_end_against_oracle(gpu):
    batch = W.c2()
    run = _FlowRun(batch, gpu, seed=5)
    k_host = _bits(run.k).reshape(run.k.shape)
    cen_before = _bits(run.cen).reshape(run.cen.shape)
    run.step()
    torch.cuda.synchronize()
    H, P = batch.num_kv_heads, batch.page_size
    ref = O.plan_decode(_np(batch.seq_lens), _np(batch.req_to_token), _np(batch.req_indices), P, H,
                        batch.topk, batch.bos, batch.eos, batch.max_chunk)
    # cache side: CMean of the pages the decode tokens close
    cen_exp, rows = O.page_reduce(k_host, cen_before, _np(run.loc), H, P, 1, O.MEAN)
    cen = _bits(run.cen).reshape(run.cen.shape)
    np.testing.assert_allclose(O.bf16_to_f32(cen), O.bf16_to_f32(cen_exp), rtol=1e-2, atol=1e-3)
    # indexer: scores within tolerance of the oracle, selection bit-exact on the GPU scores
    qm = O.q_group_mean(_bits(run.q).reshape(tuple(run.q.shape)))
    sc_exp, cov = O.gemv(qm, cen, ref["dense_indices"], ref["winfo_q"], ref["winfo_off"], ref["winfo_len"],
                         ref["num_workloads"], run.flow.gemv.output_buffer.numel())
    sc = _bits(run.flow.gemv.output_buffer)
    np.testing.assert_allclose(O.bf16_to_f32(sc)[cov], O.bf16_to_f32(sc_exp)[cov], rtol=1e-2, atol=1e-3)
    sel, _ = O.topk(sc, ref["dense_indptr"], ref["sparse_indptr"], ref["dense_indices"], ref["sparse_indices"],
                    batch.batch * H, batch.topk, batch.bos, batch.eos)
    np.testing.assert_array_equal(_np(run.ic.sparse_kv_indices), sel)


def test_c3_configured_inputs_cmean_then_fused_indexer(gpu):
    """C3 with the inputs its configuration names: K = N(0, 1) noise plus a
    per-(page, head) offset ~ N(0, 0.5), the centroid pool written by the
    package's CMean over every page, then plan and the fused indexer at full
    size (64 segments of 2046 middle pages: the split layout with the topK
    op's workspace).  CMean within tolerance of the oracle on a sample of
    pages; every covered score within tolerance of the oracle's GeMV; the
    selection the oracle's top-k of the GPU's scores, bit for bit."""
    dev = gpu
    batch = W.c3()
    assert batch.extra.get("k_page_offsets")
    ic, _ = W.make_contexts(batch, dev)
    _plan(batch, ic, dev)
    H, G, D, P = batch.num_kv_heads, batch.group_size, batch.head_dim, batch.page_size
    S = batch.batch * H
    k = W.k_pool(batch, 11, dev, page_offsets=True)
    cen = W.centroids_from_k(k, batch)
    rng = np.random.default_rng(3)
    pages = rng.choice(batch.pool_pages, 256, replace=False)
    srows = (pages[:, None] * H + np.arange(H)[None, :]).reshape(-1)
    sel_rows = torch.as_tensor(srows, device=dev)
    xs = _bits(k[sel_rows]).reshape(len(srows), P, D)
    exp, _ = O.page_reduce(xs, np.zeros((len(srows), 1, D), np.uint16), np.arange(len(pages)) * P + (P - 1), H, P,
                           1, O.MEAN)
    got = _bits(cen[sel_rows]).reshape(len(srows), 1, D)
    np.testing.assert_allclose(O.bf16_to_f32(got), O.bf16_to_f32(exp), rtol=1e-2, atol=1e-3)
    del k

    q = W.randn_bf16((S, G, D), 12, dev)
    qm = torch.full((S, 1, D), 3.0, device=dev, dtype=torch.bfloat16)
    sc = torch.full((ic.dense_kv_indices.numel(), 1, 1), -5.0, device=dev, dtype=torch.bfloat16)
    sp = ic.sparse_kv_indices.clone()
    ws = torch.zeros(_hip.indexer_fused_workspace_len(S), dtype=torch.int32, device=dev)
    _hip.indexer_fused(q, qm, cen, sc, ic.dense_kv_indptr, ic.sparse_kv_indptr, ic.dense_kv_indices, sp, S,
                       batch.topk, batch.bos, batch.eos, batch.max_pages_per_request, seg_counters=ws,
                       mode=_hip.FUSED_AUTO)
    torch.cuda.synchronize()
    ref = O.plan_decode(_np(batch.seq_lens), _np(batch.req_to_token), _np(batch.req_indices), P, H, batch.topk,
                        batch.bos, batch.eos, batch.max_chunk)
    qm_exp = O.q_group_mean(_bits(q).reshape(S, G, D))
    np.testing.assert_array_equal(_bits(qm).reshape(qm_exp.shape), qm_exp)
    sc_exp, cov = O.gemv(qm_exp, _bits(cen).reshape(cen.shape), ref["dense_indices"], ref["winfo_q"],
                         ref["winfo_off"], ref["winfo_len"], ref["num_workloads"], sc.numel())
    got_sc = _bits(sc)
    np.testing.assert_allclose(O.bf16_to_f32(got_sc)[cov], O.bf16_to_f32(sc_exp)[cov], rtol=1e-2, atol=1e-3)
    sel, _ = O.topk(got_sc, ref["dense_indptr"], ref["sparse_indptr"], ref["dense_indices"], ref["sparse_indices"],
                    S, batch.topk, batch.bos, batch.eos)
    np.testing.assert_array_equal(_np(sp), sel)
    # the offsets separate the pages: a segment's best score stands well above its median
    f = O.bf16_to_f32(got_sc)
    dip = ref["dense_indptr"]
    spread = [np.max(f[dip[s] + 1:dip[s + 1] - 1]) - np.median(f[dip[s] + 1:dip[s + 1] - 1]) for s in range(S)]
    assert min(spread) > 0.0


@pytest.mark.parametrize("name", ["c2", "c3"])
def test_flow_graph_replay(gpu, name):
    # C2 runs one workgroup per segment, C3 (64 segments) the split layout
    batch = getattr(W, name)()
    run = _FlowRun(batch, gpu, seed=9)
    stream = torch.cuda.Stream(gpu)
    stream.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(stream):
        run.step()
    torch.cuda.synchronize()
    with torch._C.DisableTorchFunctionSubclass():
        eager_o = run.ic.sparse_kv_indices.clone()
        eager_s = run.flow.gemv.output_buffer.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        run.step()
    torch.cuda.synchronize()
    for rep in range(4):
        # eager work between replays, then clobber the outputs
        run.ic.sparse_kv_indices.fill_(-3)
        with torch._C.DisableTorchFunctionSubclass():
            run.flow.gemv.output_buffer.fill_(0.5)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        with torch._C.DisableTorchFunctionSubclass():
            assert torch.equal(run.ic.sparse_kv_indices, eager_o), f"replay {rep}: selection differs"
            s = run.flow.gemv.output_buffer
            assert torch.equal(s[s != 0.5], eager_s[s != 0.5])
            nseg = run.ic.dense_kv_indptr.numel() - 1
            assert int(run.flow.output_func.seg_counters[:nseg].abs().sum()) == 0


def test_deferred_mean_materializes_on_use(gpu):
    """A recorded q-mean read by other torch code sees torch.mean's result."""
    from vortex_torch import _deferred

    q = as_vtensor(W.randn_bf16((16, 2, 128), 7, gpu), FORMAT.BATCHED)
    with _deferred.scope(True):
        m = q.mean(dim=1, keepdim=True)
        assert isinstance(m, _deferred.DeferredTensor) and m.is_pending
        assert tuple(m.shape) == (16, 1, 128)  # metadata does not materialise
        assert m.is_pending
        doubled = m * 2
        assert not m.is_pending
    with torch._C.DisableTorchFunctionSubclass():
        expect = q.as_subclass(torch.Tensor).mean(dim=1, keepdim=True)
        assert torch.equal(m.as_subclass(torch.Tensor), expect)
        assert torch.equal(doubled.as_subclass(torch.Tensor), expect * 2)


# ------------------------------------------- CMean inside the fused launch
def _cmean_case(name):
    return W.cmean_case(name)


@pytest.mark.parametrize("mode", [_hip.FUSED_AUTO, _hip.FUSED_SPLIT])
@pytest.mark.parametrize("name", ["c1", "c2", "c3", "eos0", "mid", "d64", "big_loc", "d256", "d576", "r3", "r6",
                                  "r9"])
def test_fused_cmean_equals_separate_launches(gpu, name, mode):
    """vtx_indexer_fused_cmean writes what vtx_page_reduce then
    vtx_indexer_fused write: centroids, q-mean, scores and block table."""
    dev = gpu
    batch, loc = _cmean_case(name)
    loc = loc.to(dev)
    ic, _ = W.make_contexts(batch, dev)
    _plan(batch, ic, dev)
    H, G, D, P = batch.num_kv_heads, batch.group_size, batch.head_dim, batch.page_size
    S = batch.batch * H
    rows = batch.pool_pages * H
    q = W.randn_bf16((S, G, D), 1, dev)
    k = W.randn_bf16((rows, P, D), 3, dev)
    y0 = W.randn_bf16((rows, 1, D), 2, dev, std=0.25)
    n_dense = ic.dense_kv_indices.numel()
    out = {}
    for fused in (False, True):
        y = y0.clone()
        qm = torch.zeros((S, 1, D), device=dev, dtype=torch.bfloat16)
        sc = torch.full((n_dense, 1, 1), -5.0, device=dev, dtype=torch.bfloat16)
        sp = ic.sparse_kv_indices.clone()
        counters = torch.zeros(S, dtype=torch.int32, device=dev)
        x_out = qm if G <= 2 else None
        qin = q if G <= 2 else q.mean(dim=1, keepdim=True)
        args = (qin, x_out, y, sc, ic.dense_kv_indptr, ic.sparse_kv_indptr, ic.dense_kv_indices, sp, S,
                batch.topk, batch.bos, batch.eos, batch.max_pages_per_request)
        if fused:
            _hip.indexer_fused(*args, seg_counters=counters, mode=mode, cmean=(k, loc, H))
        else:
            _hip.page_reduce(k, y, loc, H, P, 1, _hip.REDUCE_MEAN)
            _hip.indexer_fused(*args, seg_counters=counters, mode=mode)
        torch.cuda.synchronize()
        out[fused] = (_bits(y), _bits(qm), _bits(sc), _np(sp))
    assert (out[True][0] != _bits(y0)).any() or int(((loc + 1) % P == 0).sum()) == 0
    for a, b in zip(out[False], out[True]):
        np.testing.assert_array_equal(a, b)



@pytest.mark.parametrize("kernel", ["mean", "gqa", "quest"])
def test_fused_cmean_segment_listing_a_closed_page_many_times(gpu, kernel):
    """A malformed table whose one segment lists the page the launch closes
    300 times: the launch with the in-kernel page-finish reduction writes
    exactly what the separate reduction followed by the same kernel writes —
    every copy scored against the fresh centroid (or envelopes), none against
    a row being rewritten — for the q-mean, GQA and Quest kernels."""
    dev = gpu
    P, D, k, rows = 16, 128, 10, 64
    G = 2 if kernel == "mean" else 4
    c = 37  # the closed page's row (H = 1)
    n_mid = 300
    dind = torch.tensor([0, n_mid + 2], dtype=torch.int32, device=dev)
    sind = torch.tensor([0, k + 2], dtype=torch.int32, device=dev)
    didx = torch.tensor([5] + [c] * n_mid + [6], dtype=torch.int32, device=dev)
    loc = torch.tensor([c * P + P - 1], dtype=torch.int64, device=dev)
    q = W.randn_bf16((1, G, D), 1, dev)
    kpool = W.randn_bf16((rows, P, D), 3, dev)
    pools0 = [W.randn_bf16((rows, 1, D), 2 + i, dev, std=0.25) for i in range(2 if kernel == "quest" else 1)]
    table = (dind, sind, didx)

    def run(in_launch):
        pools = [t.clone() for t in pools0]
        sidx = torch.full((k + 2,), -1, dtype=torch.int32, device=dev)
        if kernel == "mean":
            outs = [torch.zeros((1, 1, D), device=dev, dtype=torch.bfloat16),
                    torch.full((n_mid + 2, 1, 1), -5.0, device=dev, dtype=torch.bfloat16)]
            if not in_launch:
                _hip.page_reduce(kpool, pools[0], loc, 1, P, 1, _hip.REDUCE_MEAN)
            _hip.indexer_fused(q, outs[0], pools[0], outs[1], *table[:2], didx, sidx, 1, k, 1, 1, n_mid + 2,
                               mode=_hip.FUSED_SEGMENT, cmean=(kpool, loc, 1) if in_launch else None)
        elif kernel == "gqa":
            outs = [torch.full((n_mid + 2, 1, G), -5.0, device=dev, dtype=torch.bfloat16),
                    torch.full((n_mid + 2, 1, 1), -5.0, device=dev, dtype=torch.bfloat16)]
            if not in_launch:
                _hip.page_reduce(kpool, pools[0], loc, 1, P, 1, _hip.REDUCE_MEAN)
            _hip.indexer_gqa_fused(q, pools[0], outs[0], outs[1], *table[:2], didx, sidx, 1, k, 1, 1, n_mid + 2,
                                   softmax_scale=0.09, cmean=(kpool, loc, 1) if in_launch else None)
        else:
            outs = [torch.full((n_mid + 2, G, 1), -5.0, device=dev, dtype=torch.bfloat16),
                    torch.full((n_mid + 2, 1, 1), -5.0, device=dev, dtype=torch.bfloat16)]
            if not in_launch:
                _hip.page_reduce_multi(kpool, pools, [_hip.REDUCE_MAX, _hip.REDUCE_MIN], loc, 1, P, 1)
            _hip.indexer_quest_fused(q, pools[0], pools[1], outs[0], outs[1], *table[:2], didx, sidx, 1, k, 1, 1,
                                     n_mid + 2, envelope=(kpool, loc, 1) if in_launch else None)
        torch.cuda.synchronize()
        return [_bits(t) for t in pools + outs] + [_np(sidx)]

    sep, fused = run(False), run(True)
    assert (sep[0] != _bits(pools0[0])).any(), "the reduction changed nothing"
    for a, b in zip(sep, fused):
        np.testing.assert_array_equal(a, b)
    assert (fused[-1][1:k + 1] == c).all()
    # every copy of the page carries one score, the fresh one
    score = (fused[-2] if kernel == "mean" else fused[-3]).reshape(n_mid + 2, -1)[1:n_mid + 1]
    assert (score == score[0]).all()


@pytest.mark.parametrize("name", ["c1", "c2", "eos0", "r3", "r9"])
def test_flow_cmean_carried_into_indexer_launch(gpu, name, monkeypatch):
    """forward_cache's CMean runs inside the next forward_indexer's fused
    launch (VORTEX_FUSE_CMEAN=1) with the same centroids, scores and block
    table as when it is launched on its own (=0)."""
    batch = _cmean_case(name)[0]
    seen = []
    real = _hip.indexer_fused
    monkeypatch.setattr(_hip, "indexer_fused", lambda *a, **k: (seen.append(k.get("cmean") is not None),
                                                                 real(*a, **k)))
    results = {}
    for carry in ("1", "0"):
        monkeypatch.setenv("VORTEX_FUSE_CMEAN", carry)
        run = _FlowRun(batch, gpu)
        seen.clear()
        run.step()
        torch.cuda.synchronize()
        with torch._C.DisableTorchFunctionSubclass():
            results[carry] = (_bits(run.cen), _np(run.ic.sparse_kv_indices), _bits(run.flow.gemv.output_buffer))
        assert seen == ([carry == "1"] if seen else [])
    np.testing.assert_array_equal(results["1"][0], results["0"][0])
    np.testing.assert_array_equal(results["1"][1], results["0"][1])
    # scores: the positions the GeMV covers (the planner's workloads)
    ref = O.plan_decode(_np(batch.seq_lens), _np(batch.req_to_token), _np(batch.req_indices), batch.page_size,
                        batch.num_kv_heads, batch.topk, batch.bos, batch.eos, batch.max_chunk)
    cov = np.zeros(results["1"][2].size, dtype=bool)
    for off, ln in zip(ref["winfo_off"], ref["winfo_len"]):
        cov[off:off + ln] = True
    np.testing.assert_array_equal(results["1"][2][cov], results["0"][2][cov])


def _c5_top64():
    b = W.c5()
    b.topk = 64  # 16 staged lists of 64: four entries per thread in the merge
    return b


@pytest.mark.parametrize("kind", ["random", "ties", "const"])
@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c5", "c5k64", "r0", "r3", "r5", "r9"])
def test_split_staged_preselect_equals_unstaged(gpu, name, kind):
    """The split layout with room for the staged pre-selection after the
    counters (every chunk workgroup stages its chunk's best k, the last one
    merges the lists) writes what it writes without that room — q-mean,
    scores and selection, bit for bit — on two calls in a row (the counters
    come back to zero, the staged lists are rewritten), and on tied scores
    the selection is the oracle's stable order."""
    dev = gpu
    batch = {"r0": lambda: W.random_small(0), "r3": lambda: W.random_small(3), "r5": lambda: W.random_small(5),
             "r9": lambda: W.random_small(9), "c5k64": _c5_top64}.get(name, getattr(W, name, None))()
    ic, _ = W.make_contexts(batch, dev)
    _plan(batch, ic, dev)
    H, G, D = batch.num_kv_heads, batch.group_size, batch.head_dim
    S = batch.batch * H
    rows = batch.pool_pages * H
    q = W.randn_bf16((S, G, D), 5, dev)
    if kind == "random":
        y = W.randn_bf16((rows, 1, D), 6, dev, std=0.25)
    else:
        base = W.randn_bf16((3, D), 6, dev, std=0.25)
        pick = (torch.zeros(rows, dtype=torch.long) if kind == "const"
                else torch.randint(0, 3, (rows,), generator=torch.Generator().manual_seed(7)))
        y = base[pick.to(dev)].view(rows, 1, D).contiguous()
    qin = q if G <= 16 else q.mean(dim=1, keepdim=True)
    out = {}
    for staged in (False, True):
        counters = torch.zeros(_hip.indexer_fused_workspace_len(S) if staged else S, dtype=torch.int32, device=dev)
        for _ in range(2):
            qm = torch.full((S, 1, D), 3.0, device=dev, dtype=torch.bfloat16)
            sc = torch.full((ic.dense_kv_indices.numel(), 1, 1), -5.0, device=dev, dtype=torch.bfloat16)
            sp = ic.sparse_kv_indices.clone()
            _hip.indexer_fused(qin, qm if G <= 16 else None, y, sc, ic.dense_kv_indptr, ic.sparse_kv_indptr,
                               ic.dense_kv_indices, sp, S, batch.topk, batch.bos, batch.eos,
                               batch.max_pages_per_request, seg_counters=counters, mode=_hip.FUSED_SPLIT)
            torch.cuda.synchronize()
            assert int(counters[:S].abs().sum()) == 0, "segment counters not reset"
        out[staged] = (_bits(qm), _bits(sc), _np(sp))
    for a, b in zip(out[False], out[True]):
        np.testing.assert_array_equal(a, b)
    if kind != "random":
        exp, _ = O.topk(out[True][1], _np(ic.dense_kv_indptr), _np(ic.sparse_kv_indptr),
                        _np(ic.dense_kv_indices), _np(ic.sparse_kv_indices), S, batch.topk, batch.bos, batch.eos)
        np.testing.assert_array_equal(out[True][2], exp)


def _split_case(batch, dev, seed):
    ic, _ = W.make_contexts(batch, dev)
    _plan(batch, ic, dev)
    H, G, D = batch.num_kv_heads, batch.group_size, batch.head_dim
    S = batch.batch * H
    q = W.randn_bf16((S, G, D), seed, dev)
    y = W.randn_bf16((batch.pool_pages * H, 1, D), seed + 1, dev, std=0.25)
    return ic, q, y, S


def _split_run(batch, case, workspace):
    ic, q, y, S = case
    D = batch.head_dim
    qm = torch.full((S, 1, D), 3.0, device=q.device, dtype=torch.bfloat16)
    sc = torch.full((ic.dense_kv_indices.numel(), 1, 1), -5.0, device=q.device, dtype=torch.bfloat16)
    sp = ic.sparse_kv_indices.clone()
    _hip.indexer_fused(q, qm, y, sc, ic.dense_kv_indptr, ic.sparse_kv_indptr, ic.dense_kv_indices, sp, S,
                       batch.topk, batch.bos, batch.eos, batch.max_pages_per_request, seg_counters=workspace,
                       mode=_hip.FUSED_SPLIT)
    torch.cuda.synchronize()
    return _bits(qm), _bits(sc), _np(sp)


def test_split_workspace_shared_by_batches_of_several_sizes(gpu):
    """One workspace serves a decode loop whose segment count changes from
    call to call (growing and shrinking, as SGLang's batches do): every call
    equals the same call on a fresh zeroed workspace and on a counters-only
    buffer (the unstaged path), bit for bit, and leaves the whole workspace
    (counters and staging zone) at zero, so that the MLA calls, whose
    selecting workgroups read the staged lists as they arrive, never meet a
    list an earlier call left behind."""
    dev = gpu
    cap = 512
    ws = torch.zeros(_hip.indexer_fused_workspace_len(cap), dtype=torch.int32, device=dev)
    small = W.make_batch([3000, 9000, 700], pool_pages=900, seed=51, num_kv_heads=2, group_size=2,
                         head_dim=128, topk=20, bos=1, eos=1)
    mid = W.make_batch([2500 + 97 * i for i in range(40)], pool_pages=12000, seed=52, num_kv_heads=8,
                       group_size=2, head_dim=128, topk=30, bos=1, eos=1)
    wide = W.make_batch([5000, 7000, 9000], pool_pages=2000, seed=53, num_kv_heads=1, group_size=16,
                        head_dim=576, topk=32, bos=1, eos=1)
    seq = [(W.c3(), 5), (small, 6), (W.c3(), 5), (mid, 7), (wide, 8), (small, 6), (mid, 7)]
    for i, (batch, seed) in enumerate(seq):
        case = _split_case(batch, dev, seed)
        S = case[3]
        assert S <= cap
        got = _split_run(batch, case, ws)
        assert int(ws[:cap].abs().sum()) == 0, f"call {i}: counters not back at zero"
        assert int(ws.abs().sum()) == 0, f"call {i}: staged lists left in the zone"
        fresh = _split_run(batch, case, torch.zeros_like(ws))
        plain = _split_run(batch, case, torch.zeros(S, dtype=torch.int32, device=dev))
        for a, b, c in zip(got, fresh, plain):
            np.testing.assert_array_equal(a, b)
            np.testing.assert_array_equal(a, c)
