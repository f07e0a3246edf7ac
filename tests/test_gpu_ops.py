"""GPU parity of the workload-walking indexer ops (GeMM, elementwise,
tile reductions, segment softmax / normalize) and of the GQA and Quest flows
run through the public API.

Each kernel is called through the C ABI on the planner's own block tables
(C1, C2, C5 and random small layouts) and compared with the oracle on the
same inputs: bit-exact for max / min / mul / add, relu / abs / add_mul and
the max / min reductions; within rtol 1e-2 / atol 1e-3 for the fp32
contractions and sums (GeMM, mean, sum, L2) and the exp-based ops (softmax,
sigmoid, SiLU; atol 1e-6 for softmax probabilities).  Positions outside the
workload list must keep their sentinel.  The flows' selections are
bit-exact against the oracle top-k of the GPU's own page scores.
"""
import numpy as np
import pytest
import torch

import workloads as W
from oracle import vortex_oracle as O
from vortex_torch import _hip
from vortex_torch.abs import FORMAT, as_vtensor

pytestmark = pytest.mark.gpu

SENTINEL = -7.0


def _np(t):
    return t.detach().cpu().numpy()


def _bits(t):
    with torch._C.DisableTorchFunctionSubclass():
        return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def _f(bits):
    return O.bf16_to_f32(bits)


def _planned(name, dev):
    from vortex_torch.indexer.utils_sglang import plan_decode

    batch = W.random_small(int(name[1:])) if name.startswith("r") else getattr(W, name)()
    ic, cc = W.make_contexts(batch, dev)
    b = batch.to(dev)
    plan_decode(b.seq_lens, b.req_to_token, b.req_indices, ic)
    return batch, ic, cc


def _winfo(ic):
    return (ic.winfo_q_indices, ic.winfo_kv_offsets, ic.winfo_kv_lens, ic.winfo_num_workloads)


def _owinfo(ic):
    return (_np(ic.winfo_q_indices), _np(ic.winfo_kv_offsets), _np(ic.winfo_kv_lens),
            int(ic.winfo_num_workloads.item()))


def _sentinel(shape, dev):
    return torch.full(shape, SENTINEL, device=dev, dtype=torch.bfloat16)


def _close(got_bits, exp_bits, covered, rtol=1e-2, atol=1e-3):
    got, exp = _f(got_bits), _f(exp_bits)
    np.testing.assert_allclose(got[covered], exp[covered], rtol=rtol, atol=atol)
    assert (got[~covered] == SENTINEL).all(), "a position outside the workload list was written"


LAYOUTS = ["c1", "c2", "c5", "r3", "r11"]


def test_bf16_rounding_matches_rne_for_every_input(gpu):
    """The kernels round fp32 to bf16 with gfx950's conversion instruction;
    every bit-exact claim against the oracle rests on it being the integer
    round-to-nearest-even of the oracle for all 2^32 inputs (NaN -> 0x7fc0)."""
    assert _hip.bf16_rounding_check(gpu) == (0, 0)


@pytest.mark.parametrize("name", LAYOUTS)
def test_gemm_bpr_matches_oracle(gpu, name):
    batch, ic, _ = _planned(name, gpu)
    H, G, D = batch.num_kv_heads, batch.group_size, batch.head_dim
    q = W.randn_bf16((batch.batch * H, G, D), 1, gpu)
    cen = W.randn_bf16((batch.pool_pages * H, 1, D), 2, gpu, std=0.25)
    o = _sentinel((ic.dense_kv_indices.numel(), 1, G), gpu)
    _hip.ragged_gemm(q, _hip.ROWS_BATCHED, cen, _hip.ROWS_PAGED, o, ic.dense_kv_indices, _winfo(ic))
    exp, cov = O.ragged_gemm(_bits(q), O.ROWS_BATCHED, _bits(cen), O.ROWS_PAGED, _bits(o), _np(ic.dense_kv_indices),
                             *_owinfo(ic))
    assert cov.any() or int(ic.winfo_num_workloads.item()) == 0
    _close(_bits(o), exp, cov)


@pytest.mark.parametrize("modes", [(_hip.ROWS_RAGGED, _hip.ROWS_RAGGED), (_hip.ROWS_RAGGED, _hip.ROWS_PAGED),
                                   (_hip.ROWS_BATCHED, _hip.ROWS_PAGED)])
@pytest.mark.parametrize("K", [64, 72, 128, 576])
def test_gemm_modes_and_tiles(gpu, modes, K):
    batch, ic, _ = _planned("r5", gpu)
    S, H = ic.dense_kv_indices.numel(), batch.num_kv_heads
    xm, ym = modes
    C, G = 2, 3
    x = W.randn_bf16((batch.batch * H if xm == _hip.ROWS_BATCHED else S, G, K), 3, gpu)
    y = W.randn_bf16((batch.pool_pages * H if ym == _hip.ROWS_PAGED else S, C, K), 4, gpu, std=0.5)
    o = _sentinel((S, C, G), gpu)
    _hip.ragged_gemm(x, xm, y, ym, o, ic.dense_kv_indices, _winfo(ic))
    exp, cov = O.ragged_gemm(_bits(x), xm, _bits(y), ym, _bits(o), _np(ic.dense_kv_indices), *_owinfo(ic))
    _close(_bits(o), exp, cov)


@pytest.mark.parametrize("op", [O.BINARY_MAXIMUM, O.BINARY_MINIMUM, O.BINARY_ADD, O.BINARY_MUL])
@pytest.mark.parametrize("case", ["bpr_quest", "rrr", "rpr_bcast", "rrr_scalar_cols"])
def test_binary_matches_oracle_bit_exact(gpu, op, case):
    batch, ic, _ = _planned("c1" if case == "bpr_quest" else "r7", gpu)
    S, H, G = ic.dense_kv_indices.numel(), batch.num_kv_heads, batch.group_size
    D = 128
    if case == "bpr_quest":  # Multiply(q, cache["max"]) of the Quest flow
        xm, ym, xs, ys, os_ = _hip.ROWS_BATCHED, _hip.ROWS_PAGED, (batch.batch * H, G, D), (batch.pool_pages * H, 1, D), (S, G, D)
    elif case == "rrr":
        xm, ym, xs, ys, os_ = _hip.ROWS_RAGGED, _hip.ROWS_RAGGED, (S, 3, 16), (S, 3, 16), (S, 3, 16)
    elif case == "rpr_bcast":
        xm, ym, xs, ys, os_ = _hip.ROWS_RAGGED, _hip.ROWS_PAGED, (S, 3, 1), (batch.pool_pages * H, 1, 16), (S, 3, 16)
    else:
        xm, ym, xs, ys, os_ = _hip.ROWS_RAGGED, _hip.ROWS_RAGGED, (S, 2, 3), (S, 1, 3), (S, 2, 3)
    x, y = W.randn_bf16(xs, 5, gpu), W.randn_bf16(ys, 6, gpu)
    o = _sentinel(os_, gpu)
    alpha, beta = 0.7, -1.3
    _hip.ragged_binary(op, alpha, beta, x, xm, y, ym, o, ic.dense_kv_indices, _winfo(ic))
    exp, cov = O.ragged_binary(op, alpha, beta, _bits(x), xm, _bits(y), ym, _bits(o), _np(ic.dense_kv_indices),
                               *_owinfo(ic))
    np.testing.assert_array_equal(_bits(o), exp)


@pytest.mark.parametrize("op", [O.UNARY_RELU, O.UNARY_SIGMOID, O.UNARY_SILU, O.UNARY_ABS, O.UNARY_ADD_MUL])
@pytest.mark.parametrize("tile", [(2, 16), (3, 5)])
def test_unary_matches_oracle(gpu, op, tile):
    batch, ic, _ = _planned("r9", gpu)
    S = ic.dense_kv_indices.numel()
    x = W.randn_bf16((S,) + tile, 7, gpu, std=3.0)
    o = _sentinel((S,) + tile, gpu)
    _hip.ragged_unary(op, 0.3, -0.8, x, o, _winfo(ic))
    _, woff, wlen, nw = _owinfo(ic)
    exp, cov = O.ragged_unary(op, 0.3, -0.8, _bits(x), _bits(o), woff, wlen, nw)
    if op in (O.UNARY_SIGMOID, O.UNARY_SILU):
        _close(_bits(o), exp, cov)
    else:
        np.testing.assert_array_equal(_bits(o), exp)


@pytest.mark.parametrize("rtype", [O.MEAN, O.MAX, O.MIN, O.L2NORM, O.REDUCE_SUM])
@pytest.mark.parametrize("dim", [1, 2])
@pytest.mark.parametrize("tile", [(1, 2), (2, 128), (3, 5)])
def test_reduce_matches_oracle(gpu, rtype, dim, tile):
    batch, ic, _ = _planned("c2" if tile == (1, 2) else "r4", gpu)
    S = ic.dense_kv_indices.numel()
    x = W.randn_bf16((S,) + tile, 8, gpu)
    oshape = (S, 1, tile[1]) if dim == 1 else (S, tile[0], 1)
    o = _sentinel(oshape, gpu)
    _hip.ragged_reduce(x, o, dim, rtype, _winfo(ic))
    _, woff, wlen, nw = _owinfo(ic)
    exp, cov = O.ragged_reduce(_bits(x), _bits(o), dim, rtype, woff, wlen, nw)
    if rtype in (O.MAX, O.MIN):
        np.testing.assert_array_equal(_bits(o), exp)
    else:
        _close(_bits(o), exp, cov)


@pytest.mark.parametrize("op", [O.SEGMENT_SOFTMAX, O.SEGMENT_NORMALIZE])
@pytest.mark.parametrize("name,cols", [("c1", 2), ("c2", 2), ("c5", 16), ("r6", 3), ("r6", 300)])
def test_segment_scan_matches_oracle(gpu, op, name, cols):
    batch, ic, _ = _planned(name, gpu)
    S = ic.dense_kv_indices.numel()
    E = batch.batch * batch.num_kv_heads
    x = W.randn_bf16((S, 1, cols), 9, gpu, std=4.0)
    before = _bits(x).copy()
    _hip.segment_scan(op, 0.09, x, ic.dense_kv_indptr, E, batch.topk, batch.bos, batch.eos)
    exp, touched = O.segment_scan(op, 0.09, before, _np(ic.dense_kv_indptr), E, batch.topk, batch.bos, batch.eos)
    got = _bits(x)
    np.testing.assert_array_equal(got[~touched], before[~touched])
    np.testing.assert_allclose(_f(got[touched]), _f(exp[touched]), rtol=1e-2,
                               atol=1e-6 if op == O.SEGMENT_SOFTMAX else 1e-3)


# ----------------------------------------------------------------- flows
class _Flow:
    """One layer of a registered flow on `batch`, through the public API."""

    def __init__(self, flow_name, batch, dev, seed=0):
        from vortex_torch import flow as vflow

        self.batch, self.dev = batch, dev
        self.ic, self.cc = W.make_contexts(batch, dev)
        H, G, D, P = batch.num_kv_heads, batch.group_size, batch.head_dim, batch.page_size
        self.flow = vflow.build_vflow(flow_name)
        rows = batch.pool_pages * H
        self.k = W.randn_bf16((rows, P, D), seed, dev)
        self.cache = {"k": as_vtensor(self.k, FORMAT.PAGED)}
        for name, (r, c) in self.flow.create_cache(P, D).items():
            self.cache[name] = as_vtensor(W.randn_bf16((rows, r, c), seed + 1 + len(self.cache), dev, std=0.25),
                                          FORMAT.PAGED)
        self.q = as_vtensor(W.randn_bf16((batch.batch * H, G, D), seed + 9, dev), FORMAT.BATCHED)
        self.o = as_vtensor(self.ic.sparse_kv_indices.view(-1, 1, 1), FORMAT.RAGGED)
        self.loc = W.decode_loc(batch).to(dev)
        self.dev_batch = batch.to(dev)
        self.ic.profile()
        self.cc.profile()
        self.flow.forward_cache(self.cache, self.loc, self.cc)
        self.flow.forward_indexer(self.q, self.o, self.cache, self.ic)
        self.ic.execute()
        self.cc.execute()
        # every op's output buffer starts as a finite sentinel, so positions no
        # workload covers hold defined values when they reach the oracle
        with torch._C.DisableTorchFunctionSubclass():
            for op in vars(self.flow).values():
                buf = getattr(op, "output_buffer", None)
                if isinstance(buf, torch.Tensor):
                    buf.fill_(-7.0 if buf.is_floating_point() else -7)

    def step(self):
        from vortex_torch.indexer.utils_sglang import plan_decode

        b = self.dev_batch
        plan_decode(b.seq_lens, b.req_to_token, b.req_indices, self.ic)
        self.flow.forward_cache(self.cache, self.loc, self.cc)
        self.flow.forward_indexer(self.q, self.o, self.cache, self.ic)


def _check_selection(run, page_score_bits):
    ic, b = run.ic, run.batch
    sel, _ = O.topk(page_score_bits.reshape(-1), _np(ic.dense_kv_indptr), _np(ic.sparse_kv_indptr),
                    _np(ic.dense_kv_indices), _np(ic.sparse_kv_indices), b.batch * b.num_kv_heads, b.topk, b.bos,
                    b.eos)
    np.testing.assert_array_equal(_np(ic.sparse_kv_indices), sel)


@pytest.mark.parametrize("name", ["c1", "c2", "r3"])
def test_gqa_block_sparse_flow(gpu, name):
    batch = W.random_small(3) if name == "r3" else getattr(W, name)()
    run = _Flow("gqa_block_sparse_attention", batch, gpu)
    run.step()
    torch.cuda.synchronize()
    f, ic = run.flow, run.ic
    cov = np.zeros(ic.dense_kv_indices.numel(), bool)
    p, _ = O.workload_positions(*_owinfo(ic))
    cov[p] = True
    # stage by stage on the GPU's own intermediates: GeMM, softmax, max over G
    raw, _ = O.ragged_gemm(_bits(run.q), O.ROWS_BATCHED, _bits(run.cache["centroids"]), O.ROWS_PAGED,
                           np.zeros(tuple(f.gemm.output_buffer.shape), np.uint16), _np(ic.dense_kv_indices),
                           *_owinfo(ic))
    sm = _bits(f.gemm.output_buffer)  # softmax ran in place on the GeMM output
    exp_sm, touched = O.segment_scan(O.SEGMENT_SOFTMAX, 0.09, raw, _np(ic.dense_kv_indptr),
                                     batch.batch * batch.num_kv_heads, batch.topk, batch.bos, batch.eos)
    np.testing.assert_allclose(_f(sm[touched]), _f(exp_sm[touched]), rtol=2e-2, atol=1e-5)
    aggr = _bits(f.max_op.output_buffer)
    exp_aggr, _ = O.ragged_reduce(sm, aggr, 2, O.MAX, *_owinfo(ic)[1:])
    np.testing.assert_array_equal(aggr[cov], exp_aggr[cov])
    _check_selection(run, aggr)


@pytest.mark.parametrize("name", ["c1", "c2", "r3"])
def test_gqa_quest_flow(gpu, monkeypatch, name):
    # stage by stage: every op launched on its own writes its output buffer
    monkeypatch.setenv("VORTEX_FUSE", "0")
    batch = W.random_small(3) if name == "r3" else getattr(W, name)()
    run = _Flow("gqa_quest_sparse_attention", batch, gpu)
    run.step()
    torch.cuda.synchronize()
    f, ic = run.flow, run.ic
    # the envelopes the cache side wrote for the closed pages
    cmax, rows = O.page_reduce(_bits(run.k), np.zeros_like(_bits(run.cache["max"])), _np(run.loc),
                               batch.num_kv_heads, batch.page_size, 1, O.MAX)
    np.testing.assert_array_equal(_bits(run.cache["max"])[rows], cmax[rows])
    dense, wi = _np(ic.dense_kv_indices), _owinfo(ic)
    s_max, cov = O.ragged_binary(O.BINARY_MUL, 1.0, 1.0, _bits(run.q), O.ROWS_BATCHED, _bits(run.cache["max"]),
                                 O.ROWS_PAGED, _bits(f.mul_max.output_buffer), dense, *wi)
    np.testing.assert_array_equal(_bits(f.mul_max.output_buffer), s_max)
    s = _bits(f.maximum_op.output_buffer)
    exp_s, _ = O.ragged_binary(O.BINARY_MAXIMUM, 1.0, 1.0, _bits(f.mul_max.output_buffer), O.ROWS_RAGGED,
                               _bits(f.mul_min.output_buffer), O.ROWS_RAGGED, s, dense, *wi)
    np.testing.assert_array_equal(s, exp_s)
    score = _bits(f.sum.output_buffer)
    exp_score, _ = O.ragged_reduce(s, score, 2, O.REDUCE_SUM, *wi[1:])
    np.testing.assert_allclose(_f(score[cov]), _f(exp_score[cov]), rtol=1e-2, atol=1e-3)
    aggr = _bits(f.max_op.output_buffer)
    exp_aggr, _ = O.ragged_reduce(score, aggr, 1, O.MAX, *wi[1:])
    np.testing.assert_array_equal(aggr[cov], exp_aggr[cov])
    _check_selection(run, aggr)


@pytest.mark.parametrize("flow_name", ["gqa_block_sparse_attention", "gqa_quest_sparse_attention"])
def test_flow_graph_replay_matches_eager(gpu, flow_name):
    run = _Flow(flow_name, W.c2(), gpu)
    run.step()
    torch.cuda.synchronize()
    eager = run.ic.sparse_kv_indices.clone()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run.step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        run.step()
    for _ in range(4):
        run.ic.sparse_kv_indices.fill_(-1)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(run.ic.sparse_kv_indices, eager)


# ------------------------------------------------------- fused GQA indexer
def _gqa_max_flow():
    """GeMM -> Max(dim=2) -> topK without the softmax (registered once)."""
    from vortex_torch.cache import Mean as CMean
    from vortex_torch.flow import registry, vFlow
    from vortex_torch.indexer import GeMM, Max, topK

    name = "test_gqa_max_only"
    if not registry.has(name):
        @registry.register(name)
        class _GqaMax(vFlow):
            def __init__(self):
                super().__init__()
                self.gemm, self.max_op, self.output_func = GeMM(), Max(dim=2), topK()
                self.reduction = CMean(dim=1)

            def forward_indexer(self, q, o, cache, ctx):
                self.output_func(self.max_op(self.gemm(q, cache["centroids"], ctx=ctx), ctx=ctx), o, ctx=ctx)

            def forward_cache(self, cache, loc, ctx):
                self.reduction(cache["k"], cache["centroids"], loc=loc, ctx=ctx)

            def create_cache(self, page_size, head_dim):
                return {"centroids": (1, head_dim)}
    return name


def _gqa_case(name):
    if name.startswith("r"):
        return W.random_small(int(name[1:]))
    if name == "g8d64":  # eight query heads per kv head, head_dim 64
        return W.make_batch([3000, 700, 5000, 40], pool_pages=600, seed=11, num_kv_heads=2, group_size=8,
                            head_dim=64, topk=17, bos=2, eos=1)
    if name == "g4d256":
        return W.make_batch([2500, 4000], pool_pages=500, seed=12, num_kv_heads=3, group_size=4, head_dim=256,
                            topk=40, bos=1, eos=0)
    if name == "staged":  # 5998 middle pages, topk 4096: scores staged in global memory, not LDS
        return W.make_batch([6000, 4500], pool_pages=10600, seed=13, page_size=1, num_kv_heads=1, group_size=8,
                            head_dim=128, topk=4096, bos=1, eos=1, max_chunk=512, min_chunk=64)
    return getattr(W, name)()


@pytest.mark.parametrize("flow", ["softmax", "max_only"])
@pytest.mark.parametrize("name", ["c1", "c2", "r3", "r5", "r8", "g8d64", "g4d256", "staged"])
def test_gqa_fused_equals_unfused(gpu, monkeypatch, flow, name):
    """The fused GQA kernel writes the same bits as GeMM, Softmax, Max and
    topK launched one by one: block table, scores (after the softmax) and
    the maximum over the query heads, at every position the ops cover."""
    flow_name = "gqa_block_sparse_attention" if flow == "softmax" else _gqa_max_flow()
    batch = _gqa_case(name)
    calls = []
    real = _hip.indexer_gqa_fused
    monkeypatch.setattr(_hip, "indexer_gqa_fused", lambda *a, **k: (calls.append(1), real(*a, **k)))
    out = {}
    for fuse in ("1", "0"):
        monkeypatch.setenv("VORTEX_FUSE", fuse)
        run = _Flow(flow_name, batch, gpu)
        n0 = len(calls)
        run.ic.sparse_kv_indices.fill_(-1)
        run.step()
        torch.cuda.synchronize()
        out[fuse] = (_np(run.ic.sparse_kv_indices), _bits(run.flow.gemm.output_buffer),
                     _bits(run.flow.max_op.output_buffer), len(calls) - n0)
        ic = run.ic
    assert out["1"][3] == 1 and out["0"][3] == 0, "fused kernel not (only) taken under VORTEX_FUSE=1"
    cov = np.zeros(ic.dense_kv_indices.numel(), bool)
    p, _ = O.workload_positions(*_owinfo(ic))
    cov[p] = True
    G = batch.group_size
    np.testing.assert_array_equal(out["1"][0], out["0"][0])
    np.testing.assert_array_equal(out["1"][1].reshape(-1, G)[cov], out["0"][1].reshape(-1, G)[cov])
    np.testing.assert_array_equal(out["1"][2].reshape(-1)[cov], out["0"][2].reshape(-1)[cov])
    if cov.any():
        assert out["1"][2].reshape(-1)[cov].any()


def test_gqa_fused_graph_replay(gpu, monkeypatch):
    monkeypatch.setenv("VORTEX_FUSE", "1")
    run = _Flow("gqa_block_sparse_attention", _gqa_case("g8d64"), gpu)
    run.step()
    torch.cuda.synchronize()
    eager = (run.ic.sparse_kv_indices.clone(), run.flow.max_op.output_buffer.clone())
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run.step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run.step()
    for _ in range(3):
        run.ic.sparse_kv_indices.fill_(-1)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(run.ic.sparse_kv_indices, eager[0])
        assert torch.equal(run.flow.max_op.output_buffer, eager[1])


def _quest_keep_flow():
    """The Quest flow that keeps the elementwise maximum alive past forward_indexer."""
    from vortex_torch.flow import algorithms, registry

    name = "test_quest_keep"
    if not registry.has(name):
        @registry.register(name)
        class _QuestKeep(algorithms.GQAQuestSparseAttention):
            def forward_indexer(self, q, o, cache, ctx):
                s_max = self.mul_max(q, cache["max"], ctx=ctx)
                s_min = self.mul_min(q, cache["min"], ctx=ctx)
                self.kept = self.maximum_op(s_max, s_min, ctx=ctx)
                self.output_func(self.max_op(self.sum(self.kept, ctx=ctx), ctx=ctx), o, ctx=ctx)
    return name


@pytest.mark.parametrize("name", ["c1", "c2", "r3", "r5", "r8", "g8d64", "g4d256", "staged"])
def test_quest_fused_equals_unfused(gpu, monkeypatch, name):
    """The fused Quest kernel writes the same block table, row sums and page
    maxima as the five separate launches; the unread [pages, G, D]
    intermediates are not written."""
    batch = _gqa_case(name)
    calls = []
    real = _hip.indexer_quest_fused
    monkeypatch.setattr(_hip, "indexer_quest_fused", lambda *a, **k: (calls.append(1), real(*a, **k)))
    out = {}
    for fuse in ("1", "0"):
        monkeypatch.setenv("VORTEX_FUSE", fuse)
        run = _Flow("gqa_quest_sparse_attention", batch, gpu)
        n0 = len(calls)
        run.ic.sparse_kv_indices.fill_(-1)
        run.flow.mul_max.output_buffer.fill_(SENTINEL)
        run.step()
        torch.cuda.synchronize()
        out[fuse] = (_np(run.ic.sparse_kv_indices), _bits(run.flow.sum.output_buffer),
                     _bits(run.flow.max_op.output_buffer), len(calls) - n0, _bits(run.flow.mul_max.output_buffer),
                     _bits(run.cache["max"]), _bits(run.cache["min"]))
        ic = run.ic
    # forward_cache: CMax + CMin as one pass (fused) equal the two launches
    np.testing.assert_array_equal(out["1"][5], out["0"][5])
    np.testing.assert_array_equal(out["1"][6], out["0"][6])
    assert out["1"][3] == 1 and out["0"][3] == 0, "fused kernel not (only) taken under VORTEX_FUSE=1"
    cov = np.zeros(ic.dense_kv_indices.numel(), bool)
    p, _ = O.workload_positions(*_owinfo(ic))
    cov[p] = True
    G = batch.group_size
    np.testing.assert_array_equal(out["1"][0], out["0"][0])
    np.testing.assert_array_equal(out["1"][1].reshape(-1, G)[cov], out["0"][1].reshape(-1, G)[cov])
    np.testing.assert_array_equal(out["1"][2].reshape(-1)[cov], out["0"][2].reshape(-1)[cov])
    sentinel = _bits(_sentinel((1,), gpu))[0]
    assert (out["1"][4] == sentinel).all(), "an elided product was written"
    if cov.any():
        assert (out["0"][4].reshape(-1, G * batch.head_dim)[cov] != sentinel).any()


def test_quest_fused_keeps_observed_intermediates(gpu, monkeypatch):
    """An intermediate still referenced after forward_indexer is computed."""
    batch = W.c1()
    got = {}
    for fuse in ("1", "0"):
        monkeypatch.setenv("VORTEX_FUSE", fuse)
        run = _Flow(_quest_keep_flow(), batch, gpu)
        run.flow.maximum_op.output_buffer.fill_(SENTINEL)
        run.step()
        torch.cuda.synchronize()
        got[fuse] = (_bits(run.flow.maximum_op.output_buffer), _np(run.ic.sparse_kv_indices))
    np.testing.assert_array_equal(got["1"][1], got["0"][1])
    np.testing.assert_array_equal(got["1"][0], got["0"][0])


@pytest.mark.parametrize("softmax", [True, False])
@pytest.mark.parametrize("name", ["c1", "c2", "eos0", "mid", "d64", "big_loc", "d256", "r3", "r9"])
def test_gqa_fused_cmean_equals_separate_launches(gpu, name, softmax):
    """vtx_indexer_gqa_fused_cmean writes what vtx_page_reduce then
    vtx_indexer_gqa_fused write: centroids, scores, maxima, block table."""
    batch, loc = W.cmean_case(name)
    loc = loc.to(gpu)
    ic, _ = W.make_contexts(batch, gpu)
    from vortex_torch.indexer.utils_sglang import plan_decode
    b = batch.to(gpu)
    plan_decode(b.seq_lens, b.req_to_token, b.req_indices, ic)
    H, G, D, P = batch.num_kv_heads, batch.group_size, batch.head_dim, batch.page_size
    S, rows, n = batch.batch * H, batch.pool_pages * H, ic.dense_kv_indices.numel()
    q = W.randn_bf16((S, G, D), 1, gpu)
    k = W.randn_bf16((rows, P, D), 3, gpu)
    y0 = W.randn_bf16((rows, 1, D), 2, gpu, std=0.25)
    out = {}
    for fused in (False, True):
        y = y0.clone()
        sc = _sentinel((n, 1, G), gpu)
        ag = _sentinel((n, 1, 1), gpu)
        sp = ic.sparse_kv_indices.clone()
        args = (q, y, sc, ag, ic.dense_kv_indptr, ic.sparse_kv_indptr, ic.dense_kv_indices, sp, S, batch.topk,
                batch.bos, batch.eos, batch.max_pages_per_request)
        scale = 0.09 if softmax else None
        if fused:
            _hip.indexer_gqa_fused(*args, softmax_scale=scale, cmean=(k, loc, H))
        else:
            _hip.page_reduce(k, y, loc, H, P, 1, _hip.REDUCE_MEAN)
            _hip.indexer_gqa_fused(*args, softmax_scale=scale)
        torch.cuda.synchronize()
        out[fused] = (_bits(y), _bits(sc), _bits(ag), _np(sp))
    for a, b in zip(out[False], out[True]):
        np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("name", ["c1", "c2", "eos0", "mid", "d64", "big_loc", "d256", "r3", "r9"])
def test_quest_fused_envelope_equals_separate_launches(gpu, name):
    """vtx_indexer_quest_fused_cmean writes what vtx_page_reduce_multi (CMax,
    CMin) then vtx_indexer_quest_fused write: envelopes, row sums, page
    maxima, block table."""
    batch, loc = W.cmean_case(name)
    loc = loc.to(gpu)
    ic, _ = W.make_contexts(batch, gpu)
    from vortex_torch.indexer.utils_sglang import plan_decode
    b = batch.to(gpu)
    plan_decode(b.seq_lens, b.req_to_token, b.req_indices, ic)
    H, G, D, P = batch.num_kv_heads, batch.group_size, batch.head_dim, batch.page_size
    S, rows, n = batch.batch * H, batch.pool_pages * H, ic.dense_kv_indices.numel()
    q = W.randn_bf16((S, G, D), 1, gpu)
    k = W.randn_bf16((rows, P, D), 3, gpu)
    mx0 = W.randn_bf16((rows, 1, D), 2, gpu, std=0.25)
    mn0 = W.randn_bf16((rows, 1, D), 4, gpu, std=0.25)
    out = {}
    for fused in (False, True):
        mx, mn = mx0.clone(), mn0.clone()
        sc = _sentinel((n, G, 1), gpu)
        ag = _sentinel((n, 1, 1), gpu)
        sp = ic.sparse_kv_indices.clone()
        args = (q, mx, mn, sc, ag, ic.dense_kv_indptr, ic.sparse_kv_indptr, ic.dense_kv_indices, sp, S,
                batch.topk, batch.bos, batch.eos, batch.max_pages_per_request)
        if fused:
            _hip.indexer_quest_fused(*args, envelope=(k, loc, H))
        else:
            _hip.page_reduce_multi(k, [mx, mn], [_hip.REDUCE_MAX, _hip.REDUCE_MIN], loc, H, P, 1)
            _hip.indexer_quest_fused(*args)
        torch.cuda.synchronize()
        out[fused] = (_bits(mx), _bits(mn), _bits(sc), _bits(ag), _np(sp))
    for a, b in zip(out[False], out[True]):
        np.testing.assert_array_equal(a, b)


def test_gqa_fused_rejects_bad_arguments(gpu):
    batch = W.c1()
    ic, _ = W.make_contexts(batch, gpu)
    q = torch.zeros((8, 2, 128), dtype=torch.bfloat16, device=gpu)
    y = torch.zeros((64, 1, 128), dtype=torch.bfloat16, device=gpu)
    score = torch.zeros((64, 1, 2), dtype=torch.bfloat16, device=gpu)
    aggr = torch.zeros((64, 1, 1), dtype=torch.bfloat16, device=gpu)
    args = (ic.dense_kv_indptr, ic.sparse_kv_indptr, ic.dense_kv_indices, ic.sparse_kv_indices)
    with pytest.raises(RuntimeError, match="head_dim"):
        _hip.indexer_gqa_fused(q[..., :100].contiguous(), y[..., :100].contiguous(), score, aggr, *args,
                               8, 30, 1, 1, 256)
    with pytest.raises(RuntimeError, match="query rows"):
        _hip.indexer_gqa_fused(q[:3], y, score, aggr, *args, 8, 30, 1, 1, 256)
    with pytest.raises(RuntimeError, match="topk_val"):
        _hip.indexer_gqa_fused(q, y, score, aggr, *args, 8, 5000, 1, 1, 256)
    assert not _hip.indexer_gqa_fused_supported(128, 9)


@pytest.mark.parametrize("dtype,D",[(torch.bfloat16, 128), (torch.float32, 128), (torch.bfloat16, 100),
                                     (torch.bfloat16, 3), (torch.bfloat16, 576)])
@pytest.mark.parametrize("kind", ["decode", "prefill"])
def test_set_kv_buffer_matches_oracle(gpu, dtype, D, kind):
    from vortex_torch.cache import set_kv_buffer_launcher

    P, H, pages = 16, 8 if D != 576 else 1, 300
    g = torch.Generator().manual_seed(5)
    k = torch.randn((pages * H, P, D), generator=g).to(dtype)
    v = torch.randn((pages * H, P, D), generator=g).to(dtype)
    if kind == "decode":
        loc = torch.randperm(pages * P, generator=g)[:64].to(torch.int64)
    else:  # every slot of 40 pages, shuffled, plus two tokens outside the pool
        pg = torch.randperm(pages, generator=g)[:40]
        loc = (pg[:, None] * P + torch.arange(P)).reshape(-1)
        loc = torch.cat([loc[torch.randperm(loc.numel(), generator=g)], torch.tensor([-3, pages * P + 1])])
    nk = torch.randn((loc.numel(), H, D), generator=g).to(dtype)
    nv = torch.randn((loc.numel(), H, D), generator=g).to(dtype)
    bits = (lambda t: t.view(torch.int16).numpy()) if dtype == torch.bfloat16 else (lambda t: t.view(torch.int32).numpy())
    ek, ev = O.set_kv_buffer(bits(k), bits(v), bits(nk), bits(nv), loc.numpy(), P)
    kd, vd = k.to(gpu), v.to(gpu)
    set_kv_buffer_launcher(kd, vd, nk.to(gpu), nv.to(gpu), loc.to(gpu), P)
    np.testing.assert_array_equal(bits(kd.cpu()), ek)
    np.testing.assert_array_equal(bits(vd.cpu()), ev)


def test_set_kv_then_cmean(gpu):
    """Decode step on the cache side: the new tokens go into the pool, then
    CMean of the pages they close equals the oracle's mean of the new pool."""
    from vortex_torch.cache import Mean as CMean, set_kv_buffer_launcher

    batch = W.c2()
    ic, cc = W.make_contexts(batch, gpu)
    H, D, P = batch.num_kv_heads, batch.head_dim, batch.page_size
    k = W.randn_bf16((batch.pool_pages * H, P, D), 1, gpu)
    v = torch.zeros_like(k)
    loc = W.decode_loc(batch).to(gpu)
    nk = W.randn_bf16((loc.numel(), H, D), 2, gpu)
    set_kv_buffer_launcher(k, v, nk, nk, loc, P)
    cen = torch.zeros((batch.pool_pages * H, 1, D), device=gpu, dtype=torch.bfloat16)
    op = CMean(dim=1)
    cc.profile()
    op(as_vtensor(k, FORMAT.PAGED), as_vtensor(cen, FORMAT.PAGED), loc=loc, ctx=cc)
    cc.execute()
    op(as_vtensor(k, FORMAT.PAGED), as_vtensor(cen, FORMAT.PAGED), loc=loc, ctx=cc)
    torch.cuda.synchronize()
    exp, rows = O.page_reduce(_bits(k), np.zeros_like(_bits(cen)), _np(loc), H, P, 1, O.MEAN)
    assert rows.size > 0
    np.testing.assert_allclose(_f(_bits(cen)[rows]), _f(exp[rows]), rtol=1e-2, atol=1e-3)
    # the written slots hold the new tokens
    pos = _np(loc)
    for i in range(0, loc.numel(), 9):
        for h in (0, H - 1):
            got = k[(int(pos[i]) // P) * H + h, int(pos[i]) % P]
            assert torch.equal(got, nk[i, h])


@pytest.mark.parametrize("name", ["c1", "c2", "c5", "r1", "r2", "r8", "r13"])
def test_plan_decode_fa3_matches_oracle(gpu, name):
    """FA3 planner through utils_sglang.plan_decode_fa3: every output bit-exact
    against the oracle; table entries the planner does not write keep their
    sentinel; kv_last_page_len is not an output."""
    from vortex_torch.indexer.utils_sglang import plan_decode_fa3

    batch = W.random_small(int(name[1:])) if name.startswith("r") else getattr(W, name)()
    ic, _ = W.make_contexts(batch, gpu)
    ic.kv_last_page_len.fill_(-9)
    S = max(1, batch.batch * batch.num_kv_heads)
    stride = batch.max_pages_per_request
    i32 = dict(dtype=torch.int32, device=gpu)
    dpt, spt = torch.full((S, stride), -5, **i32), torch.full((S, stride), -5, **i32)
    dcs, scs = torch.full((S,), -5, **i32), torch.full((S,), -5, **i32)
    b = batch.to(gpu)
    plan_decode_fa3(b.seq_lens, b.req_to_token, b.req_indices, dpt, dcs, spt, scs, ic)
    ref = O.plan_decode_fa3(batch.seq_lens.numpy(), batch.req_to_token.numpy(), batch.req_indices.numpy(),
                            batch.page_size, batch.num_kv_heads, batch.topk, batch.bos, batch.eos, batch.max_chunk,
                            stride)
    n = batch.batch * batch.num_kv_heads
    np.testing.assert_array_equal(_np(ic.dense_kv_indptr)[:n + 1], ref["dense_indptr"])
    np.testing.assert_array_equal(_np(ic.sparse_kv_indptr)[:n + 1], ref["sparse_indptr"])
    nd = ref["dense_indices"].size
    np.testing.assert_array_equal(_np(ic.dense_kv_indices)[:nd], ref["dense_indices"])
    w = ref["sparse_written"]
    np.testing.assert_array_equal(_np(ic.sparse_kv_indices)[:w.size][w], ref["sparse_indices"][w])
    nw = ref["num_workloads"]
    assert int(ic.winfo_num_workloads.item()) == nw
    np.testing.assert_array_equal(_np(ic.winfo_kv_offsets)[:nw], ref["winfo_off"])
    np.testing.assert_array_equal(_np(ic.winfo_kv_lens)[:nw], ref["winfo_len"])
    np.testing.assert_array_equal(_np(ic.winfo_q_indices)[:nw], ref["winfo_q"])
    if n:
        np.testing.assert_array_equal(_np(dcs)[:n], ref["dense_cache_seqlens"])
        np.testing.assert_array_equal(_np(scs)[:n], ref["sparse_cache_seqlens"])
        for got, exp, wm in ((dpt, ref["dense_page_table"], ref["dense_pt_written"]),
                             (spt, ref["sparse_page_table"], ref["sparse_pt_written"])):
            g = _np(got)[:n]
            np.testing.assert_array_equal(g[wm], exp[wm])
            assert (g[~wm] == -5).all()
    assert (_np(ic.kv_last_page_len) == -9).all()


def _attn_inputs(batch, dev, G, D, seed):
    H, P = batch.num_kv_heads, batch.page_size
    k = W.randn_bf16((batch.pool_pages * H, P, D), seed, dev)
    v = W.randn_bf16((batch.pool_pages * H, P, D), seed + 1, dev)
    q = W.randn_bf16((batch.batch * H * G, D), seed + 2, dev)
    return q, k, v


@pytest.mark.parametrize("table", ["dense", "sparse"])
@pytest.mark.parametrize("name", ["c1", "c2", "r1", "r2", "r6", "r13"])
def test_decode_attention_matches_oracle(gpu, name, table):
    from vortex_torch.decode_attention import dense_decode_attention, sparse_decode_attention

    batch, ic, _ = _planned(name, gpu)
    G, D = 2, 128
    q, k, v = _attn_inputs(batch, gpu, G, D, 3)
    if table == "sparse":  # select with topK on random scores first
        S = batch.batch * batch.num_kv_heads
        sc = W.randn_bf16((ic.dense_kv_indices.numel(), 1, 1), 4, gpu)
        _hip.topk_select(sc, ic.dense_kv_indptr, ic.sparse_kv_indptr, ic.dense_kv_indices, ic.sparse_kv_indices,
                         S, batch.topk, batch.bos, batch.eos, batch.max_pages_per_request)
        o = sparse_decode_attention(q, k, v, ic)
        ip, idx = ic.sparse_kv_indptr, ic.sparse_kv_indices
    else:
        o = dense_decode_attention(q, k, v, ic)
        ip, idx = ic.dense_kv_indptr, ic.dense_kv_indices
    exp = O.paged_decode_attention(_bits(q), _bits(k), _bits(v), _np(ip), _np(idx), _np(ic.kv_last_page_len),
                                   batch.batch, batch.num_kv_heads, 1.0 / np.sqrt(D))
    np.testing.assert_allclose(_f(_bits(o)), _f(exp), rtol=1e-2, atol=1e-3)


@pytest.mark.parametrize("D,G", [(64, 1), (64, 8), (128, 3), (128, 8), (256, 2), (256, 5)])
def test_decode_attention_head_shapes(gpu, D, G):
    from vortex_torch.decode_attention import dense_decode_attention

    batch, ic, _ = _planned("r4", gpu)
    q, k, v = _attn_inputs(batch, gpu, G, D, 7)
    o = dense_decode_attention(q, k, v, ic, sm_scale=0.05)
    exp = O.paged_decode_attention(_bits(q), _bits(k), _bits(v), _np(ic.dense_kv_indptr), _np(ic.dense_kv_indices),
                                   _np(ic.kv_last_page_len), batch.batch, batch.num_kv_heads, 0.05)
    np.testing.assert_allclose(_f(_bits(o)), _f(exp), rtol=1e-2, atol=1e-3)


@pytest.mark.parametrize("G", [1, 2, 4])
def test_decode_attention_long_segment(gpu, G):
    """Segments of more pages than the kernel stages in LDS (2048) read their
    page rows from the table; a short and an empty request beside them."""
    from vortex_torch.decode_attention import dense_decode_attention
    from vortex_torch.indexer.utils_sglang import plan_decode

    batch = W.make_batch([33600, 700, 0], pool_pages=2600, seed=31, num_kv_heads=2)
    ic, _ = W.make_contexts(batch, gpu)
    b = batch.to(gpu)
    plan_decode(b.seq_lens, b.req_to_token, b.req_indices, ic)
    assert int(ic.dense_kv_indptr[1]) - int(ic.dense_kv_indptr[0]) > 2048
    q, k, v = _attn_inputs(batch, gpu, G, 128, 11)
    o = dense_decode_attention(q, k, v, ic)
    exp = O.paged_decode_attention(_bits(q), _bits(k), _bits(v), _np(ic.dense_kv_indptr), _np(ic.dense_kv_indices),
                                   _np(ic.kv_last_page_len), batch.batch, batch.num_kv_heads, 1.0 / np.sqrt(128))
    np.testing.assert_allclose(_f(_bits(o)), _f(exp), rtol=1e-2, atol=1e-3)


def test_sparse_attention_equals_dense_when_budget_covers_all(gpu):
    """With a budget no smaller than any request, the sparse table is the
    dense one and so is the attention, bit for bit."""
    from vortex_torch.decode_attention import dense_decode_attention, sparse_decode_attention
    from vortex_torch.indexer.utils_sglang import plan_decode

    batch = W.c1()
    batch.topk = 300  # 256 pages per request < topk + bos + eos
    ic, _ = W.make_contexts(batch, gpu)
    b = batch.to(gpu)
    plan_decode(b.seq_lens, b.req_to_token, b.req_indices, ic)
    q, k, v = _attn_inputs(batch, gpu, 2, 128, 9)
    assert torch.equal(sparse_decode_attention(q, k, v, ic), dense_decode_attention(q, k, v, ic))
