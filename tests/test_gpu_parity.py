"""GPU parity of the gfx950 kernels against the CPU oracle.

Integer outputs (block tables, workload list, top-k selections, CMax/CMin)
must be bit-exact; floating outputs (GeMV scores, CMean, CL2Norm) must be
within rtol 1e-2 / atol 1e-3 of the oracle (fp32-accurate accumulation,
bf16 inputs).  Top-k is compared on the same score tensor.
Every call goes through the C ABI of libvortex_hip.so.
"""
import numpy as np
import pytest
import torch

import workloads as W
from oracle import vortex_oracle as O
from vortex_torch import _hip

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-2, 1e-3


def _np(t):
    return t.detach().cpu().numpy()


def _bits(t):
    return _np(t.contiguous().view(torch.int16)).view(np.uint16)


def plan_on_gpu(batch: W.DecodeBatch, dev, sentinel=-7):
    b = batch.to(dev)
    B, H = batch.batch, batch.num_kv_heads
    i32 = dict(dtype=torch.int32, device=dev)
    out = {
        "dense_indptr": torch.full((B * H + 1,), sentinel, **i32),
        "dense_indices": torch.full((max(1, batch.dense_capacity()),), sentinel, **i32),
        "sparse_indptr": torch.full((B * H + 1,), sentinel, **i32),
        "sparse_indices": torch.full((max(1, batch.sparse_capacity()),), sentinel, **i32),
        "kv_last_page_len": torch.full((max(1, B * H),), sentinel, **i32),
        "winfo_q": torch.full((batch.workload_capacity() + 1,), sentinel, **i32),
        "winfo_off": torch.full((batch.workload_capacity() + 1,), sentinel, **i32),
        "winfo_len": torch.full((batch.workload_capacity() + 1,), sentinel, **i32),
        "num_workloads": torch.full((1,), sentinel, **i32),
        "chunk_size": torch.full((1,), sentinel, **i32),
    }
    _hip.plan_decode(b.seq_lens, out["dense_indptr"], out["dense_indices"], out["sparse_indptr"],
                     out["sparse_indices"], out["kv_last_page_len"], b.req_to_token, b.req_indices,
                     out["winfo_q"], out["winfo_off"], out["winfo_len"], out["num_workloads"],
                     out["chunk_size"], batch.page_size, H, batch.topk, batch.bos, batch.eos,
                     batch.max_chunk, batch.min_chunk)
    return out


def plan_oracle(batch: W.DecodeBatch):
    return O.plan_decode(_np(batch.seq_lens), _np(batch.req_to_token), _np(batch.req_indices),
                         batch.page_size, batch.num_kv_heads, batch.topk, batch.bos, batch.eos,
                         batch.max_chunk)


def assert_plan_equal(g, ref, sentinel=-7):
    BH1 = ref["dense_indptr"].shape[0]
    np.testing.assert_array_equal(_np(g["dense_indptr"])[:BH1], ref["dense_indptr"])
    np.testing.assert_array_equal(_np(g["sparse_indptr"])[:BH1], ref["sparse_indptr"])
    nd = ref["dense_indices"].shape[0]
    np.testing.assert_array_equal(_np(g["dense_indices"])[:nd], ref["dense_indices"])
    sp = _np(g["sparse_indices"])[:ref["sparse_indices"].shape[0]]
    w = ref["sparse_written"]
    np.testing.assert_array_equal(sp[w], ref["sparse_indices"][w])
    assert (sp[~w] == sentinel).all(), "planner wrote the top-k slots"
    BH = BH1 - 1
    if BH:
        np.testing.assert_array_equal(_np(g["kv_last_page_len"])[:BH], ref["kv_last_page_len"])
    nw = ref["num_workloads"]
    assert int(g["num_workloads"].item()) == nw
    assert int(g["chunk_size"].item()) == ref["chunk_size"]
    np.testing.assert_array_equal(_np(g["winfo_q"])[:nw], ref["winfo_q"])
    np.testing.assert_array_equal(_np(g["winfo_off"])[:nw], ref["winfo_off"])
    np.testing.assert_array_equal(_np(g["winfo_len"])[:nw], ref["winfo_len"])
    assert (_np(g["winfo_q"])[nw:] == sentinel).all()


# ------------------------------------------------------------------ planner
@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c5"])
def test_plan_configs(gpu, name):
    batch = getattr(W, name)()
    assert_plan_equal(plan_on_gpu(batch, gpu), plan_oracle(batch))


@pytest.mark.parametrize("seed", range(12))
def test_plan_random_small(gpu, seed):
    batch = W.random_small(seed)
    assert_plan_equal(plan_on_gpu(batch, gpu), plan_oracle(batch))


def test_plan_large_batch(gpu):
    # beyond the reference planner's limits (1024 requests, 8192 segments)
    g = torch.Generator().manual_seed(11)
    lens = torch.randint(0, 700, (1500,), generator=g)
    batch = W.make_batch(lens, pool_pages=int(((lens + 15) // 16).sum()) + 5, seed=11, num_kv_heads=8,
                         topk=8, bos=1, eos=2)
    assert_plan_equal(plan_on_gpu(batch, gpu), plan_oracle(batch))


def test_plan_empty_batch(gpu):
    batch = W.make_batch([], pool_pages=4, seed=3)
    g = plan_on_gpu(batch, gpu)
    assert int(g["dense_indptr"][0]) == 0 and int(g["sparse_indptr"][0]) == 0
    assert int(g["num_workloads"].item()) == 0


# ------------------------------------------------------------------ top-k
def topk_case(batch, dev, scores_bits_np, max_pages=None):
    ref_plan = plan_oracle(batch)
    g = plan_on_gpu(batch, dev)
    sc = torch.from_numpy(scores_bits_np.view(np.int16)).to(dev).view(torch.bfloat16)
    eff = batch.batch * batch.num_kv_heads
    mp = batch.max_pages_per_request if max_pages is None else max_pages
    _hip.topk_select(sc, g["dense_indptr"], g["sparse_indptr"], g["dense_indices"], g["sparse_indices"],
                     eff, batch.topk, batch.bos, batch.eos, mp)
    exp, written = O.topk(scores_bits_np, ref_plan["dense_indptr"], ref_plan["sparse_indptr"],
                          ref_plan["dense_indices"], ref_plan["sparse_indices"], eff, batch.topk,
                          batch.bos, batch.eos)
    got = _np(g["sparse_indices"])[:exp.shape[0]]
    mask = written | ref_plan["sparse_written"]
    np.testing.assert_array_equal(got[mask], exp[mask])
    assert mask.all(), "every sparse slot is filled after plan + top-k"
    return got


def _random_scores(n, seed, kind):
    rng = np.random.default_rng(seed)
    if kind == "normal":
        v = rng.standard_normal(n).astype(np.float32) * 2.0
    elif kind == "ties":
        v = rng.integers(-3, 4, n).astype(np.float32) * 0.5
    elif kind == "zeros":
        v = np.where(rng.random(n) < 0.5, -0.0, 0.0).astype(np.float32)
        v[rng.random(n) < 0.1] = 1.0
    elif kind == "const":
        v = np.full(n, 0.25, dtype=np.float32)
    else:
        raise ValueError(kind)
    return O.f32_to_bf16(v)


@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c5"])
@pytest.mark.parametrize("kind", ["normal", "ties"])
def test_topk_configs(gpu, name, kind):
    batch = getattr(W, name)()
    n = batch.dense_capacity()
    topk_case(batch, gpu, _random_scores(n, 5, kind))


@pytest.mark.parametrize("seed", range(10))
@pytest.mark.parametrize("kind", ["normal", "ties", "zeros", "const"])
def test_topk_random_small(gpu, seed, kind):
    batch = W.random_small(100 + seed)
    n = max(1, batch.dense_capacity())
    topk_case(batch, gpu, _random_scores(n, seed, kind))


def test_topk_streaming_path(gpu):
    # max_num_pages smaller than the segments forces the global-memory path
    batch = W.c3()
    n = batch.dense_capacity()
    topk_case(batch, gpu, _random_scores(n, 9, "ties"), max_pages=64)


def test_topk_large_k(gpu):
    batch = W.make_batch([16 * 3000, 16 * 900, 77], pool_pages=4000, seed=21, num_kv_heads=2,
                         topk=1000, bos=2, eos=3)
    n = batch.dense_capacity()
    topk_case(batch, gpu, _random_scores(n, 3, "ties"))
    topk_case(batch, gpu, _random_scores(n, 4, "normal"))


# ------------------------------------------------------------------ GeMV
def gemv_case(batch, dev, seed=0, std=1.0):
    g = plan_on_gpu(batch, dev)
    ref_plan = plan_oracle(batch)
    H, D = batch.num_kv_heads, batch.head_dim
    x = W.randn_bf16((batch.batch * H, 1, D), seed, dev)
    y = W.randn_bf16((batch.pool_pages * H, 1, D), seed + 1, dev, std=std)
    o = torch.full((max(1, batch.dense_capacity()), 1, 1), -3.0, device=dev, dtype=torch.bfloat16)
    _hip.gemv_paged(x, y, o, g["dense_indices"], g["winfo_q"], g["winfo_off"], g["winfo_len"],
                    g["num_workloads"], batch.max_chunk)
    exp, cov = O.gemv(_bits(x), _bits(y), ref_plan["dense_indices"], ref_plan["winfo_q"],
                      ref_plan["winfo_off"], ref_plan["winfo_len"], ref_plan["num_workloads"],
                      o.numel())
    got = O.bf16_to_f32(_bits(o).reshape(-1))
    np.testing.assert_allclose(got[cov], O.bf16_to_f32(exp)[cov], rtol=RTOL, atol=ATOL)
    assert (got[~cov] == -3.0).all(), "GeMV wrote outside the workloads"
    return got, cov


@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c5"])
def test_gemv_configs(gpu, name):
    gemv_case(getattr(W, name)(), gpu)


@pytest.mark.parametrize("seed", range(8))
def test_gemv_random_small(gpu, seed):
    gemv_case(W.random_small(200 + seed), gpu, seed)


@pytest.mark.parametrize("dim", [64, 256, 512, 96, 100])
def test_gemv_head_dims(gpu, dim):
    batch = W.make_batch([16 * 70, 16 * 33 + 5, 300], pool_pages=200, seed=31, num_kv_heads=2,
                         head_dim=dim, topk=4, bos=1, eos=1, max_chunk=48)
    gemv_case(batch, gpu, seed=dim)


# ------------------------------------------------------------------ page reduce
def reduce_case(dev, rows_pages, H, R, C, loc, rtype, dim=1, out_dtype=torch.bfloat16, seed=0):
    x = W.randn_bf16((rows_pages * H, R, C), seed, dev)
    oshape = (rows_pages * H, 1, C) if dim == 1 else (rows_pages * H, R, 1)
    out = torch.full(oshape, 7.0, device=dev, dtype=out_dtype)
    loc_t = torch.as_tensor(loc, dtype=torch.int64, device=dev)
    _hip.page_reduce(x, out, loc_t, H, R, dim, rtype)
    init = np.full(oshape, 7.0, dtype=np.float32)
    if out_dtype == torch.bfloat16:
        init = O.f32_to_bf16(init)
    exp, rows = O.page_reduce(_bits(x), init, np.asarray(loc, dtype=np.int64), H, R, dim, rtype)
    got = _bits(out) if out_dtype == torch.bfloat16 else _np(out)
    if out_dtype == torch.bfloat16:
        got_f, exp_f = O.bf16_to_f32(got), O.bf16_to_f32(exp)
    else:
        got_f, exp_f = got, exp
    if rtype in (O.MAX, O.MIN):
        np.testing.assert_array_equal(got_f, exp_f)
    else:
        np.testing.assert_allclose(got_f, exp_f, rtol=RTOL, atol=ATOL)
    return x, out, rows


def _burst_loc(n_pages_pool, n_pages, P, seed):
    rng = np.random.default_rng(seed)
    pages = rng.permutation(n_pages_pool)[:n_pages]
    loc = (pages[:, None] * P + np.arange(P)[None, :]).reshape(-1)
    return rng.permutation(loc)


@pytest.mark.parametrize("rtype", [O.MEAN, O.MAX, O.MIN, O.L2NORM])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_reduce_types(gpu, rtype, out_dtype):
    loc = _burst_loc(300, 120, 16, 1)
    reduce_case(gpu, 300, 8, 16, 128, loc, rtype, out_dtype=out_dtype)


@pytest.mark.parametrize("R,C", [(16, 64), (16, 256), (16, 512), (16, 576), (8, 128), (16, 100), (5, 40)])
def test_reduce_shapes(gpu, R, C):
    loc = _burst_loc(50, 20, R, 2)
    reduce_case(gpu, 50, 2, R, C, loc, O.MEAN)
    reduce_case(gpu, 50, 2, R, C, loc, O.MAX)


@pytest.mark.parametrize("rtype", [O.MEAN, O.MAX, O.L2NORM])
def test_reduce_dim2(gpu, rtype):
    loc = _burst_loc(40, 15, 16, 3)
    reduce_case(gpu, 40, 4, 16, 128, loc, rtype, dim=2)


def test_reduce_decode_loc(gpu):
    # decode step: one new token per request, a few of them close a page
    batch = W.c2()
    P = batch.page_size
    loc = []
    for b in range(batch.batch):
        L = int(batch.seq_lens[b])
        j = L - 1
        loc.append(int(batch.pages[b][j // P]) * P + j % P)
    reduce_case(gpu, batch.pool_pages, 8, 16, 128, loc, O.MEAN)


def test_reduce_multi_matches_single(gpu):
    dev = gpu
    loc = torch.as_tensor(_burst_loc(500, 300, 16, 4), device=dev)
    x = W.randn_bf16((500 * 8, 16, 128), 5, dev)
    outs_single, outs_multi = [], []
    types = [O.MEAN, O.MAX, O.MIN, O.L2NORM]
    for i, t in enumerate(types):
        dt = torch.bfloat16 if i % 2 == 0 else torch.float32
        a = torch.zeros((500 * 8, 1, 128), device=dev, dtype=dt)
        b = torch.zeros_like(a)
        _hip.page_reduce(x, a, loc, 8, 16, 1, t)
        outs_single.append(a)
        outs_multi.append(b)
    _hip.page_reduce_multi(x, outs_multi, types, loc, 8, 16, 1)
    for a, b in zip(outs_single, outs_multi):
        assert torch.equal(a, b)


def test_reduce_negative_and_out_of_range_loc(gpu):
    # C semantics: loc = -1 closes "page 0"; rows beyond the pool are skipped
    loc = [-1, 15, 16 * 49 + 15, 16 * 1000 + 15]
    reduce_case(gpu, 50, 2, 16, 128, loc, O.MAX)


def _f32_bits_to_bf16(a):
    """fp32 array -> bf16 bits, round to nearest even (no NaNs here)."""
    u = a.astype(np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


@pytest.mark.parametrize("C", [64, 128, 256, 512])
@pytest.mark.parametrize("R", [1, 3, 16, 24])
def test_reduce_row_group_order_bits(gpu, C, R):
    """The dim-1 CMean's fp32 summation order, bit for bit, for both tile
    layouts of the page-reduce kernel (one lane per column vector for tiles of
    up to 16 rows, row groups folded by a shuffle tree above that): rows are
    split into G = 512 / C groups (group g: rows g, g + G, ... in order, from
    0.0), the groups folded pairwise ((0 + 1) + (2 + 3)) + ..., divided by R
    and rounded to bf16.  The in-launch decode CMean of the fused indexer uses
    the same order (test_gpu_flow compares it with this launch bit for bit)."""
    dev = gpu
    H, n_pool, n_pages = 2, 40, 25
    loc = torch.as_tensor(_burst_loc(n_pool, n_pages, R, 7), device=dev)
    x = W.randn_bf16((n_pool * H, R, C), 11, dev)
    out = torch.full((n_pool * H, 1, C), 7.0, device=dev, dtype=torch.bfloat16)
    out2 = torch.full((n_pool * H, 1, C), 7.0, device=dev, dtype=torch.bfloat16)
    _hip.page_reduce(x, out, loc, H, R, 1, _hip.REDUCE_MEAN)
    _hip.page_reduce_multi(x, [out2], [O.MEAN], loc, H, R, 1)
    torch.cuda.synchronize()
    xf = _np(x.float()).astype(np.float32)  # [rows, R, C]
    G = 512 // C

    def fold(lo, hi):
        if hi - lo == 1:
            acc = np.zeros((xf.shape[0], C), np.float32)
            for r in range(lo, R, G):
                acc = (acc + xf[:, r, :]).astype(np.float32)
            return acc
        mid = (lo + hi) // 2
        return (fold(lo, mid) + fold(mid, hi)).astype(np.float32)

    mean = (fold(0, G) / np.float32(R)).astype(np.float32)
    expect = _f32_bits_to_bf16(mean)
    closed = sorted({int(v) // R for v in _np(loc) if (int(v) + 1) % R == 0})
    rows = np.array([p * H + h for p in closed for h in range(H)])
    got = _bits(out)[:, 0, :]
    np.testing.assert_array_equal(got[rows], expect[rows])
    np.testing.assert_array_equal(_bits(out2)[:, 0, :][rows], expect[rows])
    untouched = np.setdiff1d(np.arange(n_pool * H), rows)
    assert (got[untouched] == _bits(torch.tensor(7.0, dtype=torch.bfloat16))).all()


def test_reduce_c4_burst_full_size(gpu):
    """C4 at full size: 65,536 pages (1,048,576 loc entries) of a 70k-page pool,
    CMean + CMax in one pass.  CMax must equal torch.amax of the same tiles
    bit for bit, CMean torch's fp32 mean within tolerance; rows of pages that
    did not close keep their contents; an fp32 CMean output holds the same
    bf16-rounded values.  A sample of pages is also checked against the oracle."""
    dev = gpu
    case = W.c4()
    H, P, D = case.num_kv_heads, case.page_size, case.head_dim
    x = W.randn_bf16((case.pool_pages * H, P, D), 3, dev)
    loc = case.loc.to(dev)
    cm = torch.full((case.pool_pages * H, 1, D), 7.0, device=dev, dtype=torch.bfloat16)
    cx = torch.full_like(cm, 7.0)
    _hip.page_reduce_multi(x, [cm, cx], [O.MEAN, O.MAX], loc, H, P, 1)
    cm32 = torch.full(cm.shape, 7.0, device=dev, dtype=torch.float32)
    _hip.page_reduce(x, cm32, loc, H, P, 1, O.MEAN)

    rows = (case.pages.to(dev)[:, None] * H + torch.arange(H, device=dev)[None, :]).reshape(-1)
    tiles = x[rows]
    assert torch.equal(cx[rows], tiles.amax(dim=1, keepdim=True)), "CMax differs from torch.amax"
    exp_mean = tiles.float().mean(dim=1, keepdim=True)
    del tiles
    torch.testing.assert_close(cm[rows].float(), exp_mean, rtol=RTOL, atol=ATOL)
    assert torch.equal(cm32[rows], cm[rows].float()), "fp32 CMean output is not the bf16-rounded mean"
    closed = torch.zeros(case.pool_pages * H, dtype=torch.bool, device=dev)
    closed[rows] = True
    for out in (cm, cx, cm32):
        assert bool((out[~closed] == 7.0).all()), "a row of an unfinished page was written"

    # oracle on a sample of 64 pages, through a compact copy of their tiles
    sample = case.pages[:64]
    srows = (sample[:, None] * H + torch.arange(H)[None, :]).reshape(-1)
    xs = _bits(x[srows.to(dev)]).reshape(len(srows), P, D)
    sloc = np.arange(len(sample)) * P + (P - 1)
    for out, rtype in ((cm, O.MEAN), (cx, O.MAX)):
        exp, _ = O.page_reduce(xs, np.zeros((len(srows), 1, D), np.uint16), sloc, H, P, 1, rtype)
        got = _bits(out[srows.to(dev)]).reshape(len(srows), 1, D)
        if rtype == O.MAX:
            np.testing.assert_array_equal(got, exp)
        else:
            np.testing.assert_allclose(O.bf16_to_f32(got), O.bf16_to_f32(exp), rtol=RTOL, atol=ATOL)
